/*
 * diagpu.h -- C ABI of the MI355X (gfx950) diagonal-format sparse kernels.
 *
 * Every entry point:
 *   - takes plain pointers and sizes (device pointers unless marked "host"),
 *     a HIP stream as void* (NULL = the default stream);
 *   - returns 0 (DIAGPU_OK) or a DIAGPU_ERR_* code, never exits; the text of
 *     the last failure on the calling thread is in diagpu_last_error();
 *   - validates its host-visible arguments before any HIP call, so argument
 *     errors are reported without touching the GPU;
 *   - is asynchronous on `stream` unless stated otherwise, allocates nothing
 *     and takes no ownership: the caller allocates and frees every buffer.
 *
 * Layouts (all square n x n for SpGEMM; rows x cols for SpMV):
 *   Recon      K x cols row-major, Recon[k][c] = H[c - d_k, c], rows sorted by
 *              offset descending (spmv/src/dia_reconstruct.cuh:9-17).
 *   HM         compact concatenation; diagonal d has length n - |d|, element
 *              (i, j) sits at position min(i, j) from starts[k]
 *              (spmspm/paper_hm.cuh:18-37, spmspm/bench_spmspm.cu:74-86).
 *   row-packed P x n, DA[i][t] = A[t, t + d_i], zero outside the diagonal
 *              (gemm_diag/gemm_diag.cu:9-15, 362-382).
 * Element starts are int64 everywhere (the reference's int starts overflow
 * for C outputs above 2^31 elements).
 */
#ifndef DIAGPU_H
#define DIAGPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DIAGPU_API __attribute__((visibility("default")))

enum {
    DIAGPU_OK            = 0,
    DIAGPU_ERR_ARG       = 1,  /* NULL pointer, negative size, bad flag          */
    DIAGPU_ERR_OFFSET    = 2,  /* |offset| >= n or length != n - |offset|        */
    DIAGPU_ERR_DUPLICATE = 3,  /* repeated diagonal offset in one operand        */
    DIAGPU_ERR_OVERFLOW  = 4,  /* an index or count exceeds its integer type     */
    DIAGPU_ERR_CAPACITY  = 5,  /* output capacity or workspace too small         */
    DIAGPU_ERR_HIP       = 6   /* HIP runtime error (launch, copy, sync)          */
};

/* Text of the last error on this thread ("" if none). */
DIAGPU_API const char* diagpu_last_error(void);
/* Static name of a status code. */
DIAGPU_API const char* diagpu_status_name(int status);
/* ABI version: major * 10000 + minor * 100 + patch. */
DIAGPU_API int diagpu_abi_version(void);

/* ======================================================================
 * SpMV on the Recon layout
 * ====================================================================== */

/* Non-owning device view of a Recon matrix.  Same members, order and types
 * as ReconView (spmv/src/dia_reconstruct.cuh:112-118), so a ReconView can be
 * passed by address. */
typedef struct diagpu_recon_view_f32 {
    int32_t        rows;
    int32_t        cols;
    int32_t        num_diags;
    const int32_t* diag_offsets;   /* device [num_diags]             */
    const float*   values;         /* device [num_diags * cols]      */
} diagpu_recon_view_f32;

typedef struct diagpu_recon_view_f64 {
    int32_t        rows;
    int32_t        cols;
    int32_t        num_diags;
    const int32_t* diag_offsets;
    const double*  values;
} diagpu_recon_view_f64;

/* Complex fp32 element (interleaved real, imaginary): the layout of
 * std::complex<float>, numpy complex64 and torch.complex64. */
typedef struct diagpu_complex64 {
    float re, im;
} diagpu_complex64;

typedef struct diagpu_recon_view_c64 {
    int32_t                 rows;
    int32_t                 cols;
    int32_t                 num_diags;
    const int32_t*          diag_offsets;
    const diagpu_complex64* values;
} diagpu_recon_view_c64;

/* y[r] = sum_k [0 <= r + d_k < min(cols, x_size)] Recon[k][r + d_k] * x[r + d_k]
 * for 0 <= r < rows; y is overwritten (beta = 0); rows == 0 is a successful
 * no-op.  Offsets may be in any order and out of range (such terms drop).
 * fp32 operands with fp32 accumulation (the reference rounds operands to
 * TF32 first; this path keeps full fp32).  x and y must not overlap.
 * Replaces launch_tc_spmv_regdirect (spmv/src/dia_reconstruct.cuh:139-144,
 * spmv/src/tc_spmv_regdirect_kernel.cu:135-147). */
DIAGPU_API int diagpu_spmv_recon_f32(const diagpu_recon_view_f32* R, const float* x,
                                     int64_t x_size, float* y, void* stream);

/* fp64 variant of diagpu_spmv_recon_f32 (no reference counterpart: the
 * reference is fp32/TF32 only; benchmark config 2 asks for fp64). */
DIAGPU_API int diagpu_spmv_recon_f64(const diagpu_recon_view_f64* R, const double* x,
                                     int64_t x_size, double* y, void* stream);

/* Complex Hamiltonians.  The reference kernels are real fp32 only, while the
 * physics they serve applies a complex H to a complex state
 * (slides/transcript.md:10-18, "H is an N-by-N complex Hamiltonian").
 * Same sum and bounds as diagpu_spmv_recon_f32, complex products,
 * fp32 accumulation of each part:
 *   _c64      complex64 Recon values, complex64 x and y;
 *   _f32_c64  real fp32 Recon values, complex64 x and y (a real H applied to
 *             a complex state; the values are read once for both parts). */
DIAGPU_API int diagpu_spmv_recon_c64(const diagpu_recon_view_c64* R, const diagpu_complex64* x,
                                     int64_t x_size, diagpu_complex64* y, void* stream);
DIAGPU_API int diagpu_spmv_recon_f32_c64(const diagpu_recon_view_f32* R,
                                         const diagpu_complex64* x, int64_t x_size,
                                         diagpu_complex64* y, void* stream);

/* ======================================================================
 * Krylov propagator: psi(t) = exp(-i t H) psi_0 (Lanczos)
 * ====================================================================== */

/* The matrix-free caller of the SpMV path (slides/transcript.md:10-18: one
 * trajectory, H applied to the state again and again, "exactly what
 * Krylov-subspace methods do"); the reference ships no driver for it. */
typedef struct diagpu_krylov_info {
    int32_t steps;         /* Lanczos steps used (m, fewer on breakdown)          */
    int32_t breakdown;     /* 1: an invariant subspace was reached (exact result)  */
    double  psi0_norm;     /* ||psi_0||                                            */
    double  err_estimate;  /* ||psi_0|| * beta_m * |[exp(-i t T_m)]_{m,1}|, 0 on
                              breakdown                                            */
} diagpu_krylov_info;

/* Device workspace (bytes, host out) for n x n H and m Lanczos steps:
 * m basis vectors of n complex64 plus O(n / 512) reduction scratch. */
DIAGPU_API int diagpu_expm_krylov_workspace(int32_t n, int32_t m, size_t* bytes);

/* psi_t = exp(-i t H) psi_0 for Hermitian H (n x n Recon, rows == cols; only
 * H's action is used, Hermitian symmetry is the caller's promise), complex64
 * psi_0 and psi_t of n elements, 1 <= m <= 64 Lanczos steps.  Two kernels per
 * step (SpMV with a fused dot product, three-term update with a fused norm),
 * deterministic fp64 reductions, scalars kept on the device; one stream
 * synchronisation after the m steps to read alpha and beta, then exp(-i t T_m)
 * e_1 on the host in fp64 and one combine kernel (async on `stream`).
 * host_scratch (optional) is a pinned host buffer (hipHostMalloc) of at least
 * 2m+1 doubles for that readback; with NULL the copy goes through pageable
 * memory, which the HIP runtime stages (tens of microseconds more per call).
 * alpha and beta (host, m entries each, optional) receive T_m's diagonal and
 * off-diagonal (zero past info->steps).  psi_t must not overlap psi_0 or the
 * workspace.
 *   _c64  complex64 Recon values;  _f32  real fp32 Recon values (real
 *         symmetric H) applied to the complex state. */
DIAGPU_API int diagpu_expm_krylov_c64(const diagpu_recon_view_c64* H,
                                      const diagpu_complex64* psi0, double t, int32_t m,
                                      diagpu_complex64* psi_t, void* workspace,
                                      size_t workspace_bytes, double* host_scratch,
                                      double* alpha, double* beta, diagpu_krylov_info* info,
                                      void* stream);
DIAGPU_API int diagpu_expm_krylov_f32(const diagpu_recon_view_f32* H,
                                      const diagpu_complex64* psi0, double t, int32_t m,
                                      diagpu_complex64* psi_t, void* workspace,
                                      size_t workspace_bytes, double* host_scratch,
                                      double* alpha, double* beta, diagpu_krylov_info* info,
                                      void* stream);

/* ======================================================================
 * DIA x DIA SpGEMM, HM layout: C = A * B
 * ====================================================================== */

/* One entry of the pair plan: C[k][p] += Av[ab + p + ash] * Bv[bb + p + bsh]
 * for positions with 0 <= p + ash < al and 0 <= p + bsh < bl.  Same layout as
 * GPair (spmspm/gather_flat.cuh:21): {size_t ab, bb; int ash, bsh, al, bl}. */
typedef struct diagpu_gpair {
    uint64_t ab, bb;
    int32_t  ash, bsh, al, bl;
} diagpu_gpair;

/* Result counts of the symbolic phase (written to host memory). */
typedef struct diagpu_spgemm_info {
    int64_t c_ndiag;         /* number of C diagonals                       */
    int64_t c_nnz;           /* sum of C lengths = C value count            */
    int64_t n_pairs;         /* number of pair-plan entries                 */
    int64_t max_pairs;       /* largest pair count of one C diagonal        */
    int64_t useful_flops;    /* 2 * sum over pairs of the overlap length    */
    int64_t a_extent;        /* values A_vals must hold: max(start + length) */
    int64_t b_extent;        /* values B_vals must hold                     */
} diagpu_spgemm_info;

/* Device workspace the symbolic phase needs for dimension n and operand
 * diagonal counts a_ndiag, b_ndiag (bytes, host out).  Capacities the caller
 * must provide: C arrays min(a_ndiag * b_ndiag, 2n - 1) entries (+1 for
 * pair_ptr), pairs a_ndiag * b_ndiag entries. */
DIAGPU_API int diagpu_spgemm_symbolic_workspace(int32_t n, int32_t a_ndiag, int32_t b_ndiag,
                                                size_t* bytes);

/* Symbolic (integer) phase, bit-exact with the reference host planners:
 *   C offsets  = every da + db with |da + db| < n, ascending, once each
 *                (make_c_structure, spmspm/bench_spmspm.cu:109-131;
 *                 compute_c_hm_structure, spmspm/paper_hm.cuh:87-117);
 *   C lengths  = n - |dc|; C starts = exclusive prefix sum of the lengths;
 *   c_lookup   = dc + n - 1 -> C index, -1 where absent (optional, 2n - 1
 *                entries; build_c_diag_lookup, spmspm/paper_hm.cuh:121-130);
 *   pair plan  = per C diagonal in order, per B diagonal in B's order, the A
 *                diagonal with da = dc - db if present, as GPair
 *                (build_pairs_only, spmspm/gather_flat.cuh:231-255);
 *                pair_ptr has c_ndiag + 1 entries.
 * Operand offsets may be in any order but must be distinct with |d| < n, and
 * lengths must equal n - |d| (DIAGPU_ERR_DUPLICATE / DIAGPU_ERR_OFFSET).
 * Synchronises `stream` and writes *info (host), including the value
 * extents max(start + length) of A and B (how many values A_vals and B_vals
 * must hold for the numeric phase).  Operand values are not read. */
DIAGPU_API int diagpu_spgemm_symbolic(
    int32_t n,
    const int32_t* A_off, const int32_t* A_len, const int64_t* A_starts, int32_t a_ndiag,
    const int32_t* B_off, const int32_t* B_len, const int64_t* B_starts, int32_t b_ndiag,
    int32_t* C_off, int32_t* C_len, int64_t* C_starts, int64_t c_capacity,
    int64_t* pair_ptr, diagpu_gpair* pairs, int64_t pair_capacity,
    int32_t* c_lookup,
    void* workspace, size_t workspace_bytes,
    diagpu_spgemm_info* info, void* stream);

/* diagpu_spgemm_symbolic without the workspace argument: for callers that
 * cannot allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The workspace is a
 * file-scope device array of DIAGPU_SYMBOLIC_SCRATCH_BYTES that each GPU
 * holds until the process ends; a problem whose workspace
 * (diagpu_spgemm_symbolic_workspace) is larger is rejected with
 * DIAGPU_ERR_CAPACITY before any GPU work (n up to about 4.7 million fits
 * for any diagonal counts).  Same arguments, outputs and errors as
 * diagpu_spgemm_symbolic otherwise; allocates nothing.  Like that call it
 * reads the counts back to the host with a synchronous copy on `stream`, so
 * it cannot be recorded into a HIP graph.  Every call on one GPU shares that
 * GPU's array: calls that overlap in one process (other host threads, other
 * streams) are serialised by a per-device lock held until the call's stream
 * has drained; each call re-initialises what it reads. */
#define DIAGPU_SYMBOLIC_SCRATCH_BYTES (40u << 20)
DIAGPU_API int diagpu_spgemm_symbolic_noalloc(
    int32_t n,
    const int32_t* A_off, const int32_t* A_len, const int64_t* A_starts, int32_t a_ndiag,
    const int32_t* B_off, const int32_t* B_len, const int64_t* B_starts, int32_t b_ndiag,
    int32_t* C_off, int32_t* C_len, int64_t* C_starts, int64_t c_capacity,
    int64_t* pair_ptr, diagpu_gpair* pairs, int64_t pair_capacity,
    int32_t* c_lookup, diagpu_spgemm_info* info, void* stream);

/* Numeric phase: C_vals[C_starts[k] + p] = sum over the plan entries of C
 * diagonal k (fp32 products, fp32 accumulation in plan order), for every
 * 0 <= p < C_len[k]; every C value is written exactly once (no atomics, no
 * pre-zeroing needed).  The shifted multiply-accumulate of
 * hm_structured_sparse_matmul_kernel (spmspm/paper_hm_kernel.cu:31-93) and
 * of the gather kernels (spmspm/spmspm.cu:196-319,
 * spmspm/gather_flat.cuh:23-64), computed from the plan of
 * diagpu_spgemm_symbolic.  c_ndiag and max_pairs come from its info. */
DIAGPU_API int diagpu_spgemm_numeric_f32(
    int32_t n, const float* A_vals, const float* B_vals,
    const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
    const int64_t* pair_ptr, const diagpu_gpair* pairs, int64_t max_pairs,
    float* C_vals, void* stream);

/* Complex64 variant of diagpu_spgemm_numeric_f32 for complex Hamiltonians
 * (the reference is real only): the same plan, complex products, fp32
 * accumulation of each part, same write-once semantics. */
DIAGPU_API int diagpu_spgemm_numeric_c64(
    int32_t n, const diagpu_complex64* A_vals, const diagpu_complex64* B_vals,
    const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
    const int64_t* pair_ptr, const diagpu_gpair* pairs, int64_t max_pairs,
    diagpu_complex64* C_vals, void* stream);

/* ----------------------------------------------------------------------
 * Narrow bands: the numeric phase with the operands staged in LDS
 * ---------------------------------------------------------------------- */

/* What diagpu_spgemm_band_prepare found out about a plan. */
typedef struct diagpu_band_info {
    int32_t a_off_min, a_off_max;   /* smallest and largest A offset          */
    int32_t rows_per_block;         /* rows one workgroup stages (rpb)         */
    int32_t eligible;               /* 1: the staged operands fit in LDS       */
                                    /* (lds_bytes <= 64 KiB)                   */
    int64_t lds_bytes;              /* per workgroup: 4 (nA rpb + nB wb) +     */
                                    /* 16 n_pairs, wb = rpb + span rounded up  */
                                    /* to a multiple of 4                      */
    int64_t n_pairs;                /* plan entries                            */
    int32_t b_off_min, b_off_max;   /* smallest and largest B offset          */
    int32_t mfma_blocks;            /* MFMA variant: 16x16x4 fp32 blocks       */
                                    /* issued per 16-row tile of C (issued     */
                                    /* flops = 2048 * mfma_blocks * 4 *        */
                                    /* ceil(n / 64): 4 tiles per 64-row slab)  */
    int32_t mfma_eligible;          /* 1: the MFMA variant takes the plan      */
    int64_t mfma_lds_bytes;         /* its LDS per workgroup                   */
} diagpu_band_info;

/* For the band kernel, per plan (once): entries[4g .. 4g+3] = {a rpb,
 * b wb + (da - min da), da, 0} for plan entry g, a and b the
 * indices of its A and B diagonals (looked up from the entry's starts), and
 * A's and B's offset spans, and the MFMA variant's geometry, in *info.
 * entries holds 4 n_pairs + 8 int32 (the last 8 are scratch).  One stream
 * synchronisation (to return *info).
 * DIAGPU_ERR_OFFSET if an A offset lies outside (-n, n); DIAGPU_ERR_ARG if an
 * entry's starts are not the starts of an A and a B diagonal, or if its
 * ash, bsh, al, bl differ from what diagpu_spgemm_symbolic writes for those
 * two diagonals (the band kernel computes each term's shifts and bounds from
 * the operand offsets, so it takes only such plans).  No reference
 * counterpart: the LDS-tiled form of the numeric phase below. */
DIAGPU_API int diagpu_spgemm_band_prepare(int32_t n, const int32_t* A_off,
                                          const int64_t* A_starts, int32_t nA,
                                          const int32_t* B_off, const int64_t* B_starts,
                                          int32_t nB,
                                          const diagpu_gpair* pairs, int64_t n_pairs,
                                          int32_t* entries, diagpu_band_info* info,
                                          void* stream);

/* The numeric phase of diagpu_spgemm_numeric_f32 (same C, bit for bit) with
 * each workgroup staging a block of A rows and the matching window of B rows
 * in LDS and evaluating every C diagonal's plan entries from there: for
 * products whose operand runs are used by many entries (narrow bands, e.g.
 * gemm_diag's contiguous offsets).  info must be an eligible band_prepare
 * result for these operands (else DIAGPU_ERR_CAPACITY). */
DIAGPU_API int diagpu_spgemm_numeric_band_f32(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA, const float* A_vals,
    const int32_t* B_off, const int64_t* B_starts, int32_t nB, const float* B_vals,
    const int32_t* C_off, const int64_t* C_starts, int64_t c_ndiag, const int64_t* pair_ptr,
    const int32_t* entries, const diagpu_band_info* info, float* C_vals, void* stream);

/* The numeric phase of diagpu_spgemm_numeric_f32 on the matrix cores, for
 * narrow bands (gemm_diag's contiguous offsets): each 16-row tile of C is the
 * sum of the dense 16 x 16 x 4 fp32 MFMA blocks (v_mfma_f32_16x16x4_f32) that
 * intersect the band, each wave staging the operands of its 64-row slabs in
 * LDS, elements outside the band read as zeros.  Same C to rounding (1e-5 of
 * each element's term sum), not bit for bit: the sums run in MFMA order.
 * Operands must be finite (a dense tile multiplies absent terms by zero).
 * info from diagpu_spgemm_band_prepare with mfma_eligible set (A's offset
 * range at most 32 wide, A's plus B's at most 48), else
 * DIAGPU_ERR_CAPACITY.  C offsets must be the plan's (sums of A's and B's).
 * Never picked by the plan's automatic choice: on gemm_diag's -10..10 band it
 * issues 2.9 times the useful flops and takes about 1.25 times the band
 * kernel's time (on every band from +-4 to +-16 x +-8 as well).  No reference counterpart: the reference's
 * tensor-core kernel is the TF32 SpMV, and gemm_diag/gemm_diag.cu:119-329
 * runs this product on scalar FMAs; this is that product as a dense tile
 * contraction. */
DIAGPU_API int diagpu_spgemm_numeric_band_mfma_f32(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA, const float* A_vals,
    const int32_t* B_off, const int64_t* B_starts, int32_t nB, const float* B_vals,
    const int32_t* C_off, const int64_t* C_starts, int64_t c_ndiag,
    const diagpu_band_info* info, float* C_vals, void* stream);

/* ----------------------------------------------------------------------
 * Medium bands: the numeric phase with A held in LDS
 * ---------------------------------------------------------------------- */

/* Largest A diagonal count diagpu_spgemm_numeric_astat_f32 takes: its
 * workgroups hold 288 rows of every A diagonal in LDS, 160 KiB at most (up to
 * 71 diagonals, 80 KiB, two workgroups share a CU; above, one). */
#define DIAGPU_ASTAT_MAX_A 142
/* The same for diagpu_spgemm_numeric_astat_c64: up to 75 A diagonals its
 * workgroups hold 272 complex rows of each (two workgroups per CU up to 37),
 * above that 144. */
#define DIAGPU_ASTAT_MAX_A_C64 142

/* For the A-stationary kernel, per plan (once): records[4g .. 4g+3] =
 * {a, lo, hi, b} for plan entry g: a the index of its A diagonal (looked up
 * from the entry's A start), [lo, hi) = [max(0, -ash, -bsh), min(al - ash,
 * bl - bsh)) the C positions where both operands hold an element, and
 * b = bb + bsh the B index of C position 0.  records holds 4 n_pairs + 4
 * int32: the last 4 are two error flags and the smallest and largest of A's
 * offsets, which the numeric entry points read.  A_off/A_starts, B_off/B_starts, C_off
 * and pair_ptr (c_ndiag + 1 entries) are the plan's device arrays.  One
 * stream synchronisation (to report errors): DIAGPU_ERR_ARG if an entry is
 * not in the symbolic plan's form (its A or B start is no diagonal's start,
 * da + db is not its C diagonal's offset, or ash, bsh, al, bl differ from
 * min0(da) - min0(dc), da + min0(db) - min0(dc), n - |da|, n - |db|) or if
 * pair_ptr is not a partition of the n_pairs entries,
 * DIAGPU_ERR_CAPACITY if a B index exceeds 2^30 - 1 (the numeric kernels
 * form B byte offsets in 32 bits).  No reference
 * counterpart: the A-stationary form of the numeric phase below. */
DIAGPU_API int diagpu_spgemm_astat_prepare(int32_t n, const int32_t* A_off,
                                           const int64_t* A_starts, int32_t nA,
                                           const int32_t* B_off, const int64_t* B_starts,
                                           int32_t nB, const int32_t* C_off,
                                           const int64_t* pair_ptr, int64_t c_ndiag,
                                           const diagpu_gpair* pairs, int64_t n_pairs,
                                           int32_t* records, void* stream);

/* diagpu_spgemm_symbolic and, in the same call, the records of
 * diagpu_spgemm_astat_prepare for the plan it builds: one stream
 * synchronisation for both (the records step runs on the device behind the
 * symbolic phase and reads its counts there), for callers that build a plan
 * per product, such as a matrix-power chain.  Same arguments, outputs and
 * errors as diagpu_spgemm_symbolic, plus records (4 pair_capacity + 4
 * int32).  When the call returns DIAGPU_OK, records[0 .. 4 n_pairs) hold the
 * plan's records, records[4 n_pairs .. 4 n_pairs + 3] = {0, 0, smallest,
 * largest A offset}, and *records_status is what diagpu_spgemm_astat_prepare
 * would return for the plan: DIAGPU_OK, or DIAGPU_ERR_CAPACITY if a B index
 * exceeds 2^30 - 1 (the records are then unusable; the plan is complete and
 * the other numeric entry points take it), DIAGPU_ERR_ARG if an entry fails
 * the prepare step's check (not expected of the plans this call builds);
 * diagpu_last_error() describes a non-zero *records_status.  No reference
 * counterpart. */
DIAGPU_API int diagpu_spgemm_symbolic_astat(
    int32_t n,
    const int32_t* A_off, const int32_t* A_len, const int64_t* A_starts, int32_t a_ndiag,
    const int32_t* B_off, const int32_t* B_len, const int64_t* B_starts, int32_t b_ndiag,
    int32_t* C_off, int32_t* C_len, int64_t* C_starts, int64_t c_capacity,
    int64_t* pair_ptr, diagpu_gpair* pairs, int64_t pair_capacity,
    int32_t* c_lookup,
    void* workspace, size_t workspace_bytes,
    int32_t* records, int32_t* records_status,
    diagpu_spgemm_info* info, void* stream);

/* The numeric phase of diagpu_spgemm_numeric_f32 (same C, bit for bit) with
 * each workgroup holding one block of 64 R rows of every A diagonal (plus the
 * 32 rows before it; R = 4, 8 or 16 rows per lane, chosen per launch) in LDS
 * and reading only B from memory: for products whose
 * A diagonals each feed many plan entries but whose B window is too wide for
 * the band kernel (e.g. the square of a 64-diagonal band over +-512).
 * records from diagpu_spgemm_astat_prepare for this plan; n < 2^30,
 * c_ndiag < 2^29 and n_pairs < 2^28 (else DIAGPU_ERR_ARG: the kernel
 * addresses its metadata by 32-bit byte offsets; the other numeric kernels
 * take n = 2^30); nA at most
 * DIAGPU_ASTAT_MAX_A (else DIAGPU_ERR_CAPACITY). */
DIAGPU_API int diagpu_spgemm_numeric_astat_f32(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA, const float* A_vals,
    const float* B_vals, const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts,
    int64_t c_ndiag, const int64_t* pair_ptr, const int32_t* records, int64_t n_pairs,
    float* C_vals, void* stream);

/* The same with complex64 values: the numeric phase of
 * diagpu_spgemm_numeric_c64 (same C, bit for bit), same records; each
 * workgroup holds a block of 256 rows (512 for a few short C diagonals, 128
 * above 75 A diagonals) plus the 16 before it; n < 2^30, c_ndiag < 2^29
 * and n_pairs < 2^28 (else DIAGPU_ERR_ARG); nA at most DIAGPU_ASTAT_MAX_A_C64 (else
 * DIAGPU_ERR_CAPACITY).  No reference counterpart (the reference is real
 * only). */
DIAGPU_API int diagpu_spgemm_numeric_astat_c64(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA,
    const diagpu_complex64* A_vals, const diagpu_complex64* B_vals, const int32_t* C_off,
    const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag, const int64_t* pair_ptr,
    const int32_t* records, int64_t n_pairs, diagpu_complex64* C_vals, void* stream);

/* C = (alpha A) B + sigma I in one pass: diagpu_spgemm_numeric_astat_f32 /
 * _c64 (same arguments, limits and records) with each staged A element
 * scaled once in LDS before any term reads it, and sigma added to the sums of
 * C's main diagonal (offset 0) before they are stored; a C without a main
 * diagonal gets no sigma (add it with diagpu_dia_axpby_*).  fp32: the C of
 * diagpu_spgemm_numeric_astat_f32 on the operand fl(alpha a), bit for bit,
 * with fl(c + sigma) on the main diagonal.  Complex: each part of alpha a is
 * one fused multiply-add over the other product.  No reference counterpart:
 * the reference ships no matrix-power driver (spmspm/gather_flat.cuh:13-14
 * describes one).  For the Taylor chain's Horner step
 * S_j = I + ((t/j) H) S_{j+1}, which otherwise takes a scaling pass over H
 * and an identity pass over C around the product. */
DIAGPU_API int diagpu_spgemm_numeric_astat_scaled_f32(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA, const float* A_vals,
    float alpha, const float* B_vals, const int32_t* C_off, const int32_t* C_len,
    const int64_t* C_starts, int64_t c_ndiag, const int64_t* pair_ptr, const int32_t* records,
    int64_t n_pairs, float sigma, float* C_vals, void* stream);

DIAGPU_API int diagpu_spgemm_numeric_astat_scaled_c64(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA,
    const diagpu_complex64* A_vals, diagpu_complex64 alpha, const diagpu_complex64* B_vals,
    const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
    const int64_t* pair_ptr, const int32_t* records, int64_t n_pairs, diagpu_complex64 sigma,
    diagpu_complex64* C_vals, void* stream);

/* ======================================================================
 * gemm_diag: row-packed operands, HM-layout C
 * ====================================================================== */

/* Starts and lengths that address a P x n row-packed array as an HM matrix:
 * starts[i] = i * n + max(-d_i, 0), lengths[i] = n - |d_i| (the HM position
 * of row t's element is t + min(d_i, 0)).  Device kernel; offsets must
 * satisfy |d| < n (checked by the symbolic phase).  Lets gemm_diag run the
 * SpGEMM symbolic and numeric phases unchanged on DA/DB as given
 * (gemm_diag/gemm_diag.cu:119-329 computes the same product with atomics). */
DIAGPU_API int diagpu_rowpacked_as_hm(int32_t n, const int32_t* offsets, int32_t ndiag,
                                      int64_t* starts, int32_t* lengths, void* stream);

/* ======================================================================
 * DIA linear combination (matrix-power / Taylor chain)
 * ====================================================================== */

/* Z = alpha * X + beta * Y for square n x n HM matrices (diagonal d holds
 * n - |d| values, element p at row max(-d, 0) + p).  Offsets of X, Y and Z
 * are ascending and distinct, and Z's set contains X's and Y's (normally it
 * is their union); a Z diagonal missing from X or Y takes 0 from it.  A zero
 * alpha (beta) means X (Y) is not read, as in BLAS.  Every Z value is
 * written.  Z may be X (or Y) in place when both describe the same
 * diagonals at the same starts (e.g. adding the identity to an existing
 * main diagonal); any other overlap is undefined.  Device kernel, async.
 * No counterpart in the reference, whose matrix-power chain
 * (spmspm/gather_flat.cuh:13-14,110-117) has no driver; the Taylor chain
 * uses it to scale H and to add each power into the running sum. */
DIAGPU_API int diagpu_dia_axpby_f32(int32_t n, const int32_t* X_off, const int64_t* X_starts,
                                    int32_t nx, const float* X_vals, float alpha,
                                    const int32_t* Y_off, const int64_t* Y_starts, int32_t ny,
                                    const float* Y_vals, float beta, const int32_t* Z_off,
                                    const int64_t* Z_starts, int32_t nz, float* Z_vals,
                                    void* stream);

/* Complex64 variant of diagpu_dia_axpby_f32 with complex factors (a zero
 * factor, both parts 0, means its operand is not read).  Used by the complex
 * Taylor chain that builds exp(-i t H); no reference counterpart. */
DIAGPU_API int diagpu_dia_axpby_c64(int32_t n, const int32_t* X_off, const int64_t* X_starts,
                                    int32_t nx, const diagpu_complex64* X_vals,
                                    diagpu_complex64 alpha, const int32_t* Y_off,
                                    const int64_t* Y_starts, int32_t ny,
                                    const diagpu_complex64* Y_vals, diagpu_complex64 beta,
                                    const int32_t* Z_off, const int64_t* Z_starts, int32_t nz,
                                    diagpu_complex64* Z_vals, void* stream);

/* ======================================================================
 * HM -> Recon on the device
 * ====================================================================== */

/* build_recon (spmv/src/dia_reconstruct.cuh:77-107) for a square n x n HM
 * matrix already on the device (for square matrices the HM layout is the
 * reference's compact DIA layout): recon_offsets[k] = offsets[ndiag-1-k]
 * (HM offsets ascending, as the SpGEMM symbolic phase produces them, give the
 * descending Recon order), recon_values[k * n + c] = the diagonal's element
 * in column c for c in [max(d,0), max(d,0) + n - |d|), 0 elsewhere.  Lets a
 * SpGEMM product be applied by the SpMV kernels without a host copy. */
DIAGPU_API int diagpu_hm_to_recon_f32(int32_t n, const int32_t* offsets, const int64_t* starts,
                                      int32_t ndiag, const float* values, int32_t* recon_offsets,
                                      float* recon_values, void* stream);
DIAGPU_API int diagpu_hm_to_recon_c64(int32_t n, const int32_t* offsets, const int64_t* starts,
                                      int32_t ndiag, const diagpu_complex64* values,
                                      int32_t* recon_offsets, diagpu_complex64* recon_values,
                                      void* stream);

/* dst[i] = (src[i], 0) for i < count, on the device: a real operator's
 * values (any layout) as complex64, e.g. to start a complex chain such as
 * the propagator exp(-i dt H) from a real H.  No counterpart in the
 * reference (its kernels are real only). */
DIAGPU_API int diagpu_promote_f32_c64(int64_t count, const float* src, diagpu_complex64* dst,
                                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DIAGPU_H */
