/*
 * dia_oracle.c -- CPU restatement of the reference DIA algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product
 * path in diagpu_amd/ is compared against.  Only tests/, the smoke() entry
 * of __graft_entry__.py and the cpu_baseline leg of bench.py may load the
 * library built from it (oracle/liboracle.so).  Nothing in the product links
 * or calls it.
 *
 * Every function names the reference file:line whose behaviour it restates
 * (paths relative to the yuchaosu/DiaGPU checkout).  Conventions:
 *   - "Recon" layout   : column-indexed padded K x cols array,
 *                        Recon[k][c] = H[c - d_k, c], offsets descending
 *                        (spmv/src/dia_reconstruct.cuh:9-17).
 *   - "HM" layout      : compact concatenation of diagonals, element
 *                        (i, j) of diagonal d = j - i at position min(i, j),
 *                        length n - |d| (spmspm/paper_hm.cuh:18-37).
 *   - "row-packed"     : P x n padded array, DA[i][t] = A[t, t + d_i]
 *                        (gemm_diag/gemm_diag.cu:9-15, 362-382).
 * Element starts are 64-bit throughout (the reference uses int in places,
 * which overflows at n = 262144 x 9.5k diagonals).
 *
 * Pinning status of each function is recorded in its comment and checked
 * by tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

static inline int imin0(int x) { return x < 0 ? x : 0; }
static inline int iabs_(int x) { return x < 0 ? -x : x; }

/* ------------------------------------------------------------------------
 * Generators
 * ------------------------------------------------------------------------ */

/* Portable LCG of spmv/test/test_tc_spmv.cu:87-91. */
static inline float lcg_next(uint32_t* s)
{
    *s = *s * 1664525u + 1013904223u;
    return (float)((*s >> 8) & 0xFFFFu) / 65536.0f * 2.0f - 1.0f;
}

/* Dense band matrix H (N x N, row-major) and x for one structural case of
 * spmv/test/test_tc_spmv.cu:86-98: seed = 0x1234567 + N, H filled row-major
 * over (r, offsets in the given order), then x. */
ORC_API void orc_tc_spmv_case(int N, const int* offsets, int K, float* H, float* x)
{
    uint32_t seed = 0x1234567u + (uint32_t)N;
    memset(H, 0, sizeof(float) * (size_t)N * (size_t)N);
    for (int r = 0; r < N; ++r)
        for (int k = 0; k < K; ++k) {
            const int c = r + offsets[k];
            if (c >= 0 && c < N) H[(size_t)r * N + c] = lcg_next(&seed);
        }
    for (int i = 0; i < N; ++i) x[i] = lcg_next(&seed);
}

/* Integer-hash band value and x value of spmv/bench/bench_cusparse.cu:70-82
 * (the same hval is in spmv/tools/gen_banded_mtx.cpp:18-23). */
ORC_API float orc_hval(int r, int d)
{
    uint32_t h = (uint32_t)r * 2654435761u ^ (uint32_t)(d + 1024) * 40503u;
    h ^= h >> 13; h *= 0x5bd1e995u; h ^= h >> 15;
    return (float)(h & 0xFFFFu) / 65536.0f * 2.0f - 1.0f;
}

ORC_API float orc_xval(int i)
{
    uint32_t h = (uint32_t)i * 2246822519u;
    h ^= h >> 13; h *= 0x85ebca6bu; h ^= h >> 16;
    return (float)(h & 0xFFFFu) / 65536.0f * 2.0f - 1.0f;
}

/* x[i] = orc_xval(i) for i < N. */
ORC_API void orc_xval_fill(int N, float* x)
{
    for (int i = 0; i < N; ++i) x[i] = orc_xval(i);
}

/* The band entries H[r, r + d] = orc_hval(r, d) that exist in an N x N
 * matrix, offset by offset in the given order, rows ascending; returns the
 * count written. */
ORC_API int64_t orc_hval_band(int N, const int* offsets, int K, float* out)
{
    int64_t o = 0;
    for (int k = 0; k < K; ++k)
        for (int r = 0; r < N; ++r)
            if (r + offsets[k] >= 0 && r + offsets[k] < N) out[o++] = orc_hval(r, offsets[k]);
    return o;
}

/* Recon array of the SpMV bench directly from offsets (any order) with the
 * hash values: spmv/bench/bench_cusparse.cu:131-144 (offsets sorted
 * descending, Recon[k][c] = hval(c - d_k, d_k) for valid rows).  Fills
 * r_offsets[K] and r_values[K * N]; x[N] = xval(i). */
ORC_API void orc_hash_band_recon(int N, const int* offsets, int K,
                                 int* r_offsets, float* r_values, float* x)
{
    for (int k = 0; k < K; ++k) r_offsets[k] = offsets[k];
    for (int a = 1; a < K; ++a) {             /* insertion sort, descending */
        int v = r_offsets[a], b = a - 1;
        while (b >= 0 && r_offsets[b] < v) { r_offsets[b + 1] = r_offsets[b]; --b; }
        r_offsets[b + 1] = v;
    }
    memset(r_values, 0, sizeof(float) * (size_t)K * (size_t)N);
    for (int k = 0; k < K; ++k) {
        const int d = r_offsets[k];
        for (int c = 0; c < N; ++c) {
            const int row = c - d;
            if (row >= 0 && row < N) r_values[(size_t)k * N + c] = orc_hval(row, d);
        }
    }
    for (int i = 0; i < N; ++i) x[i] = orc_xval(i);
}

/* ------------------------------------------------------------------------
 * SpMV: compact DIA <-> Recon
 * ------------------------------------------------------------------------ */

/* Count pass of dense_to_dia (spmv/test/test_reconstruct.cpp:93-116): number
 * of diagonals holding a nonzero and their total length. */
ORC_API void orc_dense_to_dia_count(const float* H, int rows, int cols,
                                    int* ndiag, int64_t* nvals)
{
    int nd = 0; int64_t nv = 0;
    for (int d = -(rows - 1); d <= cols - 1; ++d) {
        const int sr = d >= 0 ? 0 : -d, sc = d >= 0 ? d : 0;
        const int len = (rows - sr) < (cols - sc) ? (rows - sr) : (cols - sc);
        if (len <= 0) continue;
        int nz = 0;
        for (int j = 0; j < len; ++j)
            if (H[(size_t)(sr + j) * cols + (sc + j)] != 0.0f) { nz = 1; break; }
        if (!nz) continue;
        ++nd; nv += len;
    }
    *ndiag = nd; *nvals = nv;
}

/* dense_to_dia (spmv/test/test_reconstruct.cpp:93-116): offsets ascending
 * from -(rows-1), only diagonals with a nonzero, element j of diagonal d is
 * H[sr + j, sc + j]. */
ORC_API void orc_dense_to_dia(const float* H, int rows, int cols, int* offsets,
                              int64_t* starts, int* lengths, float* values)
{
    int nd = 0; int64_t nv = 0;
    for (int d = -(rows - 1); d <= cols - 1; ++d) {
        const int sr = d >= 0 ? 0 : -d, sc = d >= 0 ? d : 0;
        const int len = (rows - sr) < (cols - sc) ? (rows - sr) : (cols - sc);
        if (len <= 0) continue;
        int nz = 0;
        for (int j = 0; j < len; ++j)
            if (H[(size_t)(sr + j) * cols + (sc + j)] != 0.0f) { nz = 1; break; }
        if (!nz) continue;
        offsets[nd] = d; starts[nd] = nv; lengths[nd] = len;
        for (int j = 0; j < len; ++j) values[nv + j] = H[(size_t)(sr + j) * cols + (sc + j)];
        ++nd; nv += len;
    }
}

/* build_recon (spmv/src/dia_reconstruct.cuh:77-107): sort the offsets
 * descending; row k of the K x cols zero array receives the values of the
 * FIRST input diagonal whose offset equals d_k (linear search), at columns
 * [max(d,0), max(d,0) + len). */
#define DEFINE_BUILD_RECON(SUF, T)                                               \
ORC_API void orc_build_recon_##SUF(int rows, int cols, int K, const int* offsets,  \
                                   const int64_t* starts, const int* lengths,      \
                                   const T* values, int* r_offsets, T* r_values)   \
{                                                                                  \
    (void)rows;                                                                    \
    for (int k = 0; k < K; ++k) r_offsets[k] = offsets[k];                         \
    for (int a = 1; a < K; ++a) {                                                  \
        int v = r_offsets[a], b = a - 1;                                           \
        while (b >= 0 && r_offsets[b] < v) { r_offsets[b + 1] = r_offsets[b]; --b; } \
        r_offsets[b + 1] = v;                                                      \
    }                                                                              \
    memset(r_values, 0, sizeof(T) * (size_t)K * (size_t)cols);                     \
    for (int k = 0; k < K; ++k) {                                                  \
        const int d = r_offsets[k];                                                \
        int di = -1;                                                               \
        for (int i = 0; i < K; ++i) if (offsets[i] == d) { di = i; break; }        \
        if (di < 0) continue;                                                      \
        const int sc = d >= 0 ? d : 0;                                             \
        for (int j = 0; j < lengths[di]; ++j)                                      \
            r_values[(size_t)k * cols + sc + j] = values[starts[di] + j];          \
    }                                                                              \
}
DEFINE_BUILD_RECON(f32, float)
DEFINE_BUILD_RECON(f64, double)

/* recon_to_dense (spmv/test/test_reconstruct.cpp:145-158). */
ORC_API void orc_recon_to_dense_f32(int rows, int cols, int K, const int* r_offsets,
                                    const float* r_values, float* H)
{
    memset(H, 0, sizeof(float) * (size_t)rows * (size_t)cols);
    for (int k = 0; k < K; ++k) {
        const int d = r_offsets[k];
        for (int c = 0; c < cols; ++c) {
            const int r = c - d;
            if (r >= 0 && r < rows) H[(size_t)r * cols + c] = r_values[(size_t)k * cols + c];
        }
    }
}

/* ------------------------------------------------------------------------
 * SpMV on Recon
 *   y[r] = sum_k [0 <= r + d_k < min(cols, x_size)] Recon[k][r + d_k] * x[r + d_k]
 * (spmv/src/dia_reconstruct.cuh:22; bounds as the kernel applies them,
 * spmv/src/tc_spmv_regdirect_kernel.cu:85-104).
 * ------------------------------------------------------------------------ */

/* spmv_from_recon (spmv/test/test_reconstruct.cpp:122-138): serial, fp32
 * accumulation, diagonals in stored order. */
ORC_API void orc_spmv_recon_f32(int rows, int cols, int K, const int* offs,
                                const float* vals, const float* x, int64_t x_size,
                                float* y)
{
    const int64_t lim = x_size < cols ? x_size : cols;
    for (int r = 0; r < rows; ++r) {
        float s = 0.0f;
        for (int k = 0; k < K; ++k) {
            const int64_t c = (int64_t)r + offs[k];
            if (c >= 0 && c < lim) s += vals[(size_t)k * cols + c] * x[c];
        }
        y[r] = s;
    }
}

/* Same sum with fp64 accumulation of fp32 data: the "fp64 host result" the
 * fp32 kernel is held to.  abs_sum[r] = sum of |term| bounds the rounding
 * error of any summation order (|err| <= K * u * abs_sum). */
ORC_API void orc_spmv_recon_f32_ref64(int rows, int cols, int K, const int* offs,
                                      const float* vals, const float* x, int64_t x_size,
                                      double* y, double* abs_sum)
{
    const int64_t lim = x_size < cols ? x_size : cols;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        double s = 0.0, a = 0.0;
        for (int k = 0; k < K; ++k) {
            const int64_t c = (int64_t)r + offs[k];
            if (c >= 0 && c < lim) {
                const double t = (double)vals[(size_t)k * cols + c] * (double)x[c];
                s += t; a += fabs(t);
            }
        }
        y[r] = s;
        if (abs_sum) abs_sum[r] = a;
    }
}

ORC_API void orc_spmv_recon_f64(int rows, int cols, int K, const int* offs,
                                const double* vals, const double* x, int64_t x_size,
                                double* y, double* abs_sum)
{
    const int64_t lim = x_size < cols ? x_size : cols;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        double s = 0.0, a = 0.0;
        for (int k = 0; k < K; ++k) {
            const int64_t c = (int64_t)r + offs[k];
            if (c >= 0 && c < lim) {
                const double t = vals[(size_t)k * cols + c] * x[c];
                s += t; a += fabs(t);
            }
        }
        y[r] = s;
        if (abs_sum) abs_sum[r] = a;
    }
}

/* Complex Recon SpMV: the same sum (spmv/src/dia_reconstruct.cuh:22) and
 * bounds with complex64 values and x (interleaved re, im), fp64
 * accumulation.  abs_sum[r] = sum over terms of |a_re x_re| + |a_im x_im| +
 * |a_re x_im| + |a_im x_re| bounds the rounding of either part in any
 * summation order.  No reference counterpart (the reference is real only);
 * pinned by tests/test_oracle.py against dense complex products and scipy's
 * dia_matrix. */
ORC_API void orc_spmv_recon_c64_ref(int rows, int cols, int K, const int* offs,
                                    const float* vals, const float* x, int64_t x_size,
                                    double* y, double* abs_sum)
{
    const int64_t lim = x_size < cols ? x_size : cols;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        double sr = 0.0, si = 0.0, a = 0.0;
        for (int k = 0; k < K; ++k) {
            const int64_t c = (int64_t)r + offs[k];
            if (c >= 0 && c < lim) {
                const double vr = vals[2 * ((size_t)k * cols + c)], vi = vals[2 * ((size_t)k * cols + c) + 1];
                const double xr = x[2 * c], xi = x[2 * c + 1];
                sr += vr * xr - vi * xi;
                si += vr * xi + vi * xr;
                a += fabs(vr * xr) + fabs(vi * xi) + fabs(vr * xi) + fabs(vi * xr);
            }
        }
        y[2 * (size_t)r] = sr;
        y[2 * (size_t)r + 1] = si;
        if (abs_sum) abs_sum[r] = a;
    }
}

/* Real fp32 Recon values applied to a complex64 x: y = H Re(x) + i H Im(x),
 * fp64 accumulation, abs_sum as above. */
ORC_API void orc_spmv_recon_f32c64_ref(int rows, int cols, int K, const int* offs,
                                       const float* vals, const float* x, int64_t x_size,
                                       double* y, double* abs_sum)
{
    const int64_t lim = x_size < cols ? x_size : cols;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        double sr = 0.0, si = 0.0, a = 0.0;
        for (int k = 0; k < K; ++k) {
            const int64_t c = (int64_t)r + offs[k];
            if (c >= 0 && c < lim) {
                const double v = vals[(size_t)k * cols + c];
                sr += v * x[2 * c];
                si += v * x[2 * c + 1];
                a += fabs(v * x[2 * c]) + fabs(v * x[2 * c + 1]);
            }
        }
        y[2 * (size_t)r] = sr;
        y[2 * (size_t)r + 1] = si;
        if (abs_sum) abs_sum[r] = a;
    }
}

/* CPU baseline: the straightforward OpenMP DIA loop over the Recon layout,
 * schedule(static) over rows, inner loop over diagonals, accumulation in the
 * element type.  Returns the thread count used. */
#define DEFINE_SPMV_OMP(SUF, T)                                                    \
ORC_API int orc_spmv_recon_omp_##SUF(int rows, int cols, int K, const int* offs,     \
                                     const T* vals, const T* x, int64_t x_size, T* y) \
{                                                                                   \
    const int64_t lim = x_size < cols ? x_size : cols;                              \
    int nthr = 1;                                                                   \
    _Pragma("omp parallel")                                                         \
    {                                                                               \
        _Pragma("omp single")                                                       \
        { nthr = omp_threads_(); }                                                  \
        _Pragma("omp for schedule(static)")                                         \
        for (int r = 0; r < rows; ++r) {                                            \
            T s = 0;                                                                \
            for (int k = 0; k < K; ++k) {                                           \
                const int64_t c = (int64_t)r + offs[k];                             \
                if (c >= 0 && c < lim) s += vals[(size_t)k * cols + c] * x[c];      \
            }                                                                       \
            y[r] = s;                                                               \
        }                                                                           \
    }                                                                               \
    return nthr;                                                                    \
}
static inline int omp_threads_(void)
{
#ifdef _OPENMP
    return omp_get_num_threads();
#else
    return 1;
#endif
}
DEFINE_SPMV_OMP(f32, float)
DEFINE_SPMV_OMP(f64, double)

ORC_API int orc_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

ORC_API void orc_set_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------------
 * SpGEMM structure (integer, the bit-exact target)
 * ------------------------------------------------------------------------ */

/* GPair of spmspm/gather_flat.cuh:21: {size_t ab, bb; int ash, bsh, al, bl}. */
typedef struct { uint64_t ab, bb; int32_t ash, bsh, al, bl; } orc_gpair;

/* make_c_structure (spmspm/bench_spmspm.cu:109-131), identical set to
 * compute_c_hm_structure (spmspm/paper_hm.cuh:87-117): presence over the
 * 2n-1 offsets of every da + db with |da + db| < n, scanned ascending;
 * lengths n - |d|, starts the exclusive prefix sum of the lengths.
 * C arrays need capacity min(nA * nB, 2n - 1).  Returns the C diagonal
 * count. */
ORC_API int orc_c_structure(int n, const int* A_off, int nA, const int* B_off, int nB,
                            int* C_off, int* C_len, int64_t* C_starts, int64_t* nnz)
{
    char* present = (char*)calloc((size_t)2 * n - 1, 1);
    for (int a = 0; a < nA; ++a)
        for (int b = 0; b < nB; ++b) {
            const int64_t dc = (int64_t)A_off[a] + B_off[b];
            if (dc > -(int64_t)n && dc < n) present[dc + (n - 1)] = 1;
        }
    int nc = 0; int64_t off = 0;
    for (int d = -(n - 1); d <= n - 1; ++d) {
        if (!present[d + (n - 1)]) continue;
        const int len = n - iabs_(d);
        if (len <= 0) continue;
        C_off[nc] = d; C_len[nc] = len; C_starts[nc] = off;
        off += len; ++nc;
    }
    free(present);
    if (nnz) *nnz = off;
    return nc;
}

/* build_c_diag_lookup (spmspm/paper_hm.cuh:121-130): lookup[d + n - 1] = C
 * index, -1 where absent. */
ORC_API void orc_c_lookup(int n, const int* C_off, int nC, int* lookup)
{
    for (int64_t i = 0; i < 2 * (int64_t)n - 1; ++i) lookup[i] = -1;
    for (int k = 0; k < nC; ++k) lookup[C_off[k] + (n - 1)] = k;
}

/* PairEntry of spmspm/spmspm.cu:40-46. */
typedef struct { int32_t a_local, b_local, c_local, a_shift, b_shift; } orc_pair_entry;

/* build_schedule (spmspm/bench_spmspm.cu:137-243): the C diagonals in groups
 * of T consecutive ones; per group, for each of its C diagonals dc in order
 * and each A diagonal ai in A's order with db = dc - da an offset of B (the
 * last B index holding it), one PairEntry{a_local, b_local, c_local,
 * min0(da) - min0(dc), da + min0(db) - min0(dc)}, where a_local / b_local
 * number the group's A / B diagonals in order of first use; halos are the
 * largest |a_shift| / |b_shift| over all groups.  Per-group lists are padded
 * to the largest group (a/b/c globals and pairs group-strided, zeros in the
 * padding), then one block per (group, n-tile): block_group = g, block_tile =
 * t * n_tile.
 * scalars[8] = {a_halo, b_halo, num_groups, max_a, max_b, max_pairs,
 * num_ntiles, num_blocks}.  With a_count == NULL only the scalars are
 * computed (to size the arrays); otherwise every array is written. */
ORC_API void orc_build_schedule(int n, const int* A_off, int nA, const int* B_off, int nB,
                                const int* C_off, int nC, int T, int n_tile, int* scalars,
                                int* a_count, int* b_count, int* pair_count, int* t_out,
                                int* a_globals, int* b_globals, int* c_globals,
                                orc_pair_entry* pairs, int* block_group, int* block_tile)
{
    const int64_t nlk = 2 * (int64_t)n - 1;
    int* blk = (int*)malloc(sizeof(int) * (size_t)nlk);
    int* aloc = (int*)malloc(sizeof(int) * (size_t)(nA > 0 ? nA : 1));
    int* bloc = (int*)malloc(sizeof(int) * (size_t)(nB > 0 ? nB : 1));
    for (int64_t i = 0; i < nlk; ++i) blk[i] = -1;
    for (int b = 0; b < nB; ++b)
        if (B_off[b] > -n && B_off[b] < n) blk[B_off[b] + (n - 1)] = b;
    const int groups = (nC + T - 1) / T;
    int a_halo = 0, b_halo = 0, max_a = 0, max_b = 0, max_p = 0;
    /* two sweeps over the groups: sizes, then (with arrays) the contents */
    for (int pass = 0; pass < (a_count ? 2 : 1); ++pass) {
        for (int g = 0; g < groups; ++g) {
            for (int i = 0; i < nA; ++i) aloc[i] = -1;
            for (int i = 0; i < nB; ++i) bloc[i] = -1;
            int na = 0, nb = 0, np = 0;
            const int c0 = g * T, c1 = c0 + T < nC ? c0 + T : nC;
            for (int cl = 0; cl < c1 - c0; ++cl) {
                const int dc = C_off[c0 + cl];
                if (pass) c_globals[(size_t)g * T + cl] = c0 + cl;
                for (int ai = 0; ai < nA; ++ai) {
                    const int64_t db = (int64_t)dc - A_off[ai];
                    if (db <= -(int64_t)n || db >= n) continue;
                    const int bi = blk[db + (n - 1)];
                    if (bi < 0) continue;
                    if (aloc[ai] < 0) {
                        if (pass) a_globals[(size_t)g * max_a + na] = ai;
                        aloc[ai] = na++;
                    }
                    if (bloc[bi] < 0) {
                        if (pass) b_globals[(size_t)g * max_b + nb] = bi;
                        bloc[bi] = nb++;
                    }
                    const int da = A_off[ai];
                    const int ash = imin0(da) - imin0(dc);
                    const int bsh = da + imin0((int)db) - imin0(dc);
                    if (pass) {
                        orc_pair_entry e = {aloc[ai], bloc[bi], cl, ash, bsh};
                        pairs[(size_t)g * max_p + np] = e;
                    } else {
                        if (iabs_(ash) > a_halo) a_halo = iabs_(ash);
                        if (iabs_(bsh) > b_halo) b_halo = iabs_(bsh);
                    }
                    ++np;
                }
            }
            if (pass) {
                a_count[g] = na; b_count[g] = nb; pair_count[g] = np; t_out[g] = c1 - c0;
            } else {
                if (na > max_a) max_a = na;
                if (nb > max_b) max_b = nb;
                if (np > max_p) max_p = np;
            }
        }
        if (!pass && a_count) {     /* zero the padding before the fill sweep */
            memset(a_globals, 0, sizeof(int) * (size_t)groups * max_a);
            memset(b_globals, 0, sizeof(int) * (size_t)groups * max_b);
            memset(c_globals, 0, sizeof(int) * (size_t)groups * T);
            memset(pairs, 0, sizeof(orc_pair_entry) * (size_t)groups * max_p);
        }
    }
    const int ntiles = (n + n_tile - 1) / n_tile;
    if (a_count)
        for (int g = 0; g < groups; ++g)
            for (int t = 0; t < ntiles; ++t) {
                block_group[(size_t)g * ntiles + t] = g;
                block_tile[(size_t)g * ntiles + t] = t * n_tile;
            }
    scalars[0] = a_halo; scalars[1] = b_halo; scalars[2] = groups; scalars[3] = max_a;
    scalars[4] = max_b; scalars[5] = max_p; scalars[6] = ntiles; scalars[7] = groups * ntiles;
    free(blk); free(aloc); free(bloc);
}

/* build_pairs_only (spmspm/gather_flat.cuh:231-255): for each C diagonal k in
 * order and each B diagonal bi in B's order, da = dc - db; skip |da| >= n or
 * an A offset that is absent (Alookup, built as the bench builds its offset
 * lookups, bench_spmspm.cu:552-553: the last index wins); emit
 *   GPair{A_starts[ai], B_starts[bi], min0(da) - min0(dc),
 *         da + min0(db) - min0(dc), A_len[ai], B_len[bi]}.
 * pair_ptr has nC + 1 entries.  Returns the pair count. */
ORC_API int64_t orc_pairs_only(int n, const int* A_off, int nA, const int* A_len,
                               const int64_t* A_starts, const int* B_off, int nB,
                               const int* B_len, const int64_t* B_starts,
                               const int* C_off, int nC, int64_t* pair_ptr,
                               orc_gpair* pairs)
{
    int* Alk = (int*)malloc(sizeof(int) * ((size_t)2 * n - 1));
    for (int64_t i = 0; i < 2 * (int64_t)n - 1; ++i) Alk[i] = -1;
    for (int a = 0; a < nA; ++a)
        if (A_off[a] > -n && A_off[a] < n) Alk[A_off[a] + (n - 1)] = a;
    int64_t np = 0;
    for (int k = 0; k < nC; ++k) {
        const int dc = C_off[k], minc = imin0(dc);
        pair_ptr[k] = np;
        for (int b = 0; b < nB; ++b) {
            const int db = B_off[b];
            const int64_t da64 = (int64_t)dc - db;
            if (da64 <= -(int64_t)n || da64 >= n) continue;
            const int da = (int)da64;
            const int ai = Alk[da + (n - 1)];
            if (ai < 0) continue;
            if (pairs) {
                orc_gpair g;
                g.ab = (uint64_t)A_starts[ai]; g.bb = (uint64_t)B_starts[b];
                g.ash = imin0(da) - minc; g.bsh = da + imin0(db) - minc;
                g.al = A_len[ai]; g.bl = B_len[b];
                pairs[np] = g;
            }
            ++np;
        }
    }
    pair_ptr[nC] = np;
    free(Alk);
    return np;
}

/* ------------------------------------------------------------------------
 * SpGEMM numeric
 * ------------------------------------------------------------------------ */

/* cpu_dia_spgemm (spmspm/bench_spmspm.cu:376-408) loop structure -- per C
 * diagonal, per position p, per A diagonal ascending with the B offset
 * looked up -- accumulated in fp64.  abs_out (optional) receives the sum of
 * |term|.  Cost nC * n * nA: small inputs only. */
ORC_API void orc_spgemm_gather_f64(int n,
                                   const int* A_off, int nA, const int* A_len,
                                   const int64_t* A_starts, const float* A_vals,
                                   const int* B_off, int nB, const int* B_len,
                                   const int64_t* B_starts, const float* B_vals,
                                   const int* C_off, int nC, const int* C_len,
                                   const int64_t* C_starts, double* out, double* abs_out)
{
    int* Blk = (int*)malloc(sizeof(int) * ((size_t)2 * n - 1));
    for (int64_t i = 0; i < 2 * (int64_t)n - 1; ++i) Blk[i] = -1;
    for (int b = 0; b < nB; ++b) Blk[B_off[b] + (n - 1)] = b;
    #pragma omp parallel for schedule(dynamic)
    for (int k = 0; k < nC; ++k) {
        const int dc = C_off[k], minc = imin0(dc);
        for (int p = 0; p < C_len[k]; ++p) {
            double acc = 0.0, aab = 0.0;
            for (int a = 0; a < nA; ++a) {
                const int da = A_off[a];
                const int64_t db64 = (int64_t)dc - da;
                if (db64 <= -(int64_t)n || db64 >= n) continue;
                const int db = (int)db64;
                const int bi = Blk[db + (n - 1)];
                if (bi < 0) continue;
                const int pa = p + imin0(da) - minc;
                const int pb = p + da + imin0(db) - minc;
                if (pa < 0 || pa >= A_len[a]) continue;
                if (pb < 0 || pb >= B_len[bi]) continue;
                const double t = (double)A_vals[A_starts[a] + pa] * (double)B_vals[B_starts[bi] + pb];
                acc += t; aab += fabs(t);
            }
            out[C_starts[k] + p] = acc;
            if (abs_out) abs_out[C_starts[k] + p] = aab;
        }
    }
    free(Blk);
}

/* Numeric phase over a pair plan, as gather_flat_kernel evaluates it
 * (spmspm/gather_flat.cuh:47-62): C[k][p] = sum over the pairs of k of
 * Av[ab + p + ash] * Bv[bb + p + bsh], terms with an operand position out of
 * [0, al) / [0, bl) dropped.  fp64 accumulation, C diagonals [kbeg, kend)
 * only; out/abs_out are indexed from C_starts[kbeg] (so a sample of C
 * diagonals can be checked without the whole C). */
ORC_API void orc_spgemm_pairs_f64(const float* A_vals, const float* B_vals,
                                  const int* C_len, const int64_t* C_starts,
                                  const int64_t* pair_ptr, const orc_gpair* pairs,
                                  int kbeg, int kend, double* out, double* abs_out)
{
    const int64_t base = C_starts[kbeg];
    #pragma omp parallel for schedule(dynamic)
    for (int k = kbeg; k < kend; ++k) {
        for (int p = 0; p < C_len[k]; ++p) {
            double acc = 0.0, aab = 0.0;
            for (int64_t q = pair_ptr[k]; q < pair_ptr[k + 1]; ++q) {
                const orc_gpair g = pairs[q];
                const int pa = p + g.ash, pb = p + g.bsh;
                if (pa < 0 || pa >= g.al || pb < 0 || pb >= g.bl) continue;
                const double t = (double)A_vals[g.ab + pa] * (double)B_vals[g.bb + pb];
                acc += t; aab += fabs(t);
            }
            out[C_starts[k] - base + p] = acc;
            if (abs_out) abs_out[C_starts[k] - base + p] = aab;
        }
    }
}

/* The same plan-driven numeric phase with complex64 values (interleaved re,
 * im) and complex products, fp64 accumulation (no reference counterpart: the
 * reference is real only).  out holds re, im pairs; abs_out[p] = sum over
 * terms of |a_re b_re| + |a_im b_im| + |a_re b_im| + |a_im b_re|.  Pinned by
 * tests/test_oracle.py against dense complex products and against
 * orc_spgemm_pairs_f64 on the four real part products. */
ORC_API void orc_spgemm_pairs_c128(const float* A_vals, const float* B_vals,
                                   const int* C_len, const int64_t* C_starts,
                                   const int64_t* pair_ptr, const orc_gpair* pairs,
                                   int kbeg, int kend, double* out, double* abs_out)
{
    const int64_t base = C_starts[kbeg];
    #pragma omp parallel for schedule(dynamic)
    for (int k = kbeg; k < kend; ++k) {
        for (int p = 0; p < C_len[k]; ++p) {
            double sr = 0.0, si = 0.0, aab = 0.0;
            for (int64_t q = pair_ptr[k]; q < pair_ptr[k + 1]; ++q) {
                const orc_gpair g = pairs[q];
                const int pa = p + g.ash, pb = p + g.bsh;
                if (pa < 0 || pa >= g.al || pb < 0 || pb >= g.bl) continue;
                const double ar = A_vals[2 * (g.ab + pa)], ai = A_vals[2 * (g.ab + pa) + 1];
                const double br = B_vals[2 * (g.bb + pb)], bi = B_vals[2 * (g.bb + pb) + 1];
                sr += ar * br - ai * bi;
                si += ar * bi + ai * br;
                aab += fabs(ar * br) + fabs(ai * bi) + fabs(ar * bi) + fabs(ai * br);
            }
            out[2 * (C_starts[k] - base + p)] = sr;
            out[2 * (C_starts[k] - base + p) + 1] = si;
            if (abs_out) abs_out[C_starts[k] - base + p] = aab;
        }
    }
}

/* CPU baseline for SpGEMM: OpenMP over C diagonals, schedule(dynamic) as
 * spmspm/bench_spmspm.cu:384, with each C diagonal's pair list resolved once
 * (the plan) rather than per element; fp32 accumulation in plan order.
 * Computes C diagonals [kbeg, kend) into out (indexed from C_starts[kbeg]).
 * Returns the thread count used. */
ORC_API int orc_spgemm_pairs_omp_f32(const float* A_vals, const float* B_vals,
                                     const int* C_len, const int64_t* C_starts,
                                     const int64_t* pair_ptr, const orc_gpair* pairs,
                                     int kbeg, int kend, float* out)
{
    const int64_t base = C_starts[kbeg];
    int nthr = 1;
    #pragma omp parallel
    {
        #pragma omp single
        { nthr = omp_threads_(); }
        #pragma omp for schedule(dynamic)
        for (int k = kbeg; k < kend; ++k) {
            float* o = out + (C_starts[k] - base);
            const int len = C_len[k];
            for (int p = 0; p < len; ++p) o[p] = 0.0f;
            for (int64_t q = pair_ptr[k]; q < pair_ptr[k + 1]; ++q) {
                const orc_gpair g = pairs[q];
                int lo = 0, hi = len;                 /* positions with both operands valid */
                if (-g.ash > lo) lo = -g.ash;
                if (-g.bsh > lo) lo = -g.bsh;
                if (g.al - g.ash < hi) hi = g.al - g.ash;
                if (g.bl - g.bsh < hi) hi = g.bl - g.bsh;
                const float* a = A_vals + g.ab + g.ash;
                const float* b = B_vals + g.bb + g.bsh;
                for (int p = lo; p < hi; ++p) o[p] += a[p] * b[p];
            }
        }
    }
    return nthr;
}

/* Haque et al. atomic algorithm (spmspm/paper_hm_kernel.cu:31-93), run
 * sequentially in fp64: for each A element i, its diagonal by binary search
 * over A_starts (find_diagonal_bs, :17-29), its (row, k) coordinates, then for
 * each B diagonal the B element in row k, the C diagonal dc = col - row via
 * the lookup, and out[C_starts + p_c] += a * b.  A different traversal from
 * the gather above; the two must agree.  out must be zeroed by the caller. */
ORC_API void orc_spgemm_hm_atomic_f64(int n,
                                      const int* A_off, int nA, const int64_t* A_starts,
                                      const int* A_len, const float* A_vals, int64_t nzA,
                                      const int* B_off, int nB, const int64_t* B_starts,
                                      const int* B_len, const float* B_vals,
                                      const int* C_len, const int64_t* C_starts,
                                      const int* C_lookup, double* out)
{
    (void)A_len;
    for (int64_t i = 0; i < nzA; ++i) {
        int lo = 0, hi = nA - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) / 2;
            if (A_starts[mid] <= i) lo = mid; else hi = mid - 1;
        }
        const int da = A_off[lo];
        const int64_t a_ind = i - A_starts[lo];
        const double a = A_vals[i];
        const int64_t row = (da >= 0 ? 0 : -da) + a_ind;
        const int64_t kk = (da >= 0 ? da : 0) + a_ind;
        for (int b = 0; b < nB; ++b) {
            const int db = B_off[b];
            const int64_t p_b = kk - (db >= 0 ? 0 : -db);
            if (p_b < 0 || p_b >= B_len[b]) continue;
            const int64_t col = (db >= 0 ? db : 0) + p_b;
            const int64_t dc = col - row;
            const int ci = C_lookup[dc + (n - 1)];
            if (ci < 0) continue;
            const int64_t p_c = row - (dc >= 0 ? 0 : -dc);
            if (p_c < 0 || p_c >= C_len[ci]) continue;
            out[C_starts[ci] + p_c] += a * (double)B_vals[B_starts[b] + p_b];
        }
    }
}

/* ------------------------------------------------------------------------
 * gemm_diag (row-packed)
 * ------------------------------------------------------------------------ */

/* C[k][t] = sum_{i + j = k} DA[i][t] * DB[j][t + d_i]
 * (gemm_diag/gemm_diag.cu:9-15), traversed as cpu_diag_multiply does
 * (:335-356: pairs (ri, rj), rows t, bt = t + d_i in range, zero operands
 * skipped, col = t + d_i + d_j in range) but accumulated in fp64 straight
 * into the compact C layout of build_c_layout (:388-423): position
 * p_c = t - max(-k, 0), lookup of k via C_lookup. */
ORC_API void orc_gemm_diag_f64(int n, const float* DA, const int* off_A, int P,
                               const float* DB, const int* off_B, int Q,
                               const int* C_lookup, const int64_t* C_starts,
                               double* out, double* abs_out)
{
    for (int ri = 0; ri < P; ++ri) {
        const int i = off_A[ri];
        for (int rj = 0; rj < Q; ++rj) {
            const int j = off_B[rj];
            for (int t = 0; t < n; ++t) {
                const float a = DA[(size_t)ri * n + t];
                const int64_t bt = (int64_t)t + i;
                if (bt < 0 || bt >= n) continue;
                const float b = DB[(size_t)rj * n + bt];
                if (a == 0.0f || b == 0.0f) continue;
                const int64_t col = (int64_t)t + i + j;
                if (col < 0 || col >= n) continue;
                const int64_t k = (int64_t)i + j;
                const int ci = C_lookup[k + (n - 1)];
                if (ci < 0) continue;
                const int64_t pc = t - (k >= 0 ? 0 : -k);
                const double v = (double)a * (double)b;
                out[C_starts[ci] + pc] += v;
                if (abs_out) abs_out[C_starts[ci] + pc] += fabs(v);
            }
        }
    }
}
