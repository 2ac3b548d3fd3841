// DIA x DIA SpGEMM numeric phase for narrow bands on the matrix cores: the
// fp32 MFMA variant of the band kernel (spgemm_band.hip) for gemm_diag-type
// products (gemm_diag/gemm_diag.cu:119-329 tiles the same product, 4 x 4
// diagonals x 32 columns, with scalar FMAs and atomics).
//
// The band product is a dense matrix product restricted to a band, so each
// 16-row tile of C is computed as the dense 16 x 16 x 4 MFMA blocks that
// intersect the band (band_mfma.hpp: for column tile ct the k steps
// ks_lo..ks_hi), with the operand elements outside the band read as zeros.
//
// Every wave works alone (no workgroup barrier after set-up) on a contiguous
// range of slabs of kMfmaRows rows, with a staging buffer of its own in LDS:
//   [zero row] A_w [a_span + 1][kMfmaStrideA] [zero row]
//              row (da - a_min) = A's diagonal da at the slab's rows
//   [zero row] B_w [b_span + 1][sb] [zero row]
//              row (db - b_min) = B's diagonal db at rows k = i0 + a_min + (0..wm-1)
// and the slab's C values, C_w [c_span + 1][kMfmaStrideC], written over the
// buffer once its matrix work is done.  The workgroup shares the C starts by
// offset and the lists of absent A and B offsets (whose rows are zeroed).
// Per slab a wave
//   1. stages the slab with direct global-to-LDS loads and waits for them;
//   2. runs, per column tile ct, the issued blocks of ct over its four
//      16-row tiles (v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16]
//      and B[l / 16][l % 16] and holds D[4 (l / 16) + j][l % 16]), the next
//      k step's operands read before the current step's matrix work, every
//      column tile's accumulators in registers, each operand row index
//      clamped into [-1, span + 1] so that rows outside the offset ranges
//      read the zero rows;
//   3. writes the slab's C values by offset into C_w (lanes outside C's range
//      into a dump past it) and stores one coalesced run of kMfmaRows values
//      per C diagonal.
// Two workgroups of 4 waves share a CU (two waves per SIMD), so one wave's
// loads are in flight while the other computes.  Slabs away from the
// matrix's ends (all A rows, the B window and the C rows inside their
// diagonals) load and store with a scalar offset per diagonal and the lane's
// fixed offset (buffer instructions, where every element's byte offset lies
// below 2^32); the others clamp each position into its diagonal.
//
// The sums run in MFMA order, not plan order, so C matches the gather and
// band kernels to rounding (1e-5 of the term sum), not bit for bit.  Terms
// whose k (= A's column, B's row) lies outside the matrix multiply a staged B
// row zeroed for the purpose (slabs at the matrix's ends); every other term
// outside the band multiplies a zero operand, so operands must be finite (as
// for any dense-tile evaluation: 0 * inf is NaN).
#include "band_mfma.hpp"
#include "common.hpp"

namespace diagpu {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const float* p)
{
    // base p, no stride, the full 32-bit range (offsets are checked to stay
    // below 2^32 before this form is used), the gfx9 raw-dword format
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, -1, 0x00020000);
}

__global__ __launch_bounds__(kMfmaThreads) void k_band_mfma(
    int32_t n, const int32_t* __restrict__ A_off, const int64_t* __restrict__ A_starts, int32_t nA,
    const float* __restrict__ Av, const int32_t* __restrict__ B_off,
    const int64_t* __restrict__ B_starts, int32_t nB, const float* __restrict__ Bv,
    const int32_t* __restrict__ C_off, const int64_t* __restrict__ C_starts, int32_t nC,
    float* __restrict__ Cv, MfmaGeom g, int32_t slabs, int32_t per_wave)
{
    extern __shared__ float lds[];
    const int aspan = g.a_max - g.a_min, bspan = g.b_max - g.b_min, cspan = aspan + bspan;
    const int c_min = g.a_min + g.b_min, c_max = g.a_max + g.b_max;
    const int WM = g.wm, SB = g.sb, BUF = g.buf, B0 = g.b0;
    const int t = (int)threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    int64_t* cst = reinterpret_cast<int64_t*>(lds);                   // [cspan + 1]
    int32_t* absent = reinterpret_cast<int32_t*>(cst + cspan + 1);   // [aspan + bspan + 2]
    int32_t* n_abs = absent + aspan + bspan + 2;                     // [2]
    float* wbuf = lds + mfma_meta_bytes(aspan, bspan) / 4 + (int64_t)wave * BUF;

    // set-up: the C start of every offset (-1: no diagonal); which A and B
    // offsets of the ranges have no diagonal
    for (int r = t; r <= cspan; r += kMfmaThreads) cst[r] = -1;
    for (int r = t; r <= aspan + bspan + 1; r += kMfmaThreads) absent[r] = 1;
    __syncthreads();
    for (int c = t; c < nC; c += kMfmaThreads) {
        const int rel = C_off[c] - c_min;
        if (rel >= 0 && rel <= cspan) cst[rel] = C_starts[c];
    }
    for (int d = t; d < nA; d += kMfmaThreads) absent[A_off[d] - g.a_min] = 0;
    for (int d = t; d < nB; d += kMfmaThreads) absent[aspan + 1 + B_off[d] - g.b_min] = 0;
    __syncthreads();
    if (t == 0) {   // compact the flags into the lists: A rows, then B rows
        int na = 0, nb = 0;
        for (int r = 0; r <= aspan; ++r)
            if (absent[r]) absent[na++] = r;
        for (int r = 0; r <= bspan; ++r)
            if (absent[aspan + 1 + r]) absent[aspan + 1 + nb++] = r;
        n_abs[0] = na;
        n_abs[1] = nb;
    }
    __syncthreads();
    const int na_abs = n_abs[0], nb_abs = n_abs[1];

    const int64_t s0 = ((int64_t)blockIdx.x * kMfmaWaves + wave) * per_wave;
    const int64_t s1 = s0 + per_wave < slabs ? s0 + per_wave : slabs;
    if (s0 >= s1) return;

    // Per-diagonal metadata, one value per lane, read with readlane (no
    // memory round trip in the staging and store loops): lane d holds A's and
    // B's diagonal d (nA <= 33, nB <= 49), lane rel the C start of offset
    // c_min + rel (c span <= 48); each diagonal's LDS row; and for the
    // buffer form, the byte offset of its row 0 (A: row i0 = 0, B: window row
    // 0 at k = a_min, C: row 0), wrapping mod 2^32 (every element's own
    // offset lies below 2^32 where that form is used).
    const int l_aoff = lane < nA ? A_off[lane] : 0;
    const int64_t l_ast = lane < nA ? A_starts[lane] : 0;
    const int l_boff = lane < nB ? B_off[lane] : 0;
    const int64_t l_bst = lane < nB ? B_starts[lane] : 0;
    const int64_t l_cst = lane <= cspan ? cst[lane] : -1;
    const int l_arow = (1 + l_aoff - g.a_min) * kMfmaStrideA;
    const int l_brow = B0 + (1 + l_boff - g.b_min) * SB;
    const uint32_t l_aso = (uint32_t)(4 * (l_ast + (l_aoff < 0 ? l_aoff : 0)));
    const uint32_t l_bso = (uint32_t)(4 * (l_bst + (l_boff < 0 ? l_boff : 0) + g.a_min));
    const uint32_t l_cso = (uint32_t)(4 * (l_cst + (c_min + lane < 0 ? c_min + lane : 0)));
    const uint64_t c_present = __builtin_amdgcn_ballot_w64(lane <= cspan && l_cst >= 0);
    constexpr int64_t kLim = (1LL << 32) - 4096;
    const bool fits = (lane >= nA || (l_ast >= 0 && 4 * (l_ast + n) < kLim)) &&
                      (lane >= nB || (l_bst >= 0 && 4 * (l_bst + n) < kLim)) &&
                      (lane > cspan || l_cst < 0 || 4 * (l_cst + n) < kLim);
    const bool buf32 = __builtin_amdgcn_ballot_w64(!fits) == 0;
    const __amdgpu_buffer_rsrc_t rA = raw_rsrc(Av), rB = raw_rsrc(Bv), rC = raw_rsrc(Cv);
    const int vo = 4 * lane;
    // A slab whose A rows, B window and C rows all lie inside their
    // diagonals: positions need no clamp and stores no test.
    auto interior = [&](int64_t s) {
        const int64_t i0 = s * kMfmaRows, k0 = i0 + g.a_min;
        return i0 + (g.a_min < 0 ? g.a_min : 0) >= 0 &&
               i0 + kMfmaRows - 1 + (g.a_max > 0 ? g.a_max : 0) <= n - 1 &&
               k0 + (g.b_min < 0 ? g.b_min : 0) >= 0 &&
               k0 + WM - 1 + (g.b_max > 0 ? g.b_max : 0) <= n - 1 &&
               i0 + (c_min < 0 ? c_min : 0) >= 0 &&
               i0 + kMfmaRows - 1 + (c_max > 0 ? c_max : 0) <= n - 1;
    };

    // One wave's 64 rows of one diagonal: lane l loads the element of row w
    // (its HM position clamped into the diagonal, so the address is valid)
    // into dst[l] with a direct global-to-LDS load.
    auto load_row = [&](const float* __restrict__ vals, int64_t st, int o, int64_t w, float* dst) {
        const int len = n - (o < 0 ? -o : o);
        int64_t pos = w + (o < 0 ? o : 0);
        pos = pos < 0 ? 0 : (pos > len - 1 ? len - 1 : pos);
        __builtin_amdgcn_global_load_lds(vals + st + pos, dst, 4, 0, 0);
    };
    // Slab s into a buffer: the zero rows and the rows of absent offsets
    // zeroed (C values of an earlier slab lie there), every other row loaded.
    auto stage = [&](int64_t s, float* buf) {
        const int64_t i0 = s * kMfmaRows;
        float* zb_lo = buf + B0;
        float* zb_hi = buf + B0 + (bspan + 2) * SB;
        buf[lane] = 0.f;
        buf[(aspan + 2) * kMfmaStrideA + lane] = 0.f;
        zb_lo[lane] = 0.f;
        zb_hi[lane] = 0.f;
        if (lane < WM - 64) {
            zb_lo[64 + lane] = 0.f;
            zb_hi[64 + lane] = 0.f;
        }
        for (int e = 0; e < na_abs; ++e) buf[(1 + absent[e]) * kMfmaStrideA + lane] = 0.f;
        for (int e = 0; e < nb_abs; ++e) {
            float* row = buf + B0 + (1 + absent[aspan + 1 + e]) * SB;
            row[lane] = 0.f;
            if (lane < WM - 64) row[64 + lane] = 0.f;
        }
        if (buf32 && interior(s)) {
            const uint32_t ib = 4 * (uint32_t)i0;
            for (int d = 0; d < nA; ++d) {
                const uint32_t so = (uint32_t)__builtin_amdgcn_readlane((int)l_aso, d) + ib;
                float* dst = buf + __builtin_amdgcn_readlane(l_arow, d);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr)dst, 4, vo, (int)so, 0, 0);
            }
            for (int d = 0; d < nB; ++d) {
                const uint32_t so = (uint32_t)__builtin_amdgcn_readlane((int)l_bso, d) + ib;
                float* dst = buf + __builtin_amdgcn_readlane(l_brow, d);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_ptr)dst, 4, vo, (int)so, 0, 0);
                if (lane < WM - 64)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_ptr)(dst + 64), 4, vo,
                                                             (int)(so + 256), 0, 0);
            }
            return;
        }
        for (int d = 0; d < nA; ++d) {
            const int o = __builtin_amdgcn_readlane(l_aoff, d);
            const int64_t st = ((int64_t)__builtin_amdgcn_readlane((int)(l_ast >> 32), d) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)l_ast, d);
            load_row(Av, st, o, i0 + lane, buf + __builtin_amdgcn_readlane(l_arow, d));
        }
        const int64_t k0 = i0 + g.a_min;
        for (int d = 0; d < nB; ++d) {
            const int o = __builtin_amdgcn_readlane(l_boff, d);
            const int64_t st = ((int64_t)__builtin_amdgcn_readlane((int)(l_bst >> 32), d) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)l_bst, d);
            float* dst = buf + __builtin_amdgcn_readlane(l_brow, d);
            load_row(Bv, st, o, k0 + lane, dst);
            if (lane < WM - 64) load_row(Bv, st, o, k0 + 64 + lane, dst + 64);
        }
    };
    // Slab sp's C values (in C_w) to memory: one coalesced
    // run of kMfmaRows values per C diagonal.  Interior slabs read the LDS
    // values in groups of 8 ahead of their stores.
    auto store = [&](int64_t sp, const float* C_w) {
        if (buf32 && interior(sp)) {
            const uint32_t ib = 4 * (uint32_t)(sp * kMfmaRows);
            for (int rel0 = 0; rel0 <= cspan; rel0 += 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    v[u] = C_w[(rel0 + u <= cspan ? rel0 + u : cspan) * kMfmaStrideC + lane];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int rel = rel0 + u;
                    if (rel <= cspan && ((c_present >> rel) & 1)) {
                        const uint32_t so = (uint32_t)__builtin_amdgcn_readlane((int)l_cso, rel) + ib;
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v[u]), rC,
                                                              vo, (int)so, 0);
                    }
                }
            }
            return;
        }
        const int64_t i = sp * kMfmaRows + lane;
        for (int rel = 0; rel <= cspan; ++rel) {
            if (!((c_present >> rel) & 1)) continue;
            const int64_t c0 = ((int64_t)__builtin_amdgcn_readlane((int)(l_cst >> 32), rel) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)l_cst, rel);
            const int dc = c_min + rel;
            const float v = C_w[rel * kMfmaStrideC + lane];
            if (i < n && i + dc >= 0 && i + dc < n) Cv[c0 + i + (dc < 0 ? dc : 0)] = v;
        }
    };

    const int q = lane >> 4, r = lane & 15;        // MFMA lane coordinates
    const int la = (q - r) * kMfmaStrideA, lb = (r - q) * SB;   // lane parts of the operand rows
    const int amax = (aspan + 1) * kMfmaStrideA, bmax = (bspan + 1) * SB;
    // Where lane (q, r) writes value j of column tile ct: C row rel = 16 ct +
    // r - 4 q - j at column 4 q + j (tile u 16 u further), or the dump past
    // the C rows where rel lies outside C's range.
    int caddr[kMfmaMaxCt][4];
#pragma unroll
    for (int ct = 0; ct < kMfmaMaxCt; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int rel = 16 * ct + r - 4 * q - j;
            caddr[ct][j] = (rel >= 0 && rel <= cspan) ? rel * kMfmaStrideC + 4 * q + j
                                                      : (cspan + 1) * kMfmaStrideC + lane;
        }

    for (int64_t s = s0; s < s1; ++s) {
        float* cur = wbuf;
        stage(s, cur);
        __builtin_amdgcn_s_waitcnt(0);   // the slab's loads have landed in LDS
        const int64_t i0 = s * kMfmaRows;
        const int64_t k0 = i0 + g.a_min;
        if (!interior(s) && (k0 < 0 || k0 + WM > n)) {
            // B rows k outside the matrix to zero: their terms A(i, k) B(k, j)
            // then vanish (A's staged values there are finite operand values)
            for (int d = 0; d < nB; ++d) {
                float* row = cur + __builtin_amdgcn_readlane(l_brow, d);
                for (int j = lane; j < WM; j += 64)
                    if (k0 + j < 0 || k0 + j >= n) row[j] = 0.f;
            }
        }
        // operand rows clamped into [-1, span + 1] (the zero rows beyond),
        // as offsets: row x stride clamped into [-stride, (span + 1) stride]
        const float* Ab = cur + kMfmaStrideA + r;
        const float* Bb = cur + B0 + SB + q;
        auto operands = [&](int ct, int ks, float (&av)[4], float (&bv)[4]) {
            const int xa = min(max(la + 4 * kMfmaStrideA * ks, -kMfmaStrideA), amax);
            const int xb = min(max(lb + SB * (16 * ct - 4 * ks), -SB), bmax);
            const float* ap = Ab + xa;
            const float* bp = Bb + xb + 4 * ks;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                av[u] = ap[16 * u];
                bv[u] = bp[16 * u];
            }
        };
        f4 acc[kMfmaMaxCt][4];
#pragma unroll
        for (int ct = 0; ct < kMfmaMaxCt; ++ct)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[ct][u] = f4{0.f, 0.f, 0.f, 0.f};
        auto mfma4 = [&](f4 (&a)[4], const float (&av)[4], const float (&bv)[4]) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                a[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv[u], a[u], 0, 0, 0);
        };
        // per column tile its k steps, two operand sets in turn: the next
        // step's LDS reads go out before the current step's matrix work
#pragma unroll
        for (int ct = 0; ct < kMfmaMaxCt; ++ct) {
            const int lo = g.ks_lo[ct], hi = g.ks_hi[ct];
            if (lo > hi) continue;
            float xa[4], xb[4], ya[4], yb[4];
            operands(ct, lo, xa, xb);
            int ks = lo;
            for (; ks + 2 <= hi; ks += 2) {
                operands(ct, ks + 1, ya, yb);
                mfma4(acc[ct], xa, xb);
                operands(ct, ks + 2, xa, xb);
                mfma4(acc[ct], ya, yb);
            }
            if (ks + 1 <= hi) {
                operands(ct, ks + 1, ya, yb);
                mfma4(acc[ct], xa, xb);
                mfma4(acc[ct], ya, yb);
            } else {
                mfma4(acc[ct], xa, xb);
            }
        }
        // the slab's C values by offset into C_w (the buffer is read no
        // more): lane (q, r), value j of tile u of column tile ct is C(i,
        // i + dc), i = i0 + 16 u + 4 q + j, dc = c_min + 16 ct + r - 4 q - j
        float* C_w = cur;
#pragma unroll
        for (int ct = 0; ct < kMfmaMaxCt; ++ct) {
            if (ct >= g.nct) break;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int u = 0; u < 4; ++u) C_w[caddr[ct][j] + 16 * u] = acc[ct][u][j];
        }
        store(s, cur);
    }
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_spgemm_numeric_band_mfma_f32(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA, const float* A_vals,
    const int32_t* B_off, const int64_t* B_starts, int32_t nB, const float* B_vals,
    const int32_t* C_off, const int64_t* C_starts, int64_t c_ndiag,
    const diagpu_band_info* info, float* C_vals, void* stream)
{
    using namespace diagpu;
    const char* fn = "diagpu_spgemm_numeric_band_mfma_f32";
    if (!info) return fail(DIAGPU_ERR_ARG, "%s: info is NULL", fn);
    if (n < 1 || nA < 1 || nB < 1 || c_ndiag < 0 || c_ndiag > 2 * (int64_t)n - 1)
        return fail(DIAGPU_ERR_ARG, "%s: bad sizes (n=%d nA=%d nB=%d c_ndiag=%lld)", fn, n, nA,
                    nB, (long long)c_ndiag);
    if (info->a_off_min > info->a_off_max || info->b_off_min > info->b_off_max ||
        info->a_off_min <= -n || info->a_off_max >= n || info->b_off_min <= -n ||
        info->b_off_max >= n)
        return fail(DIAGPU_ERR_ARG, "%s: info holds no band_prepare result", fn);
    const MfmaGeom g = mfma_geom(info->a_off_min, info->a_off_max, info->b_off_min,
                                 info->b_off_max);
    if (!g.ok || !info->mfma_eligible || info->mfma_blocks != g.nblk ||
        info->mfma_lds_bytes != g.lds_bytes)
        return fail(DIAGPU_ERR_CAPACITY, "%s: the operands' offset ranges (A %d..%d, B %d..%d) "
                    "are too wide for the MFMA band kernel", fn, info->a_off_min,
                    info->a_off_max, info->b_off_min, info->b_off_max);
    if (c_ndiag == 0) return DIAGPU_OK;
    if (!A_off || !A_starts || !A_vals || !B_off || !B_starts || !B_vals || !C_off ||
        !C_starts || !C_vals)
        return fail(DIAGPU_ERR_ARG, "%s: a pointer is NULL", fn);
    int st = check_hip(hipFuncSetAttribute((const void*)k_band_mfma,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)kMfmaLdsBudget), fn);
    if (st) return st;
    const int64_t slabs = ceil_div<int64_t>(n, kMfmaRows);
    int per_cu = 0;
    st = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_band_mfma,
                                                               kMfmaThreads, (size_t)g.lds_bytes),
                   fn);
    if (st) return st;
    // persistent: as many waves as fit at once (two workgroups per CU), each
    // on a contiguous range of slabs (a slab's B window overlaps the next
    // one's, which then comes from the same XCD's L2)
    const int64_t waves = (int64_t)cu_count() * (per_cu > 0 ? per_cu : 1) * kMfmaWaves;
    const int64_t per_wave = ceil_div<int64_t>(slabs, waves);
    const int64_t wg = ceil_div<int64_t>(ceil_div<int64_t>(slabs, per_wave), kMfmaWaves);
    hipLaunchKernelGGL(k_band_mfma, dim3((unsigned)wg), dim3(kMfmaThreads), (size_t)g.lds_bytes,
                       as_stream(stream), n, A_off, A_starts, nA, A_vals, B_off, B_starts, nB,
                       B_vals, C_off, C_starts, (int32_t)c_ndiag, C_vals, g, (int32_t)slabs,
                       (int32_t)per_wave);
    return check_launch(fn);
}

}  // extern "C"
