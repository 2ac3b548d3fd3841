// DIA x DIA SpGEMM numeric phase for narrow bands on the matrix cores: the
// fp32 MFMA variant of the band kernel (spgemm_band.hip) for gemm_diag-type
// products (gemm_diag/gemm_diag.cu:119-329 tiles the same product, 4 x 4
// diagonals x 32 columns, with scalar FMAs and atomics).
//
// The band product is a dense matrix product restricted to a band, so each
// 16-row tile of C is computed as the dense 16 x 16 x 4 MFMA blocks that
// intersect the band (band_mfma.hpp: the issued (ct, ks) blocks), with the
// operand elements outside the band read as zeros.  Every wave works alone
// on slabs of kMfmaRows rows (no workgroup barrier after set-up), with its
// own LDS (row strides kMfmaStrideA / B / C, chosen against bank conflicts):
//   A_z, B_z                     zero rows, read for offsets outside A's /
//                                B's range
//   A_w [a_span + 1][kMfmaRows]  row (da - a_min) = A's diagonal da at the
//                                slab's rows (zeros for absent offsets)
//   B_w [b_span + 1][wm]         row (db - b_min) = B's diagonal db at rows
//                                k = i0 + a_min + (0..wm-1)
//   C_w [c_span + 1][kMfmaRows]  row (dc - c_min) = the slab's C values,
//                                written over A_w and B_w after the matrix work
// and the workgroup shares the C starts by offset and the lists of absent A
// and B offsets.  Per slab a wave zeroes the rows of absent offsets, stages
// the others with direct global-to-LDS loads, waits for its own loads only,
// and runs, per column tile ct, the issued blocks of ct over its four 16-row
// tiles (v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16] and holds D[4 (l / 16) + j][l % 16]), with every column
// tile's accumulators in registers; then it writes the slab's C values by
// offset into C_w and stores one coalesced run of kMfmaRows values per C
// diagonal.  Eight waves per CU (two workgroups) overlap one slab's loads
// with another's matrix work.
//
// The sums run in MFMA order, not plan order, so C matches the gather and
// band kernels to rounding (1e-5 of the term sum), not bit for bit.  Terms
// whose k (= A's column, B's row) lies outside the matrix are zeroed; every
// other term outside the band multiplies a zero operand, so operands must be
// finite (as for any dense-tile evaluation: 0 * inf is NaN).
#include "band_mfma.hpp"
#include "common.hpp"

namespace diagpu {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kMfmaThreads) void k_band_mfma(
    int32_t n, const int32_t* __restrict__ A_off, const int64_t* __restrict__ A_starts, int32_t nA,
    const float* __restrict__ Av, const int32_t* __restrict__ B_off,
    const int64_t* __restrict__ B_starts, int32_t nB, const float* __restrict__ Bv,
    const int32_t* __restrict__ C_off, const int64_t* __restrict__ C_starts, int32_t nC,
    float* __restrict__ Cv, MfmaGeom g, int32_t slabs)
{
    extern __shared__ float lds[];
    const int aspan = g.a_max - g.a_min, bspan = g.b_max - g.b_min, cspan = aspan + bspan;
    const int c_min = g.a_min + g.b_min, WM = g.wm;
    const int t = (int)threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    const int64_t per_wave = mfma_wave_floats(aspan, bspan);
    float* A_z = lds + wave * per_wave;
    float* B_z = A_z + kMfmaStrideA;
    float* A_w = B_z + kMfmaStrideB;
    float* B_w = A_w + (aspan + 1) * kMfmaStrideA;
    float* C_w = A_w;
    int64_t* cst = reinterpret_cast<int64_t*>(lds + kMfmaWaves * per_wave);   // [cspan + 1]
    int32_t* absent = reinterpret_cast<int32_t*>(cst + cspan + 1);  // [aspan + bspan + 2]
    int32_t* n_abs = absent + aspan + bspan + 2;                     // [2]

    // set-up: zero this wave's rows; the C start of every offset (-1: no
    // diagonal); which A and B offsets of the ranges have no diagonal
    for (int64_t i = lane; i < per_wave; i += 64) A_z[i] = 0.f;
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

    // One wave's 64 rows of one diagonal: lane l loads the element of row w
    // (its HM position clamped into the diagonal, so the address is valid)
    // into dst[l] with a direct global-to-LDS load.
    auto load_row = [&](const float* __restrict__ vals, int64_t st, int o, int64_t w, float* dst) {
        const int len = n - (o < 0 ? -o : o);
        int64_t pos = w + (o < 0 ? o : 0);
        pos = pos < 0 ? 0 : (pos > len - 1 ? len - 1 : pos);
        __builtin_amdgcn_global_load_lds(vals + st + pos, dst, 4, 0, 0);
    };
    const int q = lane >> 4, r = lane & 15;        // MFMA lane coordinates
    const int64_t stride = (int64_t)gridDim.x * kMfmaWaves;
    for (int64_t slab = (int64_t)blockIdx.x * kMfmaWaves + wave; slab < slabs; slab += stride) {
        const int64_t i0 = slab * kMfmaRows;
        // rows of absent offsets: zero again (the last slab's C values lie there)
        for (int e = 0; e < na_abs; ++e) A_w[absent[e] * kMfmaStrideA + lane] = 0.f;
        for (int e = 0; e < nb_abs; ++e)
            for (int seg = 0; seg < WM / 64; ++seg)
                B_w[absent[aspan + 1 + e] * kMfmaStrideB + 64 * seg + lane] = 0.f;
        for (int d = 0; d < nA; ++d) {
            const int o = A_off[d];
            load_row(Av, A_starts[d], o, i0 + lane, A_w + (o - g.a_min) * kMfmaStrideA);
        }
        for (int d = 0; d < nB; ++d) {
            const int o = B_off[d];
            float* dst = B_w + (o - g.b_min) * kMfmaStrideB;
            for (int seg = 0; seg < WM / 64; ++seg)
                load_row(Bv, B_starts[d], o, i0 + g.a_min + 64 * seg + lane, dst + 64 * seg);
        }
        __builtin_amdgcn_s_waitcnt(0);   // this wave's direct loads have landed in LDS

        // every k of the slab inside the matrix: no masking
        const bool interior = i0 + g.a_min >= 0 && i0 + WM + g.a_min <= n;
        f4 acc[kMfmaMaxCt][4];
#pragma unroll
        for (int ct = 0; ct < kMfmaMaxCt; ++ct)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[ct][u] = f4{0.f, 0.f, 0.f, 0.f};
        int b = 0;
#pragma unroll
        for (int ct = 0; ct < kMfmaMaxCt; ++ct) {
            for (; b < g.nblk && (g.blk[b] >> 5) == ct; ++b) {
                const int ks = g.blk[b] & 31;
                const int da = g.a_min + 4 * ks + q - r;
                const int db = c_min + 16 * ct + r - (g.a_min + 4 * ks + q);
                const float* ap = (da >= g.a_min && da <= g.a_max)
                                      ? A_w + (da - g.a_min) * kMfmaStrideA + r
                                      : A_z + r;
                const float* bp = (db >= g.b_min && db <= g.b_max)
                                      ? B_w + (db - g.b_min) * kMfmaStrideB + 4 * ks + q
                                      : B_z + q;
                float av[4], bv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    av[u] = ap[16 * u];
                    bv[u] = bp[16 * u];
                }
                if (!interior) {
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int64_t k = i0 + 16 * u + g.a_min + 4 * ks + q;
                        if (k < 0 || k >= n) av[u] = bv[u] = 0.f;
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc[ct][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv[u], acc[ct][u], 0,
                                                                      0, 0);
            }
        }
        // The slab's C values by offset into C_w (A_w and B_w are read no
        // more): lane (q, r), value j of tile u of column tile ct is C(i,
        // i + dc), i = i0 + 16 u + 4 q + j, dc = c_min + 16 ct + r - 4 q - j.
#pragma unroll
        for (int ct = 0; ct < kMfmaMaxCt; ++ct) {
            if (ct >= g.nct) break;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int rel = 16 * ct + r - 4 * q - j;
                if (rel >= 0 && rel <= cspan) {
#pragma unroll
                    for (int u = 0; u < 4; ++u) C_w[rel * kMfmaStrideC + 16 * u + 4 * q + j] = acc[ct][u][j];
                }
            }
        }
        // then one coalesced run of kMfmaRows values per C diagonal
        for (int rel = 0; rel <= cspan; ++rel) {
            const int64_t c0 = cst[rel];
            if (c0 < 0) continue;
            const int dc = c_min + rel;
            const int64_t i = i0 + lane;
            const float v = C_w[rel * kMfmaStrideC + lane];
            if (i < n && i + dc >= 0 && i + dc < n) Cv[c0 + i + (dc < 0 ? dc : 0)] = v;
        }
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
    // persistent: as many workgroups as fit at once, each wave on slabs
    // wave, wave + stride, ...
    int64_t wg = (int64_t)cu_count() * (per_cu > 0 ? per_cu : 1);
    const int64_t need = ceil_div<int64_t>(slabs, kMfmaWaves);
    if (wg > need) wg = need;
    hipLaunchKernelGGL(k_band_mfma, dim3((unsigned)wg), dim3(kMfmaThreads), (size_t)g.lds_bytes,
                       as_stream(stream), n, A_off, A_starts, nA, A_vals, B_off, B_starts, nB,
                       B_vals, C_off, C_starts, (int32_t)c_ndiag, C_vals, g, (int32_t)slabs);
    return check_launch(fn);
}

}  // extern "C"
