// DIA SpMV on the column-indexed Recon layout, gfx950.
//
//   y[r] = sum_k [0 <= r + d_k < lim] Recon[k][r + d_k] * x[r + d_k],
//   lim = min(cols, x_size)
//
// (spmv/src/dia_reconstruct.cuh:22, bounds as in
// spmv/src/tc_spmv_regdirect_kernel.cu:85-104).  The reference lifts the band
// to a TF32 MMA and keeps 1/16 of the product; here the sum is what it is, an
// HBM stream: every useful value is read once and fused into its row's
// accumulator.
//
// Mapping.  A workgroup of 256 lanes owns a tile of 256 x R consecutive rows,
// R = 16 / sizeof(T) (4 floats or 2 doubles): each lane owns R consecutive
// rows r..r+R-1.  For diagonal k the lane needs Recon[k][r+d_k ..] and
// x[r+d_k ..]: both are 16-byte runs at the same column, one 128-bit load
// each (dword aligned: gfx950 serves unaligned global loads), and the 64
// lanes of a wave cover 1 KiB of each stream.  Value loads and the y store are
// non-temporal: each value is used once, while x stays in L2 for the tiles
// that re-read it.
//
// Memory-level parallelism.  What bounds this kernel is how many HBM bytes
// each CU keeps in flight, not the x re-reads or the misalignment (measured:
// a 64-stream read with the same offsets and no x runs at 80% of 8 TB/s, and
// adding the x loads costs 3 points).  So loads are never drained in chunks:
// the ring kernel keeps W diagonals' loads in flight per lane at all times --
// step j consumes slot j and refills it with the diagonal W ahead, and
// sched_barrier pins that order so the compiler emits a steady
// s_waitcnt vmcnt(2W-2) instead of hoisting or sinking the loads.  Offsets
// travel 64 at a time in one VGPR (lane l holds d_{g0+l}) and are broadcast
// with readlane, which needs no memory wait.  For K <= 5 the short kernel
// takes the offsets with scalar loads (the scalar cache does not queue behind
// the HBM stream) and issues all 2K loads straight-line.
//
// Edge tiles.  A tile whose rows or columns leave the matrix for some
// diagonal runs the same ring with per-element loads at clamped (always
// valid) columns and masked FMAs: no branch around a load, so the loads
// pipeline like the interior ones.  An edge tile is also dispatched early
// (odd XCDs walk their row range from the end), since the slowest tile sets
// the kernel's end.
//
// XCD awareness: workgroup b runs on XCD b mod 8; tiles are remapped so each
// XCD owns one contiguous eighth of the rows.  x[c] is used by rows c - d_k
// of every diagonal, i.e. by this tile and by tiles up to max|d_k| rows away,
// which then sit on the same XCD and find x in its L2.
#include <climits>

#include "common.hpp"

namespace diagpu {
namespace {

constexpr int kBlock = 256;

template <typename T> struct Vec16;   // 16 bytes of T, element-aligned
template <> struct Vec16<float> {
    typedef float type __attribute__((ext_vector_type(4), aligned(4)));
};
template <> struct Vec16<double> {
    typedef double type __attribute__((ext_vector_type(2), aligned(8)));
};

template <typename T> constexpr int rows_per_lane() { return 16 / (int)sizeof(T); }
template <typename T> constexpr int tile_rows() { return kBlock * rows_per_lane<T>(); }

// Diagonals in flight per lane: interior ring (16-byte loads) and edge ring
// (per-element loads).  Chosen so the kernel stays within 64 VGPRs (8 waves
// per SIMD).
constexpr int kRing = 6;
constexpr int kRingEdge = 3;
constexpr int kShortMax = 5;   // K <= kShortMax: straight-line kernel

template <typename T>
__device__ __forceinline__ typename Vec16<T>::type ld16_stream(const T* p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const typename Vec16<T>::type*>(p));
}
template <typename T>
__device__ __forceinline__ typename Vec16<T>::type ld16(const T* p)
{
    return *reinterpret_cast<const typename Vec16<T>::type*>(p);
}
template <typename T>
__device__ __forceinline__ void st16_stream(T* p, typename Vec16<T>::type v)
{
    __builtin_nontemporal_store(v, reinterpret_cast<typename Vec16<T>::type*>(p));
}

__device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_(double a, double b, double c) { return __builtin_fma(a, b, c); }

// Lane-wise helpers on 16-byte vectors.
template <typename V>
__device__ __forceinline__ V vfma(const V& a, const V& b, const V& c)
{
    V r;
#pragma unroll
    for (int e = 0; e < (int)(16 / sizeof(a[0])); ++e) r[e] = fma_(a[e], b[e], c[e]);
    return r;
}

// Tile index of workgroup b: XCD x = b mod 8 owns tiles [x*per_xcd,
// (x+1)*per_xcd); even XCDs walk their range upwards, odd ones downwards, so
// the last tile of the matrix (an edge tile) is among the first dispatched.
__device__ __forceinline__ int tile_of_block(int per_xcd)
{
    const int x = (int)(blockIdx.x % kNumXcd);
    const int l = (int)(blockIdx.x / kNumXcd);
    return x * per_xcd + ((x & 1) ? per_xcd - 1 - l : l);
}

// min and max of a group of offsets held one per lane (lanes >= gn hold a
// copy of a valid offset), uniform across the wave.
__device__ __forceinline__ void wave_minmax(int v, int& lo, int& hi)
{
    int a = v, b = v;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) {
        const int oa = __shfl_xor(a, s);
        const int ob = __shfl_xor(b, s);
        a = oa < a ? oa : a;
        b = ob > b ? ob : b;
    }
    lo = __builtin_amdgcn_readfirstlane(a);
    hi = __builtin_amdgcn_readfirstlane(b);
}

// One group of gn <= 64 diagonals (offsets in `ov`, lane l = d_{g0+l};
// values `vg` = Recon row g0) accumulated into `acc` for the lane's R rows
// starting at row `r`.  W loads in flight; every index is clamped to the
// group so all loads are valid, and the slots past the group are masked.
//
// EDGE = false: the whole tile is in range (rows < `rows`, every column in
// [0, lim)); 16-byte loads.  EDGE = true: per-element loads at columns
// clamped into [0, lim), terms whose column is outside masked.
template <typename T, int W, bool EDGE>
__device__ __forceinline__ void ring_group(int64_t r, int64_t cols, int64_t lim, int gn, int ov,
                                           const T* __restrict__ vg, const T* __restrict__ x,
                                           typename Vec16<T>::type& acc)
{
    typedef typename Vec16<T>::type V;
    constexpr int R = rows_per_lane<T>();
    V a[W], b[W];
    // EDGE: the lane's first column for the slot's diagonal, clamped to
    // [-R, lim] (a column outside that range is as out of range as its clamp)
    int32_t c0[W];
    (void)c0;
    auto issue = [&](int j, int k) {
        const int d = __builtin_amdgcn_readlane(ov, k);
        if constexpr (!EDGE) {
            a[j] = ld16_stream<T>(vg + (int64_t)k * cols + r + d);
            b[j] = ld16<T>(x + r + d);
        } else {
            const int64_t c = r + d;
            c0[j] = (int32_t)(c < -R ? -R : (c > lim ? lim : c));
            const T* vk = vg + (int64_t)k * cols;
#pragma unroll
            for (int e = 0; e < R; ++e) {
                int64_t cc = c + e;
                cc = cc < 0 ? 0 : (cc >= lim ? lim - 1 : cc);   // always a valid address
                a[j][e] = __builtin_nontemporal_load(vk + (uint32_t)cc);
                b[j][e] = x[(uint32_t)cc];
            }
        }
    };
    auto consume = [&](int j, bool on) {
        if constexpr (!EDGE) {
            const V t = vfma(a[j], b[j], acc);
            acc = on ? t : acc;
        } else {
#pragma unroll
            for (int e = 0; e < R; ++e) {
                const int64_t c = (int64_t)c0[j] + e;
                const bool ok = on && c >= 0 && c < lim;
                const T t = fma_(a[j][e], b[j][e], acc[e]);
                acc[e] = ok ? t : acc[e];
            }
        }
    };

#pragma unroll
    for (int j = 0; j < W; ++j) issue(j, j < gn ? j : gn - 1);
    __builtin_amdgcn_sched_barrier(0);
    int k0 = 0;
    while (k0 + 2 * W <= gn) {   // every refill of this round is in range
#pragma unroll
        for (int j = 0; j < W; ++j) {
            consume(j, true);
            __builtin_amdgcn_sched_barrier(0);
            issue(j, k0 + W + j);
            __builtin_amdgcn_sched_barrier(0);
        }
        k0 += W;
    }
    // Last two rounds: slots hold k0 .. k0+W-1 (those >= gn are clamped
    // copies); refills are clamped the same way.
#pragma unroll
    for (int j = 0; j < W; ++j) {
        consume(j, k0 + j < gn);
        __builtin_amdgcn_sched_barrier(0);
        const int kn = k0 + W + j;
        issue(j, kn < gn ? kn : gn - 1);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < W - 1; ++j) consume(j, k0 + W + j < gn);
}

template <typename T>
__device__ __forceinline__ void store_rows(T* __restrict__ y, int64_t r, int64_t rows,
                                           const typename Vec16<T>::type& acc, bool full)
{
    if (full) {
        st16_stream<T>(y + r, acc);
    } else {
#pragma unroll
        for (int e = 0; e < rows_per_lane<T>(); ++e)
            if (r + e < rows) y[r + e] = acc[e];
    }
}

// General K: groups of 64 diagonals, each through the ring (MULTI = false:
// K <= 64, one group, the offsets VGPR loaded once).
template <typename T, bool MULTI>
__global__ __launch_bounds__(kBlock) void spmv_ring_kernel(
    int32_t rows, int32_t cols, int64_t lim, int32_t K, const int32_t* __restrict__ offs,
    const T* __restrict__ vals, const T* __restrict__ x, T* __restrict__ y, int32_t tiles,
    int32_t per_xcd)
{
    typedef typename Vec16<T>::type V;
    constexpr int TILE = tile_rows<T>();
    const int tile = tile_of_block(per_xcd);
    if (tile >= tiles) return;
    const int lane = (int)threadIdx.x & 63;
    const int64_t r0 = (int64_t)tile * TILE;
    const int64_t r = r0 + (int64_t)threadIdx.x * rows_per_lane<T>();

    // offset range over all groups (one vector load per 64 offsets)
    const int g0n = K < 64 ? K : 64;
    const int ov0 = offs[lane < g0n ? lane : g0n - 1];
    int dmin, dmax;
    wave_minmax(ov0, dmin, dmax);
    if constexpr (MULTI) {
        for (int g0 = 64; g0 < K; g0 += 64) {
            const int gn = (K - g0) < 64 ? (K - g0) : 64;
            int lo, hi;
            wave_minmax(offs[g0 + (lane < gn ? lane : gn - 1)], lo, hi);
            dmin = lo < dmin ? lo : dmin;
            dmax = hi > dmax ? hi : dmax;
        }
    }
    const bool interior = r0 + TILE <= rows && r0 + dmin >= 0 && r0 + TILE + (int64_t)dmax <= lim;

    V acc;
#pragma unroll
    for (int e = 0; e < rows_per_lane<T>(); ++e) acc[e] = T(0);
    if constexpr (!MULTI) {
        if (interior)
            ring_group<T, kRing, false>(r, cols, lim, K, ov0, vals, x, acc);
        else
            ring_group<T, kRingEdge, true>(r, cols, lim, K, ov0, vals, x, acc);
    } else {
        for (int g0 = 0; g0 < K; g0 += 64) {
            const int gn = (K - g0) < 64 ? (K - g0) : 64;
            const int ov = g0 == 0 ? ov0 : offs[g0 + (lane < gn ? lane : gn - 1)];
            const T* vg = vals + (int64_t)g0 * cols;
            if (interior)
                ring_group<T, kRing, false>(r, cols, lim, gn, ov, vg, x, acc);
            else
                ring_group<T, kRingEdge, true>(r, cols, lim, gn, ov, vg, x, acc);
        }
    }
    store_rows<T>(y, r, rows, acc, interior);
}

// K == KF <= kShortMax: offsets by scalar loads, all 2K loads straight-line.
template <typename T, int KF>
__global__ __launch_bounds__(kBlock) void spmv_short_kernel(
    int32_t rows, int32_t cols, int64_t lim, int32_t K, const int32_t* __restrict__ offs,
    const T* __restrict__ vals, const T* __restrict__ x, T* __restrict__ y, int32_t tiles,
    int32_t per_xcd)
{
    typedef typename Vec16<T>::type V;
    constexpr int TILE = tile_rows<T>();
    const int tile = tile_of_block(per_xcd);
    if (tile >= tiles) return;
    const int64_t r0 = (int64_t)tile * TILE;
    const int64_t r = r0 + (int64_t)threadIdx.x * rows_per_lane<T>();
    (void)K;

    int d[KF > 0 ? KF : 1];
    int dmin = INT_MAX, dmax = INT_MIN;
#pragma unroll
    for (int k = 0; k < KF; ++k) {
        d[k] = offs[k];
        dmin = d[k] < dmin ? d[k] : dmin;
        dmax = d[k] > dmax ? d[k] : dmax;
    }
    const bool interior =
        r0 + TILE <= rows && (KF == 0 || (r0 + dmin >= 0 && r0 + TILE + (int64_t)dmax <= lim));

    V acc;
#pragma unroll
    for (int e = 0; e < rows_per_lane<T>(); ++e) acc[e] = T(0);
    if constexpr (KF > 0) {
        if (interior) {
            V a[KF], b[KF];
#pragma unroll
            for (int k = 0; k < KF; ++k) {
                a[k] = ld16_stream<T>(vals + (int64_t)k * cols + r + d[k]);
                b[k] = ld16<T>(x + r + d[k]);
            }
#pragma unroll
            for (int k = 0; k < KF; ++k) acc = vfma(a[k], b[k], acc);
        } else {
            const int lane = (int)threadIdx.x & 63;
            const int ov = offs[lane < KF ? lane : KF - 1];
            ring_group<T, kRingEdge, true>(r, cols, lim, KF, ov, vals, x, acc);
        }
    }
    store_rows<T>(y, r, rows, acc, interior);
}

template <typename T>
using SpmvKernel = void (*)(int32_t, int32_t, int64_t, int32_t, const int32_t*, const T*,
                            const T*, T*, int32_t, int32_t);

template <typename T>
SpmvKernel<T> pick_kernel(int K)
{
    switch (K) {
    case 0: return spmv_short_kernel<T, 0>;
    case 1: return spmv_short_kernel<T, 1>;
    case 2: return spmv_short_kernel<T, 2>;
    case 3: return spmv_short_kernel<T, 3>;
    case 4: return spmv_short_kernel<T, 4>;
    case 5: return spmv_short_kernel<T, 5>;
    default: return K <= 64 ? spmv_ring_kernel<T, false> : spmv_ring_kernel<T, true>;
    }
}
static_assert(kShortMax == 5, "pick_kernel covers K = 0..5");

template <typename T, typename View>
int spmv_launch(const View* R, const T* x, int64_t x_size, T* y, void* stream, const char* name)
{
    if (!R) return fail(DIAGPU_ERR_ARG, "%s: R is NULL", name);
    if (R->rows < 0 || R->cols < 0 || R->num_diags < 0)
        return fail(DIAGPU_ERR_ARG, "%s: negative size (rows=%d cols=%d num_diags=%d)", name,
                    R->rows, R->cols, R->num_diags);
    if (x_size < 0) return fail(DIAGPU_ERR_ARG, "%s: negative x_size %lld", name, (long long)x_size);
    if (R->rows == 0) return DIAGPU_OK;
    if (!y) return fail(DIAGPU_ERR_ARG, "%s: y is NULL", name);
    const int64_t lim = x_size < R->cols ? x_size : (int64_t)R->cols;
    int K = R->num_diags;
    if (K > 0) {
        if (!R->diag_offsets) return fail(DIAGPU_ERR_ARG, "%s: diag_offsets is NULL", name);
        if (R->cols > 0 && !R->values) return fail(DIAGPU_ERR_ARG, "%s: values is NULL", name);
        if (lim > 0 && !x) return fail(DIAGPU_ERR_ARG, "%s: x is NULL", name);
    }
    if (lim == 0) K = 0;   // no column in range: y = 0 without touching values or x
    const int32_t tiles = (int32_t)ceil_div<int64_t>(R->rows, tile_rows<T>());
    const int32_t per_xcd = ceil_div<int32_t>(tiles, kNumXcd);
    hipLaunchKernelGGL(pick_kernel<T>(K), dim3(per_xcd * kNumXcd), dim3(kBlock), 0,
                       as_stream(stream), R->rows, R->cols, lim, K, R->diag_offsets, R->values, x,
                       y, tiles, per_xcd);
    return check_launch(name);
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_spmv_recon_f32(const diagpu_recon_view_f32* R, const float* x,
                                     int64_t x_size, float* y, void* stream)
{
    return diagpu::spmv_launch<float>(R, x, x_size, y, stream, "diagpu_spmv_recon_f32");
}

DIAGPU_API int diagpu_spmv_recon_f64(const diagpu_recon_view_f64* R, const double* x,
                                     int64_t x_size, double* y, void* stream)
{
    return diagpu::spmv_launch<double>(R, x, x_size, y, stream, "diagpu_spmv_recon_f64");
}

}  // extern "C"
