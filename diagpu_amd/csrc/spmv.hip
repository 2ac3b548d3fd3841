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
// Mapping.  A workgroup of 256 lanes owns a tile of 1024 consecutive rows;
// each lane owns 4 consecutive rows r..r+3.  For diagonal k the lane needs
// Recon[k][r+d_k .. r+d_k+3] and x[r+d_k .. r+d_k+3]: both are contiguous
// quads at the same column, so one 128-bit load each (dword-aligned: gfx950
// serves unaligned global loads), and the 64 lanes of a wave cover 1 KiB of
// each stream.  Diagonals are processed in chunks of 4 whose 8 loads are all
// issued before the first FMA (a larger chunk costs more VGPRs than its
// extra loads in flight buy back in occupancy).  Value loads and the y store
// are non-temporal: each value is used once, while x stays in L2 for the
// tiles that re-read it.  The diagonal offsets are wave-uniform.  Tiles whose rows and columns are all in range (every tile of a large
// matrix except the first and last few) run without per-element bounds
// checks; the others take a checked path.
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
constexpr int kRowsPerLane = 4;
constexpr int kTile = kBlock * kRowsPerLane;   // rows per workgroup
constexpr int kChunk = 4;                       // diagonals per load batch

template <typename T> struct QuadOf;
template <> struct QuadOf<float> {
    typedef float type __attribute__((ext_vector_type(4), aligned(4)));
};
template <> struct QuadOf<double> {
    typedef double type __attribute__((ext_vector_type(4), aligned(8)));
};

template <typename T>
__device__ __forceinline__ typename QuadOf<T>::type load_quad(const T* p)
{
    return *reinterpret_cast<const typename QuadOf<T>::type*>(p);
}

// Streaming (non-temporal) load: the value stream is read once, so it should
// not displace x, which neighbouring tiles re-read from L2.
template <typename T>
__device__ __forceinline__ typename QuadOf<T>::type load_quad_stream(const T* p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const typename QuadOf<T>::type*>(p));
}

template <typename T>
__device__ __forceinline__ void store_quad_stream(T* p, typename QuadOf<T>::type v)
{
    __builtin_nontemporal_store(v, reinterpret_cast<typename QuadOf<T>::type*>(p));
}

__device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_(double a, double b, double c) { return __builtin_fma(a, b, c); }

// min and max of the diagonal offsets, uniform across the wave.  `first` is
// offs[lane] (lane < K), loaded once and reused by the main loop.
__device__ __forceinline__ void offset_range(const int32_t* __restrict__ offs, int K, int first,
                                             int& dmin, int& dmax)
{
    const int lane = threadIdx.x & 63;
    int lo = lane < K ? first : INT_MAX, hi = lane < K ? first : INT_MIN;
    for (int k = lane + 64; k < K; k += 64) {
        const int d = offs[k];
        lo = d < lo ? d : lo;
        hi = d > hi ? d : hi;
    }
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) {
        const int olo = __shfl_xor(lo, s);
        const int ohi = __shfl_xor(hi, s);
        lo = olo < lo ? olo : lo;
        hi = ohi > hi ? ohi : hi;
    }
    dmin = __builtin_amdgcn_readfirstlane(lo);
    dmax = __builtin_amdgcn_readfirstlane(hi);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void spmv_recon_kernel(
    int32_t rows, int32_t cols, int64_t lim, int32_t K, const int32_t* __restrict__ offs,
    const T* __restrict__ vals, const T* __restrict__ x, T* __restrict__ y, int32_t tiles,
    int32_t tiles_per_xcd)
{
    typedef typename QuadOf<T>::type Quad;
    const int tile = (int)(blockIdx.x % kNumXcd) * tiles_per_xcd + (int)(blockIdx.x / kNumXcd);
    if (tile >= tiles) return;
    const int64_t r0 = (int64_t)tile * kTile;
    const int64_t r = r0 + (int64_t)threadIdx.x * kRowsPerLane;

    // One vector load of the first 64 offsets serves the range test and the
    // first group of the main loop (one dependent round trip per tile).
    const int lane = threadIdx.x & 63;
    const int first = lane < K ? offs[lane] : 0;
    int dmin = 0, dmax = 0;
    offset_range(offs, K, first, dmin, dmax);
    const bool interior = (r0 + kTile <= rows) &&
                          (K == 0 || (r0 + dmin >= 0 && r0 + kTile + (int64_t)dmax <= lim));

    if (interior) {
        Quad acc = {0, 0, 0, 0};
        const T* __restrict__ vr = vals + r;
        const T* __restrict__ xr = x + r;
        // Offsets travel 64 at a time as one vector load (lane l holds
        // offset g0 + l) and are broadcast with readlane, so the loads of a
        // chunk issue back to back without a scalar-load wait per diagonal.
        for (int g0 = 0; g0 < K; g0 += 64) {
            const int dl = g0 == 0 ? first : ((g0 + lane < K) ? offs[g0 + lane] : 0);
            const int gn = (K - g0) < 64 ? (K - g0) : 64;
            const T* __restrict__ vg = vr + (int64_t)g0 * cols;
            for (int k0 = 0; k0 < gn; k0 += kChunk) {
                // Broadcast the chunk's offsets first: a readlane placed
                // between the loads would make the compiler drain every
                // outstanding load before it.
                int d[kChunk];
#pragma unroll
                for (int j = 0; j < kChunk; ++j) d[j] = __builtin_amdgcn_readlane(dl, (k0 + j) & 63);
                Quad a[kChunk], b[kChunk];
#pragma unroll
                for (int j = 0; j < kChunk; ++j) {
                    if (k0 + j < gn) {
                        a[j] = load_quad_stream<T>(vg + (int64_t)(k0 + j) * cols + d[j]);
                        b[j] = load_quad<T>(xr + d[j]);
                    }
                }
#pragma unroll
                for (int j = 0; j < kChunk; ++j) {
                    if (k0 + j < gn) {
                        acc.x = fma_(a[j].x, b[j].x, acc.x);
                        acc.y = fma_(a[j].y, b[j].y, acc.y);
                        acc.z = fma_(a[j].z, b[j].z, acc.z);
                        acc.w = fma_(a[j].w, b[j].w, acc.w);
                    }
                }
            }
        }
        store_quad_stream<T>(y + r, acc);
        return;
    }

    // Boundary tile: per-element bounds, same summation order.
#pragma unroll
    for (int e = 0; e < kRowsPerLane; ++e) {
        const int64_t rr = r + e;
        if (rr >= rows) break;
        T acc = 0;
        for (int k = 0; k < K; ++k) {
            const int64_t c = rr + offs[k];
            if (c >= 0 && c < lim) acc = fma_(vals[(int64_t)k * cols + c], x[c], acc);
        }
        y[rr] = acc;
    }
}

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
    if (R->num_diags > 0) {
        if (!R->diag_offsets) return fail(DIAGPU_ERR_ARG, "%s: diag_offsets is NULL", name);
        if (R->cols > 0 && !R->values) return fail(DIAGPU_ERR_ARG, "%s: values is NULL", name);
        if (lim > 0 && !x) return fail(DIAGPU_ERR_ARG, "%s: x is NULL", name);
    }
    const int32_t tiles = (int32_t)ceil_div<int64_t>(R->rows, kTile);
    const int32_t per_xcd = ceil_div<int32_t>(tiles, kNumXcd);
    hipLaunchKernelGGL(spmv_recon_kernel<T>, dim3(per_xcd * kNumXcd), dim3(kBlock), 0,
                       as_stream(stream), R->rows, R->cols, lim, R->num_diags, R->diag_offsets,
                       R->values, x, y, tiles, per_xcd);
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
