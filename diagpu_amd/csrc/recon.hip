// build_recon on the device: an HM (compact diagonal) square matrix to the
// column-indexed Recon layout the SpMV kernels read.
//
// For a square n x n matrix the HM layout is the reference's compact DIA
// layout (element j of diagonal d is H[max(-d, 0) + j, max(d, 0) + j]), so
// this is build_recon of spmv/src/dia_reconstruct.cuh:77-107 with the input
// already on the GPU: offsets reversed from ascending (as the SpGEMM symbolic
// phase produces them) to descending, and Recon row k holding its diagonal at
// columns [max(d, 0), max(d, 0) + n - |d|), zero elsewhere.  It lets a product
// built by SpGEMM (a propagator, a matrix power) be applied by the SpMV path
// without a trip through host memory.  One streaming pass: every Recon value
// written once, every HM value read once.  Also the real -> complex64
// promotion of a value array (diagpu_promote_f32_c64).
#include "common.hpp"
#include "elem.hpp"

namespace diagpu {
namespace {

constexpr int kBlock = 256;
constexpr int kSpan = kBlock * 4;   // columns per workgroup iteration

template <typename T>
__global__ __launch_bounds__(kBlock) void k_hm_to_recon(int32_t n,
                                                       const int32_t* __restrict__ off,
                                                       const int64_t* __restrict__ starts,
                                                       int32_t K, const T* __restrict__ hm,
                                                       int32_t* __restrict__ r_off,
                                                       T* __restrict__ r_vals, int32_t spans)
{
    for (int64_t w = blockIdx.x; w < (int64_t)K * spans; w += gridDim.x) {
        const int kr = (int)(w / spans);              // Recon row
        const int sb = (int)(w - (int64_t)kr * spans);
        const int ks = K - 1 - kr;                    // HM diagonal (ascending order)
        const int d = off[ks];
        const int64_t first = d > 0 ? d : 0;
        const int64_t len = (int64_t)n - (d < 0 ? -d : d);
        const T* src = hm + starts[ks] - first;       // src[c] = element of column c
        T* dst = r_vals + (int64_t)kr * n;
        if (sb == 0 && threadIdx.x == 0) r_off[kr] = d;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t c = (int64_t)sb * kSpan + (int64_t)e * kBlock + threadIdx.x;
            if (c < n) dst[c] = (c >= first && c < first + len) ? src[c] : zero_of<T>();
        }
    }
}

template <typename T>
int hm_to_recon(int32_t n, const int32_t* off, const int64_t* starts, int32_t K, const T* vals,
                int32_t* r_off, T* r_vals, void* stream, const char* fn)
{
    if (n < 1 || K < 0) return fail(DIAGPU_ERR_ARG, "%s: need n >= 1 and ndiag >= 0", fn);
    if (K == 0) return DIAGPU_OK;
    if (!off || !starts || !vals || !r_off || !r_vals)
        return fail(DIAGPU_ERR_ARG, "%s: a pointer is NULL", fn);
    const int32_t spans = (int32_t)ceil_div<int64_t>(n, kSpan);
    int64_t grid = (int64_t)K * spans;
    const int64_t cap = (int64_t)cu_count() * 16;
    if (grid > cap) grid = cap;
    hipLaunchKernelGGL(k_hm_to_recon<T>, dim3((unsigned)grid), dim3(kBlock), 0, as_stream(stream),
                       n, off, starts, K, vals, r_off, r_vals, spans);
    return check_launch(fn);
}

// dst[i] = (src[i], 0): a real operator's values as complex64.  Grid-stride,
// 16-byte stores.
__global__ __launch_bounds__(kBlock) void k_promote(int64_t count, const float* __restrict__ src,
                                                   cf32* __restrict__ dst)
{
    const int64_t stride = (int64_t)gridDim.x * kBlock * 2;
    for (int64_t i = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * 2; i < count; i += stride) {
        if (i + 2 <= count) {
            const float a = src[i], b = src[i + 1];
            const f4dw q = {a, 0.f, b, 0.f};
            *reinterpret_cast<f4dw*>(dst + i) = q;
        } else {
            dst[i] = cf32{src[i], 0.f};
        }
    }
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_promote_f32_c64(int64_t count, const float* src, diagpu_complex64* dst,
                                      void* stream)
{
    const char* fn = "diagpu_promote_f32_c64";
    if (count < 0) return diagpu::fail(DIAGPU_ERR_ARG, "%s: negative count", fn);
    if (count == 0) return DIAGPU_OK;
    if (!src || !dst) return diagpu::fail(DIAGPU_ERR_ARG, "%s: a pointer is NULL", fn);
    using diagpu::cf32;
    const int64_t pairs = (count + 1) / 2;
    int64_t grid = diagpu::ceil_div<int64_t>(pairs, diagpu::kBlock);
    const int64_t cap = (int64_t)diagpu::cu_count() * 16;
    if (grid > cap) grid = cap;
    hipLaunchKernelGGL(diagpu::k_promote, dim3((unsigned)grid), dim3(diagpu::kBlock), 0,
                       diagpu::as_stream(stream), count, src, reinterpret_cast<cf32*>(dst));
    return diagpu::check_launch(fn);
}

DIAGPU_API int diagpu_hm_to_recon_f32(int32_t n, const int32_t* offsets, const int64_t* starts,
                                      int32_t ndiag, const float* values, int32_t* recon_offsets,
                                      float* recon_values, void* stream)
{
    return diagpu::hm_to_recon<float>(n, offsets, starts, ndiag, values, recon_offsets,
                                      recon_values, stream, "diagpu_hm_to_recon_f32");
}

DIAGPU_API int diagpu_hm_to_recon_c64(int32_t n, const int32_t* offsets, const int64_t* starts,
                                      int32_t ndiag, const diagpu_complex64* values,
                                      int32_t* recon_offsets, diagpu_complex64* recon_values,
                                      void* stream)
{
    using diagpu::cf32;
    return diagpu::hm_to_recon<cf32>(n, offsets, starts, ndiag,
                                     reinterpret_cast<const cf32*>(values), recon_offsets,
                                     reinterpret_cast<cf32*>(recon_values), stream,
                                     "diagpu_hm_to_recon_c64");
}

}  // extern "C"
