// Z = alpha * X + beta * Y for HM (compact diagonal) matrices, gfx950.
//
// Z's diagonal set is given by the caller and must contain every diagonal of
// X and of Y (normally their union); a Z diagonal absent from X (or Y) takes
// 0 from it.  All three offset lists are ascending and duplicate-free, so the
// X / Y diagonal behind each Z diagonal is found by binary search.  Diagonals
// of equal offset have equal length n - |d| and the same position meaning,
// so the update is elementwise along each diagonal: one coalesced streaming
// pass over Z (12 bytes per position where both X and Y hold the diagonal).
//
// No reference counterpart: the reference describes a matrix-power chain
// (spmspm/gather_flat.cuh:13-14,110-117) but ships no driver for it.  The
// Taylor chain uses it to form I + (t/K) H and, in steps not fused into the
// product (diagpu_spgemm_numeric_astat_scaled_*), to scale H and to add I.
//
// Work: (Z diagonal, span) items, spans fastest, in contiguous ranges per
// workgroup, so a workgroup looks up X's and Y's diagonal (two binary
// searches of dependent scalar loads) only when its Z diagonal changes.  A
// span is kRuns 16-byte runs per lane, all loaded before any store.  The
// spans of a diagonal are shifted back by less than one 128-byte line so
// that they start on a line of Z: a line written in two parts by two
// workgroups at different times costs a read-modify-write in HBM.
#include "common.hpp"
#include "elem.hpp"

namespace diagpu {
namespace {

constexpr int kBlock = 256;
constexpr int kRuns = 4;   // 16-byte runs per lane per span

template <typename T> constexpr int run_len() { return (int)(16 / sizeof(T)); }
template <typename T> constexpr int span_len() { return kBlock * kRuns * run_len<T>(); }
template <typename T> constexpr int line_len() { return (int)(128 / sizeof(T)); }

__device__ __forceinline__ int find_offset(const int32_t* __restrict__ off, int cnt, int d)
{
    int lo = 0, hi = cnt - 1;
    while (lo <= hi) {
        const int mid = (lo + hi) >> 1;
        const int v = off[mid];
        if (v == d) return mid;
        if (v < d) lo = mid + 1; else hi = mid - 1;
    }
    return -1;
}

__device__ __forceinline__ float axpby_(float a, float x, float b, float y) { return a * x + b * y; }
__device__ __forceinline__ cf32 axpby_(cf32 a, cf32 x, cf32 b, cf32 y)
{
    cf32 r;
    r.re = a.re * x.re - a.im * x.im + (b.re * y.re - b.im * y.im);
    r.im = a.re * x.im + a.im * x.re + (b.re * y.im + b.im * y.re);
    return r;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_axpby(
    int32_t n, const int32_t* __restrict__ X_off, const int64_t* __restrict__ X_starts, int32_t nx,
    const T* Xv, T alpha, const int32_t* __restrict__ Y_off,
    const int64_t* __restrict__ Y_starts, int32_t ny, const T* Yv, T beta,
    const int32_t* __restrict__ Z_off, const int64_t* __restrict__ Z_starts, int32_t nz,
    T* Zv, int32_t spans, int64_t per_wg)
{
    constexpr int E = run_len<T>(), SPAN = span_len<T>(), L = line_len<T>();
    typedef Run<T, E> V;
    const int64_t total = (int64_t)nz * spans;
    const int64_t w0 = (int64_t)blockIdx.x * per_wg;
    const int64_t w1 = w0 + per_wg < total ? w0 + per_wg : total;
    int zc = -1, len = 0;
    int64_t shift = 0;
    // Z may be X (or Y) itself, element for element: each lane reads its
    // positions before it writes them, so the value pointers are not restrict.
    const T* xp = nullptr;
    const T* yp = nullptr;
    T* zp = nullptr;
    for (int64_t w = w0; w < w1; ++w) {
        const int z = (int)(w / spans);
        const int sb = (int)(w - (int64_t)z * spans);
        if (z != zc) {
            zc = z;
            const int d = Z_off[z];
            len = n - (d < 0 ? -d : d);
            const int xi = find_offset(X_off, nx, d);
            const int yi = find_offset(Y_off, ny, d);
            xp = xi >= 0 ? Xv + X_starts[xi] : nullptr;
            yp = yi >= 0 ? Yv + Y_starts[yi] : nullptr;
            const int64_t zs = Z_starts[z];
            zp = Zv + zs;
            shift = zs & (L - 1);   // Z + zs - shift starts a line
        }
        const int64_t p0 = (int64_t)sb * SPAN - shift;
        if (p0 >= len) continue;
        V xv[kRuns], yv[kRuns];
#pragma unroll
        for (int q = 0; q < kRuns; ++q) {           // all loads first, then the stores
            const int64_t p = p0 + ((int64_t)q * kBlock + threadIdx.x) * E;
            if (p >= 0 && p + E <= len) {
#pragma unroll
                for (int e = 0; e < E; ++e) xv[q].v[e] = yv[q].v[e] = zero_of<T>();
                if (xp) xv[q] = load_run<T, E, false>(xp + p);
                if (yp) yv[q] = load_run<T, E, false>(yp + p);
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const bool ok = p + e >= 0 && p + e < len;
                    xv[q].v[e] = (xp && ok) ? xp[p + e] : zero_of<T>();
                    yv[q].v[e] = (yp && ok) ? yp[p + e] : zero_of<T>();
                }
            }
        }
#pragma unroll
        for (int q = 0; q < kRuns; ++q) {
            const int64_t p = p0 + ((int64_t)q * kBlock + threadIdx.x) * E;
            V r;
#pragma unroll
            for (int e = 0; e < E; ++e) r.v[e] = axpby_(alpha, xv[q].v[e], beta, yv[q].v[e]);
            if (p >= 0 && p + E <= len) {
                store_run<T, E>(zp + p, r);          // zs + p is a multiple of E: 16-byte aligned
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e)
                    if (p + e >= 0 && p + e < len) zp[p + e] = r.v[e];
            }
        }
    }
}

inline bool is_zero(float a) { return a == 0.0f; }
inline bool is_zero(cf32 a) { return a.re == 0.0f && a.im == 0.0f; }

template <typename T>
int axpby_launch(int32_t n, const int32_t* X_off, const int64_t* X_starts, int32_t nx,
                 const T* X_vals, T alpha, const int32_t* Y_off, const int64_t* Y_starts,
                 int32_t ny, const T* Y_vals, T beta, const int32_t* Z_off,
                 const int64_t* Z_starts, int32_t nz, T* Z_vals, void* stream, const char* fn)
{
    if (n < 1 || n > (1 << 30) || nx < 0 || ny < 0 || nz < 0)
        return fail(DIAGPU_ERR_ARG, "%s: need 1 <= n <= 2^30 and counts >= 0", fn);
    if (nz == 0) return DIAGPU_OK;
    if (!Z_off || !Z_starts || !Z_vals) return fail(DIAGPU_ERR_ARG, "%s: Z arrays are NULL", fn);
    if (nx > 0 && (!X_off || !X_starts || !X_vals)) return fail(DIAGPU_ERR_ARG, "%s: X arrays are NULL", fn);
    if (ny > 0 && (!Y_off || !Y_starts || !Y_vals)) return fail(DIAGPU_ERR_ARG, "%s: Y arrays are NULL", fn);
    if (is_zero(alpha)) nx = 0;      // BLAS convention: a zero factor's operand is not read
    if (is_zero(beta)) ny = 0;
    // spans per diagonal: n positions plus a shift of less than one line
    const int32_t spans = (int32_t)ceil_div<int64_t>((int64_t)n + line_len<T>() - 1, span_len<T>());
    const int64_t total = (int64_t)nz * spans;
    const int64_t slots = (int64_t)cu_count() * 8;
    const int64_t per_wg = ceil_div<int64_t>(total, slots);
    const int64_t grid = ceil_div<int64_t>(total, per_wg);
    hipLaunchKernelGGL(k_axpby<T>, dim3((unsigned)grid), dim3(kBlock), 0, as_stream(stream), n,
                       X_off, X_starts, nx, X_vals, alpha, Y_off, Y_starts, ny, Y_vals, beta,
                       Z_off, Z_starts, nz, Z_vals, spans, per_wg);
    return check_launch(fn);
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_dia_axpby_f32(int32_t n, const int32_t* X_off, const int64_t* X_starts,
                                    int32_t nx, const float* X_vals, float alpha,
                                    const int32_t* Y_off, const int64_t* Y_starts, int32_t ny,
                                    const float* Y_vals, float beta, const int32_t* Z_off,
                                    const int64_t* Z_starts, int32_t nz, float* Z_vals, void* stream)
{
    return diagpu::axpby_launch<float>(n, X_off, X_starts, nx, X_vals, alpha, Y_off, Y_starts, ny,
                                       Y_vals, beta, Z_off, Z_starts, nz, Z_vals, stream,
                                       "diagpu_dia_axpby_f32");
}

DIAGPU_API int diagpu_dia_axpby_c64(int32_t n, const int32_t* X_off, const int64_t* X_starts,
                                    int32_t nx, const diagpu_complex64* X_vals,
                                    diagpu_complex64 alpha, const int32_t* Y_off,
                                    const int64_t* Y_starts, int32_t ny,
                                    const diagpu_complex64* Y_vals, diagpu_complex64 beta,
                                    const int32_t* Z_off, const int64_t* Z_starts, int32_t nz,
                                    diagpu_complex64* Z_vals, void* stream)
{
    using diagpu::cf32;
    return diagpu::axpby_launch<cf32>(
        n, X_off, X_starts, nx, reinterpret_cast<const cf32*>(X_vals), cf32{alpha.re, alpha.im},
        Y_off, Y_starts, ny, reinterpret_cast<const cf32*>(Y_vals), cf32{beta.re, beta.im}, Z_off,
        Z_starts, nz, reinterpret_cast<cf32*>(Z_vals), stream, "diagpu_dia_axpby_c64");
}

}  // extern "C"
