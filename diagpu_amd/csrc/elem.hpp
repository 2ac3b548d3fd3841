// Element types and arithmetic shared by the SpMV and SpGEMM kernels: fp32,
// fp64 and complex fp32 (cf32) elements, fused multiply-adds over
// (matrix element, vector element) pairs, and 16- or 32-byte runs of
// elements moved as 16-byte vectors (dword aligned: gfx950 serves unaligned
// global vector loads).
#pragma once

#include <hip/hip_runtime.h>

#include "spmv_internal.hpp"   // cf32

namespace diagpu {

__device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_(double a, double b, double c) { return __builtin_fma(a, b, c); }

// acc + a * x for (matrix element, vector element)
__device__ __forceinline__ float mad(float acc, float a, float x) { return fma_(a, x, acc); }
__device__ __forceinline__ double mad(double acc, double a, double x) { return fma_(a, x, acc); }
__device__ __forceinline__ cf32 mad(cf32 acc, cf32 a, cf32 x)
{
    cf32 r;
    r.re = fma_(-a.im, x.im, fma_(a.re, x.re, acc.re));
    r.im = fma_(a.im, x.re, fma_(a.re, x.im, acc.im));
    return r;
}
__device__ __forceinline__ cf32 mad(cf32 acc, float a, cf32 x)
{
    cf32 r;
    r.re = fma_(a, x.re, acc.re);
    r.im = fma_(a, x.im, acc.im);
    return r;
}

// alpha * x rounded once per real part (fp32: one multiply; complex: each
// part one fused multiply-add over the other product, written out so that
// no compiler contraction choice changes it)
__device__ __forceinline__ float scale_(float a, float x) { return a * x; }
__device__ __forceinline__ cf32 scale_(cf32 a, cf32 x)
{
    cf32 r;
    r.re = fma_(a.re, x.re, -(a.im * x.im));
    r.im = fma_(a.re, x.im, a.im * x.re);
    return r;
}
__device__ __forceinline__ float add_(float a, float b) { return a + b; }
__device__ __forceinline__ cf32 add_(cf32 a, cf32 b) { return cf32{a.re + b.re, a.im + b.im}; }

__device__ __forceinline__ float sel(bool c, float a, float b) { return c ? a : b; }
__device__ __forceinline__ double sel(bool c, double a, double b) { return c ? a : b; }
__device__ __forceinline__ cf32 sel(bool c, cf32 a, cf32 b)
{
    cf32 r;
    r.re = c ? a.re : b.re;
    r.im = c ? a.im : b.im;
    return r;
}

template <typename T> __device__ __forceinline__ T zero_of();
template <> __device__ __forceinline__ float zero_of<float>() { return 0.f; }
template <> __device__ __forceinline__ double zero_of<double>() { return 0.0; }
template <> __device__ __forceinline__ cf32 zero_of<cf32>() { return cf32{0.f, 0.f}; }

// Re(conj(u) * y) in fp64
__device__ __forceinline__ double dotpart(float u, float y) { return (double)u * (double)y; }
__device__ __forceinline__ double dotpart(double u, double y) { return u * y; }
__device__ __forceinline__ double dotpart(cf32 u, cf32 y) { return (double)u.re * y.re + (double)u.im * y.im; }

// One element, loaded as a plain vector register value.
template <typename T> struct ElemRaw { typedef T type; };
template <> struct ElemRaw<cf32> { typedef float type __attribute__((ext_vector_type(2))); };

template <typename T, bool NT>
__device__ __forceinline__ T load_elem(const T* p)
{
    typedef typename ElemRaw<T>::type Raw;
    Raw v = NT ? __builtin_nontemporal_load(reinterpret_cast<const Raw*>(p))
               : *reinterpret_cast<const Raw*>(p);
    T r;
    __builtin_memcpy(&r, &v, sizeof(T));
    return r;
}

// A lane's run of R consecutive elements (8, 16 or 32 bytes), moved as one
// 8-byte or whole 16-byte vectors.
template <typename T, int R> struct Run { T v[R]; };

typedef float f4dw __attribute__((ext_vector_type(4), aligned(4)));
typedef float f2dw __attribute__((ext_vector_type(2), aligned(4)));

template <typename T, int R, bool NT>
__device__ __forceinline__ Run<T, R> load_run(const T* p)
{
    Run<T, R> r;
    if constexpr (R * sizeof(T) == 8) {
        const f2dw q = NT ? __builtin_nontemporal_load(reinterpret_cast<const f2dw*>(p))
                          : *reinterpret_cast<const f2dw*>(p);
        __builtin_memcpy(&r, &q, sizeof(r));
    } else {
        static_assert((R * sizeof(T)) % 16 == 0, "runs are 8 bytes or whole 16-byte vectors");
        constexpr int NQ = (int)(R * sizeof(T) / 16);
        f4dw q[NQ];
#pragma unroll
        for (int i = 0; i < NQ; ++i)
            q[i] = NT ? __builtin_nontemporal_load(reinterpret_cast<const f4dw*>(p) + i)
                      : reinterpret_cast<const f4dw*>(p)[i];
        __builtin_memcpy(&r, q, sizeof(r));
    }
    return r;
}

template <typename T, int R>
__device__ __forceinline__ void store_run_nt(T* p, const Run<T, R>& r)
{
    constexpr int NQ = (int)(R * sizeof(T) / 16);
    f4dw q[NQ];
    __builtin_memcpy(q, &r, sizeof(r));
#pragma unroll
    for (int i = 0; i < NQ; ++i) __builtin_nontemporal_store(q[i], reinterpret_cast<f4dw*>(p) + i);
}

template <typename T, int R>
__device__ __forceinline__ void store_run(T* p, const Run<T, R>& r)
{
    constexpr int NQ = (int)(R * sizeof(T) / 16);
    f4dw q[NQ];
    __builtin_memcpy(q, &r, sizeof(r));
#pragma unroll
    for (int i = 0; i < NQ; ++i) reinterpret_cast<f4dw*>(p)[i] = q[i];
}

}  // namespace diagpu
