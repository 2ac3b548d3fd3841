// Workgroup-wide prefix sums for 64-lane waves (device helpers).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace diagpu {

// Inclusive prefix sum across the 64 lanes of a wave.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
        const T o = __shfl_up(v, s, 64);
        if (lane >= s) v += o;
    }
    return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v)
{
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
    return v;
}

// Exclusive prefix sum over a workgroup of BLOCK threads (BLOCK a multiple
// of 64, at most 1024).  `total` receives the workgroup sum.  `lds` must hold
// BLOCK / 64 values.  Contains barriers: every thread must call it.
template <typename T, int BLOCK>
__device__ __forceinline__ T block_exclusive_scan(T v, T& total, T* lds)
{
    constexpr int kWaves = BLOCK / 64;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const T incl = wave_inclusive_scan(v);
    if (lane == 63) lds[wave] = incl;
    __syncthreads();
    T before = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const T s = lds[w];
        before += (w < wave) ? s : T(0);
        sum += s;
    }
    __syncthreads();
    total = sum;
    return before + incl - v;
}

}  // namespace diagpu
