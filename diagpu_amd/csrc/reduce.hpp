// Deterministic fp64 sums across a grid: every workgroup stores one partial
// with a plain store; a one-workgroup kernel launched after it adds the
// partials in index order.  The launch boundary makes the partials visible,
// so no device-scope fence is needed inside the producing kernel (on gfx950
// such a fence writes back and invalidates the XCD's L2 -- per workgroup,
// that cost more than the kernels themselves).
#pragma once

#include <hip/hip_runtime.h>

namespace diagpu {

// Sum of `s` over the calling workgroup (kBlockSize lanes, every lane
// calls).  The result is valid in every lane.
template <int kBlockSize>
__device__ __forceinline__ double block_sum(double s)
{
    __shared__ double wsum[kBlockSize / 64];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
    __syncthreads();   // wsum may still be read by a previous call
    if (lane == 0) wsum[wave] = s;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < kBlockSize / 64; ++w) t += wsum[w];
    return t;
}

// Workgroup `part` stores the sum of its lanes' `s` into partials[part].
template <int kBlockSize>
__device__ __forceinline__ void store_partial(double s, int part, double* partials)
{
    const double t = block_sum<kBlockSize>(s);
    if (threadIdx.x == 0) partials[part] = t;
}

}  // namespace diagpu
