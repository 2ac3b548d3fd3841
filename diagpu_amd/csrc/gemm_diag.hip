// gemm_diag on gfx950: row-packed operands through the HM SpGEMM phases.
//
// The reference's gemm_diag computes C[k][t] = sum_{i+j=k} DA[i][t] DB[j][t+i]
// (gemm_diag/gemm_diag.cu:9-15) with 4x4 diagonal tiles, a shared-memory
// k-map of at most 7 outputs per tile and float atomics (:119-329); that map
// drops terms when a tile's offsets are not contiguous.  Here the row-packed
// arrays are addressed as HM matrices instead: row t of diagonal d sits at
// DA[i * n + t] and its HM position is t + min(d, 0), so
//   starts[i] = i * n + max(-d, 0),  lengths[i] = n - |d|
// make DA an HM operand in place (the zero padding is never read).  The
// symbolic and numeric SpGEMM phases then give the product for any offsets,
// in the compact C layout of build_c_layout (:388-423), with C overwritten.
#include "common.hpp"

namespace diagpu {
namespace {

__global__ __launch_bounds__(256) void k_rowpacked_starts(int32_t n,
                                                          const int32_t* __restrict__ off,
                                                          int32_t nd, int64_t* __restrict__ starts,
                                                          int32_t* __restrict__ lengths)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nd) return;
    const int d = off[i];
    const int ad = d < 0 ? -d : d;
    starts[i] = (int64_t)i * n + (d < 0 ? -d : 0);
    lengths[i] = n - ad;
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_rowpacked_as_hm(int32_t n, const int32_t* offsets, int32_t ndiag,
                                      int64_t* starts, int32_t* lengths, void* stream)
{
    using namespace diagpu;
    const char* fn = "diagpu_rowpacked_as_hm";
    if (n < 1 || n > (1 << 30) || ndiag < 0)
        return fail(DIAGPU_ERR_ARG, "%s: need 1 <= n <= 2^30, ndiag >= 0 (n=%d ndiag=%d)", fn, n,
                    ndiag);
    if (ndiag == 0) return DIAGPU_OK;
    if (!offsets || !starts || !lengths)
        return fail(DIAGPU_ERR_ARG, "%s: NULL array", fn);
    hipLaunchKernelGGL(k_rowpacked_starts, dim3(ceil_div(ndiag, 256)), dim3(256), 0,
                       as_stream(stream), n, offsets, ndiag, starts, lengths);
    return check_launch(fn);
}

}  // extern "C"
