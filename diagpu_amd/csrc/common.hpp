// Shared host/device helpers of libdiagpu (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "diagpu.h"

namespace diagpu {

// MI355X in SPX mode: 8 XCDs, workgroup i of a launch is dispatched to XCD
// (i mod 8).  Kernels remap blockIdx so that the workgroups of one XCD work
// on one contiguous range of rows and share its L2.
constexpr int kNumXcd = 8;

// Record `status` with a printf-style message for diagpu_last_error() and
// return it.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Map the last HIP error (after a launch or runtime call) to DIAGPU_ERR_HIP.
int check_hip(hipError_t err, const char* what);
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units of the current device (cached per device).
int cu_count();

template <typename T>
__host__ __device__ constexpr T ceil_div(T a, T b) { return (a + b - 1) / b; }

// *(base + o bytes) for a uniform base and offset: compiled to a scalar load
// with the offset in an SGPR (s_load ... sbase, soffset), so the address
// costs no 64-bit arithmetic.  A constant part of the offset belongs in the
// pointer (base + 1), where it becomes the instruction's immediate and
// neighbouring loads can merge.
template <typename V>
__device__ __forceinline__ V at_byte(const V* __restrict__ base, uint32_t o)
{
    return *reinterpret_cast<const V*>(reinterpret_cast<const char*>(base) + o);
}

}  // namespace diagpu
