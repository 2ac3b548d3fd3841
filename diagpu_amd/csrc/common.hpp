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

}  // namespace diagpu
