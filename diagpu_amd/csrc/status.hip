// Status reporting and device queries of the C ABI.
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "common.hpp"

namespace diagpu {

namespace {
thread_local char g_last_error[512] = "";
}

int fail(int status, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_hip(hipError_t err, const char* what)
{
    if (err == hipSuccess) return DIAGPU_OK;
    return fail(DIAGPU_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

int cu_count()
{
    static std::mutex mu;
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

}  // namespace diagpu

extern "C" {

DIAGPU_API const char* diagpu_last_error(void) { return diagpu::g_last_error; }

DIAGPU_API const char* diagpu_status_name(int status)
{
    switch (status) {
    case DIAGPU_OK: return "DIAGPU_OK";
    case DIAGPU_ERR_ARG: return "DIAGPU_ERR_ARG";
    case DIAGPU_ERR_OFFSET: return "DIAGPU_ERR_OFFSET";
    case DIAGPU_ERR_DUPLICATE: return "DIAGPU_ERR_DUPLICATE";
    case DIAGPU_ERR_OVERFLOW: return "DIAGPU_ERR_OVERFLOW";
    case DIAGPU_ERR_CAPACITY: return "DIAGPU_ERR_CAPACITY";
    case DIAGPU_ERR_HIP: return "DIAGPU_ERR_HIP";
    default: return "DIAGPU_ERR_UNKNOWN";
    }
}

DIAGPU_API int diagpu_abi_version(void) { return 100; }

}  // extern "C"
