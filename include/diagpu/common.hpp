// Shared pieces of the C++ drop-in headers: errors and device buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>
#include <string>
#include <vector>

#include "diagpu.h"

namespace diagpu {

// A non-zero status from libdiagpu, or a failed HIP runtime call.
struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string& what) : std::runtime_error(what), status(s) {}
};

inline void check(int status)
{
    if (status != DIAGPU_OK)
        throw Error(status, std::string(diagpu_status_name(status)) + ": " + diagpu_last_error());
}

inline void check_hip(hipError_t e, const char* what)
{
    if (e != hipSuccess)
        throw Error(DIAGPU_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Owning device array (hipMalloc / hipFree), move-only.
template <typename T>
class DeviceArray {
public:
    DeviceArray() = default;
    explicit DeviceArray(size_t n) { resize(n); }
    explicit DeviceArray(const std::vector<T>& h) { upload(h); }
    DeviceArray(const DeviceArray&) = delete;
    DeviceArray& operator=(const DeviceArray&) = delete;
    DeviceArray(DeviceArray&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
    DeviceArray& operator=(DeviceArray&& o) noexcept
    {
        if (this != &o) { release(); p_ = o.p_; n_ = o.n_; o.p_ = nullptr; o.n_ = 0; }
        return *this;
    }
    ~DeviceArray() { release(); }

    void resize(size_t n)
    {
        release();
        if (n) check_hip(hipMalloc(reinterpret_cast<void**>(&p_), n * sizeof(T)), "hipMalloc");
        n_ = n;
    }
    void upload(const std::vector<T>& h)
    {
        resize(h.size());
        if (n_) check_hip(hipMemcpy(p_, h.data(), n_ * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
    }
    std::vector<T> download(size_t count) const
    {
        std::vector<T> h(count);
        if (count) check_hip(hipMemcpy(h.data(), p_, count * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
        return h;
    }
    std::vector<T> download() const { return download(n_); }
    T* data() { return p_; }
    const T* data() const { return p_; }
    size_t size() const { return n_; }

private:
    void release()
    {
        if (p_) (void)hipFree(p_);
        p_ = nullptr;
        n_ = 0;
    }
    T* p_ = nullptr;
    size_t n_ = 0;
};

}  // namespace diagpu
