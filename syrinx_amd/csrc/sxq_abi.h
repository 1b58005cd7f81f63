// sxq_abi.h -- error reporting and device scoping shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/sxq.h"

namespace sxq {
namespace abi {

// Record `fmt` as this thread's sxq_last_error() and return `code`.
sxq_status fail(sxq_status code, const char* fmt, ...);
// Map a HIP error to SXQ_ERR_OOM / SXQ_ERR_DEVICE with its text.
sxq_status hip_fail(hipError_t e, const char* what);

#define HIP_TRY(expr, what)                                      \
    do {                                                         \
        hipError_t e_ = (expr);                                  \
        if (e_ != hipSuccess) return ::sxq::abi::hip_fail(e_, what); \
    } while (0)

// Makes `dev` current for the scope and restores the caller's device afterwards.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) err = hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;
};

}  // namespace abi
}  // namespace sxq
