// Host-side helpers for the C ABI implementation: error strings, HIP checks,
// the per-process device state (current device, library stream).
#pragma once

#include "navi_amd.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

namespace navi_amd {

inline void set_err(char *err, size_t errlen, const char *fmt, ...) {
    if (!err || errlen == 0) return;
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

// Process-wide device state: navi_device_open() fills it; every entry point
// enqueues on `stream` (one GPU owner, one stream: device.cpp:96-97).
struct DeviceState {
    bool open = false;
    int device = -1;
    hipStream_t stream = nullptr;
    hipDeviceProp_t prop{};
};
DeviceState &device_state();

// Opens the device on first use so the ABI works without an explicit open.
navi_status ensure_device(char *err, size_t errlen);

#define NAVI_TRY_HIP(expr, err, errlen)                                                              \
    do {                                                                                             \
        const hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess) {                                                                      \
            ::navi_amd::set_err((err), (errlen), "%s failed: %s", #expr, hipGetErrorString(e_));    \
            return NAVI_ERR_HIP;                                                                     \
        }                                                                                            \
    } while (0)

} // namespace navi_amd
