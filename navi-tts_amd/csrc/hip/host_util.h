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

inline const navi_tensor_ref *find_tensor(const navi_tensor_ref *t, int n, const std::string &name) {
    for (int i = 0; i < n; ++i)
        if (t[i].name && name == t[i].name) return &t[i];
    return nullptr;
}

// Looks a weight up by name and checks its dtype, shape and 16-byte alignment (the contract of
// DeviceWeights::get + Params::validate). d1 == 0: a 1-D tensor [d0]; else [d0, d1].
template <class T>
navi_status bind_tensor(const char *who, const navi_tensor_ref *t, int n, const std::string &name, int dtype, uint64_t d0,
                        uint64_t d1, const T *&out, char *err, size_t errlen) {
    const navi_tensor_ref *r = find_tensor(t, n, name);
    if (!r) {
        set_err(err, errlen, "%s: missing tensor '%s'", who, name.c_str());
        return NAVI_ERR_INVALID;
    }
    const int nd = d1 ? 2 : 1;
    const bool ok = r->dtype == dtype && r->ndim == nd && r->dims[0] == d0 && (nd == 1 || r->dims[1] == d1);
    if (!ok) {
        set_err(err, errlen, "%s: tensor '%s' has an unexpected dtype or shape", who, name.c_str());
        return NAVI_ERR_INVALID;
    }
    if (reinterpret_cast<uintptr_t>(r->ptr) & 15u) {
        set_err(err, errlen, "%s: tensor '%s' is not 16-byte aligned", who, name.c_str());
        return NAVI_ERR_INVALID;
    }
    out = static_cast<const T *>(r->ptr);
    return NAVI_OK;
}

#define NAVI_TRY_HIP(expr, err, errlen)                                                              \
    do {                                                                                             \
        const hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess) {                                                                      \
            ::navi_amd::set_err((err), (errlen), "%s failed: %s", #expr, hipGetErrorString(e_));    \
            return NAVI_ERR_HIP;                                                                     \
        }                                                                                            \
    } while (0)

} // namespace navi_amd
