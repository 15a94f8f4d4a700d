// Device selection and device memory behind the C ABI.
// Device::open (runtime/device/device.cpp:77-108) and the DeviceWeights arena /
// Impl::alloc helpers (device_weights.cpp:18-76, frame.hip:604-610) go through here.
#include "host_util.h"

#include <cstring>

namespace navi_amd {

DeviceState &device_state() {
    static DeviceState s;
    return s;
}

static std::string arch_of(const hipDeviceProp_t &p) {
    std::string a = p.gcnArchName;
    const auto c = a.find(':');
    return c == std::string::npos ? a : a.substr(0, c);
}

navi_status ensure_device(char *err, size_t errlen) {
    DeviceState &s = device_state();
    if (s.open) {
        NAVI_TRY_HIP(hipSetDevice(s.device), err, errlen);
        return NAVI_OK;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        set_err(err, errlen, "no HIP device visible");
        return NAVI_ERR_UNSUPPORTED;
    }
    for (int i = 0; i < n; ++i) {
        hipDeviceProp_t p{};
        if (hipGetDeviceProperties(&p, i) != hipSuccess) continue;
        if (arch_of(p) != "gfx950") continue;
        NAVI_TRY_HIP(hipSetDevice(i), err, errlen);
        (void) hipSetDeviceFlags(hipDeviceScheduleSpin);
        int coop = 0;
        NAVI_TRY_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, i), err, errlen);
        if (!coop) {
            set_err(err, errlen, "device %d (%s) does not support cooperative launch", i, p.name);
            return NAVI_ERR_UNSUPPORTED;
        }
        NAVI_TRY_HIP(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking), err, errlen);
        s.device = i;
        s.prop = p;
        s.open = true;
        return NAVI_OK;
    }
    set_err(err, errlen, "no gfx950 device among %d visible; this build runs on MI355X only", n);
    return NAVI_ERR_UNSUPPORTED;
}

} // namespace navi_amd

using namespace navi_amd;

extern "C" {

const char *navi_build_arch(void) { return "gfx950"; }

navi_status navi_device_open(navi_device_info *out, char *err, size_t errlen) {
    const navi_status st = ensure_device(err, errlen);
    if (st != NAVI_OK) return st;
    if (!out) return NAVI_OK;
    const DeviceState &s = device_state();
    const hipDeviceProp_t &p = s.prop;
    std::memset(out, 0, sizeof(*out));
    out->index = s.device;
    std::snprintf(out->name, sizeof(out->name), "%s", p.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", arch_of(p).c_str());
    out->multiprocessors = p.multiProcessorCount;
    out->warp_size = p.warpSize;
    out->cooperative_launch = 1;
    out->max_threads_per_block = p.maxThreadsPerBlock;
    out->lds_per_block = p.sharedMemPerBlock;
    out->clock_khz = p.clockRate;
    out->mem_clock_khz = p.memoryClockRate;
    out->mem_bus_width = p.memoryBusWidth;
    out->l2_bytes = static_cast<uint64_t>(p.l2CacheSize);
    size_t fr = 0, tot = 0;
    if (hipMemGetInfo(&fr, &tot) == hipSuccess) { out->vram_free = fr; out->vram_total = tot; }
    int rv = 0;
    (void) hipRuntimeGetVersion(&rv);
    out->hip_runtime_version = rv;
    return NAVI_OK;
}

void *navi_device_stream(void) { return device_state().stream; }

navi_status navi_device_close(void) {
    DeviceState &s = device_state();
    if (!s.open) return NAVI_OK;
    const hipError_t e = hipStreamSynchronize(s.stream);
    const hipError_t e2 = hipStreamDestroy(s.stream);
    s.stream = nullptr;
    s.open = false;
    return e == hipSuccess && e2 == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

navi_status navi_device_synchronize(void) {
    if (!device_state().open) return NAVI_OK;
    return hipStreamSynchronize(device_state().stream) == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

navi_status navi_mem_alloc(void **dptr, size_t bytes) {
    if (!dptr) return NAVI_ERR_INVALID;
    *dptr = nullptr;
    if (ensure_device(nullptr, 0) != NAVI_OK) return NAVI_ERR_UNSUPPORTED;
    if (bytes == 0) return NAVI_OK;
    if (hipMalloc(dptr, bytes) != hipSuccess) { *dptr = nullptr; return NAVI_ERR_HIP; }
    if (hipMemsetAsync(*dptr, 0, bytes, device_state().stream) != hipSuccess) return NAVI_ERR_HIP;
    return hipStreamSynchronize(device_state().stream) == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

navi_status navi_mem_free(void *dptr) {
    if (!dptr) return NAVI_OK;
    return hipFree(dptr) == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

static navi_status copy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind) {
    if (bytes == 0) return NAVI_OK;
    if (!dst || !src) return NAVI_ERR_INVALID;
    if (ensure_device(nullptr, 0) != NAVI_OK) return NAVI_ERR_UNSUPPORTED;
    hipStream_t st = device_state().stream;
    if (hipMemcpyAsync(dst, src, bytes, kind, st) != hipSuccess) return NAVI_ERR_HIP;
    return hipStreamSynchronize(st) == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

navi_status navi_mem_h2d(void *dst, const void *src, size_t bytes) { return copy(dst, src, bytes, hipMemcpyHostToDevice); }
navi_status navi_mem_d2h(void *dst, const void *src, size_t bytes) { return copy(dst, src, bytes, hipMemcpyDeviceToHost); }
navi_status navi_mem_d2d(void *dst, const void *src, size_t bytes) { return copy(dst, src, bytes, hipMemcpyDeviceToDevice); }

navi_status navi_mem_zero(void *dptr, size_t bytes) {
    if (bytes == 0) return NAVI_OK;
    if (!dptr) return NAVI_ERR_INVALID;
    if (ensure_device(nullptr, 0) != NAVI_OK) return NAVI_ERR_UNSUPPORTED;
    hipStream_t st = device_state().stream;
    if (hipMemsetAsync(dptr, 0, bytes, st) != hipSuccess) return NAVI_ERR_HIP;
    return hipStreamSynchronize(st) == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

} // extern "C"
