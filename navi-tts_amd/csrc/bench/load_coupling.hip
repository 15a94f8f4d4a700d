// Load coupling of the frame kernel's polls on MI355X: does a wave's agent-scope poll wait behind
// other waves' in-flight loads on the same CU, or only behind its own (vector loads retire in order
// per wave)?
// 256 blocks x 512 threads (one per CU, cooperative). Waves 4..7 of block 0 and block 129 (another XCD) bounce a
// tagged word R times (lane 0 of wave 4); waves 0..3 of every block ("loaders", mode 1) stream a
// 1 GiB buffer in batches of 16 x 16 B per lane. Mode 2: no loaders, but the pinging wave issues
// one batch of 16 x 16 B loads before each ping (its own in-order load counter). Every wait has a cap.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>

typedef unsigned u4 __attribute__((ext_vector_type(4)));
#define G __attribute__((address_space(1)))

__device__ __forceinline__ void put(uint64_t *p, uint64_t w) { __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ uint64_t peek(uint64_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

constexpr int R = 200;
constexpr unsigned long long CAP = 4000000ull;

__global__ void __launch_bounds__(512) k(int mode, const u4 *buf, size_t n16, uint64_t *mb, uint32_t *done, uint32_t *fail,
                                          unsigned long long *out, unsigned *sink) {
    const int w = threadIdx.x / 64, l = threadIdx.x & 63, b = blockIdx.x;
    if (w < 4) {
        if (mode != 1) return;
        u4 acc = {0, 0, 0, 0};
        size_t base = (static_cast<size_t>(b) * 4 + w) * 4096 * 64;   // distinct start per wave
        for (int it = 0; it < 200000; ++it) {
            u4 v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = __builtin_nontemporal_load((const G u4 *) (buf + (base + (static_cast<size_t>(it) * 16 + i) * 64 + l) % n16));
#pragma unroll
            for (int i = 0; i < 16; ++i) acc += v[i];
            if ((it & 7) == 0 && __hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
        }
        if (acc.x == 0x12345u) sink[b] = acc.y;
        return;
    }
    if (w != 4 || (b != 0 && b != 129)) return;
    const bool leader = b == 0;
    uint64_t *mine = mb + (leader ? 0 : 64), *theirs = mb + (leader ? 64 : 0);
    unsigned long long t0 = 0, t1 = 0;
    u4 acc = {0, 0, 0, 0};
    size_t base = static_cast<size_t>(b) * 999 * 64;
    bool ok = true;
    for (int r = 1; r <= R && ok; ++r) {
        if (r == 21) t0 = wall_clock64();
        if (mode == 2) {
            u4 v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = __builtin_nontemporal_load((const G u4 *) (buf + (base + (static_cast<size_t>(r) * 16 + i) * 64 + l) % n16));
            // keep them live without waiting: fold after the ping below
#pragma unroll
            for (int i = 0; i < 16; ++i) acc += v[i];
        }
        if (leader) {
            if (l == 0) put(mine, (static_cast<uint64_t>(r) << 32) | 1u);
            unsigned long long s = 0;
            uint64_t x = 0;
            if (l == 0) { do { x = peek(theirs); } while ((x >> 32) != static_cast<uint64_t>(r) && ++s < CAP); }
            ok = __shfl(static_cast<int>(s < CAP), 0) != 0;
        } else {
            unsigned long long s = 0;
            uint64_t x = 0;
            if (l == 0) { do { x = peek(theirs); } while ((x >> 32) != static_cast<uint64_t>(r) && ++s < CAP); }
            ok = __shfl(static_cast<int>(s < CAP), 0) != 0;
            if (l == 0) put(mine, (static_cast<uint64_t>(r) << 32) | 1u);
        }
    }
    t1 = wall_clock64();
    if (!ok && l == 0) atomicExch(fail, 1u);
    if (leader && l == 0) { out[0] = t1 - t0; __hip_atomic_store(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
    if (acc.x == 0x12345u) sink[b] = acc.y;
}

int main() {
    const size_t bytes = 1ull << 30, n16 = bytes / 16;
    u4 *buf; uint64_t *mb; uint32_t *done, *fail; unsigned long long *out; unsigned *sink;
    if (hipMalloc(&buf, bytes) || hipMalloc(&mb, 4096) || hipMalloc(&done, 4) || hipMalloc(&fail, 4) || hipMalloc(&out, 8) || hipMalloc(&sink, 1024 * 4)) { printf("alloc failed\n"); return 1; }
    (void) hipMemset(buf, 0, bytes);
    int dev = 0; hipDeviceProp_t p; (void) hipGetDeviceProperties(&p, dev);
    int clk = 0; (void) hipDeviceGetAttribute(&clk, hipDeviceAttributeWallClockRate, dev);   // kHz
    printf("CUs %d wall clock %d kHz\n", p.multiProcessorCount, clk);
    const char *names[] = {"no loads", "other waves of the CU stream 1 GiB", "the pinging wave loads 16 KB before each ping"};
    for (int rep = 0; rep < 2; ++rep)
    for (int mode = 0; mode < 3; ++mode) {
        (void) hipMemset(mb, 0, 4096); (void) hipMemset(done, 0, 4); (void) hipMemset(fail, 0, 4); (void) hipMemset(out, 0, 8);
        int m = mode; const u4 *bp = buf; size_t n = n16;
        void *args[] = {&m, &bp, &n, &mb, &done, &fail, &out, &sink};
        hipError_t e = hipLaunchCooperativeKernel((const void *) k, dim3(256), dim3(512), args, 0, 0);
        if (e != hipSuccess) { printf("launch: %s\n", hipGetErrorString(e)); return 1; }
        if (hipDeviceSynchronize() != hipSuccess) { printf("sync failed\n"); return 1; }
        unsigned long long t = 0; uint32_t f = 0;
        (void) hipMemcpy(&t, out, 8, hipMemcpyDeviceToHost); (void) hipMemcpy(&f, fail, 4, hipMemcpyDeviceToHost);
        printf("mode %d (%s): round trip %.3f us%s\n", mode, names[mode], t * 1000.0 / clk / (R - 20), f ? " (a wait was capped)" : "");
        fflush(stdout);
    }
    return 0;
}
