// Cost of one dependent phase of a persistent grid whose phases exchange the multi-stream decode's
// 32-row f32 activations through plain stores and loads ordered by a grid-wide counter barrier
// (the alternative to k_frame's tagged words, whose bytes double and whose per-word polls grow with
// the operand): 256 co-resident blocks x 512 threads (the row projections' grid), R rounds in one
// cooperative launch. A round: every block reads the whole ROWS x K activation (float4 loads, all
// in flight), writes its ROWS x K/256 tile of the next one, and waits at the barrier; the two
// activation buffers alternate, so a buffer is rewritten only after every block has passed the
// barrier that ends its reads. Barriers:
//   release/acquire   : agent-scope release add on one counter (the L2 writeback the plain stores
//                       need), relaxed polls by one thread, agent-scope acquire fence (the L2
//                       invalidate the plain loads need) -- the standard grid barrier;
//   + sleep           : the same with s_sleep 1 between polls;
//   relaxed, no fences: relaxed add and polls only -- the synchronisation alone, with no ordering
//                       of the activation's stores and loads (a lower bound, not a usable barrier);
//   two-level         : release add on the block's XCD counter (blocks b % 8 == x), the 32nd arriver
//                       adds to the global counter, the 8th global arriver writes the round into 8
//                       per-XCD flags (one cache line each), blocks poll their XCD's flag, acquire fence.
// Every wait has a spin cap; a capped wait sets the fail word, every later wait gives up, and the
// run is reported as failed.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define CHECK(x)                                                                              \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) {                                                               \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);        \
            return 1;                                                                         \
        }                                                                                     \
    } while (0)

constexpr int NB = 256, BT = 512;
constexpr unsigned CAP = 4000000u;

// MODE 0: release add + relaxed polls + agent acquire fence (the standard grid barrier)
// MODE 1: MODE 0 with s_sleep between polls
// MODE 2: relaxed add, relaxed polls with s_sleep, no fences (sync cost alone; no data ordering)
// MODE 3: two levels: release add on the XCD's counter; its 32nd arriver adds to the global counter;
//         the 8th global arriver writes the round into 8 per-XCD flags; blocks poll their XCD's flag
//         (sleep between polls), then an agent acquire fence
template <int MODE>
__device__ __forceinline__ bool grid_wait(unsigned *ctr, unsigned r1, unsigned *fail) {
    __shared__ int bad;
    __syncthreads();
    if (threadIdx.x == 0) {
        bad = 0;
        unsigned s = 0;
        if (MODE == 3) {
            const int x = blockIdx.x % 8;
            unsigned *xc = ctr + 64 + 64 * x, *fl = ctr + 1024 + 64 * x;
            const unsigned old = __hip_atomic_fetch_add(xc, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            if (old == 32u * r1 - 1u) {
                const unsigned g = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
                if (g == 8u * r1 - 1u)
                    for (int y = 0; y < 8; ++y) __hip_atomic_store(ctr + 1024 + 64 * y, r1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            }
            while (__hip_atomic_load(fl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < r1) {
                __builtin_amdgcn_s_sleep(1);
                if (++s >= CAP || __hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                    __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    bad = 1;
                    break;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        } else {
            const unsigned target = 256u * r1;
            if (MODE == 2) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                if (MODE >= 1) __builtin_amdgcn_s_sleep(1);
                if (++s >= CAP || __hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                    __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    bad = 1;
                    break;
                }
            }
            if (MODE != 2) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
    }
    __syncthreads();
    return bad == 0;
}

// ROWS x K activation read by every block; each block writes ROWS x (K/NB) of the next one.
template <int ROWS, int K, int MODE>
__global__ void __launch_bounds__(BT) k_phase(float *a0, float *a1, unsigned *ctr, unsigned *fail, int R, float *sink) {
    constexpr int NV = ROWS * K / 4 / BT;  // float4 per thread
    float acc = 0.f;
    for (int r = 0; r < R; ++r) {
        const float *src = (r & 1) ? a1 : a0;
        float *dst = (r & 1) ? a0 : a1;
        float s = 0.f;
        if (NV > 0) {
            float4 v[NV > 0 ? NV : 1];
#pragma unroll
            for (int i = 0; i < NV; ++i) v[i] = reinterpret_cast<const float4 *>(src)[threadIdx.x + BT * i];
#pragma unroll
            for (int i = 0; i < NV; ++i) s += v[i].x + v[i].y + v[i].z + v[i].w;
        }
        constexpr int CPB = K / NB > 0 ? K / NB : 1;  // columns per block
        if (ROWS * K > 0 && threadIdx.x < ROWS * CPB) {
            const int row = threadIdx.x / CPB, col = blockIdx.x * CPB + threadIdx.x % CPB;
            dst[row * K + col] = s * 1e-30f + 1.f;
        }
        acc += s;
        if (!grid_wait<MODE>(ctr, static_cast<unsigned>(r + 1), fail)) break;
    }
    if (acc == 12345.f) sink[blockIdx.x] = acc;
}

template <int ROWS, int K, int MODE>
static int run(const char *name, int R, float *a0, float *a1, unsigned *ctr, unsigned *fail, float *sink, hipStream_t st) {
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    float best = 1e30f;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipMemsetAsync(ctr, 0, 4 * 2048, st));
        CHECK(hipMemsetAsync(fail, 0, 4, st));
        void *args[] = {&a0, &a1, &ctr, &fail, &R, &sink};
        CHECK(hipEventRecord(e0, st));
        CHECK(hipLaunchCooperativeKernel(reinterpret_cast<void *>(k_phase<ROWS, K, MODE>), dim3(NB), dim3(BT), args, 0, st));
        CHECK(hipEventRecord(e1, st));
        CHECK(hipEventSynchronize(e1));
        float ms;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        unsigned f;
        CHECK(hipMemcpy(&f, fail, 4, hipMemcpyDeviceToHost));
        if (f) {
            std::printf("%s: capped wait\n", name);
            return 1;
        }
        if (ms < best) best = ms;
    }
    std::printf("%-60s %7.3f us/round\n", name, best * 1e3f / R);
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
    return 0;
}

template <int ROWS, int K>
static int run4(const char *label, int R, float *a0, float *a1, unsigned *ctr, unsigned *fail, float *sink, hipStream_t st) {
    static const char *mn[4] = {"release/acquire", "+ sleep", "relaxed, no fences", "two-level, XCD flags"};
    char nm[128];
    std::snprintf(nm, sizeof nm, "%s [%s]", label, mn[0]);
    if (run<ROWS, K, 0>(nm, R, a0, a1, ctr, fail, sink, st)) return 1;
    std::snprintf(nm, sizeof nm, "%s [%s]", label, mn[1]);
    if (run<ROWS, K, 1>(nm, R, a0, a1, ctr, fail, sink, st)) return 1;
    std::snprintf(nm, sizeof nm, "%s [%s]", label, mn[2]);
    if (run<ROWS, K, 2>(nm, R, a0, a1, ctr, fail, sink, st)) return 1;
    std::snprintf(nm, sizeof nm, "%s [%s]", label, mn[3]);
    if (run<ROWS, K, 3>(nm, R, a0, a1, ctr, fail, sink, st)) return 1;
    return 0;
}

int main(int argc, char **argv) {
    const int R = argc > 1 ? std::atoi(argv[1]) : 2000;
    hipStream_t st;
    CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    float *a0, *a1, *sink;
    unsigned *ctr, *fail;
    const size_t n = 32 * 3072 + 64;
    CHECK(hipMalloc(&a0, n * 4));
    CHECK(hipMalloc(&a1, n * 4));
    CHECK(hipMalloc(&sink, NB * 4));
    CHECK(hipMalloc(&ctr, 4 * 2048));
    CHECK(hipMalloc(&fail, 4));
    CHECK(hipMemset(a0, 0, n * 4));
    CHECK(hipMemset(a1, 0, n * 4));
    if (run4<0, 0>("barrier only", R, a0, a1, ctr, fail, sink, st)) return 1;
    if (run4<32, 1024>("read 32x1024 f32", R, a0, a1, ctr, fail, sink, st)) return 1;
    if (run4<32, 3072>("read 32x3072 f32", R, a0, a1, ctr, fail, sink, st)) return 1;
    return 0;
}
