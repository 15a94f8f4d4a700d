// Dependent-launch floor on MI355X: the cost of one link in a chain of kernels on one stream, the
// way the multi-stream decode (streams.hip, 582 launches per step, replayed from a HIP graph) and
// the prompt prefill (prefill.hip, 170 launches) run. R launches of the same kernel, each waiting
// for the one before (same stream), timed with events, eagerly and as a replayed graph:
//   empty       : a kernel of the row projections' grid (256 blocks x 512 threads) that does nothing;
//   rows qkv    : the multi-stream q|k|v projection (rows.h k_rows<2, PLAIN, norm, 8 waves x 4 steps>:
//                 32 rows, K 1024, N 4096);
//   rows o      : the residual o projection (k_rows<1, RESID, 16 x 4>: 32 rows, K 2048, N 1024);
//   rows down   : the residual down projection (k_rows<1, RESID, 16 x 6>: 32 rows, K 3072, N 1024);
//   rows gate|up: k_rows<2, SWIGLU, norm, 8 x 4> (32 rows, K 1024, F 3072).
// Each projection runs with the input rows K floats apart (strides of 4, 8 or 12 KB) and 8 floats
// further apart (the padding the decode and the prefill lay their activations out with), every
// launch on the same weights (cache-resident after the warm-up chain). The padded projections then
// run on a ring of weight copies, launch i reading copy i mod n: a ring of ~128 MB stays in the
// 256 MB memory-side cache (MALL) but not in the L2s, one of ~400 MB comes from HBM. The last
// variant adds, to the 400 MB ring, a prefetch of launch i + 2's weights (a 32 x 256 kernel reading
// them) on a second captured stream that forks after launch i and joins at the end of the chain.
// Buffers are zero-filled; every launch reads and writes inside them.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <functional>
#include <utility>

#include "rows.h"

using namespace navi_amd::rows;

#define CHECK(x)                                                                              \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) {                                                               \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            return 1;                                                                         \
        }                                                                                     \
    } while (0)

__global__ void __launch_bounds__(512) k_empty(int *p) {
    if (p && threadIdx.x == 0 && blockIdx.x == 0) p[0] = 0;
}

// Reads n16 16-byte words from p (8 loads in flight per thread) and drops them: the prefetch.
__global__ void __launch_bounds__(256) k_touch(const uint4 *p, size_t n16, unsigned *sink) {
    unsigned acc = 0;
    const size_t stride = static_cast<size_t>(gridDim.x) * 256 * 8;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 * 8 + threadIdx.x; i < n16; i += stride) {
        uint4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = i + 256 * j < n16 ? p[i + 256 * j] : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

static hipStream_t s, s2;
static hipEvent_t e0, e1, ef, ej;
static unsigned *g_sink;
static int g_pfblocks = 32;

// chain of R launches (launch(i)), each launch i also forks a prefetch of the weights of launch
// i + 2 (bytes returned by pf(i + 2)) onto s2, dependent on launch i; graph only
static int chain_pf(const char *name, int R, const std::function<void(int)> &launch,
                    const std::function<std::pair<const void *, size_t>(int)> &pf) {
    hipGraph_t g;
    hipGraphExec_t ge;
    CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < R; ++i) {
        launch(i);
        CHECK(hipEventRecord(ef, s));
        CHECK(hipStreamWaitEvent(s2, ef, 0));
        auto r = pf(i + 2);
        hipLaunchKernelGGL(k_touch, dim3(g_pfblocks), dim3(256), 0, s2, static_cast<const uint4 *>(r.first), r.second / 16, g_sink);
    }
    CHECK(hipEventRecord(ej, s2));
    CHECK(hipStreamWaitEvent(s, ej, 0));
    CHECK(hipStreamEndCapture(s, &g));
    CHECK(hipGraphInstantiateWithFlags(&ge, g, 0));
    CHECK(hipGraphLaunch(ge, s));
    CHECK(hipStreamSynchronize(s));
    float best = 1e30f, ms = 0.f;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(e0, s));
        CHECK(hipGraphLaunch(ge, s));
        CHECK(hipEventRecord(e1, s));
        CHECK(hipEventSynchronize(e1));
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        if (ms < best) best = ms;
    }
    std::printf("%-64s                 graph %6.2f us per launch\n", name, best * 1e3f / R);
    CHECK(hipGraphExecDestroy(ge));
    CHECK(hipGraphDestroy(g));
    return 0;
}

static int chain(const char *name, int R, const std::function<void(int)> &launch) {
    for (int i = 0; i < R; ++i) launch(i);
    CHECK(hipStreamSynchronize(s));
    float ms = 0.f;
    CHECK(hipEventRecord(e0, s));
    for (int i = 0; i < R; ++i) launch(i);
    CHECK(hipEventRecord(e1, s));
    CHECK(hipEventSynchronize(e1));
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const float eager = ms * 1e3f / R;
    hipGraph_t g;
    hipGraphExec_t ge;
    CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < R; ++i) launch(i);
    CHECK(hipStreamEndCapture(s, &g));
    CHECK(hipGraphInstantiateWithFlags(&ge, g, 0));
    CHECK(hipGraphLaunch(ge, s));
    CHECK(hipStreamSynchronize(s));
    float best = 1e30f;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(e0, s));
        CHECK(hipGraphLaunch(ge, s));
        CHECK(hipEventRecord(e1, s));
        CHECK(hipEventSynchronize(e1));
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        if (ms < best) best = ms;
    }
    std::printf("%-64s eager %6.2f us   graph %6.2f us per launch\n", name, eager, best * 1e3f / R);
    CHECK(hipGraphExecDestroy(ge));
    CHECK(hipGraphDestroy(g));
    return 0;
}

int main(int argc, char **argv) {
    const int R = argc > 1 ? std::atoi(argv[1]) : 200;
    if (argc > 2) g_pfblocks = std::atoi(argv[2]);
    CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    CHECK(hipStreamCreateWithFlags(&s2, hipStreamNonBlocking));
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    CHECK(hipEventCreateWithFlags(&ef, hipEventDisableTiming));
    CHECK(hipEventCreateWithFlags(&ej, hipEventDisableTiming));
    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, 0));
    std::printf("device %s, %d CUs; chains of %d dependent launches; prefetch grid %d x 256\n", prop.gcnArchName, prop.multiProcessorCount, R, g_pfblocks);
    const int M = 32, KMAX = 3072 + 8, NMAX = 6144 + 8;
    const size_t WBYTES = size_t(1300) << 20;
    float *A, *Y, *ln;
    uint16_t *W;
    uint32_t *flag;
    CHECK(hipMalloc(&A, sizeof(float) * M * KMAX));
    CHECK(hipMalloc(&Y, sizeof(float) * M * NMAX));
    CHECK(hipMalloc(&ln, sizeof(float) * KMAX));
    CHECK(hipMalloc(&W, WBYTES));
    CHECK(hipMalloc(&flag, 4));
    CHECK(hipMalloc(&g_sink, 4));
    CHECK(hipMemset(A, 0, sizeof(float) * M * KMAX));
    CHECK(hipMemset(Y, 0, sizeof(float) * M * NMAX));
    CHECK(hipMemset(ln, 0, sizeof(float) * KMAX));
    CHECK(hipMemset(W, 0, WBYTES));
    CHECK(hipMemset(flag, 0, 4));
    if (chain("empty (256 x 512)", R, [&](int) { hipLaunchKernelGGL(k_empty, dim3(256), dim3(512), 0, s, nullptr); })) return 1;
    for (int pad : {0, 8}) {
        char nm[96];
        {
            const RowArgs ra{A, ln, W, W, W, Y, flag, 1024 + pad, M, 1024, 4096, 4096, 0, 4096, 1e-6f};
            std::snprintf(nm, sizeof nm, "rows qkv (32 x 1024 -> 4096, norm), lda %d", 1024 + pad);
            if (chain(nm, R, [&](int) {
                    hipLaunchKernelGGL((k_rows<2, EPI_PLAIN, true, 8, 4>), dim3(4096 / 16, 1), dim3(512), 0, s, ra);
                }))
                return 1;
        }
        {
            const RowArgs ra{A, nullptr, W, nullptr, nullptr, Y, flag, 2048 + pad, M, 2048, 1024, 1024, 0, 1024 + pad, 0.f};
            std::snprintf(nm, sizeof nm, "rows o (32 x 2048 -> 1024, residual), lda %d", 2048 + pad);
            if (chain(nm, R, [&](int) {
                    hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 4>), dim3(1024 / 16, 2), dim3(1024), 0, s, ra);
                }))
                return 1;
        }
        {
            const RowArgs ra{A, nullptr, W, nullptr, nullptr, Y, flag, 3072 + pad, M, 3072, 1024, 1024, 0, 1024 + pad, 0.f};
            std::snprintf(nm, sizeof nm, "rows down (32 x 3072 -> 1024, residual), lda %d", 3072 + pad);
            if (chain(nm, R, [&](int) {
                    hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 6>), dim3(1024 / 16, 2), dim3(1024), 0, s, ra);
                }))
                return 1;
        }
        {
            const RowArgs ra{A, ln, W, W + size_t(3072) * 1024, nullptr, Y, flag, 1024 + pad, M, 1024, 3072, 6144, 3072, 3072 + pad, 1e-6f};
            std::snprintf(nm, sizeof nm, "rows gate|up (32 x 1024 -> 3072, SwiGLU), lda %d", 1024 + pad);
            if (chain(nm, R, [&](int) {
                    hipLaunchKernelGGL((k_rows<2, EPI_SWIGLU, true, 8, 4>), dim3(3072 / 16, 1), dim3(512), 0, s, ra);
                }))
                return 1;
        }
    }
    struct P { const char *nm; int K, N; };
    const P ps[4] = {{"qkv", 1024, 4096}, {"o", 2048, 1024}, {"down", 3072, 1024}, {"gate|up", 1024, 6144}};
    const size_t targets[2] = {size_t(128) << 20, size_t(400) << 20};
    for (int pi = 0; pi < 4; ++pi) {
        const P &p = ps[pi];
        const size_t wel = size_t(p.N) * p.K, wb = wel * 2;
        for (int ti = 0; ti < 3; ++ti) {
            const size_t tgt = targets[ti < 2 ? ti : 1];
            const int ring = static_cast<int>((tgt + wb - 1) / wb);
            if (size_t(ring) * wb > WBYTES) return 1;
            auto wp = [&](int i) { return W + size_t(i % ring) * wel; };
            auto launch = [&](int i) {
                const uint16_t *w = wp(i);
                if (pi == 0) {
                    const RowArgs ra{A, ln, w, w, w, Y, flag, 1024 + 8, M, 1024, 4096, 4096, 0, 4096, 1e-6f};
                    hipLaunchKernelGGL((k_rows<2, EPI_PLAIN, true, 8, 4>), dim3(4096 / 16, 1), dim3(512), 0, s, ra);
                } else if (pi == 1) {
                    const RowArgs ra{A, nullptr, w, nullptr, nullptr, Y, flag, 2048 + 8, M, 2048, 1024, 1024, 0, 1024 + 8, 0.f};
                    hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 4>), dim3(1024 / 16, 2), dim3(1024), 0, s, ra);
                } else if (pi == 2) {
                    const RowArgs ra{A, nullptr, w, nullptr, nullptr, Y, flag, 3072 + 8, M, 3072, 1024, 1024, 0, 1024 + 8, 0.f};
                    hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 6>), dim3(1024 / 16, 2), dim3(1024), 0, s, ra);
                } else {
                    const RowArgs ra{A, ln, w, w + size_t(3072) * 1024, nullptr, Y, flag, 1024 + 8, M, 1024, 3072, 6144, 3072, 3072 + 8, 1e-6f};
                    hipLaunchKernelGGL((k_rows<2, EPI_SWIGLU, true, 8, 4>), dim3(3072 / 16, 1), dim3(512), 0, s, ra);
                }
            };
            char nm[128];
            std::snprintf(nm, sizeof nm, "rows %s (32 x %d -> %d), lda +8, ring %d x %.1f MB = %.0f MB%s", p.nm, p.K, pi == 3 ? 3072 : p.N, ring,
                          wb / 1048576.0, ring * wb / 1048576.0, ti == 2 ? ", prefetch i+2" : "");
            if (ti < 2) {
                if (chain(nm, R, launch)) return 1;
            } else {
                if (chain_pf(nm, R, launch, [&](int i) { return std::make_pair(static_cast<const void *>(wp(i)), wb); })) return 1;
            }
        }
    }
    return 0;
}
