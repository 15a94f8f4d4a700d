// Dependent-launch floor on MI355X: the cost of one link in a chain of kernels on one stream, the
// way the multi-stream decode (streams.hip, 582 launches per step, replayed from a HIP graph) and
// the prompt prefill (prefill.hip, 170 launches) run. R launches of the same kernel, each waiting
// for the one before (same stream), timed with events, eagerly and as a replayed graph:
//   empty       : a kernel of the row projections' grid (256 blocks x 512 threads) that does nothing;
//   rows qkv    : the multi-stream q|k|v projection (rows.h k_rows<2, PLAIN, norm, 8 waves x 4 steps>:
//                 32 rows, K 1024, N 4096), weights and inputs already in the caches after warm-up;
//   rows o      : the residual o projection (k_rows<1, RESID, 16 x 4>: 32 rows, K 2048, N 1024);
//   rows down   : the residual down projection (k_rows<1, RESID, 16 x 6>: 32 rows, K 3072, N 1024);
//   rows gate|up: k_rows<2, SWIGLU, norm, 8 x 4> (32 rows, K 1024, F 3072).
// Each projection runs twice: with the input rows K floats apart (strides of 4, 8 or 12 KB) and
// 8 floats further apart, the padding the decode and the prefill lay their activations out with.
// Buffers are zero-filled; every launch reads and writes inside them.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <functional>

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

static hipStream_t s;
static hipEvent_t e0, e1;

static int chain(const char *name, int R, const std::function<void()> &launch) {
    for (int i = 0; i < R; ++i) launch();
    CHECK(hipStreamSynchronize(s));
    float ms = 0.f;
    CHECK(hipEventRecord(e0, s));
    for (int i = 0; i < R; ++i) launch();
    CHECK(hipEventRecord(e1, s));
    CHECK(hipEventSynchronize(e1));
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const float eager = ms * 1e3f / R;
    hipGraph_t g;
    hipGraphExec_t ge;
    CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < R; ++i) launch();
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
    std::printf("%-56s eager %6.2f us   graph %6.2f us per launch\n", name, eager, best * 1e3f / R);
    CHECK(hipGraphExecDestroy(ge));
    CHECK(hipGraphDestroy(g));
    return 0;
}

int main(int argc, char **argv) {
    const int R = argc > 1 ? std::atoi(argv[1]) : 200;
    CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, 0));
    std::printf("device %s, %d CUs; chains of %d dependent launches\n", prop.gcnArchName, prop.multiProcessorCount, R);
    const int M = 32, KMAX = 3072 + 8, NMAX = 6144 + 8;
    float *A, *Y, *ln;
    uint16_t *W;
    uint32_t *flag;
    CHECK(hipMalloc(&A, sizeof(float) * M * KMAX));
    CHECK(hipMalloc(&Y, sizeof(float) * M * NMAX));
    CHECK(hipMalloc(&ln, sizeof(float) * KMAX));
    CHECK(hipMalloc(&W, sizeof(uint16_t) * NMAX * KMAX));
    CHECK(hipMalloc(&flag, 4));
    CHECK(hipMemset(A, 0, sizeof(float) * M * KMAX));
    CHECK(hipMemset(Y, 0, sizeof(float) * M * NMAX));
    CHECK(hipMemset(ln, 0, sizeof(float) * KMAX));
    CHECK(hipMemset(W, 0, sizeof(uint16_t) * NMAX * KMAX));
    CHECK(hipMemset(flag, 0, 4));
    if (chain("empty (256 x 512)", R, [&] { hipLaunchKernelGGL(k_empty, dim3(256), dim3(512), 0, s, nullptr); })) return 1;
    for (int pad : {0, 8}) {
        char nm[96];
        {
            const RowArgs ra{A, ln, W, W, W, Y, flag, 1024 + pad, M, 1024, 4096, 4096, 0, 4096, 1e-6f};
            std::snprintf(nm, sizeof nm, "rows qkv (32 x 1024 -> 4096, norm), lda %d", 1024 + pad);
            if (chain(nm, R, [&] {
                    hipLaunchKernelGGL((k_rows<2, EPI_PLAIN, true, 8, 4>), dim3(4096 / 16, 1), dim3(512), 0, s, ra);
                }))
                return 1;
        }
        {
            const RowArgs ra{A, nullptr, W, nullptr, nullptr, Y, flag, 2048 + pad, M, 2048, 1024, 1024, 0, 1024 + pad, 0.f};
            std::snprintf(nm, sizeof nm, "rows o (32 x 2048 -> 1024, residual), lda %d", 2048 + pad);
            if (chain(nm, R, [&] {
                    hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 4>), dim3(1024 / 16, 2), dim3(1024), 0, s, ra);
                }))
                return 1;
        }
        {
            const RowArgs ra{A, nullptr, W, nullptr, nullptr, Y, flag, 3072 + pad, M, 3072, 1024, 1024, 0, 1024 + pad, 0.f};
            std::snprintf(nm, sizeof nm, "rows down (32 x 3072 -> 1024, residual), lda %d", 3072 + pad);
            if (chain(nm, R, [&] {
                    hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 6>), dim3(1024 / 16, 2), dim3(1024), 0, s, ra);
                }))
                return 1;
        }
        {
            const RowArgs ra{A, ln, W, W, nullptr, Y, flag, 1024 + pad, M, 1024, 3072, 6144, 3072, 3072 + pad, 1e-6f};
            std::snprintf(nm, sizeof nm, "rows gate|up (32 x 1024 -> 3072, SwiGLU), lda %d", 1024 + pad);
            if (chain(nm, R, [&] {
                    hipLaunchKernelGGL((k_rows<2, EPI_SWIGLU, true, 8, 4>), dim3(3072 / 16, 1), dim3(512), 0, s, ra);
                }))
                return 1;
        }
    }
    return 0;
}
