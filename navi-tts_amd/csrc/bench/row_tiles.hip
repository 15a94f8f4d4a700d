// The row projections on the row-major layout (rows.h launch_rows, activation rows padded by 8
// floats) against the MFMA tile layouts (rows.h launch_rows_pk) at the row counts of the prompt
// prefill (10, 130), the multi-stream decode (32) and the code predictor's first pass (64): the
// talker's four shapes, q|k|v (K 1024 -> 4096, RMSNorm fused), o (2048 -> 1024, residual add),
// down (3072 -> 1024, residual add) and gate|up (1024 -> 2 x 3072, RMSNorm and SwiGLU fused).
// A chain of 100 dependent launches per line (best of 3), each launch reading a different weight
// copy of a ~400 MB ring, so the weights come from HBM as in a prefill or a decode step. Timing only:
// the buffers are zero-filled and every launch reads and writes inside them.
#include <hip/hip_runtime.h>

#include <cstdio>
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

static hipStream_t s;
static hipEvent_t e0, e1;

static float chain(int R, const std::function<void(int)> &launch) {
    for (int i = 0; i < R; ++i) launch(i);
    (void) hipStreamSynchronize(s);
    float best = 1e30f, ms = 0.f;
    for (int rep = 0; rep < 3; ++rep) {
        (void) hipEventRecord(e0, s);
        for (int i = 0; i < R; ++i) launch(i);
        (void) hipEventRecord(e1, s);
        (void) hipEventSynchronize(e1);
        (void) hipEventElapsedTime(&ms, e0, e1);
        if (ms < best) best = ms;
    }
    return best * 1e3f / R;
}

int main() {
    CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    constexpr int MMAX = 144, KMAX = 3072 + 8, NMAX = 6144 + 8;   // rows padded to whole 16-row tiles
    const size_t WBYTES = size_t(1300) << 20;
    float *A, *Y, *ln;
    uint16_t *W;
    uint32_t *flag;
    CHECK(hipMalloc(&A, sizeof(float) * MMAX * KMAX));
    CHECK(hipMalloc(&Y, sizeof(float) * MMAX * NMAX));
    CHECK(hipMalloc(&ln, sizeof(float) * KMAX));
    CHECK(hipMalloc(&W, WBYTES));
    CHECK(hipMalloc(&flag, 4));
    CHECK(hipMemset(A, 0, sizeof(float) * MMAX * KMAX));
    CHECK(hipMemset(Y, 0, sizeof(float) * MMAX * NMAX));
    CHECK(hipMemset(ln, 0, sizeof(float) * KMAX));
    CHECK(hipMemset(W, 0, WBYTES));
    CHECK(hipMemset(flag, 0, 4));
    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, 0));
    std::printf("device %s, %d CUs; chains of 100 dependent launches, weights from a ~400 MB ring\n", prop.gcnArchName,
                prop.multiProcessorCount);
    struct P {
        const char *name;
        int epi, K, N;        // N: output columns (gate|up: F, the weight has 2F rows)
        bool norm;
    };
    const P ps[4] = {{"q|k|v", EPI_PLAIN, 1024, 4096, true},
                     {"o", EPI_RESID, 2048, 1024, false},
                     {"down", EPI_RESID, 3072, 1024, false},
                     {"gate|up", EPI_SWIGLU, 1024, 3072, true}};
    for (int M : {10, 32, 64, 130}) {
        float sum[2] = {0.f, 0.f};
        for (const P &p : ps) {
            const int wrows = p.epi == EPI_SWIGLU ? 2 * p.N : p.N;
            const size_t wel = static_cast<size_t>(wrows) * p.K;
            const int ring = static_cast<int>(((size_t(400) << 20) + 2 * wel - 1) / (2 * wel));
            if (static_cast<size_t>(ring) * wel * 2 > WBYTES) return 1;
            auto wp = [&](int i) { return W + static_cast<size_t>(i % ring) * wel; };
            const float t_rows = chain(100, [&](int i) {
                const uint16_t *w = wp(i);
                if (p.epi == EPI_SWIGLU)
                    launch_rows(p.epi, true, A, p.K + 8, M, p.K, ln, 1e-6f, w, p.N, w + static_cast<size_t>(p.N) * p.K, p.N,
                                nullptr, 0, Y, p.N + 8, flag, s);
                else
                    launch_rows(p.epi, p.norm, A, p.K + 8, M, p.K, ln, 1e-6f, w, p.N, nullptr, 0, nullptr, 0, Y, p.N + 8, flag, s);
            });
            bool ok = true;
            const float t_tiled = chain(100, [&](int i) {
                ok &= launch_rows_pk(p.epi, p.norm, A, M, p.K, ln, 1e-6f, wp(i), p.N, Y, p.N, flag, s);
            });
            if (!ok) {
                std::printf("launch_rows_pk refused %s at %d rows\n", p.name, M);
                return 1;
            }
            sum[0] += t_rows;
            sum[1] += t_tiled;
            std::printf("%3d rows  %-8s row-major %6.2f us   tiled %6.2f us\n", M, p.name, t_rows, t_tiled);
        }
        std::printf("%3d rows  a layer's four projections: row-major %6.2f us, tiled %6.2f us\n", M, sum[0], sum[1]);
    }
    CHECK(hipStreamSynchronize(s));
    return 0;
}
