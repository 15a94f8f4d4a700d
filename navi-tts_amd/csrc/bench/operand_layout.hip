// Read rate of the MFMA operand loads by memory layout on MI355X: the row projections' A (f32
// activations) and W (f16 weights) fragments, read from L2-resident data, as the row-major layout
// gives them (one wave instruction = 16 rows x 4 lanes x 16 bytes, 16 cache lines half used) against
// the tile layout of rows.h (one wave instruction = 1 KB contiguous, 8 lines), plus 8 rows x 128 bytes.
//
// Each block (512 threads) reads 16 instructions x 16 bytes per lane = 128 KB and drops it. Block b
// reads region (b / 8) % nreg of 140 KB regions (blocks of one XCD share regions, so the data stays in
// that XCD's L2 for nreg 16 but not in the CUs' L1s; nreg 64 spills to the memory-side cache and HBM).
// Each line is the best of 3 timed chains of 50 launches; the rate is over the time above a 2.5 us
// launch floor (the empty-kernel chain of launch_floor.hip). All reads stay inside one 256 MB buffer.
#include <hip/hip_runtime.h>

#include <cstdio>

#define CHECK(x)                                                                              \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) {                                                               \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            return 1;                                                                         \
        }                                                                                     \
    } while (0)

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int NI = 16;                   // load instructions per wave
constexpr size_t REGION = 140 << 10;     // bytes between regions
constexpr int RS = 4128;                 // row stride of the row-major layouts (1032 floats)

// PAT 0: tile layout, instruction i of wave w reads 1 KB at (w NI + i) KB.
// PAT 1: row-major MFMA operand, lane 16 kq + c reads row c at byte 32 kq + 16 (i & 1) of its
//        128-byte step i / 2 (the two instructions of a step take the two halves of 16 lines).
// PAT 2: 8 rows x 128 bytes per instruction (lane l: row l / 8, bytes 16 (l % 8)).
template <int PAT>
__global__ void __launch_bounds__(512) k_read(const char *base, int nreg, float *sink) {
    const int w = threadIdx.x / 64, l = threadIdx.x & 63, c = l & 15, kq = l >> 4;
    const char *p = base + static_cast<size_t>((blockIdx.x / 8) % nreg) * REGION;
    f4 v[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        size_t off;
        if (PAT == 0) off = static_cast<size_t>(w) * NI * 1024 + static_cast<size_t>(i) * 1024 + 16 * l;
        else if (PAT == 1)
            off = static_cast<size_t>(16 * (w & 1) + c) * RS + static_cast<size_t>(w >> 1) * (NI / 2) * 128 +
                  static_cast<size_t>(i >> 1) * 128 + 32 * kq + 16 * (i & 1);
        else off = static_cast<size_t>(8 * (w & 3) + (l >> 3)) * RS + static_cast<size_t>(w >> 2) * NI * 128 + static_cast<size_t>(i) * 128 + 16 * (l & 7);
        v[i] = *reinterpret_cast<const f4 *>(p + off);
    }
    f4 s = v[0];
#pragma unroll
    for (int i = 1; i < NI; ++i) s += v[i];
    if (s[0] + s[1] + s[2] + s[3] == 1234.5f) sink[0] = 1.f;   // keeps the loads; never true for zeros
}

int main() {
    hipStream_t s;
    hipEvent_t e0, e1;
    CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    const size_t TOT = size_t(256) << 20;     // >= 64 regions x 140 KB; every offset above stays < 140 KB
    char *buf;
    float *sink;
    CHECK(hipMalloc(&buf, TOT));
    CHECK(hipMalloc(&sink, 4));
    CHECK(hipMemset(buf, 0, TOT));
    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, 0));
    std::printf("device %s, %d CUs; 128 KB per 512-thread block, 16 load instructions per wave\n", prop.gcnArchName,
                prop.multiProcessorCount);
    auto run = [&](const char *name, void (*kern)(const char *, int, float *), int blocks, int nreg) -> int {
        constexpr int R = 50;
        for (int i = 0; i < 5; ++i) hipLaunchKernelGGL(kern, dim3(blocks), dim3(512), 0, s, buf, nreg, sink);
        CHECK(hipStreamSynchronize(s));
        float best = 1e30f, ms = 0.f;
        for (int rep = 0; rep < 3; ++rep) {
            CHECK(hipEventRecord(e0, s));
            for (int i = 0; i < R; ++i) hipLaunchKernelGGL(kern, dim3(blocks), dim3(512), 0, s, buf, nreg, sink);
            CHECK(hipEventRecord(e1, s));
            CHECK(hipEventSynchronize(e1));
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            if (ms < best) best = ms;
        }
        const double us = best * 1e3 / R, bytes = double(blocks) * (128 << 10);
        std::printf("%-44s blocks %4d  regions %2d  %7.2f us/launch  %6.1f TB/s above the floor\n", name, blocks, nreg, us,
                    us > 2.6 ? bytes / (us - 2.5) / 1e6 : 0.0);
        return 0;
    };
    for (int nreg : {16, 64})
        for (int blocks : {256, 1024}) {
            if (run("tile layout (1 KB per instruction)", k_read<0>, blocks, nreg)) return 1;
            if (run("row-major operand (16 rows x 64 B)", k_read<1>, blocks, nreg)) return 1;
            if (run("8 rows x 128 B", k_read<2>, blocks, nreg)) return 1;
        }
    return 0;
}
