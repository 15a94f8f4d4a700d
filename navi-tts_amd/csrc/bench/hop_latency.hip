// Hop latency of the frame kernel's communication primitive on MI355X: a persistent grid of one
// 256-thread block per CU exchanging tagged 64-bit words {f32, u32 tag} with agent-scope relaxed
// stores and loads (what k_frame's phases do between layers, frame.hip). Each pattern runs R
// rounds in one cooperative launch; a round is one complete exchange (every block publishes its
// share, then waits for and reads everything it needs), so us/round is the cost of one hop with
// no compute around it. Rounds alternate two mailbox regions: a region is rewritten only after
// every block has finished reading it (a block publishes round r only after its round r - 1
// gather, which needed every block's round r - 1 words, published after their round r - 2 reads).
//
// Patterns:
//   all-gather N, 8 copies : every block publishes N/256 words to 8 copies (one per XCD) and
//                            gathers all N words from its own XCD's copy (k_frame's broadcast);
//   all-gather N, 1 copy   : the same from a single copy;
//   all-gather N, chunk polls: 8 copies, but every thread polls all words of its producer's chunk
//                            until every tag matches, so the poll that succeeds delivers the data
//                            (no sentinel round and no second read after a barrier);
//   reduce-scatter 1024    : every block publishes 4 words to each of the 256 blocks (one copy)
//                            and gathers the 1024 words addressed to it (the shape of a split
//                            matvec whose partial sums go to the row owners);
//   XCD-local all-gather   : the 32 blocks of one XCD exchange 1024 words among themselves;
//   one-way, same / other XCD : block 0 and one partner bounce a word; half a round trip.
// Every wait has a spin cap; a capped wait sets the fail word, every later wait gives up, and
// the pattern is reported as failed.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

#define CHECK(x)                                                                              \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) {                                                               \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);        \
            return 1;                                                                         \
        }                                                                                     \
    } while (0)

namespace {

constexpr int NB = 256, BT = 256, NREP = 8, NQ = NB / 64;
constexpr unsigned long long CAP = 2000000ull;

__device__ __forceinline__ void put(uint64_t *p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t peek(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t tag_of(uint64_t w) { return static_cast<uint32_t>(w >> 32); }
__device__ __forceinline__ uint64_t word(uint32_t tag, float v) { return (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v); }
__device__ __forceinline__ int xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15; }

// Wave 0 polls the sentinel of each of `np` producer chunks (chunk q's last word at
// base + q * stride + stride - 1), all in flight at once; then the block reads the N words from
// base, every thread's N / BT loads issued before any is checked. Returns false on a capped wait
// (and sets *fail).
template <int N>
__device__ bool wait_and_read(const uint64_t *base, int np, int stride, uint32_t tag, uint32_t *fail, float *dst, int &bad) {
    if (threadIdx.x < 64) {
        uint64_t sw[NQ];
        const int l = threadIdx.x;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int pr = l + 64 * q;
            sw[q] = pr < np ? peek(base + static_cast<size_t>(pr) * stride + stride - 1) : static_cast<uint64_t>(tag) << 32;
        }
        unsigned long long s = 0;
        for (;;) {
            bool done = true;
#pragma unroll
            for (int q = 0; q < NQ; ++q) done &= tag_of(sw[q]) == tag;
            if (done) break;
            if (++s >= CAP || ((s & 63) == 0 && peek(reinterpret_cast<const uint64_t *>(fail)) != 0)) {
                bad = 1;
                break;
            }
#pragma unroll
            for (int q = 0; q < NQ; ++q)
                if (tag_of(sw[q]) != tag) sw[q] = peek(base + static_cast<size_t>(l + 64 * q) * stride + stride - 1);
        }
    }
    __syncthreads();
    if (bad) {
        if (threadIdx.x == 0) __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    constexpr int PER = N / BT;
    uint64_t w[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) w[k] = peek(base + threadIdx.x + k * BT);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        unsigned long long s = 0;
        while (tag_of(w[k]) != tag) {
            if (++s >= CAP) {
                bad = 1;
                break;
            }
            w[k] = peek(base + threadIdx.x + k * BT);
        }
        dst[threadIdx.x + k * BT] = __uint_as_float(static_cast<uint32_t>(w[k]));
    }
    __syncthreads();
    if (bad && threadIdx.x == 0) __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return bad == 0;
}

// every thread polls its own PER contiguous words (producer t's whole chunk when CH == PER) until
// every tag matches: the poll that succeeds delivers the data (no second read after a barrier)
template <int N>
__device__ bool wait_full(const uint64_t *base, uint32_t tag, uint32_t *fail, float *dst, int &bad) {
    constexpr int PER = N / BT;
    const uint64_t *p = base + threadIdx.x * PER;
    uint64_t w[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) w[k] = peek(p + k);
    unsigned long long s = 0;
    for (;;) {
        bool done = true;
#pragma unroll
        for (int k = 0; k < PER; ++k) done &= tag_of(w[k]) == tag;
        if (done) break;
        if (++s >= CAP || ((s & 63) == 0 && peek(reinterpret_cast<const uint64_t *>(fail)) != 0)) {
            bad = 1;
            break;
        }
#pragma unroll
        for (int k = 0; k < PER; ++k)
            if (tag_of(w[k]) != tag) w[k] = peek(p + k);
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) dst[threadIdx.x * PER + k] = __uint_as_float(static_cast<uint32_t>(w[k]));
    __syncthreads();
    if (bad && threadIdx.x == 0) __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return bad == 0;
}

// MODE 0: all-gather over the grid (N words, REPL copies); 1: reduce-scatter (1024 words per
// block); 2: all-gather among the blocks of one XCD (1024 words); 3: MODE 0 with chunk polls.
template <int MODE, int N, int REPL>
__global__ void __launch_bounds__(BT, 1) k_hops(uint64_t *mb, size_t region, int rounds, uint32_t base_tag, uint32_t *fail,
                                                int *xcc_of_block) {
    __shared__ float buf[N];
    __shared__ int bad;
    if (threadIdx.x == 0) bad = 0;
    if (threadIdx.x == 0) xcc_of_block[blockIdx.x] = xcc_id();
    __syncthreads();
    const int b = blockIdx.x, x = xcc_id();
    float acc = 0.f;
    for (int r = 1; r <= rounds; ++r) {
        const uint32_t tag = base_tag + r;
        uint64_t *reg = mb + (r & 1) * region;
        if (MODE == 0) {
            constexpr int CH = N / NB;
            for (int i = threadIdx.x; i < CH * REPL; i += BT) {
                const int c = i % CH, rep = i / CH;
                put(reg + static_cast<size_t>(rep) * N + b * CH + c, word(tag, acc + c));
            }
            if (!wait_and_read<N>(reg + static_cast<size_t>(REPL > 1 ? x % REPL : 0) * N, NB, CH, tag, fail, buf, bad)) return;
        } else if (MODE == 3) {
            constexpr int CH = N / NB;
            for (int i = threadIdx.x; i < CH * REPL; i += BT) {
                const int c = i % CH, rep = i / CH;
                put(reg + static_cast<size_t>(rep) * N + b * CH + c, word(tag, acc + c));
            }
            if (!wait_full<N>(reg + static_cast<size_t>(REPL > 1 ? x % REPL : 0) * N, tag, fail, buf, bad)) return;
        } else if (MODE == 1) {
            // 4 words to every block d: slot d * 1024 + b * 4 .. + 3
            for (int i = threadIdx.x; i < NB * 4; i += BT) {
                const int d = i / 4, k = i % 4;
                put(reg + static_cast<size_t>(d) * 1024 + b * 4 + k, word(tag, acc + k));
            }
            if (!wait_and_read<1024>(reg + static_cast<size_t>(b) * 1024, NB, 4, tag, fail, buf, bad)) return;
        } else {
            // the 32 blocks of XCD x: block b is member b / 8 of group b % 8 (round-robin dispatch,
            // checked on the host from xcc_of_block)
            const int g = b % 8, m = b / 8;
            uint64_t *gr = reg + static_cast<size_t>(g) * 1024;
            for (int i = threadIdx.x; i < 32; i += BT) put(gr + m * 32 + i, word(tag, acc + i));
            if (!wait_and_read<1024>(gr, 32, 32, tag, fail, buf, bad)) return;
        }
        acc = buf[(threadIdx.x * 7 + r) % N] * 1e-9f;
        __syncthreads();
    }
}

// block 0 and block `other` (lane 0 of each) bounce a word `rounds` times.
__global__ void k_pingpong(uint64_t *w, int rounds, int other, uint32_t base, uint32_t *fail) {
    if (threadIdx.x != 0) return;
    const int b = blockIdx.x;
    if (b != 0 && b != other) return;
    for (int r = 1; r <= rounds; ++r) {
        const uint64_t ping = (static_cast<uint64_t>(base) << 32) + 2ull * r - 1, pong = ping + 1;
        unsigned long long s = 0;
        if (b == 0) {
            put(w, ping);
            while (peek(w + 16) != pong)
                if (++s >= CAP) { *fail = 1; return; }
        } else {
            while (peek(w) != ping)
                if (++s >= CAP) { *fail = 1; return; }
            put(w + 16, pong);
        }
    }
}

} // namespace

int main(int argc, char **argv) {
    int dev_count = 0;
    CHECK(hipGetDeviceCount(&dev_count));
    if (dev_count < 1) { std::printf("no device\n"); return 1; }
    hipDeviceProp_t prop{};
    CHECK(hipGetDeviceProperties(&prop, 0));
    if (prop.multiProcessorCount < NB) {
        std::printf("needs %d CUs, device has %d\n", NB, prop.multiProcessorCount);
        return 1;
    }
    const int rounds = argc > 1 ? std::atoi(argv[1]) : 2000;
    const size_t region = static_cast<size_t>(NB) * 1024 * NREP;   // words per region, the largest pattern's need
    uint64_t *mb = nullptr;
    uint32_t *fail = nullptr;
    int *xob = nullptr;
    CHECK(hipMalloc(&mb, 2 * region * sizeof(uint64_t)));
    CHECK(hipMemset(mb, 0, 2 * region * sizeof(uint64_t)));
    CHECK(hipMalloc(&fail, 8));
    CHECK(hipMemset(fail, 0, 8));
    CHECK(hipMalloc(&xob, NB * sizeof(int)));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    uint32_t base = 1000;
    std::printf("device %s, %d CUs; %d rounds per pattern, best of 3 launches\n", prop.name, prop.multiProcessorCount, rounds);
    struct P { const char *name; const void *fn; };
    const P pats[] = {
        {"all-gather 1024 words, 8 copies (per XCD)", reinterpret_cast<const void *>(k_hops<0, 1024, 8>)},
        {"all-gather 1024 words, 1 copy", reinterpret_cast<const void *>(k_hops<0, 1024, 1>)},
        {"all-gather 3072 words, 8 copies (per XCD)", reinterpret_cast<const void *>(k_hops<0, 3072, 8>)},
        {"all-gather 2048 words, 8 copies (per XCD)", reinterpret_cast<const void *>(k_hops<0, 2048, 8>)},
        {"all-gather 1024 words, 8 copies, chunk polls", reinterpret_cast<const void *>(k_hops<3, 1024, 8>)},
        {"all-gather 3072 words, 8 copies, chunk polls", reinterpret_cast<const void *>(k_hops<3, 3072, 8>)},
        {"reduce-scatter 1024 words (4 from each block)", reinterpret_cast<const void *>(k_hops<1, 1024, 1>)},
        {"XCD-local all-gather 1024 words (32 blocks)", reinterpret_cast<const void *>(k_hops<2, 1024, 1>)},
    };
    for (const P &p : pats) {
        float best = 1e30f;
        for (int rep = 0; rep < 3; ++rep) {
            size_t reg = region;
            int rr = rounds;
            void *args[] = {&mb, &reg, &rr, &base, &fail, &xob};
            CHECK(hipEventRecord(e0));
            CHECK(hipLaunchCooperativeKernel(p.fn, dim3(NB), dim3(BT), args, 0, 0));
            CHECK(hipEventRecord(e1));
            CHECK(hipEventSynchronize(e1));
            float ms = 0.f;
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            base += rounds + 8;
            uint32_t f = 0;
            CHECK(hipMemcpy(&f, fail, 4, hipMemcpyDeviceToHost));
            if (f) {
                std::printf("%-48s FAILED (a wait hit its cap)\n", p.name);
                return 2;
            }
            if (ms < best) best = ms;
        }
        if (p.fn == reinterpret_cast<const void *>(k_hops<2, 1024, 1>)) {
            int h[NB];
            CHECK(hipMemcpy(h, xob, sizeof h, hipMemcpyDeviceToHost));
            bool rr = true;
            for (int b = 0; b < NB; ++b) rr = rr && h[b] == h[b % 8];
            for (int g = 0; g < 8; ++g)
                for (int g2 = g + 1; g2 < 8; ++g2) rr = rr && h[g] != h[g2];
            std::printf("%-48s %7.3f us/hop%s\n", p.name, best * 1000.f / rounds,
                        rr ? "" : "  (dispatch was not round-robin over XCDs: groups span XCDs)");
        } else {
            std::printf("%-48s %7.3f us/hop\n", p.name, best * 1000.f / rounds);
        }
        std::fflush(stdout);
    }
    // one-way latency: partner 1 (another XCD under round-robin dispatch), partner 8 (the same XCD)
    int h[NB];
    CHECK(hipMemcpy(h, xob, sizeof h, hipMemcpyDeviceToHost));
    for (int other : {1, 8}) {
        float best = 1e30f;
        for (int rep = 0; rep < 3; ++rep) {
            uint64_t *w = mb;
            int rr = rounds;
            void *args[] = {&w, &rr, &other, &base, &fail};
            CHECK(hipEventRecord(e0));
            CHECK(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(k_pingpong), dim3(NB), dim3(64), args, 0, 0));
            CHECK(hipEventRecord(e1));
            CHECK(hipEventSynchronize(e1));
            float ms = 0.f;
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            base += 1;
            uint32_t f = 0;
            CHECK(hipMemcpy(&f, fail, 4, hipMemcpyDeviceToHost));
            if (f) {
                std::printf("one-way block 0 <-> %d FAILED\n", other);
                return 2;
            }
            if (ms < best) best = ms;
        }
        std::printf("one-way, block 0 (XCD %d) <-> block %d (XCD %d)%*s %7.3f us\n", h[0], other, h[other],
                    other < 10 ? 13 : 12, "", best * 1000.f / rounds / 2);
    }
    CHECK(hipFree(mb));
    CHECK(hipFree(fail));
    CHECK(hipFree(xob));
    return 0;
}
