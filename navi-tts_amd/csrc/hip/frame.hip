// The per-frame token loop on gfx950: talker decode step at n_past -> codebook-0
// sampling -> 16-position code-predictor pass with 15 sampled codebooks ->
// next step embedding, in one persistent launch.
//
// Replaces k_frame and its phases (model/qwen3tts/frame.hip:85-579) and the
// host side of Frame (frame.hip:590-810). MI355X design:
//
//  * Grid: one 256-thread block (4 wave64s, one per SIMD, so each wave may use
//    the full 512 VGPR+AGPR budget) per CU, 256 blocks. Every matrix
//    is partitioned into fixed per-block row slices (q/k/v 16 rows, o 4, gate+up
//    12+12, down 4, talker head 12, cp lm_head 8) so each block streams the same
//    slice of every layer, and the slice of the NEXT layer for a phase is loaded
//    into registers as soon as the current one has been consumed.
//  * No grid barriers. Every activation vector is published as 64-bit tagged
//    words {f32, u32 epoch} with device-scope relaxed stores; each consumer
//    polls exactly the words it needs. A hop costs one store and one load
//    instead of a barrier's fence + atomic + poll + data load.
//  * Sampling (greedy argmax or exact top-k + PCG32 draw) runs redundantly in
//    every block on identical inputs, so the sampled code never costs a hop.
//  * Code-predictor positions 0 and 1 run as one 2-row pass (15 weight passes
//    instead of 16); each attention block keeps its kv head's cp K/V in LDS.
//  * Every wait has a spin cap; the first block to exceed it stamps the
//    launch's epoch into the abort word and every other wait gives up, so a
//    frame fails with "timed out" instead of hanging (frame.hip:78-99 contract).
#include "dev_common.h"
#include "host_util.h"
#include "sampler.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace navi_amd {
namespace fk {

constexpr int NB = 256, BT = 256, NW = BT / WAVE;   // one block per CU, one wave per SIMD
constexpr int H = 1024, NH = 16, NKV = 8, HD = 128, FF = 3072, VT = 3072, VC = 2048;
constexpr int QD = NH * HD, KVD = NKV * HD, QKV = QD + 2 * KVD;
constexpr int NCB = 16, CPH = NCB - 1, GRP = NH / NKV;
constexpr int MAX_TL = 32, MAX_CL = 5;
constexpr int MAX_POS = 4096;          // talker KV positions a frame may attend over
constexpr int MAX_RUN = 4096;          // frames per navi_frame_run_many call
constexpr int KCH = 256;               // talker K/V rows staged in LDS per chunk
constexpr float ATT_SCALE = 0.08838834764831845f;   // 1/sqrt(128)

static_assert(QKV / NB == 4 * NW, "q/k/v: 4 rows per wave");
static_assert(H / NB == NW, "o/down: 1 row per wave");
static_assert(2 * FF / NB == 6 * NW, "gate+up: 6 rows per wave");
static_assert(VT / NB == 3 * NW, "talker head: 3 rows per wave");
static_assert(VC / NB == 2 * NW, "cp head: 2 rows per wave");

// mailbox layout, in 64-bit words
constexpr int MB_X = 0, MB_QKV = MB_X + 2 * H, MB_ATT = MB_QKV + 2 * QKV, MB_X2 = MB_ATT + 2 * QD,
              MB_H = MB_X2 + 2 * H, MB_LG = MB_H + 2 * FF, MB_WORDS = MB_LG + VT;
// Every vector that all 256 blocks gather (att, x2, h, x, logits) is published in NREP copies,
// MB_WORDS apart, and each block reads the copy of its XCD: the 32 CUs of an XCD then share one
// copy's lines instead of all 256 CUs hammering the same few memory channels (all-to-all hop
// of 1024 words on MI355X: 2.5 us with one copy, 1.6 us with one per XCD). q/k/v, read by the
// 16 attention blocks only, stays in copy 0.
constexpr int NREP = 8;
// Talker attention partials: NR key ranges per head, one AP_W-word chunk each ({o[128], max, sum,
// padding}), single copy after the replicated mailboxes.
constexpr int NR = NB / NH, AP_W = 144, MB_AP = NREP * MB_WORDS, MB_TOTAL = MB_AP + NH * NR * AP_W;
static_assert(NR * AP_W % BT == 0 && AP_W > HD + 1, "partial chunk layout");

// This wave's XCD (HW_REG_XCC_ID, a scalar register read): the mailbox copy it gathers from.
__device__ __forceinline__ int xcc_copy() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & (NREP - 1); }
constexpr uint32_t EPOCH_STRIDE = 4096;   // > tags used by one launch

struct LayerPtrs {
    const uint16_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float *ln1, *ln2, *qn, *kn;
};

struct Weights {
    LayerPtrs tl[MAX_TL];
    LayerPtrs cp[MAX_CL];
    const float *tl_norm, *cp_norm;
    const uint16_t *codec_head, *codec_emb;
    const uint16_t *cp_emb[CPH], *lm_head[CPH];
    float invf_t[HD / 2], invf_c[HD / 2];
    float eps_t, eps_c;
};

struct Args {
    uint64_t *mb;
    uint32_t *abort_word;
    int32_t *codes_out;
    int n_tl, n_cl, n_past, skip_talker;
    const float *hidden_in, *logits_in, *step_in, *trailing;
    float *step_out;
    uint8_t *seen;
    float temperature, rep_penalty, cp_temperature, eps_t, eps_c;
    int top_k, cp_top_k, min_frames, frame_index, eos_id, suppress_from;
    uint64_t talker_seed, cp_seed, spin_cap;
    uint32_t epoch;
    float *tap_hidden, *tap_logits, *tap_cp_logits;
    uint64_t *prof;       // per block [PROF_SLOTS] s_memrealtime stamps (null: off)
    uint32_t *stop;       // frame loop: nonzero = an earlier frame of the loop ended it (null: single frame)
};

// This block's slice of one layer (and of the heads), 160 registers per lane:
// with one wave per SIMD the unified VGPR/AGPR file holds it without scratch.
struct Regs {
    uint4 qkv[4][2];   // [row][512-col chunk]
    uint4 o[4];
    uint4 gu[6][2];
    uint4 dn[6];
    uint4 th[3][2];    // talker head rows
    uint4 lm[2][2];    // cp lm head rows
    float ln1[H / BT];   // next input RMSNorm weights of this thread's elements
    float ln2[H / BT];   // next post-attention RMSNorm weights
    float qkw;           // q_norm (waves 0-1) or k_norm (waves 2-3) weight of dim tid % 128
    float fn[H / BT];    // final RMSNorm weights (talker norm, then the cp norm)
};

struct Smem {
    float x[2][H];                  // residual stream rows
    float xn[2][H];                 // normed rows
    union {
        struct {                    // talker attention: one chunk of cached K/V rows, f16,
            uint16_t k[KCH][HD];    // 16-byte chunk c of row j stored at slot c ^ (j & 15)
            uint16_t v[KCH][HD];
        } tkv;
        struct {
            union {
                float big[2 * FF];  // att [T][QD] | h [T][FF]
                struct { float lg[VT]; alignas(16) int idx[VT]; } samp;   // idx: the sampler's counters
            };
            // this block's cp K/V (kv head att_head() / 2), whole frame, zero until written; K rows
            // keep 16-byte chunk c at slot c ^ (row & 15)
            uint16_t ckv[2][MAX_CL][NCB][HD];
            float rope[2][NCB][HD / 2];      // cp RoPE cos / sin of positions 0..15, dim pairs
        } m;
    } u;
    float invf[2][HD / 2];          // RoPE inverse frequencies (talker, cp)
    float trope[2][HD / 2];         // talker RoPE cos / sin at this frame's position
    LayerPtrs lp[MAX_TL + MAX_CL];  // weight pointers, copied once: a scalar load of the table in
    const uint16_t *emb[CPH];       // global memory misses the scalar cache under the weight stream
    const uint16_t *lmh[CPH];
    float red[4 * NW];
    float q[2][HD], k[2][HD], v[2][HD];
    float qw[NW][HD];               // talker attention: each wave's copy of the rotated q
    float nw[2 * HD];               // attention: q_norm (0..127) and k_norm (128..255) weights
    float sc[KCH];                  // attention weights of one key chunk (cp: [T][NCB])
    float opart[NW][HD];
    unsigned hist[256];
    int isel[4];
    float sred[2 * NW];             // sampling: per-wave maxima / sums
    int sidx[NW];                   // sampling: per-wave argmax
    int codes[NCB];
    int fail;
    int prof_i;
};

constexpr int PROF_SLOTS = 4096;
// Profiling (reference: NAVI_FRAME_PROFILE, frame.hip:71-73/522-529): when enabled, thread 0
// of every block stamps the 100 MHz real-time counter at each wait's start and end.
#define PROF_MARK(a, S)                                                                         \
    do {                                                                                        \
        if ((a).prof && threadIdx.x == 0 && (S).prof_i < PROF_SLOTS)                            \
            gst((a).prof + static_cast<size_t>(blockIdx.x) * PROF_SLOTS + (S).prof_i++, static_cast<uint64_t>(wall_clock64())); \
    } while (0)

// The weight table and the per-layer KV pointers are separate `const __restrict__` kernel
// arguments so their loads are scalar (s_load, counted by lgkmcnt): a vector load here would
// wait behind every in-flight weight prefetch (vmcnt retires in order).
struct Ctx {
    const Weights *__restrict__ W;
    uint16_t *const *__restrict__ kv;    // [0, MAX_TL): K per layer, [MAX_TL, 2 MAX_TL): V
};

__device__ __forceinline__ int tid() { return static_cast<int>(threadIdx.x); }
__device__ __forceinline__ int lane() { return static_cast<int>(threadIdx.x) & (WAVE - 1); }
__device__ __forceinline__ int wave() { return static_cast<int>(threadIdx.x) / WAVE; }
__device__ __forceinline__ int blk() { return static_cast<int>(blockIdx.x); }

// Blocks are dispatched to the XCDs round-robin (block b on XCD b % 8), and kv group g's q|k|v
// rows and its attention are kept on XCD g, so the q|k|v -> attention hop stays inside one L2:
// the 32 blocks of XCD g (j = b / 8) compute q heads 2g and 2g + 1 (j < 16), k of group g
// (16 <= j < 24) and v of group g (j >= 24), 16 rows each; q head h's attention blocks are the
// blocks b with b % 8 == h / 2 and (b / 8) % 2 == h % 2.
__device__ __forceinline__ int qkv_row0() {
    const int x = blk() % NKV, j = blk() / NKV;
    return j < 16 ? 2 * HD * x + 16 * j : j < 24 ? QD + HD * x + 16 * (j - 16) : QD + KVD + HD * x + 16 * (j - 24);
}
__device__ __forceinline__ int att_head() { return 2 * (blk() % NKV) + ((blk() / NKV) & 1); }

// ---- block reductions (fixed order: every block gets bit-identical results) ----

__device__ __forceinline__ float block_sum(float v, Smem &S) {
    v = wave_sum(v);
    if (lane() == 0) S.red[wave()] = v;
    __syncthreads();
    float r = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) r += S.red[w];
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_max(float v, Smem &S) {
    v = wave_max(v);
    if (lane() == 0) S.red[wave()] = v;
    __syncthreads();
    float r = S.red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = fmaxf(r, S.red[w]);
    __syncthreads();
    return r;
}

// ---- waits ----------------------------------------------------------------

__device__ __forceinline__ bool aborted(const Args &a) { return ctl_peek(a.abort_word) == a.epoch; }

// The first wait over its spin cap: every other wait of this launch gives up, and a frame loop
// runs no further frame.
__device__ __forceinline__ void abort_frame(const Args &a) {
    ctl_put(a.abort_word, a.epoch);
    if (a.stop) ctl_put(a.stop, 2u);
}

// Polls one word until it carries `tag`; false on spin cap or abort.
__device__ __forceinline__ bool poll_word(const Args &a, uint64_t *p, uint32_t tag, uint64_t &w) {
    uint64_t spins = 0;
    while (tag_of(w) != tag) {
        if (++spins >= a.spin_cap || ((spins & 63u) == 0 && aborted(a))) {
            abort_frame(a);
            return false;
        }
        w = mb_peek(p);
    }
    return true;
}

// RMSNorm weights of this thread's elements (tid + k * BT), by value so they stay in registers.
struct NormW {
    float v[H / BT];
};
__device__ __forceinline__ NormW normw(const float (&w)[H / BT]) {
    NormW n;
#pragma unroll
    for (int k = 0; k < H / BT; ++k) n.v[k] = w[k];
    return n;
}

// How a gather waits for its vector: every thread issues the loads of all its words at once and,
// round by round, re-issues only those whose tag is not yet this phase's, so the vector is in LDS
// one coherent round trip after the last producer's store becomes visible. The alternative, wave 0
// polling one sentinel word per producer and then every thread reading the vector (a second round
// trip, but 1/CH of the polling traffic while the producers still compute), measured on MI355X at
// n_past 256: sentinels everywhere 1.775 ms; words for the residual, MLP, talker-logit and
// attention-partial gathers 1.612 ms; once every first poll waited a pause (below), words for the
// attention output and the code-predictor logits too: 1.462 -> 1.438 ms.

// A pause before a gather's first poll, in s_sleep units of 64 clocks, per gather site. Polls that
// go out while the producers are still computing only add coherent traffic to the mailbox lines
// the producers' stores are headed for, and slow those stores down. A frame at n_past 256 on
// MI355X: no pause 1.614 ms; 16 before the residual, MLP, talker-logit and attention-partial
// gathers 1.564; the values below 1.534 (32 before the residual gathers: 1.558); with the late
// q|k|v prefetch of the attention blocks (run_layer) the attention output's pause went from 24
// to 12 (1.509 -> 1.487 ms; 32: 1.532).
constexpr int D_X2 = 24;    // x2 (after o; its prefetch is 16 KB per CU)
constexpr int D_H = 16;     // MLP activation (after gate|up and its 48 KB prefetch)
constexpr int D_X = 24;     // x (after down)
constexpr int D_ATT = 12;   // attention output (every block; the 16 attention blocks publish it)
constexpr int D_AP = 24;    // talker attention partials (the combining blocks)
constexpr int D_TLG = 32;   // talker logits
constexpr int D_CLG = 32;   // code-predictor logits
constexpr int D_QKV = 8;    // q/k/v at the attention blocks

template <int D>
__device__ __forceinline__ void pause() {
    if constexpr (D > 0) __builtin_amdgcn_s_sleep(D);
}

// Block-wide: N tagged words at mailbox offset `off` -> dst (LDS f32). Uniform result.
// With NORM (N == H) the same pass does norm_prep's work: xn[i] = x[i] * w[i] and this wave's
// sum of x^2 in S.red[red + wave] (same order, so the same bits), published by the final barrier.
template <int N, bool REPL = true, bool NORM = false, int D = 0>
__device__ __forceinline__ bool gather(const Args &a, int off, uint32_t tag, float *dst, Smem &S, NormW nw = {},
                                       float *xn = nullptr, int red = 0) {
    static_assert(N % BT == 0, "gather size");
    static_assert(!NORM || N == H, "norm of the residual stream");
    constexpr int PER = N / BT;
    uint64_t *const mb = sgpr_ptr(a.mb + (REPL ? xcc_copy() * MB_WORDS : 0) + off);
    PROF_MARK(a, S);
    uint64_t w[PER];
    pause<D>();
#pragma unroll
    for (int k = 0; k < PER; ++k) w[k] = mb_peek(mb + tid() + k * BT);
    uint64_t spins = 0;
    bool ok = true;
    for (;;) {                                 // per thread: the wave runs until every lane is done
        bool done = true;
#pragma unroll
        for (int k = 0; k < PER; ++k) done &= tag_of(w[k]) == tag;
        if (done) break;
        if (++spins >= a.spin_cap || ((spins & 63u) == 0 && aborted(a))) {
            abort_frame(a);
            ok = false;
            break;
        }
#pragma unroll
        for (int k = 0; k < PER; ++k)
            if (tag_of(w[k]) != tag) w[k] = mb_peek(mb + tid() + k * BT);
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = tid() + k * BT;
        const float v = val_of(w[k]);
        dst[i] = v;
        if constexpr (NORM) {
            ss = fmaf(v, v, ss);
            xn[i] = v * nw.v[k];
        }
    }
    if constexpr (NORM) {
        ss = wave_sum(ss);
        if (lane() == 0) S.red[red + wave()] = ss;
    }
    if (!ok) S.fail = 1;
    __syncthreads();
    PROF_MARK(a, S);
    return S.fail == 0;
}

// Two rows of N words (row stride N in the mailbox and in dst) in one wait: both rows' words
// of a thread in flight at once, so the second row costs no round trip of its own. Per row the
// same values, order and norm partial sums (S.red[t * NW + wave]) as gather<>.
template <int N, bool NORM, int D>
__device__ __forceinline__ bool gather_two_rows(const Args &a, int off, uint32_t tag, float *dst, Smem &S, NormW nw,
                                                float *xn) {
    static_assert(N % BT == 0, "gather size");
    constexpr int PER = N / BT;
    uint64_t *const mb = sgpr_ptr(a.mb + xcc_copy() * MB_WORDS + off);
    PROF_MARK(a, S);
    uint64_t w[2][PER];
    pause<D>();
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int k = 0; k < PER; ++k) w[t][k] = mb_peek(mb + t * N + tid() + k * BT);
    uint64_t spins = 0;
    bool ok = true;
    for (;;) {
        bool done = true;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int k = 0; k < PER; ++k) done &= tag_of(w[t][k]) == tag;
        if (done) break;
        if (++spins >= a.spin_cap || ((spins & 63u) == 0 && aborted(a))) {
            abort_frame(a);
            ok = false;
            break;
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int k = 0; k < PER; ++k)
                if (tag_of(w[t][k]) != tag) w[t][k] = mb_peek(mb + t * N + tid() + k * BT);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = t * N + tid() + k * BT;
            const float v = val_of(w[t][k]);
            dst[i] = v;
            if constexpr (NORM) {
                ss = fmaf(v, v, ss);
                xn[i] = v * nw.v[k];
            }
        }
        if constexpr (NORM) {
            ss = wave_sum(ss);
            if (lane() == 0) S.red[t * NW + wave()] = ss;
        }
    }
    if (!ok) S.fail = 1;
    __syncthreads();
    PROF_MARK(a, S);
    return S.fail == 0;
}

// T rows of N words each (row stride N in the mailbox and in dst), two rows in one wait.
template <int T, int N, bool NORM = false, int D = 0>
__device__ __forceinline__ bool gather_rows(const Args &a, int off, uint32_t tag, float *dst, Smem &S, NormW nw = {},
                                            float *xn = nullptr) {
    static_assert(T == 1 || T == 2, "one or two rows");
    if constexpr (T == 2) return gather_two_rows<N, NORM, D>(a, off, tag, dst, S, nw, xn);
    else return gather<N, true, NORM, D>(a, off, tag, dst, S, nw, NORM ? xn : nullptr, 0);
}

// ---- RMSNorm of T rows (every block, redundantly) ---------------------------

// RMSNorm, split (every block, redundantly): out[t] = x[t] * w elementwise and this wave's partial
// sum of x[t]^2 in S.red, published by one barrier; the scalar rsqrt(mean(x^2) + eps) (norm_scale)
// multiplies the matvec results instead of every element (block_rmsnorm, frame.hip:107-114).
template <int T>
__device__ __forceinline__ void norm_prep(const float (*x)[H], const float (&w)[H / BT], float (*out)[H], Smem &S) {
    constexpr int PER = H / BT;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const float e = x[t][tid() + k * BT];
            ss = fmaf(e, e, ss);
            out[t][tid() + k * BT] = e * w[k];
        }
        ss = wave_sum(ss);
        if (lane() == 0) S.red[t * NW + wave()] = ss;
    }
    __syncthreads();
}

__device__ __forceinline__ float norm_scale_row(float eps, int row, const Smem &S) {
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) ss += S.red[row * NW + w];
    return rsqrtf(ss / static_cast<float>(H) + eps);
}

template <int T>
__device__ __forceinline__ void norm_scale(float eps, float (&sc)[T], const Smem &S) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float ss = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) ss += S.red[t * NW + w];
        sc[t] = rsqrtf(ss / static_cast<float>(H) + eps);
    }
}

// This thread's RMSNorm weights (elements tid + k * BT).
__device__ __forceinline__ void load_norm(float (&w)[H / BT], const float *g) {
#pragma unroll
    for (int k = 0; k < H / BT; ++k) w[k] = gld(g + tid() + k * BT);
}

// x fragment a lane multiplies with 512-col chunks: cols base + c*512 + lane*8 .. +8
template <int NC>
__device__ __forceinline__ void xfrag(const float *x, int base, float (&xf)[NC][8]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const f32x4_t p = *reinterpret_cast<const f32x4_t *>(x + base + c * 512 + lane() * 8);
        const f32x4_t q = *reinterpret_cast<const f32x4_t *>(x + base + c * 512 + lane() * 8 + 4);
        xf[c][0] = p.x; xf[c][1] = p.y; xf[c][2] = p.z; xf[c][3] = p.w;
        xf[c][4] = q.x; xf[c][5] = q.y; xf[c][6] = q.z; xf[c][7] = q.w;
    }
}

// ---- weight prefetch: this block's slice of one layer -----------------------
// Talker weights are read once per frame and stream past with the non-temporal hint. The code
// predictor's 5 layers and heads (220 MB) are read 15 times per frame: plain loads let the
// memory-side cache serve the repeats (60 us per frame less at n_past 256 than streaming them).
__device__ __forceinline__ uint4 ldw(const uint16_t *p, bool reuse) { return reuse ? ldg16(p) : ldg16_stream(p); }

__device__ __forceinline__ void load_qkv(Regs &R, const LayerPtrs &L, bool reuse) {
    const int rb = qkv_row0();
    const uint16_t *M;
    int base;
    if (rb < QD) { M = L.wq; base = rb; }
    else if (rb < QD + KVD) { M = L.wk; base = rb - QD; }
    else { M = L.wv; base = rb - QD - KVD; }
    M = sgpr_ptr(M + static_cast<size_t>(base) * H);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint16_t *p = M + static_cast<size_t>(wave() * 4 + r) * H + lane() * 8;
        R.qkv[r][0] = ldw(p, reuse);
        R.qkv[r][1] = ldw(p + 512, reuse);
    }
    load_norm(R.ln1, L.ln1);
    R.qkw = gld((wave() < 2 ? L.qn : L.kn) + (tid() & (HD - 1)));
}

__device__ __forceinline__ void load_o(Regs &R, const LayerPtrs &L, bool reuse) {
    const uint16_t *p = sgpr_ptr(L.wo + static_cast<size_t>(blk() * (H / NB)) * QD) + static_cast<size_t>(wave()) * QD + lane() * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c) R.o[c] = ldw(p + c * 512, reuse);
}

__device__ __forceinline__ void load_gu(Regs &R, const LayerPtrs &L, bool reuse) {
    constexpr int RB = FF / NB;   // 12 gate + 12 up rows per block
#pragma unroll
    for (int r = 0; r < 6; ++r) {
        const int vr = wave() * 3 + (r % 3);               // r < 3: gate row vr, r >= 3: up row vr
        const uint16_t *M = sgpr_ptr((r < 3 ? L.wg : L.wu) + static_cast<size_t>(blk() * RB) * H);
        const uint16_t *p = M + static_cast<size_t>(vr) * H + lane() * 8;
        R.gu[r][0] = ldw(p, reuse);
        R.gu[r][1] = ldw(p + 512, reuse);
    }
    load_norm(R.ln2, L.ln2);
}

__device__ __forceinline__ void load_dn(Regs &R, const LayerPtrs &L, bool reuse) {
    const uint16_t *p = sgpr_ptr(L.wd + static_cast<size_t>(blk() * (H / NB)) * FF) + static_cast<size_t>(wave()) * FF + lane() * 8;
#pragma unroll
    for (int c = 0; c < 6; ++c) R.dn[c] = ldw(p + c * 512, reuse);
}

__device__ __forceinline__ void load_th(Regs &R, const uint16_t *head) {
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        const uint16_t *p = head + static_cast<size_t>(blk() * (VT / NB) + wave() * 3 + r) * H + lane() * 8;
        R.th[r][0] = ldg16_stream(p);
        R.th[r][1] = ldg16_stream(p + 512);
    }
}

__device__ __forceinline__ void load_lm(Regs &R, const uint16_t *head) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint16_t *p = head + static_cast<size_t>(blk() * (VC / NB) + wave() * 2 + r) * H + lane() * 8;
        R.lm[r][0] = ldg16(p);
        R.lm[r][1] = ldg16(p + 512);
    }
}

// ---- matvec phases --------------------------------------------------------

template <int T>
__device__ __forceinline__ void qkv_phase(const Args &a, const Regs &R, Smem &S, uint32_t tag, const float (&sc)[T]) {
    const int row0 = qkv_row0() + wave() * 4;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float xf[2][8], d[4];
        xfrag<2>(S.xn[t], 0, xf);
        dot16_rows<4>(R.qkv, xf, d);
        wave_sum_n<4>(d);
        const int L = lane();
        if (L < 4) mb_put(a.mb + MB_QKV + t * QKV + row0 + L, (L == 0 ? d[0] : L == 1 ? d[1] : L == 2 ? d[2] : d[3]) * sc[t], tag);
    }
}

// x2[row] = x[row] + Wo . att  (att gathered into S.u.m.big as [T][QD])
template <int T>
__device__ __forceinline__ void o_phase(const Args &a, const Regs &R, Smem &S, uint32_t tag) {
    const int row = blk() * (H / NB) + wave();
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float acc = 0.f;
#pragma unroll
        for (int c2 = 0; c2 < 4; c2 += 2) {
            float xf[2][8];
            xfrag<2>(S.u.m.big + t * QD, c2 * 512, xf);
            acc = dot8(R.o[c2 + 1], xf[1], dot8(R.o[c2], xf[0], acc));
        }
        const float d = wave_sum(acc);
        if (lane() < NREP) mb_put(a.mb + lane() * MB_WORDS + MB_X2 + t * H + row, S.x[t][row] + d, tag);
    }
}

// h[row] = silu(Wg . xn) * (Wu . xn)
template <int T>
__device__ __forceinline__ void gu_phase(const Args &a, const Regs &R, Smem &S, uint32_t tag, const float (&sc)[T]) {
    constexpr int RB = FF / NB;   // wave w holds gate rows 3w..3w+2 (r < 3) and the matching up rows (r >= 3)
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float xf[2][8];
        xfrag<2>(S.xn[t], 0, xf);
        float d[6];
        dot16_rows<6>(R.gu, xf, d);
        wave_sum_n<6>(d);
#pragma unroll
        for (int r = 0; r < 6; ++r) d[r] *= sc[t];
        // lane 8r + c publishes h row 3w + r to copy c
        const int r = lane() >> 3, c = lane() & 7;
        if (r < 3) {
            const float g = r == 0 ? d[0] : r == 1 ? d[1] : d[2];
            const float u = r == 0 ? d[3] : r == 1 ? d[4] : d[5];
            mb_put(a.mb + c * MB_WORDS + MB_H + t * FF + blk() * RB + wave() * 3 + r, g / (1.f + expf(-g)) * u, tag);
        }
    }
}

// x[row] = x2[row] + Wd . h  (x2 in S.x, h gathered into S.u.m.big as [T][FF])
template <int T>
__device__ __forceinline__ void down_phase(const Args &a, const Regs &R, Smem &S, uint32_t tag) {
    const int row = blk() * (H / NB) + wave();
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float acc = 0.f;
#pragma unroll
        for (int c2 = 0; c2 < 6; c2 += 2) {
            float xf[2][8];
            xfrag<2>(S.u.m.big + t * FF, c2 * 512, xf);
            acc = dot8(R.dn[c2 + 1], xf[1], dot8(R.dn[c2], xf[0], acc));
        }
        const float d = wave_sum(acc);
        if (lane() < NREP) mb_put(a.mb + lane() * MB_WORDS + MB_X + t * H + row, S.x[t][row] + d, tag);
    }
}

// ---- attention --------------------------------------------------------------

// RMSNorm of one 128-dim head row with weights nw, lane l's elements (l, l + 64) into (x0, x1).
__device__ __forceinline__ void head_norm_pair(const float *row, const float *nw, float eps, float &x0, float &x1) {
    const int l = lane();
    const float a0 = row[l], a1 = row[l + HD / 2];
    const float sc = rsqrtf(wave_sum(fmaf(a0, a0, a1 * a1)) / static_cast<float>(HD) + eps);
    x0 = a0 * sc * nw[l];
    x1 = a1 * sc * nw[l + HD / 2];
}

__device__ __forceinline__ void rope_pair(float *v, int i, float c, float s) {
    const float x0 = v[i], x1 = v[i + HD / 2];
    v[i] = x0 * c - x1 * s;
    v[i + HD / 2] = x0 * s + x1 * c;
}

// Waits for q head h and kv head g of T rows: S.q/S.k/S.v[t].
template <int T>
__device__ __forceinline__ bool gather_head(const Args &a, int h, int g, uint32_t tag, Smem &S) {
    constexpr int PER = (T * 3 * HD + BT - 1) / BT;
    int off[PER];
    uint64_t w[PER];
    pause<D_QKV>();
#pragma unroll
    for (int k = 0; k < PER; ++k) {                   // all of this thread's words in flight at once
        const int i = tid() + k * BT;
        const int t = i / (3 * HD), seg = (i % (3 * HD)) / HD, d = i % HD;
        off[k] = MB_QKV + t * QKV + (seg == 0 ? h * HD : seg == 1 ? QD + g * HD : QD + KVD + g * HD) + d;
        if (i < T * 3 * HD) w[k] = mb_peek(a.mb + off[k]);
    }
    bool ok = true;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = tid() + k * BT;
        if (i >= T * 3 * HD) continue;
        if (ok) ok = poll_word(a, a.mb + off[k], tag, w[k]);
        const int t = i / (3 * HD), seg = (i % (3 * HD)) / HD, d = i % HD;
        (seg == 0 ? S.q[t] : seg == 1 ? S.k[t] : S.v[t])[d] = val_of(w[k]);
    }
    if (!ok) S.fail = 1;
    __syncthreads();
    return S.fail == 0;
}

typedef __attribute__((address_space(1))) void gmem_t;
typedef __attribute__((address_space(3))) void lmem_t;

__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// LDS-DMA (global_load_lds_dwordx4) of cached K and V rows [j0, j0 + n), n <= KCH, of one kv head
// into S.u.tkv. A wave instruction moves 1 KB = 4 rows; lane l fills LDS slot l % 16 of row l / 16
// with the row's 16-byte chunk (l % 16) ^ (row & 15). No VGPRs; completion is the wave's vmcnt.
__device__ __forceinline__ void stage_kv(const uint16_t *Kc, const uint16_t *Vc, int j0, int n, Smem &S) {
    const int nblk = (n + 3) / 4;
    for (int bi = wave(); bi < 2 * nblk; bi += NW) {
        const bool isv = bi >= nblk;
        const int r4 = (isv ? bi - nblk : bi) * 4, jj = r4 + (lane() >> 4), c = (lane() & 15) ^ (jj & 15);
        const int jsrc = j0 + min(jj, n - 1);
        const uint16_t *src = (isv ? Vc : Kc) + static_cast<size_t>(jsrc) * KVD + c * 8;
        uint16_t *dst = isv ? &S.u.tkv.v[r4][0] : &S.u.tkv.k[r4][0];
        __builtin_amdgcn_global_load_lds((gmem_t *) src, (lmem_t *) dst, 16, 0, 0);
    }
}

// Talker attention, spread over all 256 blocks: block b takes q head h = att_head() and range
// r = b / NH of the cached keys (NR ranges of ceil(pos / NR) keys; the current key at pos goes
// to the last range, whose even-head block also writes the new f16 K/V row). A block stages its
// range's K/V rows in LDS by DMA while this step's q/k/v are in flight, normalises and rotates
// q (and the current k), runs a per-wave online softmax over its keys and publishes the range's
// partial (max, sum, unnormalised V sum) as one AP_W-word chunk. The range-0 block of head h
// gathers the NR partials of head h, combines them in range order and publishes the head's
// output. Every range of head h sits on XCD h / 2 with the blocks that produce its q|k|v, so
// both the q|k|v hop and the partial hop stay within one L2.
__device__ bool talker_attention(const Args &a, const Ctx &cx, float qkw, int il, uint32_t tag_qkv, uint32_t tag_ap,
                                 uint32_t tag_att, Smem &S) {
    const int h = att_head(), r = blk() / NH, g = h / GRP, pos = a.n_past;
    const int R = (pos + NR - 1) / NR, j0 = min(pos, r * R), n = max(0, min(pos, j0 + R) - j0);   // n <= KCH
    const bool last = r == NR - 1;
    uint16_t *const Kbase = cx.kv[il], *const Vbase = cx.kv[MAX_TL + il];
    const uint16_t *Kc = Kbase + g * HD;
    uint16_t *Vc = Vbase + g * HD;
    if (n > 0) stage_kv(Kc, Vc, j0, n, S);
    PROF_MARK(a, S);
    S.nw[tid()] = qkw;                                     // published by gather_head's barrier
    if (!gather_head<1>(a, h, g, tag_qkv, S)) return false;
    PROF_MARK(a, S);
    // Every wave, redundantly (no barrier): head RMSNorm and RoPE of q (and, in the last range, of
    // the current k) with the pair (l, l + 64) in lane l, q copied to the wave's own LDS row for
    // the score loop, the current key's score and value in registers.
    const int L = lane(), w = wave();
    const float cs = S.trope[0][L], sn = S.trope[1][L];
    float qa, qb;
    head_norm_pair(S.q[0], S.nw, a.eps_t, qa, qb);
    S.qw[w][L] = qa * cs - qb * sn;
    S.qw[w][L + HD / 2] = qa * sn + qb * cs;
    float s_cur = -INFINITY, vc0 = 0.f, vc1 = 0.f;
    if (last) {
        float ka, kb;
        head_norm_pair(S.k[0], S.nw + HD, a.eps_t, ka, kb);
        const float kra = round_f16(ka * cs - kb * sn), krb = round_f16(ka * sn + kb * cs);
        s_cur = wave_sum(fmaf(S.qw[w][L], kra, S.qw[w][L + HD / 2] * krb)) * ATT_SCALE;
        vc0 = round_f16(S.v[0][2 * L]);
        vc1 = round_f16(S.v[0][2 * L + 1]);
        if (w == 0 && (h & 1) == 0) {
            uint16_t *kw = Kbase + static_cast<size_t>(pos) * KVD + g * HD;
            gst(kw + L, f2h(kra));
            gst(kw + L + HD / 2, f2h(krb));
            uint16_t *vw = Vc + static_cast<size_t>(pos) * KVD;
            gst(vw + 2 * L, f2h(vc0));
            gst(vw + 2 * L + 1, f2h(vc1));
        }
    }
    wait_vm_all();
    __syncthreads();                                       // every wave's part of the range has landed
    PROF_MARK(a, S);
    // Scores of the range's keys, every wave: lanes 16q..16q+15 take key j = base + q (base =
    // 4w + 16i), lane 16q + c multiplying the key's 16-byte chunk c with q[8c .. 8c+7]; the 16
    // lanes sum by DPP within their row and lane 16q keeps the score in S.sc[j].
    {
        const int q4 = L >> 4, c = L & 15;
        float qf[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[e] = S.qw[w][c * 8 + e];
        for (int base = 4 * w; base < n; base += 4 * NW) {   // base <= 252: rows base + q4 < KCH
            const int j = base + q4;
            const u32x4_t kv4 = *reinterpret_cast<const u32x4_t *>(&S.u.tkv.k[j][(c ^ (j & 15)) * 8]);
            uint4 kk;
            __builtin_memcpy(&kk, &kv4, 16);
            float acc = dot8(kk, qf, 0.f);
            acc += dpp_red<0xB1>(acc);
            acc += dpp_red<0x4E>(acc);
            acc += dpp_red<0x141>(acc);
            acc += dpp_red<0x140>(acc);
            if (c == 0 && j < n) S.sc[j] = acc * ATT_SCALE;
        }
    }
    __syncthreads();
    // Per-wave softmax over the wave's keys (wave w: rows w*per .. w*per + per - 1, per =
    // ceil(n / 4) <= 64, lane-per-key); wave 0 of the last range also takes the current key. Lane L
    // owns value dims 2L, 2L + 1.
    float mw = -INFINITY, lw = 0.f, acc0 = 0.f, acc1 = 0.f;
    const int slot8 = 2 * (L & 3);
    {
        const int per = (n + NW - 1) / NW;
        const int jw = w * per, cnt = max(0, min(per, n - jw));
        const float sj = L < cnt ? S.sc[jw + L] : -INFINITY;
        const bool cur = last && w == 0;
        float mn = wave_max(sj);
        if (cur) mn = fmaxf(mn, s_cur);
        if (mn != -INFINITY) {
            const float e = L < cnt ? expf(sj - mn) : 0.f;
            const float ec = cur ? expf(s_cur - mn) : 0.f;
            lw = wave_sum(e) + ec;
            mw = mn;
            // V sum in groups of 8 keys: the 8 LDS reads are issued before the first FMA (rows
            // past cnt repeat the last row with weight 0), and 2 independent accumulator pairs
            // halve the FMA chains (key j's weight: lane j's e)
            float b0[2] = {ec * vc0, 0.f}, b1[2] = {ec * vc1, 0.f};
            for (int j = 0; j < cnt; j += 8) {
                half2_t hv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int jj = jw + min(j + u, cnt - 1);
                    __builtin_memcpy(&hv[u], &S.u.tkv.v[jj][((L >> 2) ^ (jj & 15)) * 8 + slot8], 4);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const float p = lane_value(e, j + u);
                    b0[u & 1] = fmaf(p, static_cast<float>(hv[u][0]), b0[u & 1]);
                    b1[u & 1] = fmaf(p, static_cast<float>(hv[u][1]), b1[u & 1]);
                }
            }
            acc0 = b0[0] + b0[1];
            acc1 = b1[0] + b1[1];
        }
    }
    PROF_MARK(a, S);
    // the four waves' (max, sum, accumulator) -> the range's partial, published as one chunk
    if (L == 0) {
        S.red[w] = mw;
        S.red[NW + w] = lw;
    }
    S.opart[w][2 * L] = acc0;
    S.opart[w][2 * L + 1] = acc1;
    __syncthreads();
    {
        float M = S.red[0];
#pragma unroll
        for (int i = 1; i < NW; ++i) M = fmaxf(M, S.red[i]);
        float sc[NW], den = 0.f;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            sc[i] = S.red[i] == -INFINITY ? 0.f : expf(S.red[i] - M);
            den = fmaf(S.red[NW + i], sc[i], den);
        }
        uint64_t *ap = a.mb + MB_AP + (h * NR + r) * AP_W;
        for (int i = tid(); i < AP_W; i += BT) {
            float v = 0.f;
            if (i < HD) {
#pragma unroll
                for (int k = 0; k < NW; ++k) v = fmaf(S.opart[k][i], sc[k], v);
            } else if (i == HD) {
                v = M;
            } else if (i == HD + 1) {
                v = den;
            }
            mb_put(ap + i, v, tag_ap);
        }
    }
    PROF_MARK(a, S);
    if (r != 0) return true;
    // combine head h's NR partials in range order: out = sum_r o_r e^(m_r - M) / sum_r l_r e^(m_r - M)
    float *P = S.u.m.big;
    if (!gather<NR * AP_W, false, false, D_AP>(a, MB_AP + h * NR * AP_W, tag_ap, P, S)) return false;
    {
        // every thread combines dim tid % 128 (the two halves of the block identically) and
        // publishes it to half of the copies; lane k (mod 16) computes partial k's weight once,
        // the weights go round by readlane
        static_assert(NR == 16, "one partial per lane of a 16-lane row");
        const int k = L & (NR - 1), d = tid() & (HD - 1);
        const float mk = P[k * AP_W + HD], lk = P[k * AP_W + HD + 1];
        const float M = wave_max(mk);
        const float wk = mk == -INFINITY ? 0.f : expf(mk - M);
        float pv[NR];
#pragma unroll
        for (int k2 = 0; k2 < NR; ++k2) pv[k2] = P[k2 * AP_W + d];
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int k2 = 0; k2 < NR; ++k2) {
            const float wv = lane_value(wk, k2);
            den = fmaf(lane_value(lk, k2), wv, den);
            num = fmaf(pv[k2], wv, num);
        }
        const float o = num / den;
        const int c0 = (tid() >> 7) * (NREP / 2);
#pragma unroll
        for (int c = 0; c < NREP / 2; ++c) mb_put(a.mb + (c0 + c) * MB_WORDS + MB_ATT + h * HD + d, o, tag_att);
    }
    PROF_MARK(a, S);
    return true;
}

// Code-predictor attention for q head h = att_head() (blocks 0..15) over T rows at positions p0..p0+T-1;
// K/V of this block's kv head live in S.u.m.ckv for the whole frame (rows not yet written are
// zero), RoPE cos/sin in S.u.m.rope (the frame's table of the 16 cp positions).
template <int T>
__device__ bool cp_attention(const Args &a, float qkw, int il, int p0, uint32_t tag_qkv, uint32_t tag_att, Smem &S) {
    const int h = att_head(), g = h / GRP;
    PROF_MARK(a, S);
    S.nw[tid()] = qkw;                                     // published by gather_head's barrier
    if (!gather_head<T>(a, h, g, tag_qkv, S)) return false;
    PROF_MARK(a, S);
    // Wave t computes row t (position p0 + t) alone: head norms and RoPE of q (into the wave's
    // own LDS row) and of the new keys 0..T-1, written with the new values into ckv (every
    // computing wave writes the same values, so each reads back what it wrote itself; later
    // positions' passes read them after many barriers). Scores: lanes 4j..4j+3 take key j, a
    // quarter of the head each (dims 32s..32s+31), summed by two DPP steps. Value sum: lane l
    // owns dims 2l, 2l+1; all 16 rows are read at once (rows >= n are zero, weight 0).
    const int L = lane(), w = wave();
    if (w >= T) return true;
    const int t = w, pos = p0 + t, n = pos + 1;
    {
        const float cs = S.u.m.rope[0][pos][L], sn = S.u.m.rope[1][pos][L];
        float x0, x1;
        head_norm_pair(S.q[t], S.nw, a.eps_c, x0, x1);
        S.qw[w][L] = x0 * cs - x1 * sn;
        S.qw[w][L + HD / 2] = x0 * sn + x1 * cs;
    }
#pragma unroll
    for (int u = 0; u < T; ++u) {
        const int pu = p0 + u;
        const float cs = S.u.m.rope[0][pu][L], sn = S.u.m.rope[1][pu][L];
        float x0, x1;
        head_norm_pair(S.k[u], S.nw + HD, a.eps_c, x0, x1);
        uint16_t *kr = S.u.m.ckv[0][il][pu];
        kr[(((L >> 3) ^ (pu & 15)) << 3) + (L & 7)] = f2h(x0 * cs - x1 * sn);
        kr[((((L + HD / 2) >> 3) ^ (pu & 15)) << 3) + (L & 7)] = f2h(x0 * sn + x1 * cs);
        S.u.m.ckv[1][il][pu][2 * L] = f2h(S.v[u][2 * L]);
        S.u.m.ckv[1][il][pu][2 * L + 1] = f2h(S.v[u][2 * L + 1]);
    }
    const int j = L >> 2, sq = L & 3;
    float sc;
    {
        const uint16_t *kr = S.u.m.ckv[0][il][j];
        const float *qr = &S.qw[w][sq * 32];
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint4 kk;
            __builtin_memcpy(&kk, kr + (((sq * 4 + c) ^ j) << 3), 16);
            acc = dot8(kk, qr + c * 8, acc);
        }
        acc += dpp_mov<0xB1>(acc);       // quad_perm [1,0,3,2]
        acc += dpp_mov<0x4E>(acc);       // quad_perm [2,3,0,1]: the 4 lanes of key j hold its dot
        sc = j < n ? acc * ATT_SCALE : -INFINITY;
    }
    const float m = wave_max(sc);
    const float e = j < n ? expf(sc - m) : 0.f;
    const float inv = 1.f / wave_sum(sq == 0 ? e : 0.f);
    half2_t hv[NCB];
#pragma unroll
    for (int r = 0; r < NCB; ++r) __builtin_memcpy(&hv[r], &S.u.m.ckv[1][il][r][2 * L], 4);
    float o0 = 0.f, o1 = 0.f, q0 = 0.f, q1 = 0.f;
#pragma unroll
    for (int r = 0; r < NCB; r += 2) {
        const float pa = lane_value(e, 4 * r), pb = lane_value(e, 4 * r + 4);
        o0 = fmaf(pa, static_cast<float>(hv[r][0]), o0);
        o1 = fmaf(pa, static_cast<float>(hv[r][1]), o1);
        q0 = fmaf(pb, static_cast<float>(hv[r + 1][0]), q0);
        q1 = fmaf(pb, static_cast<float>(hv[r + 1][1]), q1);
    }
    o0 = (o0 + q0) * inv;
    o1 = (o1 + q1) * inv;
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
        uint64_t *dst = a.mb + r * MB_WORDS + MB_ATT + t * QD + h * HD + 2 * L;
        mb_put(dst, o0, tag_att);
        mb_put(dst + 1, o1, tag_att);
    }
    PROF_MARK(a, S);
    return true;
}

// ---- sampling: block_sample (sampler.h) on this block's LDS ----------------------

__device__ __forceinline__ SampleLds sample_lds(Smem &S) {
    static_assert(VT >= SAMPLE_LDS_WORDS, "sampler counters fit the idx array");
    return SampleLds{S.u.m.samp.lg, reinterpret_cast<unsigned *>(S.u.m.samp.idx), S.sred, S.sidx, &S.isel[2]};
}

// ---- the frame ---------------------------------------------------------------

struct Seq {           // tags: epoch + running phase number, identical in every block
    uint32_t base, n;
    __device__ uint32_t next() { return base + (++n); }
};

__device__ __forceinline__ const LayerPtrs &layer_at(const Args &a, const Smem &S, int gi) {
    return S.lp[gi < a.n_tl ? gi : MAX_TL + (gi - a.n_tl) % a.n_cl];
}

// One decoder layer over T rows held in S.x (its input); leaves its output in S.x.
// gi: global layer index (talker layers, then n_cl cp layers per cp pass).
// normed: S.xn and the norm's partial sums are already there (the previous layer's last gather
// made them). next_final: the output feeds the final norm (R.fn) and a head, not another layer.
template <int T, bool TALKER>
__device__ __forceinline__ bool run_layer(const Args &a, const Ctx &cx, Regs &R, int gi, int p0, Seq &seq, Smem &S,
                                          const uint16_t *head, bool normed, bool next_final) {
    const int n_total = a.n_tl + CPH * a.n_cl;
    const bool has_next = gi + 1 < n_total;
    const LayerPtrs &N = layer_at(a, S, has_next ? gi + 1 : gi);
    const bool next_cp = gi + 1 >= a.n_tl;
    const float eps = TALKER ? a.eps_t : a.eps_c;

    if (!normed) norm_prep<T>(S.x, R.ln1, S.xn, S);
    float sc[T];
    norm_scale<T>(eps, sc, S);
    const uint32_t t_qkv = seq.next();
    qkv_phase<T>(a, R, S, t_qkv, sc);
    const float qkw = R.qkw;     // this layer's q/k norm weight; the prefetch below replaces it
    // The next layer's q|k|v slice. Blocks with attention work of their own (the talker's key-range
    // blocks, the code predictor's attention blocks) issue it once that work is published, so its
    // loads do not sit in front of their q/k/v polls; the talker's combining blocks and the code
    // predictor's other blocks issue it now (1.537 -> 1.518 ms per frame at n_past 256).
    const bool pf_late = TALKER ? blk() >= NH : blk() < NH;
    if (has_next && !pf_late) load_qkv(R, N, next_cp);

    const uint32_t t_ap = TALKER ? seq.next() : 0u;
    const uint32_t t_att = seq.next();
    if constexpr (TALKER) {
        if (!talker_attention(a, cx, qkw, gi, t_qkv, t_ap, t_att, S)) return false;
    } else if (blk() < NH) {
        if (!cp_attention<T>(a, qkw, (gi - a.n_tl) % a.n_cl, p0, t_qkv, t_att, S)) return false;
    }
    if (has_next && pf_late) load_qkv(R, N, next_cp);
    if (!gather_rows<T, QD, false, D_ATT>(a, MB_ATT, t_att, S.u.m.big, S)) return false;
    const uint32_t t_x2 = seq.next();
    o_phase<T>(a, R, S, t_x2);
    if (has_next) load_o(R, N, next_cp);

    if (!gather_rows<T, H, true, D_X2>(a, MB_X2, t_x2, &S.x[0][0], S, normw(R.ln2), &S.xn[0][0])) return false;
    norm_scale<T>(eps, sc, S);
    const uint32_t t_h = seq.next();
    gu_phase<T>(a, R, S, t_h, sc);
    if (has_next) load_gu(R, N, next_cp);

    if (!gather_rows<T, FF, false, D_H>(a, MB_H, t_h, S.u.m.big, S)) return false;
    const uint32_t t_x = seq.next();
    down_phase<T>(a, R, S, t_x);
    if (has_next) load_dn(R, N, next_cp);
    if (head) {                  // the pass's head slice, issued one phase before it is needed
        if constexpr (TALKER) load_th(R, head);
        else load_lm(R, head);
    }

    // R.ln1 holds the next layer's weights by now (load_qkv above); the last layer of the frame
    // is always next_final
    return gather_rows<T, H, true, D_X>(a, MB_X, t_x, &S.x[0][0], S, next_final ? normw(R.fn) : normw(R.ln1),
                                           &S.xn[0][0]);
}

__device__ __forceinline__ void load_row_f16(const uint16_t *src, float *dst) {
    for (int i = tid(); i < H; i += BT) dst[i] = h2f(gld(src + i));
}

__global__ void __launch_bounds__(BT, 1) k_frame(Args a, const Weights *__restrict__ Wp, uint16_t *const *__restrict__ kvp) {
    __shared__ Smem S;
    // frame loop: an earlier frame (a finished launch, so every block reads the same word) sampled
    // EOS or timed out; this frame does not run
    if (a.stop && ctl_peek(a.stop) != 0u) return;
    if (tid() == 0) { S.fail = 0; S.prof_i = 0; }
    const Ctx cx{Wp, kvp};
    const Weights &W = *Wp;
    Seq seq{a.epoch, 0};
    Regs R;
    // small per-thread state first: nothing is in flight yet, so these loads drain nothing
    if (tid() < HD / 2) S.invf[0][tid()] = gld(W.invf_t + tid());
    else if (tid() < HD) S.invf[1][tid() - HD / 2] = gld(W.invf_c + tid() - HD / 2);
    {
        constexpr int NP = static_cast<int>(sizeof(LayerPtrs) / sizeof(void *));
        const void *const *src_t = reinterpret_cast<const void *const *>(W.tl);
        const void *const *src_c = reinterpret_cast<const void *const *>(W.cp);
        const void **dst = reinterpret_cast<const void **>(S.lp);
        for (int i = tid(); i < (MAX_TL + MAX_CL) * NP; i += BT)
            dst[i] = i < MAX_TL * NP ? gld(src_t + i) : gld(src_c + i - MAX_TL * NP);
        if (tid() < CPH) { S.emb[tid()] = gld(W.cp_emb + tid()); S.lmh[tid()] = gld(W.lm_head + tid()); }
    }
    __syncthreads();
    if (tid() < HD / 2) {
        float sn, cs;
        sincosf(static_cast<float>(a.n_past) * S.invf[0][tid()], &sn, &cs);
        S.trope[0][tid()] = cs;
        S.trope[1][tid()] = sn;
    }
    uint32_t seen_bits = 0;
    for (int k = 0; k < VT / BT; ++k) seen_bits |= (gld(a.seen + tid() + k * BT) ? 1u : 0u) << k;
    load_norm(R.fn, a.skip_talker ? W.cp_norm : W.tl_norm);
    const int first = a.skip_talker ? a.n_tl : 0;
    {
        const LayerPtrs &L0 = layer_at(a, S, first);
        const bool cp0 = first >= a.n_tl;
        load_qkv(R, L0, cp0); load_o(R, L0, cp0); load_gu(R, L0, cp0); load_dn(R, L0, cp0);
    }
    __syncthreads();

    // ---- talker step (or frame 0's prefill outputs) ----
    if (!a.skip_talker) {
        for (int i = tid(); i < H; i += BT) S.x[0][i] = gld(a.step_in + i);
        __syncthreads();
        for (int il = 0; il < a.n_tl; ++il)
            if (!run_layer<1, true>(a, cx, R, il, a.n_past, seq, S, il == a.n_tl - 1 ? W.codec_head : nullptr, il > 0,
                                    il == a.n_tl - 1))
                return;
        float hsc[1];
        norm_scale<1>(a.eps_t, hsc, S);
        load_norm(R.fn, W.cp_norm);
        const uint32_t t_lg = seq.next();
        {
            float xf[2][8], d[3];
            xfrag<2>(S.xn[0], 0, xf);
            dot16_rows<3>(R.th, xf, d);
            wave_sum_n<3>(d);
#pragma unroll
            for (int r = 0; r < 3; ++r)
                if (lane() < NREP) mb_put(a.mb + lane() * MB_WORDS + MB_LG + blk() * (VT / NB) + wave() * 3 + r, d[r] * hsc[0], t_lg);
        }
        if (!gather<VT, true, false, D_TLG>(a, MB_LG, t_lg, S.u.m.samp.lg, S)) return;
        // the post-norm hidden the code predictor takes: each thread scales the elements it wrote
        // (and is the only one to read below), after the gather's barriers ended the head's reads
        for (int i = tid(); i < H; i += BT) S.xn[0][i] *= hsc[0];
    } else {
        for (int i = tid(); i < H; i += BT) S.xn[0][i] = gld(a.hidden_in + i);
        for (int i = tid(); i < VT; i += BT) S.u.m.samp.lg[i] = gld(a.logits_in + i);
        __syncthreads();
    }
    if (a.tap_hidden && blk() == 0) {
        for (int i = tid(); i < H; i += BT) gst(a.tap_hidden + i, S.xn[0][i]);
        for (int i = tid(); i < VT; i += BT) gst(a.tap_logits + i, S.u.m.samp.lg[i]);
    }

    // ---- codebook 0: suppression, min-frames EOS, repetition penalty (frame.hip:413-419) ----
#pragma unroll
    for (int k = 0; k < VT / BT; ++k) {
        const int i = tid() + k * BT;
        float v = S.u.m.samp.lg[i];
        if (i >= a.suppress_from && i != a.eos_id) v = -INFINITY;
        else if (i == a.eos_id && a.frame_index < a.min_frames) v = -INFINITY;
        else if (a.rep_penalty > 0.f && ((seen_bits >> k) & 1u)) v = v > 0.f ? v / a.rep_penalty : v * a.rep_penalty;
        S.u.m.samp.lg[i] = v;
    }
    __syncthreads();
    PROF_MARK(a, S);
    const int cb0 = block_sample<VT, BT>(a.temperature, a.top_k, a.talker_seed, sample_lds(S));
    PROF_MARK(a, S);
    if (tid() == 0) S.codes[0] = cb0;

    // ---- code predictor: positions {0,1} as one 2-row pass, then 2..15 ----
    int gi = a.n_tl;
    for (int i = tid(); i < H; i += BT) {
        S.x[0][i] = S.xn[0][i];
        S.x[1][i] = h2f(gld(W.codec_emb + static_cast<size_t>(cb0) * H + i));
    }
    if (blk() < NH) {            // the cp attention blocks: K/V rows not yet written read as zero
        constexpr int NV = static_cast<int>(sizeof(S.u.m.ckv) / sizeof(u32x4_t));
        u32x4_t *z = reinterpret_cast<u32x4_t *>(&S.u.m.ckv[0][0][0][0]);
        for (int i = tid(); i < NV; i += BT) z[i] = u32x4_t{0u, 0u, 0u, 0u};
        for (int i = tid(); i < NCB * HD / 2; i += BT) {
            const int pos = i / (HD / 2), l = i % (HD / 2);
            float sn, cs;
            sincosf(static_cast<float>(pos) * S.invf[1][l], &sn, &cs);
            S.u.m.rope[0][pos][l] = cs;
            S.u.m.rope[1][pos][l] = sn;
        }
    }
    __syncthreads();
    for (int il = 0; il < a.n_cl; ++il, ++gi)
        if (!run_layer<2, false>(a, cx, R, gi, 0, seq, S, il == a.n_cl - 1 ? S.lmh[0] : nullptr, il > 0, il == a.n_cl - 1))
            return;
    for (int pos = 1; pos < NCB; ++pos) {
        if (pos > 1) {
            for (int il = 0; il < a.n_cl; ++il, ++gi)
                if (!run_layer<1, false>(a, cx, R, gi, pos, seq, S, il == a.n_cl - 1 ? S.lmh[pos - 1] : nullptr, il > 0,
                                         il == a.n_cl - 1))
                    return;
        }
        // the last layer's gather normed every row with the cp norm; the head takes the last row
        const int row = pos == 1 ? 1 : 0;
        const float hsc0 = norm_scale_row(a.eps_c, row, S);
        const uint32_t t_lg = seq.next();
        {
            float xf[2][8], d[2];
            xfrag<2>(S.xn[row], 0, xf);
            dot16_rows<2>(R.lm, xf, d);
            wave_sum_n<2>(d);
#pragma unroll
            for (int r = 0; r < 2; ++r)
                if (lane() < NREP) mb_put(a.mb + lane() * MB_WORDS + MB_LG + blk() * (VC / NB) + wave() * 2 + r, d[r] * hsc0, t_lg);
        }
        if (!gather<VC, true, false, D_CLG>(a, MB_LG, t_lg, S.u.m.samp.lg, S)) return;
        if (a.tap_cp_logits && blk() == 0) {
            for (int i = tid(); i < VC; i += BT) gst(a.tap_cp_logits + (pos - 1) * VC + i, S.u.m.samp.lg[i]);
            __syncthreads();
        }
        PROF_MARK(a, S);
        const int code = block_sample<VC, BT>(a.cp_temperature, a.cp_top_k, a.cp_seed + static_cast<uint64_t>(pos) * 0xD1B54A32D192ED03ull, sample_lds(S));
        PROF_MARK(a, S);
        if (tid() == 0) S.codes[pos] = code;
        if (pos + 1 < NCB) {
            load_row_f16(S.emb[pos - 1] + static_cast<size_t>(code) * H, S.x[0]);
            __syncthreads();
        }
    }

    // ---- next step embedding (frame.hip:503-513 order) and outputs ----
    __syncthreads();
    if (tid() < H / NB) {
        const int i = blk() * (H / NB) + tid();
        float v = h2f(gld(W.codec_emb + static_cast<size_t>(S.codes[0]) * H + i));
        for (int cb = 0; cb < CPH; ++cb) v += h2f(gld(S.emb[cb] + static_cast<size_t>(S.codes[cb + 1]) * H + i));
        gst(a.step_out + i, v + gld(a.trailing + i));
    }
    PROF_MARK(a, S);
    if (blk() == 0 && tid() == 0) {
        for (int c = 0; c < NCB; ++c) gst(a.codes_out + c, static_cast<int32_t>(S.codes[c]));
        if (S.codes[0] != a.eos_id) gst(a.seen + S.codes[0], static_cast<uint8_t>(1u));
        else if (a.stop) ctl_put(a.stop, 1u);
    }
}

uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

} // namespace fk
} // namespace navi_amd

// ---------------------------------------------------------------------------
// Host side (Frame::Impl, frame.hip:590-810)
// ---------------------------------------------------------------------------

using namespace navi_amd;
using namespace navi_amd::fk;

struct navi_frame {
    navi_model_params p{};
    navi_frame_options opt{};
    Weights hw{};
    Weights *dw = nullptr;
    uint64_t *mb = nullptr;
    uint32_t *ctl = nullptr;       // [0..15] codes, [16] abort epoch
    float *step_out = nullptr;
    uint8_t *seen = nullptr;
    float *tap = nullptr;          // hidden | logits | cp logits
    bool taps = false;
    uint16_t **kv_dev = nullptr;   // [2][MAX_TL] per-layer K/V pointers as the kernel reads them
    uint64_t *prof = nullptr;      // [NB][PROF_SLOTS] when profiling is on
    int32_t *run_codes = nullptr;  // frame loop: [MAX_RUN][16] codes of each frame
    uint32_t *stop = nullptr;      // frame loop: 1 = EOS sampled, 2 = a frame timed out
    // pinned host copies read back after a call's one synchronization: [MAX_RUN][16] loop codes,
    // then ctl ([16] codes, abort epoch), then the loop's stop word
    uint32_t *h_rb = nullptr;
    uint16_t *kv_host[2][MAX_TL] = {};
    uint32_t epoch = 0;
    int grid = NB, occ = 0;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::vector<void *> owned;

    ~navi_frame() {
        if (ev0) (void) hipEventDestroy(ev0);
        if (ev1) (void) hipEventDestroy(ev1);
        if (h_rb) (void) hipHostFree(h_rb);
        for (void *q : owned) (void) hipFree(q);
    }
    uint32_t *h_ctl() const { return h_rb + static_cast<size_t>(MAX_RUN) * NCB; }
    uint32_t *h_stop() const { return h_ctl() + NCB + 1; }
    template <class T> navi_status alloc(T *&ptr, size_t n, char *err, size_t errlen) {
        void *q = nullptr;
        NAVI_TRY_HIP(hipMalloc(&q, n * sizeof(T)), err, errlen);
        owned.push_back(q);
        NAVI_TRY_HIP(hipMemset(q, 0, n * sizeof(T)), err, errlen);
        ptr = static_cast<T *>(q);
        return NAVI_OK;
    }
};

namespace {

#define NAVI_BIND(T, name, dt, d0, d1, out)                                                       \
    do {                                                                                          \
        const navi_status s_ = bind_tensor<T>("frame", tensors, n_tensors, (name), (dt), (d0), (d1), (out), err, errlen); \
        if (s_ != NAVI_OK) return s_;                                                             \
    } while (0)

navi_status bind_layers(const navi_tensor_ref *tensors, int n_tensors, const std::string &prefix, int n, LayerPtrs *L,
                        char *err, size_t errlen) {
    for (int l = 0; l < n; ++l) {
        const std::string p = prefix + ".layers." + std::to_string(l) + ".";
        NAVI_BIND(float, p + "input_layernorm.weight", NAVI_DT_F32, H, 0, L[l].ln1);
        NAVI_BIND(float, p + "post_attention_layernorm.weight", NAVI_DT_F32, H, 0, L[l].ln2);
        NAVI_BIND(float, p + "self_attn.q_norm.weight", NAVI_DT_F32, HD, 0, L[l].qn);
        NAVI_BIND(float, p + "self_attn.k_norm.weight", NAVI_DT_F32, HD, 0, L[l].kn);
        NAVI_BIND(uint16_t, p + "self_attn.q_proj.weight", NAVI_DT_F16, QD, H, L[l].wq);
        NAVI_BIND(uint16_t, p + "self_attn.k_proj.weight", NAVI_DT_F16, KVD, H, L[l].wk);
        NAVI_BIND(uint16_t, p + "self_attn.v_proj.weight", NAVI_DT_F16, KVD, H, L[l].wv);
        NAVI_BIND(uint16_t, p + "self_attn.o_proj.weight", NAVI_DT_F16, H, QD, L[l].wo);
        NAVI_BIND(uint16_t, p + "mlp.gate_proj.weight", NAVI_DT_F16, FF, H, L[l].wg);
        NAVI_BIND(uint16_t, p + "mlp.up_proj.weight", NAVI_DT_F16, FF, H, L[l].wu);
        NAVI_BIND(uint16_t, p + "mlp.down_proj.weight", NAVI_DT_F16, H, FF, L[l].wd);
    }
    return NAVI_OK;
}

bool shape_is(const navi_xformer_params &x, int vocab) {
    return x.hidden == H && x.n_head == NH && x.n_kv_head == NKV && x.head_dim == HD && x.ff == FF && x.vocab == vocab;
}

} // namespace

extern "C" {

navi_status navi_frame_create(const navi_model_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                              const navi_frame_options *opt, navi_frame **out, char *err, size_t errlen) {
    if (!p || !tensors || !out) { set_err(err, errlen, "frame: null argument"); return NAVI_ERR_INVALID; }
    *out = nullptr;
    navi_status st = ensure_device(err, errlen);
    if (st != NAVI_OK) return st;
    if (!shape_is(p->talker, VT) || !shape_is(p->cp, VC) || p->n_code_groups != NCB) {
        set_err(err, errlen, "frame: kernel is built for the Qwen3-TTS-0.6B shapes (hidden 1024, 16/8 heads x 128, ff 3072, vocab 3072/2048, 16 codebooks)");
        return NAVI_ERR_UNSUPPORTED;
    }
    if (p->talker.n_layer < 1 || p->talker.n_layer > MAX_TL || p->cp.n_layer < 1 || p->cp.n_layer > MAX_CL) {
        set_err(err, errlen, "frame: layer counts %d/%d exceed the kernel's %d/%d", p->talker.n_layer, p->cp.n_layer, MAX_TL, MAX_CL);
        return NAVI_ERR_UNSUPPORTED;
    }
    navi_frame_options o{1, 0};
    if (opt) o = *opt;
    if (o.blocks_per_mp != 1) { set_err(err, errlen, "frame: blocks_per_mp must be 1 (one persistent block per CU)"); return NAVI_ERR_INVALID; }
    if (o.spin_cap == 0) o.spin_cap = 2000000ull;   // ~1-2 s of polling at MALL latency

    const DeviceState &ds = device_state();
    if (ds.prop.multiProcessorCount < NB) {
        set_err(err, errlen, "frame: needs %d co-resident blocks, device has %d CUs", NB, ds.prop.multiProcessorCount);
        return NAVI_ERR_UNSUPPORTED;
    }
    int occ = 0;
    NAVI_TRY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_frame, BT, 0), err, errlen);
    if (occ < 1) { set_err(err, errlen, "frame: k_frame cannot be resident"); return NAVI_ERR_UNSUPPORTED; }

    auto *f = new navi_frame();
    f->p = *p;
    f->opt = o;
    f->occ = occ;
    Weights &w = f->hw;
    auto fail = [&](navi_status s) { delete f; return s; };
    if ((st = bind_layers(tensors, n_tensors, "talker.model", p->talker.n_layer, w.tl, err, errlen)) != NAVI_OK) return fail(st);
    if ((st = bind_layers(tensors, n_tensors, "talker.code_predictor.model", p->cp.n_layer, w.cp, err, errlen)) != NAVI_OK) return fail(st);
    {
        const int n_tensors_ = n_tensors;
        auto b16 = [&](const uint16_t *&dst, const std::string &name, uint64_t d0, uint64_t d1) {
            return bind_tensor<uint16_t>("frame", tensors, n_tensors_, name, NAVI_DT_F16, d0, d1, dst, err, errlen);
        };
        auto b32 = [&](const float *&dst, const std::string &name, uint64_t d0) {
            return bind_tensor<float>("frame", tensors, n_tensors_, name, NAVI_DT_F32, d0, 0, dst, err, errlen);
        };
        if ((st = b32(w.tl_norm, "talker.model.norm.weight", H)) != NAVI_OK) return fail(st);
        if ((st = b32(w.cp_norm, "talker.code_predictor.model.norm.weight", H)) != NAVI_OK) return fail(st);
        if ((st = b16(w.codec_head, "talker.codec_head.weight", VT, H)) != NAVI_OK) return fail(st);
        if ((st = b16(w.codec_emb, "talker.model.codec_embedding.weight", VT, H)) != NAVI_OK) return fail(st);
        for (int i = 0; i < CPH; ++i) {
            if ((st = b16(w.cp_emb[i], "talker.code_predictor.model.codec_embedding." + std::to_string(i) + ".weight", VC, H)) != NAVI_OK) return fail(st);
            if ((st = b16(w.lm_head[i], "talker.code_predictor.lm_head." + std::to_string(i) + ".weight", VC, H)) != NAVI_OK) return fail(st);
        }
    }
    for (int i = 0; i < HD / 2; ++i) {
        w.invf_t[i] = static_cast<float>(1.0 / std::pow(p->talker.rope_theta, 2.0 * i / HD));
        w.invf_c[i] = static_cast<float>(1.0 / std::pow(p->cp.rope_theta, 2.0 * i / HD));
    }
    w.eps_t = p->talker.rms_eps;
    w.eps_c = p->cp.rms_eps;

    if ((st = f->alloc(f->dw, 1, err, errlen)) != NAVI_OK) return fail(st);
    if ((st = f->alloc(f->mb, static_cast<size_t>(MB_TOTAL), err, errlen)) != NAVI_OK) return fail(st);
    if ((st = f->alloc(f->ctl, 32, err, errlen)) != NAVI_OK) return fail(st);
    if ((st = f->alloc(f->run_codes, static_cast<size_t>(MAX_RUN) * NCB, err, errlen)) != NAVI_OK) return fail(st);
    if ((st = f->alloc(f->stop, 1, err, errlen)) != NAVI_OK) return fail(st);
    if ((st = f->alloc(f->step_out, H, err, errlen)) != NAVI_OK) return fail(st);
    if ((st = f->alloc(f->seen, VT, err, errlen)) != NAVI_OK) return fail(st);
    if ((st = f->alloc(f->tap, H + VT + CPH * VC, err, errlen)) != NAVI_OK) return fail(st);
    if ((st = f->alloc(f->kv_dev, 2 * MAX_TL, err, errlen)) != NAVI_OK) return fail(st);
    if (hipMemcpy(f->dw, &f->hw, sizeof(Weights), hipMemcpyHostToDevice) != hipSuccess) {
        set_err(err, errlen, "frame: weight table upload failed");
        return fail(NAVI_ERR_HIP);
    }
    if (hipEventCreate(&f->ev0) != hipSuccess || hipEventCreate(&f->ev1) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void **>(&f->h_rb), sizeof(uint32_t) * (static_cast<size_t>(MAX_RUN) * NCB + NCB + 2),
                      hipHostMallocDefault) != hipSuccess) {
        set_err(err, errlen, "frame: hipEventCreate or the pinned readback allocation failed");
        return fail(NAVI_ERR_HIP);
    }
    f->grid = NB;
    *out = f;
    return NAVI_OK;
}

void navi_frame_destroy(navi_frame *f) { delete f; }

navi_status navi_frame_reset(navi_frame *f) {
    if (!f) return NAVI_ERR_INVALID;
    return hipMemsetAsync(f->seen, 0, VT, device_state().stream) == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

navi_status navi_frame_set_profile(navi_frame *f, int32_t enabled) {
    if (!f) return NAVI_ERR_INVALID;
    if (enabled && !f->prof) {
        if (f->alloc(f->prof, static_cast<size_t>(NB) * PROF_SLOTS, nullptr, 0) != NAVI_OK) return NAVI_ERR_HIP;
    }
    if (!enabled && f->prof) {
        (void) hipFree(f->prof);
        f->owned.erase(std::remove(f->owned.begin(), f->owned.end(), static_cast<void *>(f->prof)), f->owned.end());
        f->prof = nullptr;
    }
    return NAVI_OK;
}

navi_status navi_frame_profile(const navi_frame *f, uint64_t *out, int32_t n_blocks, int32_t n_slots) {
    if (!f || !out || !f->prof || n_blocks > NB || n_slots > PROF_SLOTS) return NAVI_ERR_INVALID;
    for (int b = 0; b < n_blocks; ++b)
        if (hipMemcpy(out + static_cast<size_t>(b) * n_slots, f->prof + static_cast<size_t>(b) * PROF_SLOTS,
                      static_cast<size_t>(n_slots) * sizeof(uint64_t), hipMemcpyDeviceToHost) != hipSuccess)
            return NAVI_ERR_HIP;
    return NAVI_OK;
}

navi_status navi_frame_set_epoch(navi_frame *f, uint32_t epoch) {
    if (!f || epoch % EPOCH_STRIDE != 0 || epoch > 0xFFFFFFFFu - EPOCH_STRIDE + 1u) return NAVI_ERR_INVALID;
    f->epoch = epoch;
    return NAVI_OK;
}

uint32_t navi_frame_epoch(const navi_frame *f) { return f ? f->epoch : 0u; }

navi_status navi_frame_set_spin_cap(navi_frame *f, uint64_t spin_cap) {
    if (!f) return NAVI_ERR_INVALID;
    f->opt.spin_cap = spin_cap ? spin_cap : 2000000ull;
    return NAVI_OK;
}

navi_status navi_frame_set_taps(navi_frame *f, int32_t enabled) {
    if (!f) return NAVI_ERR_INVALID;
    f->taps = enabled != 0;
    return NAVI_OK;
}

const float *navi_frame_tap_hidden(const navi_frame *f) { return f ? f->tap : nullptr; }
const float *navi_frame_tap_logits(const navi_frame *f) { return f ? f->tap + H : nullptr; }
const float *navi_frame_tap_cp_logits(const navi_frame *f) { return f ? f->tap + H + VT : nullptr; }
float *navi_frame_step_out(navi_frame *f) { return f ? f->step_out : nullptr; }
int32_t navi_frame_grid_blocks(const navi_frame *f) { return f ? f->grid : 0; }
int32_t navi_frame_occupancy_per_mp(const navi_frame *f) { return f ? f->occ : 0; }

} // extern "C"

namespace {

// KV view checks for frames up to n_past_max, and the per-layer pointer table upload when the
// cache changed (frame.hip:787-810 run's checks). msg: the reference's error text on failure.
navi_status frame_kv(navi_frame *f, const navi_kv_view *kv, int n_past_min, int n_past_max, const char *&msg) {
    if (!kv || !kv->k || !kv->v) { msg = "frame: run needs a KV cache"; return NAVI_ERR_INVALID; }
    if (n_past_max >= kv->max_pos || n_past_max >= MAX_POS) { msg = "KV cache full"; return NAVI_ERR_KV_FULL; }
    if (n_past_min < 0) { msg = "frame: negative n_past"; return NAVI_ERR_INVALID; }
    if (kv->n_layer != f->p.talker.n_layer || kv->kv_dim != KVD) { msg = "KV cache layer count mismatch"; return NAVI_ERR_INVALID; }
    bool same = true;
    for (int l = 0; l < kv->n_layer; ++l) same = same && f->kv_host[0][l] == kv->k[l] && f->kv_host[1][l] == kv->v[l];
    if (!same) {
        for (int l = 0; l < kv->n_layer; ++l) { f->kv_host[0][l] = kv->k[l]; f->kv_host[1][l] = kv->v[l]; }
        if (hipMemcpyAsync(f->kv_dev, f->kv_host, sizeof(f->kv_host), hipMemcpyHostToDevice, device_state().stream) != hipSuccess ||
            hipStreamSynchronize(device_state().stream) != hipSuccess) {
            msg = "frame: KV pointer upload failed";
            return NAVI_ERR_HIP;
        }
    }
    return NAVI_OK;
}

// The launch arguments of one frame (Impl::launch, frame.hip:653-681: per-frame seeds, a new epoch).
Args frame_args(navi_frame *f, int n_past, bool skip_talker, const float *d_hidden, const float *d_logits,
                const float *d_trailing, const navi_sampling *s, uint64_t seed, int frame_index, int32_t *codes_out) {
    Args a{};
    a.hidden_in = skip_talker ? d_hidden : nullptr;
    a.logits_in = skip_talker ? d_logits : nullptr;
    a.mb = f->mb;
    a.eps_t = f->p.talker.rms_eps;
    a.eps_c = f->p.cp.rms_eps;
    a.abort_word = f->ctl + NCB;
    a.codes_out = codes_out;
    a.n_tl = f->p.talker.n_layer;
    a.n_cl = f->p.cp.n_layer;
    a.n_past = n_past;
    a.skip_talker = skip_talker ? 1 : 0;
    a.step_in = f->step_out;
    a.trailing = d_trailing;
    a.step_out = f->step_out;
    a.seen = f->seen;
    a.temperature = s->temperature;
    a.top_k = s->top_k;
    a.rep_penalty = s->repetition_penalty;
    a.cp_temperature = s->cp_temperature;
    a.cp_top_k = s->cp_top_k;
    a.min_frames = s->min_frames;
    a.frame_index = frame_index;
    a.eos_id = f->p.codec_eos_id;
    a.suppress_from = VT - 1024;   // HF suppress_tokens = range(vocab - 1024, vocab) minus EOS
    a.talker_seed = splitmix64(seed ^ (static_cast<uint64_t>(frame_index) * 0xA24BAED4963EE407ull));
    a.cp_seed = splitmix64(a.talker_seed ^ 0x9FB21C651E98DF25ull);
    a.spin_cap = f->opt.spin_cap;
    a.epoch = f->epoch;
    a.prof = f->prof;
    if (f->taps) {
        a.tap_hidden = f->tap;
        a.tap_logits = f->tap + H;
        a.tap_cp_logits = f->tap + H + VT;
    }
    return a;
}

// Advances the launch epoch (Impl::launch's barrier reset, frame.hip:660). Tags are epoch + phase in
// 32 bits, so epochs repeat after 2^20 launches. When the epoch wraps, the mailboxes and the abort
// word are cleared on the stream before the next launch (tag 0 is never used): neither a stale
// mailbox word nor the stamp of an old timed-out launch can then match a tag of a later launch.
hipError_t advance_epoch(navi_frame *f) {
    uint64_t next = static_cast<uint64_t>(f->epoch) + EPOCH_STRIDE;
    if (next > (1ull << 32) - EPOCH_STRIDE) {
        hipStream_t st = device_state().stream;
        hipError_t e = hipMemsetAsync(f->mb, 0, static_cast<size_t>(MB_TOTAL) * sizeof(uint64_t), st);
        if (e == hipSuccess) e = hipMemsetAsync(f->ctl + NCB, 0, sizeof(uint32_t), st);
        if (e != hipSuccess) return e;
        next = EPOCH_STRIDE;
    }
    f->epoch = static_cast<uint32_t>(next);
    return hipSuccess;
}

// The frame's grid is one block per CU and every block waits for the others, so all of them must
// be resident at once. navi_frame_create checked that one block fits on every CU; kernels on one
// stream run one after the other; and a block whose peers never become resident ends at the spin
// cap with "timed out" rather than hanging. So the grid goes out as an ordinary launch: on MI355X
// it measured 1.464 against 1.479 ms per frame for a cooperative launch (the reference's
// Impl::launch, frame.hip:663), and rocprofv3 ends a process that made cooperative launches with
// SIGSEGV inside exit() while the same process with ordinary launches exits cleanly.
// NAVI_FRAME_LAUNCH=cooperative in the environment selects the cooperative launch.
bool cooperative_launch() {
    static const bool coop = [] {
        const char *e = std::getenv("NAVI_FRAME_LAUNCH");
        return e && std::strcmp(e, "cooperative") == 0;
    }();
    return coop;
}

hipError_t frame_launch(navi_frame *f, Args &a) {
    const Weights *wp = f->dw;
    uint16_t *const *kvp = f->kv_dev;
    if (cooperative_launch()) {
        void *args[] = {&a, &wp, &kvp};
        return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(k_frame), dim3(f->grid), dim3(BT), args, 0,
                                          device_state().stream);
    }
    hipLaunchKernelGGL(k_frame, dim3(f->grid), dim3(BT), 0, device_state().stream, a, wp, kvp);
    return hipGetLastError();
}

} // namespace

extern "C" {

navi_status navi_frame_run(navi_frame *f, const navi_kv_view *kv, int32_t n_past, int32_t skip_talker,
                           const float *d_hidden, const float *d_logits, const float *d_trailing,
                           const navi_sampling *s, uint64_t seed, int32_t frame_index, navi_frame_result *out) {
    if (!out) return NAVI_ERR_INVALID;
    std::memset(out, 0, sizeof(*out));
    auto fail = [&](navi_status st, const char *msg) {
        out->ok = 0;
        out->status = st;
        std::snprintf(out->error, sizeof(out->error), "%s", msg);
        return st;
    };
    if (!f || !s || !d_trailing) return fail(NAVI_ERR_INVALID, "frame: null argument");
    if (skip_talker) {
        if (!d_hidden || !d_logits) return fail(NAVI_ERR_INVALID, "frame: run_first needs the prefill's hidden and logits");
    } else {
        const char *msg = nullptr;
        const navi_status st = frame_kv(f, kv, n_past, n_past, msg);
        if (st != NAVI_OK) return fail(st, msg);
    }
    if (advance_epoch(f) != hipSuccess) return fail(NAVI_ERR_HIP, "frame: epoch reset failed");
    Args a = frame_args(f, n_past, skip_talker != 0, d_hidden, d_logits, d_trailing, s, seed, frame_index,
                        reinterpret_cast<int32_t *>(f->ctl));
    hipStream_t st = device_state().stream;
    if (hipEventRecord(f->ev0, st) != hipSuccess) return fail(NAVI_ERR_HIP, "frame: hipEventRecord failed");
    const hipError_t e = frame_launch(f, a);
    if (e != hipSuccess) {
        std::string m = std::string("frame launch failed: ") + hipGetErrorString(e);
        return fail(NAVI_ERR_LAUNCH, m.c_str());
    }
    uint32_t *h = f->h_ctl();
    if (hipEventRecord(f->ev1, st) != hipSuccess ||
        hipMemcpyAsync(h, f->ctl, sizeof(uint32_t) * (NCB + 1), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fail(NAVI_ERR_HIP, "frame: launch or readback failed");
    float ms = 0.f;
    (void) hipEventElapsedTime(&ms, f->ev0, f->ev1);
    out->us = ms * 1000.0;
    if (h[NCB] == f->epoch) return fail(NAVI_ERR_TIMEOUT, "frame dataflow wait timed out: the persistent grid could not run to completion");
    for (int c = 0; c < NCB; ++c) out->codes[c] = static_cast<int32_t>(h[c]);
    out->eos = out->codes[0] == f->p.codec_eos_id;
    out->ok = 1;
    out->status = NAVI_OK;
    return NAVI_OK;
}

navi_status navi_frame_run_many(navi_frame *f, const navi_kv_view *kv, int32_t n_past0, int32_t skip_first,
                                const float *d_hidden, const float *d_logits, const float *d_trailing, int32_t n_trailing,
                                const float *d_tts_pad, const navi_sampling *s, uint64_t seed, int32_t frame_index0,
                                int32_t n_frames, int32_t *codes_out, int32_t *n_done, int32_t *eos, double *us, char *err,
                                size_t errlen) {
    if (!f || !s || !codes_out || !n_done || (!d_trailing && n_trailing > 0) || !d_tts_pad || n_trailing < 0) {
        set_err(err, errlen, "frame: null argument");
        return NAVI_ERR_INVALID;
    }
    *n_done = 0;
    if (eos) *eos = 0;
    if (us) *us = 0.0;
    if (n_frames < 1 || n_frames > MAX_RUN) {
        set_err(err, errlen, "frame: %d frames per loop, 1..%d allowed", n_frames, MAX_RUN);
        return NAVI_ERR_INVALID;
    }
    if (skip_first && (!d_hidden || !d_logits)) {
        set_err(err, errlen, "frame: run_first needs the prefill's hidden and logits");
        return NAVI_ERR_INVALID;
    }
    const int first_talker = skip_first ? 1 : 0;
    if (first_talker < n_frames) {
        const char *msg = nullptr;
        const navi_status st = frame_kv(f, kv, n_past0 + first_talker, n_past0 + n_frames - 1, msg);
        if (st != NAVI_OK) {
            set_err(err, errlen, "%s", msg);
            return st;
        }
    }
    hipStream_t st = device_state().stream;
    std::vector<uint32_t> epochs(static_cast<size_t>(n_frames));
    NAVI_TRY_HIP(hipMemsetAsync(f->stop, 0, sizeof(uint32_t), st), err, errlen);
    NAVI_TRY_HIP(hipEventRecord(f->ev0, st), err, errlen);
    for (int i = 0; i < n_frames; ++i) {
        const bool skip = skip_first && i == 0;
        const float *trail = i < n_trailing ? d_trailing + static_cast<size_t>(i) * H : d_tts_pad;
        NAVI_TRY_HIP(advance_epoch(f), err, errlen);
        epochs[static_cast<size_t>(i)] = f->epoch;
        Args a = frame_args(f, skip ? 0 : n_past0 + i, skip, d_hidden, d_logits, trail, s, seed, frame_index0 + i,
                            f->run_codes + static_cast<size_t>(i) * NCB);
        a.stop = f->stop;
        const hipError_t e = frame_launch(f, a);
        if (e != hipSuccess) {
            (void) hipStreamSynchronize(st);
            set_err(err, errlen, "frame launch failed: %s", hipGetErrorString(e));
            return NAVI_ERR_LAUNCH;
        }
    }
    NAVI_TRY_HIP(hipEventRecord(f->ev1, st), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(f->h_rb, f->run_codes, static_cast<size_t>(n_frames) * NCB * sizeof(int32_t),
                                hipMemcpyDeviceToHost, st), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(f->h_ctl(), f->ctl, sizeof(uint32_t) * (NCB + 1), hipMemcpyDeviceToHost, st), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(f->h_stop(), f->stop, sizeof(uint32_t), hipMemcpyDeviceToHost, st), err, errlen);
    NAVI_TRY_HIP(hipStreamSynchronize(st), err, errlen);
    std::memcpy(codes_out, f->h_rb, static_cast<size_t>(n_frames) * NCB * sizeof(int32_t));
    const uint32_t *ctl = f->h_ctl(), stop = *f->h_stop();
    float ms = 0.f;
    (void) hipEventElapsedTime(&ms, f->ev0, f->ev1);
    if (us) *us = ms * 1000.0;
    // A timed-out frame stamped its epoch and stopped the loop. A stamp older than this loop holds an
    // epoch below all of this loop's (epochs rise between wraps, and a wrap clears the stamp).
    int bad = -1;
    for (int i = 0; i < n_frames && bad < 0; ++i)
        if (epochs[static_cast<size_t>(i)] == ctl[NCB]) bad = i;
    if (stop == 2u || bad >= 0) {
        *n_done = bad > 0 ? bad : 0;
        set_err(err, errlen, "frame %d: frame dataflow wait timed out: the persistent grid could not run to completion",
                frame_index0 + *n_done);
        return NAVI_ERR_TIMEOUT;
    }
    int done = n_frames;
    for (int i = 0; i < n_frames; ++i)
        if (codes_out[static_cast<size_t>(i) * NCB] == f->p.codec_eos_id) {
            done = i + 1;
            if (eos) *eos = 1;
            break;
        }
    *n_done = done;
    return NAVI_OK;
}

} // extern "C"
