// Prompt rows and the causal prefill of the talker on gfx950, plus the linear layer they are
// built from (the C ABI's navi_talker_* and navi_linear).
//
// Replaces Talker (model/qwen3tts/talker.hip:20-399) and the GEMMs it runs through
// Talker::Impl::gemm (k_gemm_skinny / k_conv<K=1>, kernels.h:72-330). MI355X design:
//
//  * Every projection is Y = X · W^T with f16 weights [N][K] and f32 activations, on the
//    matrix cores (v_mfma_f32_16x16x32_f16). Each activation is split into an f16 pair
//    x = hi + lo (hi = f16(x), lo = f16(x - hi)), so two MFMAs per weight fragment carry ~22
//    bits of the activation: the products keep f32-level accuracy while the weights stream
//    at the matrix cores' f16 rate. Activations must lie inside the f16 range; a device flag
//    turns anything else into an error instead of an infinity.
//  * The linear (navi_linear, the prompt's text projection): a block owns 64 output columns (one
//    16-column MFMA tile per wave) and up to 64 rows; K is split across blocks so that even
//    N = 1024 fills the 256 CUs. Split-K partials go to a workspace and are summed in a fixed
//    order by the "finish" kernels, which also apply the epilogue (bias, SiLU, residual):
//    deterministic results.
//  * The prefill's layers: five launches each. q|k|v, o, gate|up and down are whole-K row
//    projections (rows.h) with the input RMSNorm, SwiGLU and the residual add fused in; the q/k
//    head norms + RoPE and the f16 K/V store run in the q|k|v projection's epilogue (above 64 rows)
//    or inside the attention (up to 64 rows); then the attention. The
//    projections read their operands in the MFMA tile layouts (rows.h pk_a / pk_w): a copy of
//    every layer's weights tiled at create, and the residual stream, the attention output and the
//    MLP hidden stored tiled by the kernels that write them.
//  * Causal prefill attention: one block per (row, q head), scores over keys 0..row from the
//    f16 cache, exactly as the frame's decode attention will later read them.
#include "dev_common.h"
#include "host_util.h"
#include "linear.h"
#include "rows.h"

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

namespace navi_amd {
namespace pf {

constexpr int BT = 256;                 // 4 wave64s
constexpr int KC = 256;                 // K elements staged in LDS per step
constexpr int LDA = KC + 8;             // padded LDS row (halves): rotates banks between rows
constexpr int HD = 128;                 // head dim the norm/rope/attention kernels are built for

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

struct LinArgs {
    const float *x;        // [M][ldx] f32
    // W as up to three row blocks (q | k | v, gate | up): output columns [0, n1) are rows of w,
    // [n1, n2) rows of w1, [n2, N) rows of w2, each [rows][K] f16
    const uint16_t *w, *w1, *w2;
    float *part;           // [S][M][ldp] f32 partial sums (columns p_off .. p_off + N)
    uint32_t *flag;        // set when an activation is outside the f16 range
    int ldx, M, K, N, kps, ldp, p_off, n1, n2;
};

__device__ __forceinline__ void split_store(float v, _Float16 *hi, _Float16 *lo, bool &bad) {
    bad |= !(fabsf(v) < 65504.f);
    const _Float16 h = static_cast<_Float16>(v);
    *hi = h;
    *lo = static_cast<_Float16>(v - static_cast<float>(h));
}

// Partial Y for one (64-column tile, MT*16-row tile, K split). Output lane layout of
// v_mfma_f32_16x16x32_f16: lane l holds column l % 16 of rows 4 * (l / 16) + r, r = 0..3.
// A and B fragments use the same lane -> k mapping (k = 8 * (l / 16) + j within a 32-k step),
// so every k of the step is summed exactly once whatever that mapping is inside the unit.
template <int MT>
__global__ void __launch_bounds__(BT) k_linear_partial(LinArgs a) {
    __shared__ __align__(16) _Float16 ahi[MT * 16][LDA];
    __shared__ __align__(16) _Float16 alo[MT * 16][LDA];
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int n0 = blockIdx.x * 64 + wv * 16;
    const int m0 = blockIdx.y * (MT * 16);
    const int kb = blockIdx.z * a.kps, ke = kb + a.kps;
    const int nc = n0 + (l & 15);
    const uint16_t *wr = nc < a.n1 ? a.w + static_cast<size_t>(nc) * a.K
                       : nc < a.n2 ? a.w1 + static_cast<size_t>(nc - a.n1) * a.K : a.w2 + static_cast<size_t>(nc - a.n2) * a.K;
    const NAVI_GLOBAL u32x4_t *wrow = (const NAVI_GLOBAL u32x4_t *) (wr + (l >> 4) * 8);
    f32x4_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    u32x4_t bcur[KC / 32], bnext[KC / 32];
    auto load_b = [&](u32x4_t (&dst)[KC / 32], int k0) {
        const int steps = min(KC, ke - k0) / 32;
#pragma unroll
        for (int c = 0; c < KC / 32; ++c)
            if (c < steps) dst[c] = __builtin_nontemporal_load(wrow + (k0 >> 3) + c * 4);
    };
    // A staging: every thread owns IT float4s of the MT*16 x kc step tile; the step's loads are
    // all issued at once (and the next step's before this step's MFMAs), never one by one.
    constexpr int IT = MT * 16 * (KC / 4) / BT;
    f32x4_t av[IT];
    auto load_a = [&](int k0) {
        const int q4 = min(KC, ke - k0) >> 2;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int i = threadIdx.x + it * BT, r = i / q4, c4 = (i - r * q4) * 4, m = m0 + r;
            av[it] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (r < MT * 16 && m < a.M) av[it] = *(const NAVI_GLOBAL f32x4_t *) (a.x + static_cast<size_t>(m) * a.ldx + k0 + c4);
        }
    };
    load_b(bcur, kb);
    load_a(kb);
    bool bad = false;
    for (int k0 = kb; k0 < ke; k0 += KC) {
        const int kc = min(KC, ke - k0);
        if (k0 + KC < ke) load_b(bnext, k0 + KC);
        __syncthreads();                                   // previous step's readers are done
        {
            const int q4 = kc >> 2;
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int i = threadIdx.x + it * BT, r = i / q4, c4 = (i - r * q4) * 4;
                if (r < MT * 16) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) split_store(av[it][j], &ahi[r][c4 + j], &alo[r][c4 + j], bad);
                }
            }
        }
        __syncthreads();
        if (k0 + KC < ke) load_a(k0 + KC);
#pragma unroll
        for (int c = 0; c < KC / 32; ++c) {
            if (c < (kc >> 5)) {
                half8v b;
                __builtin_memcpy(&b, &bcur[c], 16);
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const half8v h = *reinterpret_cast<const half8v *>(&ahi[i * 16 + (l & 15)][c * 32 + (l >> 4) * 8]);
                    const half8v o = *reinterpret_cast<const half8v *>(&alo[i * 16 + (l & 15)][c * 32 + (l >> 4) * 8]);
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, b, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o, b, acc[i], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < KC / 32; ++c) bcur[c] = bnext[c];
    }
    if (bad) gst(a.flag, 1u);
    float *p = a.part + static_cast<size_t>(blockIdx.z) * a.M * a.ldp + a.p_off + n0 + (l & 15);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + i * 16 + (l >> 4) * 4 + r;
            if (m < a.M) gst(p + static_cast<size_t>(m) * a.ldp, acc[i][r]);
        }
}

__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}



__device__ __forceinline__ float silu(float g) { return g / (1.f + expf(-g)); }

// y[m][n] = act(sum_s part + bias) + residual (Talker::Impl::gemm epilogues, kernels.h:315-321).
__global__ void __launch_bounds__(BT) k_finish_linear(const float *part, int S, int M, int N, const float *bias,
                                                      const float *residual, int act, float *y, int ldy) {
    const int m = blockIdx.x;
    for (int n = threadIdx.x * 4; n < N; n += BT * 4) {
        f32x4_t v = sum_parts4(part, S, static_cast<size_t>(M) * N, static_cast<size_t>(m) * N + n);
        if (bias) v += ld4(bias + n);
        if (act == 1)
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = silu(v[j]);
        if (residual) v += ld4(residual + static_cast<size_t>(m) * ldy + n);
        st4(y + static_cast<size_t>(m) * ldy + n, v);
    }
}

// x[m] = (S > 0 ? sum_s part + x[m] : src[m]); xn[m] = RMSNorm(x[m]) * w (k_rmsnorm, kernels.h:342-350,
// fused with the residual epilogue of the o / down projections).
__global__ void __launch_bounds__(BT) k_resid_norm(const float *part, int S, const float *src, float *x, const float *w,
                                                   float eps, float *xn, int M, int H) {
    __shared__ float red[4];
    const int m = blockIdx.x, i = threadIdx.x * 4;            // H == 4 * BT
    const size_t idx = static_cast<size_t>(m) * H + i;
    const f32x4_t v = S > 0 ? sum_parts4(part, S, static_cast<size_t>(M) * H, idx) + ld4(x + idx) : ld4(src + idx);
    const f32x4_t wv = ld4(w + i);
    st4(x + idx, v);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) ss = fmaf(v[j], v[j], ss);
    ss = block_sum256(ss, red);
    const float scale = rsqrtf(ss / static_cast<float>(H) + eps);
    f32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = v[j] * scale * wv[j];
    st4(xn + idx, o);
}

// h[m][c] = SiLU(gate) * up from the [gate | up] partials (PRO_SILU_GATE / k_silu_gate, kernels.h:334-340).
__global__ void __launch_bounds__(BT) k_swiglu(const float *part, int S, int M, int F, float *h) {
    const int m = blockIdx.x;
    const size_t stride = static_cast<size_t>(M) * 2 * F;
    for (int c = threadIdx.x * 4; c < F; c += BT * 4) {
        const f32x4_t g = sum_parts4(part, S, stride, static_cast<size_t>(m) * 2 * F + c);
        const f32x4_t u = sum_parts4(part, S, stride, static_cast<size_t>(m) * 2 * F + F + c);
        f32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = silu(g[j]) * u[j];
        st4(h + static_cast<size_t>(m) * F + c, o);
    }
}

// Causal GQA attention for rows with at most SHORT_KEYS keys (prompts of up to 256 rows; above,
// k_attn_prefill_long), one block per (row m, kv group g) for its two q heads over keys 0..pos0 + m
// of the f16 cache (k_prefill_attention, talker.hip:88-117). Wave w takes
// keys 64w .. 64w + 63; lane 16r + c reads 16-byte chunk c of key 4i + r, so one load instruction
// covers four whole 256-byte key rows, and every K chunk of the block is issued before the first
// score (the fused variant stages K and V in LDS; the other issues its V chunks after the scores,
// so they fly during the softmax and K and V never share the registers): one or two memory
// latencies per block.
// Scores are summed over a key's 16 lanes by DPP; thread t owns key t for the softmax.
// The score and value loops skip the key groups past the row's keys: per group of four keys when
// every key of the launch falls in wave 0's range (FEW, the fused prompts of up to 64 rows), per
// wave otherwise (a per-group exit in the unrolled loops of the longer rows measured slower).
constexpr int SHORT_KEYS = 256;
// FUSED (prompts of up to FUSED_ROWS rows from position 0; FEW): the q/k head norms, RoPE and the
// f16 K/V store are folded in (k_qk_norm_rope, talker.hip:46-82). The block of row m forms, from
// the raw q|k|v rows of the projection (`raw`, [rows][nq + 2 nkv heads] f32), its two q heads and
// the normed, rotated f16 keys and the f16 values 0..m of kv group g in LDS, one wave per head row
// with the arithmetic of the EPI_QKV epilogue (rows.h: lane l holding dims l and l + 64, the values
// 0 + x), and it stores K/V row m into the cache; the attention then reads its keys and values from
// LDS instead of the cache.
constexpr int FUSED_ROWS = 64;
struct HeadNorm {
    const float *raw, *qn, *kn, *invf;
    float eps;
};
template <bool FEW, bool FUSED = false>
__global__ void __launch_bounds__(BT) k_attn_prefill_short(const float *q, uint16_t *kc, uint16_t *vc, int nq,
                                                           int nkv, int pos0, float scale, float *out, int ldo,
                                                           HeadNorm hn = {}) {
    constexpr int NWV = BT / WAVE, KW = SHORT_KEYS / NWV, KI = KW / 4;
    static_assert(SHORT_KEYS == BT, "one key per thread in the softmax");
    static_assert(FEW == FUSED && (!FUSED || FUSED_ROWS <= KW), "fused (the only FEW case): every key in wave 0's range");
    __shared__ float qs[2][HD], sc[2][SHORT_KEYS], red[2][NWV], opart[NWV][4][2][HD];
    __shared__ uint16_t ks[FUSED ? FUSED_ROWS : 1][HD], vs[FUSED ? FUSED_ROWS : 1][HD];
    // grid (kv groups, rows): blocks go out in row order from the last row (the most keys) down,
    // every kv group of a row together, so the blocks that wait for a free slot are the shortest;
    // and kv group g's blocks all land on XCD g (block id % 8), whose L2 then holds its keys
    const int m = static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y), g = blockIdx.x, n = pos0 + m + 1;
    const int QD = nq * HD, KVD = nkv * HD;
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, r = l >> 4;
    u32x4_t kr[KI], vr[KI];
    if constexpr (FUSED) {
        // task t: q head 2g + t of row m (t < 2), else key / value row j = t - 2 of kv group g
        const int W = QD + 2 * KVD;
        for (int t = wv; t < 2 + n; t += NWV) {
            const bool isq = t < 2;
            const int row = isq ? m : t - 2;
            const float *hp = hn.raw + static_cast<size_t>(row) * W + (isq ? (2 * g + t) * HD : QD + g * HD);
            const float *vp = hn.raw + static_cast<size_t>(row) * W + QD + KVD + g * HD;
            const float a0 = 0.f + gld(hp + l), a1 = 0.f + gld(hp + l + HD / 2);
            float b0 = 0.f, b1 = 0.f;
            if (!isq) {
                b0 = 0.f + gld(vp + l);
                b1 = 0.f + gld(vp + l + HD / 2);
            }
            float sn, cs;
            sincosf(static_cast<float>(row) * gld(hn.invf + l), &sn, &cs);
            const float *nw = isq ? hn.qn : hn.kn;
            const float scl = rsqrtf(wave_sum(fmaf(a0, a0, a1 * a1)) / static_cast<float>(HD) + hn.eps);
            const float x0 = a0 * scl * gld(nw + l), x1 = a1 * scl * gld(nw + l + HD / 2);
            const float y0 = x0 * cs - x1 * sn;
            const float y1 = x1 * cs + x0 * sn;
            if (isq) {
                qs[t][l] = y0;
                qs[t][l + HD / 2] = y1;
            } else {
                const uint16_t k0 = f2h(y0), k1 = f2h(y1), v0 = f2h(b0), v1 = f2h(b1);
                ks[row][l] = k0;
                ks[row][l + HD / 2] = k1;
                vs[row][l] = v0;
                vs[row][l + HD / 2] = v1;
                if (row == m) {
                    uint16_t *kd = kc + static_cast<size_t>(m) * KVD + g * HD, *vd = vc + static_cast<size_t>(m) * KVD + g * HD;
                    gst(kd + l, k0);
                    gst(kd + l + HD / 2, k1);
                    gst(vd + l, v0);
                    gst(vd + l + HD / 2, v1);
                }
            }
        }
        __syncthreads();                                  // qs, ks, vs
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int j = wv * KW + 4 * i + r;
            kr[i] = j < n ? *reinterpret_cast<const u32x4_t *>(&ks[j][c * 8]) : u32x4_t{0u, 0u, 0u, 0u};
            vr[i] = j < n ? *reinterpret_cast<const u32x4_t *>(&vs[j][c * 8]) : u32x4_t{0u, 0u, 0u, 0u};
        }
    } else {
        qs[threadIdx.x >> 7][threadIdx.x & (HD - 1)] = gld(q + static_cast<size_t>(m) * QD + g * 2 * HD + threadIdx.x);
        const uint16_t *kb = kc + g * HD + c * 8;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int j = wv * KW + 4 * i + r;
            kr[i] = j < n ? *(const NAVI_GLOBAL u32x4_t *) (kb + static_cast<size_t>(j) * KVD) : u32x4_t{0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();                                      // qs
    {
        float q0[8], q1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            q0[e] = qs[0][c * 8 + e];
            q1[e] = qs[1][c * 8 + e];
        }
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            if (wv * KW + (FEW ? 4 * i : 0) >= n) break;  // this wave's remaining keys are past the row's
            uint4 k4;
            __builtin_memcpy(&k4, &kr[i], 16);
            float a0 = dot8(k4, q0, 0.f), a1 = dot8(k4, q1, 0.f);
            a0 += dpp_red<0xB1>(a0);
            a1 += dpp_red<0xB1>(a1);
            a0 += dpp_red<0x4E>(a0);
            a1 += dpp_red<0x4E>(a1);
            a0 += dpp_red<0x141>(a0);
            a1 += dpp_red<0x141>(a1);
            a0 += dpp_red<0x140>(a0);
            a1 += dpp_red<0x140>(a1);
            if (c == 0) {
                const int j = wv * KW + 4 * i + r;
                sc[0][j] = a0 * scale;
                sc[1][j] = a1 * scale;
            }
        }
    }
    if constexpr (!FUSED) {
        // prompts of 65-256 rows: the V chunks go out after the scores and fly during the softmax,
        // so K and V are never in registers together (about 100 VGPRs instead of 156: four blocks
        // per CU instead of three; the sums are unchanged)
        const uint16_t *vb = vc + g * HD + c * 8;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int j = wv * KW + 4 * i + r;
            vr[i] = j < n ? *(const NAVI_GLOBAL u32x4_t *) (vb + static_cast<size_t>(j) * KVD) : u32x4_t{0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();
    const bool mine = static_cast<int>(threadIdx.x) < n;
    const float d0 = mine ? sc[0][threadIdx.x] : -INFINITY, d1 = mine ? sc[1][threadIdx.x] : -INFINITY;
    float mx0 = wave_max(d0), mx1 = wave_max(d1);
    if (l == 0) { red[0][wv] = mx0; red[1][wv] = mx1; }
    __syncthreads();
    mx0 = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    mx1 = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    const float e0 = mine ? expf(d0 - mx0) : 0.f, e1 = mine ? expf(d1 - mx1) : 0.f;
    sc[0][threadIdx.x] = e0;                              // 0 past the last key
    sc[1][threadIdx.x] = e1;
    const float s0 = wave_sum(e0), s1 = wave_sum(e1);
    __syncthreads();                                      // red reads done, probabilities published
    if (l == 0) { red[0][wv] = s0; red[1][wv] = s1; }
    {
        float o0[8], o1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o0[e] = o1[e] = 0.f;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            if (wv * KW + (FEW ? 4 * i : 0) >= n) break;  // zero weights (and zero rows) from here on
            const int j = wv * KW + 4 * i + r;
            const float p0 = sc[0][j], p1 = sc[1][j];
            half8_t hv;
            __builtin_memcpy(&hv, &vr[i], 16);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = static_cast<float>(hv[e]);
                o0[e] = fmaf(p0, v, o0[e]);
                o1[e] = fmaf(p1, v, o1[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            opart[wv][r][0][c * 8 + e] = o0[e];
            opart[wv][r][1][c * 8 + e] = o1[e];
        }
    }
    __syncthreads();
    const int hh = threadIdx.x >> 7, d = threadIdx.x & (HD - 1);
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; ++w)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) acc += opart[w][rr][hh][d];
    const float sum = red[hh][0] + red[hh][1] + red[hh][2] + red[hh][3];
    gst(out + rows::pk_a(m, (g * 2 + hh) * HD + d, ldo), acc / sum);
}

// Causal attention of prompts of more than 256 rows on the matrix cores: block (16-row tile qt,
// q head h) over keys 0..min(T, 16 qt + 16) - 1 of kv group h / (nq / nkv), in chunks of 256 keys
// with a running softmax. Per chunk: S = Q K^T on v_mfma_f32_16x16x32_f16 with q split into f16
// hi + lo (f32-level products of the f32 q and the f16 keys; wave w takes the chunk's key tiles w,
// w + 4, ...), scaled and causally masked into LDS; per row (16 lanes) the chunk's max m_c, the
// new running max m = max(m_run, m_c), corr = e^(m_run - m), p = e^(s - m) in place, l_run =
// l_run corr + sum p; the output rows scaled by corr, then O += P V with P split hi + lo against
// the chunk's V staged transposed in LDS ([dim][key] f16: one 16-byte read per B fragment), wave w
// taking dims 32w .. 32w + 31. Finally O / l_run to the tile layout of width ldo (rows.h pk_a).
// Key 0 is in the first chunk of every row, so m_run is finite from the first chunk on.
constexpr int LONG_CHUNK = 256;
__global__ void __launch_bounds__(BT) k_attn_prefill_long(const float *q, const uint16_t *kc, const uint16_t *vc, int nq,
                                                          int nkv, int T, float scale, float *out, int ldo) {
    constexpr int KT = LONG_CHUNK / 16 / 4;              // key tiles per wave per chunk
    constexpr int LDS_S = LONG_CHUNK + 4, LDV = LONG_CHUNK + 8;
    constexpr int VCH = LONG_CHUNK * (HD / 8) / BT;       // 16-byte V chunks per thread per chunk
    __shared__ float sS[16][LDS_S];
    __shared__ __align__(16) _Float16 vt[HD][LDV];
    __shared__ float mrun[16], lrun[16], corr[16];
    // grid (q heads, row tiles): tiles go out from the last (the most keys) down, every head of a
    // tile together
    const int qt = static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y), h = blockIdx.x, g = h / (nq / nkv),
              r0 = 16 * qt;
    const int QD = nq * HD, KVD = nkv * HD;
    const int nk = min(T, r0 + 16);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, kq = l >> 4;
    half8_t qh[4], ql[4];
    {
        const int row = min(r0 + c, T - 1);
        const float *qp = q + static_cast<size_t>(row) * QD + h * HD + 8 * kq;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const f32x4_t a0 = ld4(qp + 32 * st), a1 = ld4(qp + 32 * st + 4);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = j < 4 ? a0[j] : a1[j - 4];
                const _Float16 hv = static_cast<_Float16>(v);
                qh[st][j] = hv;
                ql[st][j] = static_cast<_Float16>(v - static_cast<float>(hv));
            }
        }
    }
    if (threadIdx.x < 16) {
        mrun[threadIdx.x] = -INFINITY;
        lrun[threadIdx.x] = 0.f;
    }
    f32x4_t o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (int k0 = 0; k0 < nk; k0 += LONG_CHUNK) {
        const int nkc = min(LONG_CHUNK, nk - k0), nkt = (nkc + 15) / 16, nks = (nkc + 31) / 32;
        // the chunk's K fragments and V rows, every load before the first MFMA
        u32x4_t kf[KT][4];
#pragma unroll
        for (int i = 0; i < KT; ++i) {
            const int kt = w + 4 * i, key = 16 * kt + c;
#pragma unroll
            for (int st = 0; st < 4; ++st)
                kf[i][st] = kt < nkt && key < nkc
                                ? *(const NAVI_GLOBAL u32x4_t *) (kc + static_cast<size_t>(k0 + key) * KVD + g * HD + 32 * st + 8 * kq)
                                : u32x4_t{0u, 0u, 0u, 0u};
        }
        u32x4_t vch[VCH];
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int e = static_cast<int>(threadIdx.x) + BT * i, key = e / (HD / 8), d8 = e % (HD / 8);
            vch[i] = key < nkc ? *(const NAVI_GLOBAL u32x4_t *) (vc + static_cast<size_t>(k0 + key) * KVD + g * HD + 8 * d8)
                               : u32x4_t{0u, 0u, 0u, 0u};
        }
        __syncthreads();                                  // the previous chunk's readers of sS, vt are done
#pragma unroll
        for (int i = 0; i < KT; ++i) {
            const int kt = w + 4 * i;
            if (kt >= nkt) break;
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                half8_t b;
                __builtin_memcpy(&b, &kf[i][st], 16);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[st], b, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[st], b, acc, 0, 0, 0);
            }
            const int key = 16 * kt + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * kq + r;
                sS[row][key] = key < nkc && k0 + key <= r0 + row ? acc[r] * scale : -INFINITY;
            }
        }
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int e = static_cast<int>(threadIdx.x) + BT * i, key = e / (HD / 8), d8 = e % (HD / 8);
            if (key < 32 * nks) {
                half8_t hv;
                __builtin_memcpy(&hv, &vch[i], 16);
#pragma unroll
                for (int j = 0; j < 8; ++j) vt[8 * d8 + j][key] = hv[j];
            }
        }
        __syncthreads();
        {
            // row threadIdx / 16, its 16 lanes take keys lane % 16 + 16 m of the chunk
            const int row = threadIdx.x >> 4, j0 = threadIdx.x & 15;
            float mc = -INFINITY;
            for (int j = j0; j < 32 * nks; j += 16) mc = fmaxf(mc, j < nkt * 16 ? sS[row][j] : -INFINITY);
            mc = fmaxf(mc, dpp_red<0xB1>(mc));
            mc = fmaxf(mc, dpp_red<0x4E>(mc));
            mc = fmaxf(mc, dpp_red<0x141>(mc));
            mc = fmaxf(mc, dpp_red<0x140>(mc));
            const float mo = mrun[row], m = fmaxf(mo, mc), cr = expf(mo - m);
            float sum = 0.f;
            for (int j = j0; j < 32 * nks; j += 16) {
                const float e = j < nkt * 16 ? expf(sS[row][j] - m) : 0.f;   // masked: e^-inf = 0
                sS[row][j] = e;
                sum += e;
            }
            sum += dpp_red<0xB1>(sum);
            sum += dpp_red<0x4E>(sum);
            sum += dpp_red<0x141>(sum);
            sum += dpp_red<0x140>(sum);
            __syncthreads();                              // every lane of the row has read mrun[row]
            if (j0 == 0) {
                mrun[row] = m;
                lrun[row] = lrun[row] * cr + sum;
                corr[row] = cr;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[u][r] *= corr[4 * kq + r];
        for (int t = 0; t < nks; ++t) {
            half8_t ph, pl;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = sS[c][32 * t + 8 * kq + j];
                const _Float16 hv = static_cast<_Float16>(v);
                ph[j] = hv;
                pl[j] = static_cast<_Float16>(v - static_cast<float>(hv));
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const half8_t b = *reinterpret_cast<const half8_t *>(&vt[32 * w + 16 * u + c][32 * t + 8 * kq]);
                o[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, b, o[u], 0, 0, 0);
                o[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, b, o[u], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * kq + r;
            if (r0 + row < T) gst(out + rows::pk_a(r0 + row, h * HD + 32 * w + 16 * u + c, ldo), o[u][r] / lrun[row]);
        }
}

// rows[t] = table[ids[t]] (f16 -> f32), k_gather_rows (talker.hip:20-25).
__global__ void __launch_bounds__(BT) k_gather_rows(const uint16_t *table, const int32_t *ids, int width, float *out) {
    const uint16_t *src = table + static_cast<size_t>(gld(ids + blockIdx.x)) * width;
    float *dst = out + static_cast<size_t>(blockIdx.x) * width;
    for (int i = threadIdx.x; i < width; i += BT) gst(dst + i, h2f(gld(src + i)));
}

// out[t] = A[ia[t]] + B[ib[t]] (+ spk on spk_row), entries < 0 absent, k_assemble_rows (talker.hip:27-41).
__global__ void __launch_bounds__(BT) k_assemble_rows(const float *A, const float *B, const float *spk, const int32_t *ia,
                                                      const int32_t *ib, int spk_row, int width, float *out) {
    const int t = blockIdx.x, a_i = gld(ia + t), b_i = gld(ib + t);
    for (int i = threadIdx.x; i < width; i += BT) {
        float v = 0.f;
        if (a_i >= 0) v += gld(A + static_cast<size_t>(a_i) * width + i);
        if (b_i >= 0) v += gld(B + static_cast<size_t>(b_i) * width + i);
        if (t == spk_row) v += gld(spk + i);
        gst(out + static_cast<size_t>(t) * width + i, v);
    }
}

// ---- host: the split-K linear ------------------------------------------------------------

int tiles_m(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : M <= 48 ? 3 : 4; }

// Number of K splits: enough blocks to cover the 256 CUs (at most 384), each split at least 256
// deep (a block's weight stream and staging amortise its fixed cost), K / S a multiple of 32.
int pick_splits(int M, int K, int N) {
    const int mt = tiles_m(M);
    const int blocks = (N / 64) * ((M + 16 * mt - 1) / (16 * mt));
    int s = 1;
    while (s * 2 * blocks <= 384 && (K / 32) % (s * 2) == 0 && K / (s * 2) >= 256) s *= 2;
    return s;
}

size_t splits_floats(int M, int K, int N) { return static_cast<size_t>(pick_splits(M, K, N)) * M * N; }

void launch_partial3(const float *x, int ldx, int M, const uint16_t *w0, int n0, const uint16_t *w1, int n1, const uint16_t *w2,
                     int n2, int K, int S, float *part, int ldp, int p_off, uint32_t *flag, hipStream_t st) {
    const int N = n0 + n1 + n2;
    LinArgs a{x, w0, w1, w2, part, flag, ldx, M, K, N, K / S, ldp, p_off, n0, n0 + n1};
    const int mt = tiles_m(M);
    const dim3 grid(N / 64, (M + 16 * mt - 1) / (16 * mt), S);
    switch (mt) {
    case 1: hipLaunchKernelGGL(k_linear_partial<1>, grid, dim3(BT), 0, st, a); break;
    case 2: hipLaunchKernelGGL(k_linear_partial<2>, grid, dim3(BT), 0, st, a); break;
    case 3: hipLaunchKernelGGL(k_linear_partial<3>, grid, dim3(BT), 0, st, a); break;
    default: hipLaunchKernelGGL(k_linear_partial<4>, grid, dim3(BT), 0, st, a); break;
    }
}

void launch_partial(const float *x, int ldx, int M, const uint16_t *w, int K, int N, int S, float *part, int ldp, int p_off,
                    uint32_t *flag, hipStream_t st) {
    launch_partial3(x, ldx, M, w, N, nullptr, 0, nullptr, 0, K, S, part, ldp, p_off, flag, st);
}

void launch_resid_norm(const float *part, int S, const float *src, float *x, const float *w, float eps, float *xn, int M,
                       int H, hipStream_t st) {
    hipLaunchKernelGGL(k_resid_norm, dim3(M), dim3(BT), 0, st, part, S, src, x, w, eps, xn, M, H);
}

void launch_swiglu(const float *part, int S, int M, int F, float *h, hipStream_t st) {
    hipLaunchKernelGGL(k_swiglu, dim3(M), dim3(BT), 0, st, part, S, M, F, h);
}

void launch_finish_linear(const float *part, int S, int M, int N, const float *bias, const float *residual, int act, float *y,
                          int ldy, hipStream_t st) {
    hipLaunchKernelGGL(k_finish_linear, dim3(M), dim3(BT), 0, st, part, S, M, N, bias, residual, act, y, ldy);
}

bool linear_shape_ok(const float *x, int ldx, int M, const uint16_t *w, int K, int N) {
    return M > 0 && K > 0 && N > 0 && K % 32 == 0 && N % 64 == 0 && ldx % 4 == 0 && ldx >= K &&
           (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
}

// Library workspace for navi_linear (grown on demand; entry points run on one host thread).
struct LinearWs {
    float *part = nullptr;
    size_t floats = 0;
    uint32_t *flag = nullptr;
} g_ws;

// navi_linear_noalloc's fixed workspace: bytes [0, 256) hold the f16-range flag, the rest the
// split-K partials. Each GPU the library runs on holds its own copy until the process ends.
constexpr size_t SCRATCH_BYTES = size_t(8) << 20;
constexpr size_t SCRATCH_FLAG_BYTES = 256;
constexpr size_t SCRATCH_FLOATS = (SCRATCH_BYTES - SCRATCH_FLAG_BYTES) / sizeof(float);
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

// Device address of `scratch` per device (the array's name in host code is only a stand-in).
constexpr int MAX_DEVICES = 64;
void *g_scratch_dev[MAX_DEVICES] = {};

__global__ void k_clear_word(uint32_t *w) {
    if (threadIdx.x == 0) gst(w, 0u);
}

struct LayerW {
    const float *ln1, *ln2, *qn, *kn;
    const uint16_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    uint16_t *qkv_t, *o_t, *gu_t, *d_t;   // the tiled copies: [q; k; v], o, [gate; up], down
};

// xn = RMSNorm(row m of the tiled residual stream x) * w: k_resid_norm's arithmetic for one row
// (thread i holds elements 4i .. 4i + 3, the same sum order), reading x in the tile layout.
__global__ void __launch_bounds__(BT) k_tiled_row_norm(const float *x, int m, const float *w, float eps, float *xn, int H,
                                                       float *xn2) {
    __shared__ float red[4];
    const int i = threadIdx.x * 4;                            // H == 4 * BT
    const f32x4_t v = ld4(x + rows::pk_a(m, i, H));
    const f32x4_t wv = ld4(w + i);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) ss = fmaf(v[j], v[j], ss);
    ss = block_sum256(ss, red);
    const float scale = rsqrtf(ss / static_cast<float>(H) + eps);
    f32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = v[j] * scale * wv[j];
    st4(xn + i, o);
    if (xn2) st4(xn2 + i, o);
}

} // namespace pf
} // namespace navi_amd

using namespace navi_amd;
using namespace navi_amd::pf;

struct navi_talker {
    // shapes
    int H = 0, NQ = 0, NKV = 0, QD = 0, KVD = 0, F = 0, V = 0, L = 0, TH = 0, TV = 0;
    float eps = 0.f;
    int max_prompt = 0, max_pos = 0, mmax = 0;
    int tts_bos = 0, tts_eos = 0, tts_pad = 0, codec_bos = 0, codec_pad = 0, think = 0, nothink = 0, think_bos = 0,
        think_eos = 0, codec_vocab = 0;
    // weights
    const uint16_t *text_emb = nullptr, *codec_emb = nullptr, *fc1 = nullptr, *fc2 = nullptr, *head = nullptr;
    const float *fc1_b = nullptr, *fc2_b = nullptr, *final_norm = nullptr;
    std::vector<LayerW> layers;
    uint16_t *tiled = nullptr;         // every layer's tiled weight copies, one allocation
    // cache
    std::vector<uint16_t *> kk, vv;
    int n_used = 0;
    // work buffers
    // x (the residual stream), att and h in the tile layout (rows.h pk_a), the rest row-major
    float *x = nullptr, *xn = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *part = nullptr, *invf = nullptr;
    size_t part_floats = 0;
    uint32_t *flag = nullptr;
    uint32_t *h_flag = nullptr;        // pinned host copy of flag, read back with the call's last sync
    int32_t *d_ids = nullptr, *d_cids = nullptr, *d_ia = nullptr, *d_ib = nullptr, *d_ta = nullptr, *d_tb = nullptr;
    float *text_rows = nullptr, *fc1_out = nullptr, *proj = nullptr, *codec_rows = nullptr, *spk = nullptr;
    float *prefill = nullptr, *trailing = nullptr, *pad_row = nullptr, *hidden = nullptr, *logits = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    double last_ms = 0;
    // each row count's layer launches captured once as a HIP graph and replayed
    std::vector<std::pair<int, hipGraphExec_t>> graphs;
    bool use_graphs = false;           // off by default: replays measured no faster than launches
    std::vector<void *> owned;

    template <class T>
    navi_status alloc(T *&p, size_t n, char *err, size_t errlen) {
        void *ptr = nullptr;
        NAVI_TRY_HIP(hipMalloc(&ptr, std::max<size_t>(n, 1) * sizeof(T)), err, errlen);
        owned.push_back(ptr);
        NAVI_TRY_HIP(hipMemsetAsync(ptr, 0, std::max<size_t>(n, 1) * sizeof(T), device_state().stream), err, errlen);
        p = static_cast<T *>(ptr);
        return NAVI_OK;
    }

    ~navi_talker() {
        for (auto &g : graphs) (void) hipGraphExecDestroy(g.second);
        if (ev0) (void) hipEventDestroy(ev0);
        if (ev1) (void) hipEventDestroy(ev1);
        if (h_flag) (void) hipHostFree(h_flag);
        for (void *p : owned) (void) hipFree(p);
    }
};

namespace {

#define TALKER_BIND(T, name, dt, d0, d1, out)                                                                   \
    do {                                                                                                        \
        const navi_status s_ = bind_tensor<T>("talker", tensors, n_tensors, (name), (dt), (d0), (d1), (out), err, errlen); \
        if (s_ != NAVI_OK) return s_;                                                                           \
    } while (0)

navi_status talker_bind(navi_talker &t, const navi_tensor_ref *tensors, int n_tensors, char *err, size_t errlen) {
    TALKER_BIND(uint16_t, "talker.model.text_embedding.weight", NAVI_DT_F16, t.TV, t.TH, t.text_emb);
    TALKER_BIND(uint16_t, "talker.model.codec_embedding.weight", NAVI_DT_F16, t.codec_vocab, t.H, t.codec_emb);
    TALKER_BIND(uint16_t, "talker.text_projection.linear_fc1.weight", NAVI_DT_F16, t.TH, t.TH, t.fc1);
    TALKER_BIND(float, "talker.text_projection.linear_fc1.bias", NAVI_DT_F32, t.TH, 0, t.fc1_b);
    TALKER_BIND(uint16_t, "talker.text_projection.linear_fc2.weight", NAVI_DT_F16, t.H, t.TH, t.fc2);
    TALKER_BIND(float, "talker.text_projection.linear_fc2.bias", NAVI_DT_F32, t.H, 0, t.fc2_b);
    TALKER_BIND(uint16_t, "talker.codec_head.weight", NAVI_DT_F16, t.V, t.H, t.head);
    TALKER_BIND(float, "talker.model.norm.weight", NAVI_DT_F32, t.H, 0, t.final_norm);
    t.layers.resize(t.L);
    for (int l = 0; l < t.L; ++l) {
        const std::string p = "talker.model.layers." + std::to_string(l) + ".";
        LayerW &w = t.layers[l];
        TALKER_BIND(float, p + "input_layernorm.weight", NAVI_DT_F32, t.H, 0, w.ln1);
        TALKER_BIND(float, p + "post_attention_layernorm.weight", NAVI_DT_F32, t.H, 0, w.ln2);
        TALKER_BIND(float, p + "self_attn.q_norm.weight", NAVI_DT_F32, HD, 0, w.qn);
        TALKER_BIND(float, p + "self_attn.k_norm.weight", NAVI_DT_F32, HD, 0, w.kn);
        TALKER_BIND(uint16_t, p + "self_attn.q_proj.weight", NAVI_DT_F16, t.QD, t.H, w.wq);
        TALKER_BIND(uint16_t, p + "self_attn.k_proj.weight", NAVI_DT_F16, t.KVD, t.H, w.wk);
        TALKER_BIND(uint16_t, p + "self_attn.v_proj.weight", NAVI_DT_F16, t.KVD, t.H, w.wv);
        TALKER_BIND(uint16_t, p + "self_attn.o_proj.weight", NAVI_DT_F16, t.H, t.QD, w.wo);
        TALKER_BIND(uint16_t, p + "mlp.gate_proj.weight", NAVI_DT_F16, t.F, t.H, w.wg);
        TALKER_BIND(uint16_t, p + "mlp.up_proj.weight", NAVI_DT_F16, t.F, t.H, w.wu);
        TALKER_BIND(uint16_t, p + "mlp.down_proj.weight", NAVI_DT_F16, t.H, t.F, w.wd);
    }
    return NAVI_OK;
}

// The most partial floats any projection of a prefill (or prompt) of up to M rows needs.
size_t talker_part_floats(const navi_talker &t) {
    size_t best = 0;
    const int shapes[][2] = {{t.H, t.QD + 2 * t.KVD}, {t.QD, t.H}, {t.H, 2 * t.F}, {t.F, t.H}, {t.H, t.V},
                             {t.TH, t.TH}, {t.TH, t.H}};
    for (int M = 1; M <= t.mmax; ++M)
        for (const auto &s : shapes) {
            // q/k/v and gate/up are split as one [q|k|v] / [gate|up] output
            best = std::max(best, splits_floats(M, s[0], s[1]));
        }
    return best;
}

// The f16-range flag as the stream's last copy left it in the pinned host word.
navi_status flag_result(const navi_talker &t, const char *what, char *err, size_t errlen) {
    if (*t.h_flag) {
        set_err(err, errlen, "talker: %s: an activation is outside the f16 range (|x| >= 65504 or NaN)", what);
        return NAVI_ERR_INVALID;
    }
    return NAVI_OK;
}

// The f16-range flag of the work enqueued so far: copied into the pinned host word on the stream
// and read after one synchronization.
navi_status check_flag(navi_talker &t, const char *what, char *err, size_t errlen) {
    NAVI_TRY_HIP(hipMemcpyAsync(t.h_flag, t.flag, 4, hipMemcpyDeviceToHost, device_state().stream), err, errlen);
    NAVI_TRY_HIP(hipStreamSynchronize(device_state().stream), err, errlen);
    return flag_result(t, what, err, errlen);
}

} // namespace

extern "C" {

navi_status navi_talker_create(const navi_model_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                               int32_t max_prompt_tokens, int32_t max_positions, navi_talker **out, char *err,
                               size_t errlen) {
    if (!p || !tensors || !out) {
        set_err(err, errlen, "talker: null argument");
        return NAVI_ERR_INVALID;
    }
    *out = nullptr;
    navi_status st = ensure_device(err, errlen);
    if (st != NAVI_OK) return st;
    const navi_xformer_params &x = p->talker;
    // the prefill's row projections are built for hidden 1024, 16 q heads (K = 2048 into o) and
    // ff 3072 (K = 3072 into down): the 0.6B talker
    if (x.head_dim != HD || x.n_head != 2 * x.n_kv_head || x.n_head != 16 || x.ff != 3072 || x.vocab % 64 != 0 ||
        p->text_hidden % 64 != 0 || x.hidden != 1024) {
        set_err(err, errlen, "talker: unsupported shape (hidden %d, head_dim %d, ff %d, vocab %d, text_hidden %d)", x.hidden,
                x.head_dim, x.ff, x.vocab, p->text_hidden);
        return NAVI_ERR_UNSUPPORTED;
    }
    if (max_prompt_tokens < 9 || max_prompt_tokens > 4096 || max_positions < max_prompt_tokens) {
        set_err(err, errlen, "talker: max_prompt_tokens %d / max_positions %d out of range", max_prompt_tokens, max_positions);
        return NAVI_ERR_INVALID;
    }
    auto t = new navi_talker();
    t->H = x.hidden; t->NQ = x.n_head; t->NKV = x.n_kv_head; t->QD = x.n_head * HD; t->KVD = x.n_kv_head * HD;
    t->F = x.ff; t->V = x.vocab; t->L = x.n_layer; t->TH = p->text_hidden; t->TV = p->text_vocab; t->eps = x.rms_eps;
    t->codec_vocab = x.vocab;
    t->max_prompt = max_prompt_tokens; t->max_pos = max_positions; t->mmax = max_prompt_tokens + 8;
    t->tts_bos = p->tts_bos_id; t->tts_eos = p->tts_eos_id; t->tts_pad = p->tts_pad_id;
    t->codec_bos = p->codec_bos_id; t->codec_pad = p->codec_pad_id; t->think = p->codec_think_id;
    t->nothink = p->codec_nothink_id; t->think_bos = p->codec_think_bos_id; t->think_eos = p->codec_think_eos_id;
    auto fail = [&](navi_status s) { delete t; return s; };
    if ((st = talker_bind(*t, tensors, n_tensors, err, errlen)) != NAVI_OK) return fail(st);
    const size_t M = t->mmax;
    t->kk.resize(t->L);
    t->vv.resize(t->L);
    for (int l = 0; l < t->L; ++l) {
        if ((st = t->alloc(t->kk[l], static_cast<size_t>(max_positions) * t->KVD, err, errlen)) != NAVI_OK) return fail(st);
        if ((st = t->alloc(t->vv[l], static_cast<size_t>(max_positions) * t->KVD, err, errlen)) != NAVI_OK) return fail(st);
    }
    t->part_floats = talker_part_floats(*t);
#define TALLOC(ptr, n)                                                           \
    do {                                                                         \
        if ((st = t->alloc(ptr, (n), err, errlen)) != NAVI_OK) return fail(st);  \
    } while (0)
    const size_t MT16 = (M + 15) / 16 * 16;     // x, att and h (tile layout) hold whole 16-row tiles
    TALLOC(t->x, MT16 * t->H);
    TALLOC(t->xn, M * t->H);
    TALLOC(t->q, M * t->QD);
    TALLOC(t->att, MT16 * t->QD);
    TALLOC(t->h, MT16 * t->F);
    const size_t per_layer = static_cast<size_t>(t->QD + 2 * t->KVD) * t->H + static_cast<size_t>(t->H) * t->QD +
                             static_cast<size_t>(2 * t->F) * t->H + static_cast<size_t>(t->H) * t->F;
    TALLOC(t->tiled, per_layer * t->L);
    TALLOC(t->part, t->part_floats);
    TALLOC(t->invf, HD / 2);
    TALLOC(t->flag, 1);
    TALLOC(t->d_ids, M);
    TALLOC(t->d_cids, 16);
    TALLOC(t->d_ia, M);
    TALLOC(t->d_ib, M);
    TALLOC(t->d_ta, M);
    TALLOC(t->d_tb, M);
    TALLOC(t->text_rows, M * t->TH);
    TALLOC(t->fc1_out, M * t->TH);
    TALLOC(t->proj, M * t->H);
    TALLOC(t->codec_rows, 16 * t->H);
    TALLOC(t->spk, t->H);
    TALLOC(t->prefill, M * t->H);
    TALLOC(t->trailing, M * t->H);
    TALLOC(t->pad_row, t->H);
    TALLOC(t->hidden, t->H);
    TALLOC(t->logits, t->V);
#undef TALLOC
    float invf[HD / 2];
    for (int i = 0; i < HD / 2; ++i) invf[i] = static_cast<float>(1.0 / std::pow(x.rope_theta, (2.0 * i) / HD));
    hipStream_t s = device_state().stream;
    {
        // the tiled copies of the layer weights the prefill's projections read
        auto tile = [&](const uint16_t *src, int n, int K, uint16_t *dst) { rows::tile_weights(src, n, K, dst, s); };
        uint16_t *p = t->tiled;
        const size_t q_el = static_cast<size_t>(t->QD) * t->H, kv_el = static_cast<size_t>(t->KVD) * t->H,
                     f_el = static_cast<size_t>(t->F) * t->H;
        for (LayerW &w : t->layers) {
            w.qkv_t = p;
            tile(w.wq, t->QD, t->H, p);
            tile(w.wk, t->KVD, t->H, p + q_el);
            tile(w.wv, t->KVD, t->H, p + q_el + kv_el);
            p += q_el + 2 * kv_el;
            w.o_t = p;
            tile(w.wo, t->H, t->QD, p);
            p += static_cast<size_t>(t->H) * t->QD;
            w.gu_t = p;
            tile(w.wg, t->F, t->H, p);
            tile(w.wu, t->F, t->H, p + f_el);
            p += 2 * f_el;
            w.d_t = p;
            tile(w.wd, t->H, t->F, p);
            p += static_cast<size_t>(t->H) * t->F;
        }
    }
    if (hipMemcpyAsync(t->invf, invf, sizeof invf, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipEventCreate(&t->ev0) != hipSuccess || hipEventCreate(&t->ev1) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void **>(&t->h_flag), 64, hipHostMallocDefault) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        set_err(err, errlen, "talker: HIP setup failed");
        return fail(NAVI_ERR_HIP);
    }
    *out = t;
    return NAVI_OK;
}

void navi_talker_destroy(navi_talker *t) {
    if (!t) return;
    (void) hipStreamSynchronize(device_state().stream);
    delete t;
}

navi_status navi_talker_build_prompt(navi_talker *t, const int32_t *ids, int32_t n_ids, int32_t language_id,
                                     const float *speaker, navi_prompt *out, char *err, size_t errlen) {
    if (!t || !ids || !speaker || !out) {
        set_err(err, errlen, "talker: null argument");
        return NAVI_ERR_INVALID;
    }
    if (n_ids < 9) {
        set_err(err, errlen, "talker: prompt ids too short (need role header, text, and the trailer)");
        return NAVI_ERR_INVALID;
    }
    if (n_ids > t->max_prompt) {
        set_err(err, errlen, "talker: prompt longer than max_prompt_tokens");
        return NAVI_ERR_INVALID;
    }
    for (int i = 0; i < n_ids; ++i)
        if (ids[i] < 0 || ids[i] >= t->TV) {
            set_err(err, errlen, "talker: token id %d at %d outside the text vocabulary", ids[i], i);
            return NAVI_ERR_INVALID;
        }
    if (language_id >= t->codec_vocab) {
        set_err(err, errlen, "talker: language id %d outside the codec vocabulary", language_id);
        return NAVI_ERR_INVALID;
    }
    const int n_text = n_ids - 8;
    // rows to project: role header (3), text ids[3:3+n_text], tts_bos, tts_eos, tts_pad
    std::vector<int32_t> tids(ids, ids + 3 + n_text);
    const int i_bos = static_cast<int>(tids.size());
    tids.push_back(t->tts_bos);
    const int i_eos = static_cast<int>(tids.size());
    tids.push_back(t->tts_eos);
    const int i_pad = static_cast<int>(tids.size());
    tids.push_back(t->tts_pad);
    const int n_rows = static_cast<int>(tids.size());
    std::vector<int32_t> cids;
    if (language_id < 0) cids = {t->nothink, t->think_bos, t->think_eos};
    else cids = {t->think, t->think_bos, language_id, t->think_eos};
    const int n_think = static_cast<int>(cids.size());
    cids.push_back(t->codec_pad);
    cids.push_back(t->codec_bos);
    for (int32_t c : cids)
        if (c < 0 || c >= t->codec_vocab) {
            set_err(err, errlen, "talker: codec control id %d outside the codec vocabulary", c);
            return NAVI_ERR_INVALID;
        }
    // prefill: role rows, think rows (+ tts_pad), speaker (+ tts_pad), tts_bos + codec_pad, text[0] + codec_bos
    std::vector<int32_t> ia, ib;
    for (int r = 0; r < 3; ++r) { ia.push_back(r); ib.push_back(-1); }
    for (int r = 0; r < n_think; ++r) { ia.push_back(i_pad); ib.push_back(r); }
    const int spk_row = static_cast<int>(ia.size());
    ia.push_back(i_pad); ib.push_back(-1);
    ia.push_back(i_bos); ib.push_back(n_think);
    ia.push_back(3); ib.push_back(n_think + 1);
    // trailing: text[1:] then tts_eos
    std::vector<int32_t> ta, tb;
    for (int r = 1; r < n_text; ++r) { ta.push_back(3 + r); tb.push_back(-1); }
    ta.push_back(i_eos); tb.push_back(-1);
    const int n_pre = static_cast<int>(ia.size()), n_trail = static_cast<int>(ta.size());

    hipStream_t s = device_state().stream;
    NAVI_TRY_HIP(hipMemsetAsync(t->flag, 0, 4, s), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(t->d_ids, tids.data(), tids.size() * 4, hipMemcpyHostToDevice, s), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(t->d_cids, cids.data(), cids.size() * 4, hipMemcpyHostToDevice, s), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(t->spk, speaker, t->H * 4, hipMemcpyHostToDevice, s), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(t->d_ia, ia.data(), ia.size() * 4, hipMemcpyHostToDevice, s), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(t->d_ib, ib.data(), ib.size() * 4, hipMemcpyHostToDevice, s), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(t->d_ta, ta.data(), ta.size() * 4, hipMemcpyHostToDevice, s), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(t->d_tb, tb.data(), tb.size() * 4, hipMemcpyHostToDevice, s), err, errlen);
    hipLaunchKernelGGL(k_gather_rows, dim3(n_rows), dim3(BT), 0, s, t->text_emb, t->d_ids, t->TH, t->text_rows);
    int S = pick_splits(n_rows, t->TH, t->TH);
    launch_partial(t->text_rows, t->TH, n_rows, t->fc1, t->TH, t->TH, S, t->part, t->TH, 0, t->flag, s);
    hipLaunchKernelGGL(k_finish_linear, dim3(n_rows), dim3(BT), 0, s, t->part, S, n_rows, t->TH, t->fc1_b, nullptr, 1,
                       t->fc1_out, t->TH);
    S = pick_splits(n_rows, t->TH, t->H);
    launch_partial(t->fc1_out, t->TH, n_rows, t->fc2, t->TH, t->H, S, t->part, t->H, 0, t->flag, s);
    hipLaunchKernelGGL(k_finish_linear, dim3(n_rows), dim3(BT), 0, s, t->part, S, n_rows, t->H, t->fc2_b, nullptr, 0,
                       t->proj, t->H);
    hipLaunchKernelGGL(k_gather_rows, dim3(static_cast<unsigned>(cids.size())), dim3(BT), 0, s, t->codec_emb, t->d_cids,
                       t->H, t->codec_rows);
    hipLaunchKernelGGL(k_assemble_rows, dim3(n_pre), dim3(BT), 0, s, t->proj, t->codec_rows, t->spk, t->d_ia, t->d_ib,
                       spk_row, t->H, t->prefill);
    hipLaunchKernelGGL(k_assemble_rows, dim3(n_trail), dim3(BT), 0, s, t->proj, t->codec_rows, t->spk, t->d_ta, t->d_tb,
                       -1, t->H, t->trailing);
    NAVI_TRY_HIP(hipMemcpyAsync(t->pad_row, t->proj + static_cast<size_t>(i_pad) * t->H, t->H * 4,
                                hipMemcpyDeviceToDevice, s), err, errlen);
    NAVI_TRY_HIP(hipGetLastError(), err, errlen);
    const navi_status st = check_flag(*t, "build_prompt", err, errlen);
    if (st != NAVI_OK) return st;
    out->prefill = t->prefill;
    out->trailing = t->trailing;
    out->tts_pad = t->pad_row;
    out->n_prefill = n_pre;
    out->n_trailing = n_trail;
    return NAVI_OK;
}

} // extern "C"

namespace {

// The prefill's kernels for T rows already in t.x (tile layout): five launches per layer (q|k|v
// with the RMSNorm fused, and above 64 rows the q/k norms + RoPE + K/V store in its epilogue ->
// attention (up to 64 rows with the norms, RoPE and K/V store) -> o (+ residual) -> gate|up with
// the RMSNorm and SwiGLU fused -> down (+ residual); every projection one whole-K MFMA kernel on
// the tiled operands, rows.h), then the last row's final RMSNorm (the post-norm hidden the frame
// takes) and the codec head. false: a projection shape the tiled kernels do not take (nothing
// after it was launched).
bool prefill_layers(navi_talker &t, int T, hipStream_t s) {
    const int H = t.H, QKVW = t.QD + 2 * t.KVD;
    const float scale = 1.f / std::sqrt(static_cast<float>(HD));
    for (int l = 0; l < t.L; ++l) {
        const LayerW &w = t.layers[l];
        if (T <= FUSED_ROWS) {         // the q/k norms, RoPE and K/V store inside the attention
            if (!rows::launch_rows_pk(rows::EPI_PLAIN, true, t.x, T, H, w.ln1, t.eps, w.qkv_t, QKVW, t.part, QKVW, t.flag, s))
                return false;
            hipLaunchKernelGGL((k_attn_prefill_short<true, true>), dim3(t.NKV, T), dim3(BT), 0, s, nullptr, t.kk[l],
                               t.vv[l], t.NQ, t.NKV, 0, scale, t.att, t.QD, HeadNorm{t.part, w.qn, w.kn, t.invf, t.eps});
        } else {                       // ... or in the q|k|v projection's epilogue
            const rows::HeadOut ho{w.qn, w.kn, t.invf, t.q, t.kk[l], t.vv[l], t.NQ, t.NKV, 0};
            if (!rows::launch_rows_pk(rows::EPI_QKV, true, t.x, T, H, w.ln1, t.eps, w.qkv_t, QKVW, nullptr, 0, t.flag, s, ho))
                return false;
            if (T <= SHORT_KEYS)
                hipLaunchKernelGGL(k_attn_prefill_short<false>, dim3(t.NKV, T), dim3(BT), 0, s, t.q, t.kk[l], t.vv[l], t.NQ,
                                   t.NKV, 0, scale, t.att, t.QD, HeadNorm{});
            else
                hipLaunchKernelGGL(k_attn_prefill_long, dim3(t.NQ, (T + 15) / 16), dim3(BT), 0, s, t.q, t.kk[l], t.vv[l],
                                   t.NQ, t.NKV, T, scale, t.att, t.QD);
        }
        if (!rows::launch_rows_pk(rows::EPI_RESID, false, t.att, T, t.QD, nullptr, 0.f, w.o_t, H, t.x, 0, t.flag, s) ||
            !rows::launch_rows_pk(rows::EPI_SWIGLU, true, t.x, T, H, w.ln2, t.eps, w.gu_t, t.F, t.h, 0, t.flag, s) ||
            !rows::launch_rows_pk(rows::EPI_RESID, false, t.h, T, t.F, nullptr, 0.f, w.d_t, H, t.x, 0, t.flag, s))
            return false;
    }
    // the last row: final RMSNorm (the post-norm hidden the frame takes), then the codec head
    float *last = t.xn + static_cast<size_t>(T - 1) * H;
    hipLaunchKernelGGL(k_tiled_row_norm, dim3(1), dim3(BT), 0, s, t.x, T - 1, t.final_norm, t.eps, last, H, t.hidden);
    rows::launch_rows(rows::EPI_PLAIN, false, last, H, 1, H, nullptr, 0.f, t.head, t.V, nullptr, 0, nullptr, 0, t.logits, t.V,
                      t.flag, s);
    return true;
}

} // namespace

extern "C" {

navi_status navi_talker_prefill(navi_talker *t, const float *d_rows, int32_t n_rows, char *err, size_t errlen) {
    if (!t || !d_rows) {
        set_err(err, errlen, "talker: null argument");
        return NAVI_ERR_INVALID;
    }
    if (n_rows < 1 || n_rows > t->mmax || n_rows > t->max_pos) {
        set_err(err, errlen, "talker: prefill of %d rows exceeds the prompt buffers or the KV cache", n_rows);
        return NAVI_ERR_INVALID;
    }
    const int T = n_rows, H = t->H;
    hipStream_t s = device_state().stream;
    NAVI_TRY_HIP(hipEventRecord(t->ev0, s), err, errlen);
    rows::tile_rows(d_rows, T, H, t->x, s, t->flag);       // also clears the f16-range flag
    // The layers and the head: a launch sequence that depends only on T (every buffer is the
    // handle's), so it can be captured once per row count as a HIP graph and replayed
    // (navi_talker_set_graphs; off by default, measured no faster than host launches).
    if (t->use_graphs) {
        hipGraphExec_t ex = nullptr;
        for (auto &g : t->graphs)
            if (g.first == T) ex = g.second;
        if (!ex) {
            NAVI_TRY_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), err, errlen);
            const bool ok = prefill_layers(*t, T, s);
            hipGraph_t graph = nullptr;
            NAVI_TRY_HIP(hipStreamEndCapture(s, &graph), err, errlen);
            if (!ok) {
                (void) hipGraphDestroy(graph);
                set_err(err, errlen, "talker: a projection shape the prefill's tiled kernels do not take");
                return NAVI_ERR_UNSUPPORTED;
            }
            const hipError_t ei = hipGraphInstantiateWithFlags(&ex, graph, 0);
            (void) hipGraphDestroy(graph);
            NAVI_TRY_HIP(ei, err, errlen);
            t->graphs.push_back({T, ex});
        }
        NAVI_TRY_HIP(hipGraphLaunch(ex, s), err, errlen);
    } else if (!prefill_layers(*t, T, s)) {
        set_err(err, errlen, "talker: a projection shape the prefill's tiled kernels do not take");
        return NAVI_ERR_UNSUPPORTED;
    }
    NAVI_TRY_HIP(hipGetLastError(), err, errlen);
    NAVI_TRY_HIP(hipEventRecord(t->ev1, s), err, errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(t->h_flag, t->flag, 4, hipMemcpyDeviceToHost, s), err, errlen);
    NAVI_TRY_HIP(hipStreamSynchronize(s), err, errlen);
    float ms = 0.f;
    NAVI_TRY_HIP(hipEventElapsedTime(&ms, t->ev0, t->ev1), err, errlen);
    t->last_ms = ms;
    const navi_status st = flag_result(*t, "prefill", err, errlen);
    if (st != NAVI_OK) return st;
    t->n_used = T;
    return NAVI_OK;
}

navi_status navi_talker_set_graphs(navi_talker *t, int32_t enabled) {
    if (!t) return NAVI_ERR_INVALID;
    t->use_graphs = enabled != 0;
    return NAVI_OK;
}

navi_status navi_talker_kv(navi_talker *t, navi_kv_view *out, int32_t *n_used) {
    if (!t || !out) return NAVI_ERR_INVALID;
    out->n_layer = t->L;
    out->max_pos = t->max_pos;
    out->kv_dim = t->KVD;
    out->k = t->kk.data();
    out->v = t->vv.data();
    if (n_used) *n_used = t->n_used;
    return NAVI_OK;
}

const float *navi_talker_hidden(const navi_talker *t) { return t ? t->hidden : nullptr; }
const float *navi_talker_logits(const navi_talker *t) { return t ? t->logits : nullptr; }
double navi_talker_last_ms(const navi_talker *t) { return t ? t->last_ms : 0.0; }

// navi_linear with its workspace in `scratch`: the same split count and kernels, so the same bits;
// no allocation on any path (the device must already be open).
navi_status navi_linear_noalloc(const float *d_x, int32_t ldx, int32_t M, const uint16_t *w, int32_t K, int32_t N,
                                const float *bias, const float *residual, int32_t act, float *d_y, int32_t ldy, char *err,
                                size_t errlen) {
    if (!d_x || !w || !d_y) {
        set_err(err, errlen, "linear: null argument");
        return NAVI_ERR_INVALID;
    }
    if (!linear_shape_ok(d_x, ldx, M, w, K, N) || ldy < N || (act != 0 && act != 1)) {
        set_err(err, errlen, "linear: unsupported shape or alignment (M %d, K %d, N %d, ldx %d, ldy %d, act %d)", M, K, N,
                ldx, ldy, act);
        return NAVI_ERR_INVALID;
    }
    DeviceState &ds = device_state();
    if (!ds.open) {
        set_err(err, errlen, "linear_noalloc: open the device first (navi_device_open)");
        return NAVI_ERR_INVALID;
    }
    NAVI_TRY_HIP(hipSetDevice(ds.device), err, errlen);
    if (ds.device < 0 || ds.device >= MAX_DEVICES) {
        set_err(err, errlen, "linear_noalloc: device index %d out of range", ds.device);
        return NAVI_ERR_UNSUPPORTED;
    }
    const int S = pick_splits(M, K, N);
    const size_t need = static_cast<size_t>(S) * M * N;
    if (need > SCRATCH_FLOATS) {
        set_err(err, errlen, "linear_noalloc: %d K-splits x %d rows x %d columns need %zu floats of workspace; the "
                "fixed scratch holds %zu (use navi_linear)", S, M, N, need, SCRATCH_FLOATS);
        return NAVI_ERR_INVALID;
    }
    void *&base = g_scratch_dev[ds.device];
    if (!base) {
        void *ptr = nullptr;
        NAVI_TRY_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), err, errlen);
        base = ptr;
    }
    uint32_t *flag = static_cast<uint32_t *>(base);
    float *part = reinterpret_cast<float *>(static_cast<unsigned char *>(base) + SCRATCH_FLAG_BYTES);
    hipStream_t s = ds.stream;
    hipLaunchKernelGGL(k_clear_word, dim3(1), dim3(64), 0, s, flag);
    launch_partial(d_x, ldx, M, w, K, N, S, part, N, 0, flag, s);
    hipLaunchKernelGGL(k_finish_linear, dim3(M), dim3(BT), 0, s, part, S, M, N, bias, residual, act, d_y, ldy);
    NAVI_TRY_HIP(hipGetLastError(), err, errlen);
    uint32_t f = 0;
    NAVI_TRY_HIP(hipMemcpyAsync(&f, flag, 4, hipMemcpyDeviceToHost, s), err, errlen);
    NAVI_TRY_HIP(hipStreamSynchronize(s), err, errlen);
    if (f) {
        set_err(err, errlen, "linear: an activation is outside the f16 range (|x| >= 65504 or NaN)");
        return NAVI_ERR_INVALID;
    }
    return NAVI_OK;
}

navi_status navi_linear(const float *d_x, int32_t ldx, int32_t M, const uint16_t *w, int32_t K, int32_t N,
                        const float *bias, const float *residual, int32_t act, float *d_y, int32_t ldy, char *err,
                        size_t errlen) {
    if (!d_x || !w || !d_y) {
        set_err(err, errlen, "linear: null argument");
        return NAVI_ERR_INVALID;
    }
    if (!linear_shape_ok(d_x, ldx, M, w, K, N) || ldy < N || (act != 0 && act != 1)) {
        set_err(err, errlen, "linear: unsupported shape or alignment (M %d, K %d, N %d, ldx %d, ldy %d, act %d)", M, K, N,
                ldx, ldy, act);
        return NAVI_ERR_INVALID;
    }
    navi_status st = ensure_device(err, errlen);
    if (st != NAVI_OK) return st;
    hipStream_t s = device_state().stream;
    const int S = pick_splits(M, K, N);
    const size_t need = static_cast<size_t>(S) * M * N;
    if (need > g_ws.floats) {
        NAVI_TRY_HIP(hipStreamSynchronize(s), err, errlen);
        if (g_ws.part) (void) hipFree(g_ws.part);
        g_ws.part = nullptr;
        g_ws.floats = 0;
        NAVI_TRY_HIP(hipMalloc(&g_ws.part, need * sizeof(float)), err, errlen);
        g_ws.floats = need;
    }
    if (!g_ws.flag) NAVI_TRY_HIP(hipMalloc(&g_ws.flag, 4), err, errlen);
    NAVI_TRY_HIP(hipMemsetAsync(g_ws.flag, 0, 4, s), err, errlen);
    launch_partial(d_x, ldx, M, w, K, N, S, g_ws.part, N, 0, g_ws.flag, s);
    hipLaunchKernelGGL(k_finish_linear, dim3(M), dim3(BT), 0, s, g_ws.part, S, M, N, bias, residual, act, d_y, ldy);
    NAVI_TRY_HIP(hipGetLastError(), err, errlen);
    uint32_t f = 0;
    NAVI_TRY_HIP(hipMemcpyAsync(&f, g_ws.flag, 4, hipMemcpyDeviceToHost, s), err, errlen);
    NAVI_TRY_HIP(hipStreamSynchronize(s), err, errlen);
    if (f) {
        set_err(err, errlen, "linear: an activation is outside the f16 range (|x| >= 65504 or NaN)");
        return NAVI_ERR_INVALID;
    }
    return NAVI_OK;
}

} // extern "C"
