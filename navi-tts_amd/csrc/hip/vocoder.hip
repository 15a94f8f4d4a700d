// The codec decoder (codes -> 24 kHz PCM) on gfx950: the C ABI's navi_vocoder_*.
//
// Replaces Vocoder (model/qwen3tts/vocoder.hip:20-644) and its conv kernel (k_conv,
// kernels.h:72-242). MI355X design:
//
//  * Every convolution and linear layer is one implicit GEMM on the matrix cores
//    (v_mfma_f32_16x16x32_f16): rows = output time steps, columns = output channels, the
//    reduction runs over (tap, input channel). Weights are re-laid out once at create to
//    [phase][Cout][tap][Cin] so that eight consecutive reduction indices are eight consecutive
//    channels of ONE input row: the A fragment of a tap is a single 16-byte LDS read from a
//    time window staged once per channel chunk, and a tap is only a row offset (j * dil) into
//    that window. Activations travel as f16 hi + lo pairs (f32-level products, as in the
//    prefill); weights stream as f16.
//  * Transposed convolutions (stride s, kernel s or 2s) are s phases of a causal conv with
//    k / s taps writing every s-th output row. The SiLU-gate prologue and bias, GELU,
//    residual, layer-scale and clamp epilogues are fused into the same kernel; the Snake that
//    starts every decoder-block conv is applied once per element by the conv producing its
//    input (a second, Snake'd output), not once per consuming block.
//  * Few output tiles (short chunks, narrow layers): the input channels are split over up to
//    S blocks per tile and the partial sums added in split order by a finish kernel, so a
//    16-frame chunk still spreads over the 256 CUs.
//  * The decoder blocks' convs (k7, k1 and the transposed convs' phases) run on k_conv_wide
//    (conv.h): v_mfma_f32_32x32x16_f16 on 128- or 64-row x 64- or 96-column tiles, the time
//    window and every tap's weights staged in LDS per 32-channel chunk, no K split. The last
//    block's 96-channel k7 and the final conv run on k_conv_c96 (whole input window and each
//    tap's weights in LDS, every output channel in one block).
//  * The transformer's projections run on the fused row kernels of rows.h (RMSNorm, SwiGLU and
//    the layer-scaled residual add inside; 5 launches per layer). RoPE and the K/V ring append
//    are folded into the windowed attention kernel; the RVQ rows are gathered by one small
//    kernel; the ConvNeXt depthwise conv + LayerNorm runs one wave per row with register-only
//    reductions.
//  * Streaming state: each causal conv keeps its last (K-1)*dil input rows (the history the
//    next chunk's first rows read), the ConvNeXt depthwise conv its last 6, the attention its
//    K/V in a ring of >= window + chunk positions: chunked decoding equals one-shot decoding.
//    A history is a pair of buffers: each launch reads one and its blocks write the next chunk's
//    into the other, so no launch exists only to update it.
#include "conv.h"
#include "dev_common.h"
#include "rows.h"
#include "host_util.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

namespace navi_amd {
namespace vc {

using namespace cv;

constexpr int ROW_PAD = 8;   // floats past a transformer activation row (navi_vocoder::lxs)

// y[t] = RMSNorm(x[t]) * w over C channels.
__global__ void __launch_bounds__(BT) k_rmsnorm(const float *x, int ldx, const float *w, int C, float eps, float *y) {
    __shared__ float red[4];
    const float *row = x + static_cast<size_t>(blockIdx.x) * ldx;
    float ss = 0.f;
    for (int c = threadIdx.x; c < C; c += BT) {
        const float v = gld(row + c);
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float scale = rsqrtf((red[0] + red[1] + red[2] + red[3]) / static_cast<float>(C) + eps);
    for (int c = threadIdx.x; c < C; c += BT) gst(y + static_cast<size_t>(blockIdx.x) * C + c, gld(row + c) * scale * gld(w + c));
}

// The ConvNeXt block's front (vocoder.hip:20-54 semantics): a causal depthwise conv over DWK time
// steps, then LayerNorm over the C channels of each row. One wave per output row and no LDS: lane
// l owns the MG groups of four channels 4 l + 256 m, so each of its loads is a 16-byte piece of a
// row that the wave reads whole (the depthwise weights tap-major, [DWK][C] f16, 8 bytes per group),
// and the row's mean and variance are two wave reductions in registers. Rows before t = 0 come from
// the DWK - 1 history rows; the block's threads then carry the next chunk's history into hnext.
template <int MG>
__global__ void __launch_bounds__(BT) k_dw_ln(const float *x, const float *hist, const uint16_t *wt, const float *bias,
                                              const float *lw, const float *lb, float eps, int R, float *y, float *hnext) {
    constexpr int DWK = 7, C = 256 * MG;
    const int l = threadIdx.x & 63, t = blockIdx.x * (BT / 64) + (threadIdx.x >> 6);
    if (t < R) {
        f32x4_t xv[DWK][MG];
        u32x2_t wv[DWK][MG];
#pragma unroll
        for (int j = 0; j < DWK; ++j) {
            const int tt = t - (DWK - 1) + j;
            const float *row = tt >= 0 ? x + static_cast<size_t>(tt) * C : hist + static_cast<size_t>(DWK - 1 + tt) * C;
#pragma unroll
            for (int m = 0; m < MG; ++m) {
                const int c = 4 * l + 256 * m;
                xv[j][m] = ld4(row + c);
                wv[j][m] = gld(reinterpret_cast<const u32x2_t *>(wt + static_cast<size_t>(j) * C + c));
            }
        }
        f32x4_t acc[MG];
        float s = 0.f;
#pragma unroll
        for (int m = 0; m < MG; ++m) {
            acc[m] = ld4(bias + 4 * l + 256 * m);
#pragma unroll
            for (int j = 0; j < DWK; ++j) {
                const u32x2_t w = wv[j][m];
                const float wf[4] = {h2f(static_cast<uint16_t>(w.x)), h2f(static_cast<uint16_t>(w.x >> 16)),
                                     h2f(static_cast<uint16_t>(w.y)), h2f(static_cast<uint16_t>(w.y >> 16))};
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[m][e] = fmaf(wf[e], xv[j][m][e], acc[m][e]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) s += acc[m][e];
        }
        const float mean = wave_sum(s) / static_cast<float>(C);
        float ss = 0.f;
#pragma unroll
        for (int m = 0; m < MG; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[m][e] -= mean;
                ss = fmaf(acc[m][e], acc[m][e], ss);
            }
        const float inv = rsqrtf(wave_sum(ss) / static_cast<float>(C) + eps);
#pragma unroll
        for (int m = 0; m < MG; ++m) {
            const int c = 4 * l + 256 * m;
            const f32x4_t g = ld4(lw + c), b = ld4(lb + c);
            st4(y + static_cast<size_t>(t) * C + c, acc[m] * inv * g + b);
        }
    }
    carry_rows(hist, x, C, R, DWK - 1, C, hnext);
}

// Sliding-window causal attention of the codec transformer (k_attention, vocoder.hip:87-122
// semantics) with RoPE (theta from invf, rotate-half) and the K/V ring append folded in. A block
// takes RT query rows of one head (16, or 4 for chunks of up to 32 frames, so that a short chunk
// still spreads over many blocks; a row's result does not depend on RT): it stages in LDS the roped keys and the values of every
// position those rows see (positions of this chunk straight from the q|k|v rows, roped here;
// earlier ones from the ring, stored roped), then each wave runs RT/4 rows: lane j scores keys
// j and j + 64 of the row's window, softmax by two wave reductions, and lane d sums p_j V[j][d]
// with p_j read from lane j (readlane). The block also writes its rows' roped k and v to the ring
// for later chunks: ring >= window + chunk, so no slot written here is one this launch reads.
template <int HD, int RT>
__global__ void __launch_bounds__(BT) k_window_attention(const float *qkv, int nh, int T, const int *pos0p, int window, int ring,
                                                         const float *invf, float *kc, float *vc, float *out, int ldo) {
    constexpr int HALF = HD / 2, KS = HD + 1, DPL = HD / 64;   // K rows padded: lanes j read rows j
    static_assert(RT % 4 == 0 && RT <= 16, "RT / 4 rows per wave; the LDS is sized for 16");
    extern __shared__ float sm[];
    const int pos0 = gld(pos0p);                 // the chunk's first position (device-side: graph replays)
    const int HDT = nh * HD, ld = 3 * HDT, h = blockIdx.y;
    const int t0 = blockIdx.x * RT, t1 = min(T, t0 + RT);
    const int kp0 = max(0, pos0 + t0 - window + 1), nk = pos0 + t1 - kp0;
    float *Ks = sm, *Vs = Ks + (window + RT - 1) * KS, *Qs = Vs + (window + RT - 1) * HD;
    // Staging: a thread takes 4 dimensions i..i+3 of a row and their rotate-half partners i+HALF..,
    // so every load is a float4; a batch of NB rows' loads is issued before any of them is used
    // (one memory latency per batch instead of one per element).
    constexpr int Q = HALF / 4, MAXE = (128 + RT - 1) * Q, NIT = (MAXE + BT - 1) / BT, NB = NIT < 5 ? NIT : 5;
    const int ne = nk * Q;
    // this thread's q element (at most one: RT * Q <= BT), loaded before the K/V staging so the two
    // loads share one memory latency
    static_assert(RT * Q <= BT, "one q element per thread");
    const int eq = static_cast<int>(threadIdx.x), rq = eq / Q, iq = (eq - rq * Q) * 4;
    const bool has_q = eq < (t1 - t0) * Q;
    f32x4_t qa0{}, qa1{}, qf{};
    if (has_q) {
        const float *row = qkv + static_cast<size_t>(t0 + rq) * ld + h * HD;
        qa0 = ld4(row + iq);
        qa1 = ld4(row + iq + HALF);
        qf = ld4(invf + iq);
    }
    for (int b0 = 0; b0 < NIT && b0 * BT < ne; b0 += NB) {
        f32x4_t ka[NB], kb[NB], va[NB], vb[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int e = static_cast<int>(threadIdx.x) + (b0 + u) * BT;
            if (b0 + u >= NIT || e >= ne) continue;
            const int r = e / Q, i = (e - r * Q) * 4, p = kp0 + r;
            if (p >= pos0) {
                const float *row = qkv + static_cast<size_t>(p - pos0) * ld + h * HD;
                ka[u] = ld4(row + HDT + i);
                kb[u] = ld4(row + HDT + i + HALF);
                va[u] = ld4(row + 2 * HDT + i);
                vb[u] = ld4(row + 2 * HDT + i + HALF);
            } else {
                const size_t o = static_cast<size_t>(p % ring) * HDT + h * HD + i;
                ka[u] = ld4(kc + o);
                kb[u] = ld4(kc + o + HALF);
                va[u] = ld4(vc + o);
                vb[u] = ld4(vc + o + HALF);
            }
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int e = static_cast<int>(threadIdx.x) + (b0 + u) * BT;
            if (b0 + u >= NIT || e >= ne) continue;
            const int r = e / Q, i = (e - r * Q) * 4, p = kp0 + r;
            f32x4_t k0 = ka[u], k1 = kb[u];
            if (p >= pos0) {
                const f32x4_t f = ld4(invf + i);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float sn, cs;
                    sincosf(static_cast<float>(p) * f[c], &sn, &cs);
                    k0[c] = ka[u][c] * cs - kb[u][c] * sn;
                    k1[c] = kb[u][c] * cs + ka[u][c] * sn;
                }
                if (p - pos0 >= t0 && p - pos0 < t1) {      // this tile's own rows go to the ring
                    const size_t o = static_cast<size_t>(p % ring) * HDT + h * HD + i;
                    st4(kc + o, k0);
                    st4(kc + o + HALF, k1);
                    st4(vc + o, va[u]);
                    st4(vc + o + HALF, vb[u]);
                }
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                Ks[r * KS + i + c] = k0[c];
                Ks[r * KS + i + HALF + c] = k1[c];
                Vs[r * HD + i + c] = va[u][c];
                Vs[r * HD + i + HALF + c] = vb[u][c];
            }
        }
    }
    if (has_q) {
        const int p = pos0 + t0 + rq;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float sn, cs;
            sincosf(static_cast<float>(p) * qf[c], &sn, &cs);
            Qs[rq * HD + iq + c] = qa0[c] * cs - qa1[c] * sn;
            Qs[rq * HD + iq + HALF + c] = qa1[c] * cs + qa0[c] * sn;
        }
    }
    __syncthreads();
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    const float scale = rsqrtf(static_cast<float>(HD));
    for (int k = 0; k < RT / 4; ++k) {
        const int rr = wv * (RT / 4) + k, t = t0 + rr;
        if (t >= t1) break;
        const int pos = pos0 + t, klo = max(0, pos - window + 1), n = pos - klo + 1, rb = klo - kp0;
        const float *q = Qs + rr * HD;
        float s[2] = {-INFINITY, -INFINITY};
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int j = l + 64 * u;
            if (j < n) {
                const float *kr = Ks + (rb + j) * KS;
                float d = 0.f;
#pragma unroll 16
                for (int i = 0; i < HD; ++i) d = fmaf(q[i], kr[i], d);
                s[u] = d * scale;
            }
        }
        const float m = wave_max(fmaxf(s[0], s[1]));
        float p[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) p[u] = l + 64 * u < n ? expf(s[u] - m) : 0.f;
        const float inv = 1.f / wave_sum(p[0] + p[1]);
        // sum over the keys in key order; the V rows of 8 keys are read before their 8 products,
        // so one LDS latency covers 8 keys
        float acc[DPL] = {};
        auto pk = [&](int j) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[j >> 6]), j & 63)); };
        const float *vb = Vs + rb * HD + l;
        int j = 0;
        for (; j + 8 <= n; j += 8) {
            float vv[8][DPL];
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int d = 0; d < DPL; ++d) vv[u][d] = vb[(j + u) * HD + 64 * d];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float pj = pk(j + u);
#pragma unroll
                for (int d = 0; d < DPL; ++d) acc[d] = fmaf(pj, vv[u][d], acc[d]);
            }
        }
        for (; j < n; ++j) {
            const float pj = pk(j);
#pragma unroll
            for (int d = 0; d < DPL; ++d) acc[d] = fmaf(pj, vb[j * HD + 64 * d], acc[d]);
        }
#pragma unroll
        for (int d = 0; d < DPL; ++d) gst(out + static_cast<size_t>(t) * ldo + h * HD + l + 64 * d, acc[d] * inv);
    }
}

// The RVQ front end's input rows (k_rvq, vocoder.hip:125-143): channel ci < CD/2 of frame t is the
// semantic codebook's row for code 0, the rest the other codebooks' rows summed in codebook order;
// one float4 per thread, all of its codebook loads issued before the sum. A kernel of its own: as
// the first conv's prologue every one of that conv's column blocks repeated the gathers.
__global__ void __launch_bounds__(BT) k_rvq_rows(ConvArgs a, float *out) {
    const int q4 = a.Cin / 4, i = blockIdx.x * BT + threadIdx.x;
    if (i >= a.T * q4) return;
    const int t = i / q4, ci = (i - t * q4) * 4;
    st4(out + static_cast<size_t>(t) * a.Cin + ci, rvq_row4(a, t, ci));
}

// Zeroes span blockIdx.x ({pointer, 32-bit words}): reset's one launch over every history buffer.
struct ZeroSpan {
    uint32_t *p;
    uint32_t n;
};
__global__ void __launch_bounds__(BT) k_zero_spans(const ZeroSpan *spans) {
    const ZeroSpan z = spans[blockIdx.x];
    for (uint32_t i = threadIdx.x; i < z.n; i += BT) gst(z.p + i, 0u);
}

// The last kernel of a chunk. pcm[t] = y[t][0] for the T rows: the last conv runs on the matrix
// cores with its one output channel padded to a 16-column tile (15 zero weight rows); this keeps
// column 0, in device memory (the stage hook's copy) and in the caller's pinned host slot. Thread
// 0 also moves the utterance position past the chunk's frames and copies the chunk's f16-range
// flag into its pinned host word (every kernel that sets it ran before this one).
__global__ void __launch_bounds__(BT) k_take_col0(const float *y, int T, int ld, float *pcm, float *pcm_host, int *pos0,
                                                 int frames, const uint32_t *flag, uint32_t *flag_host) {
    const int t = blockIdx.x * BT + threadIdx.x;
    if (t < T) {
        const float v = gld(y + static_cast<size_t>(t) * ld);
        gst(pcm + t, v);
        gst(pcm_host + t, v);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        gst(pos0, gld(pos0) + frames);
        gst(flag_host, gld(flag));
    }
}

// ---- weight preparation (vocoder.hip:350-420, done here on the device) ----------------

// ConvTranspose1d [Cin][Cout][k] (stride s) -> [s][Cout][k/s][Cin]:
// out[p][co][j][ci] = W[ci][co][p + (k/s - 1 - j) * s]   (tap k/s-1 is the current input row)
__global__ void k_relayout_tconv(const uint16_t *w, int Cin, int Cout, int k, int s, uint16_t *out) {
    const size_t i = static_cast<size_t>(blockIdx.x) * BT + threadIdx.x, n = static_cast<size_t>(Cin) * Cout * k;
    if (i >= n) return;
    const int kk = k / s;
    const int ci = static_cast<int>(i % Cin);
    size_t r = i / Cin;
    const int j = static_cast<int>(r % kk);
    r /= kk;
    const int co = static_cast<int>(r % Cout), p = static_cast<int>(r / Cout);
    gst(out + i, gld(w + (static_cast<size_t>(ci) * Cout + co) * k + p + (kk - 1 - j) * s));
}

// Depthwise conv weights [C][1][K] -> tap-major [K][C] (k_dw_ln reads a tap's channels at once).
__global__ void k_tap_major(const uint16_t *w, int C, int K, uint16_t *out) {
    const int i = blockIdx.x * BT + threadIdx.x;
    if (i >= C * K) return;
    const int j = i / C, c = i - j * C;
    gst(out + i, gld(w + static_cast<size_t>(c) * K + j));
}

__global__ void k_snake_prep(const float *alpha, const float *beta, int n, float *sa, float *sb) {
    const int i = blockIdx.x * BT + threadIdx.x;
    if (i >= n) return;
    gst(sa + i, expf(gld(alpha + i)));
    gst(sb + i, 1.f / (expf(gld(beta + i)) + 1e-9f));
}

// ---- host ------------------------------------------------------------------------------

struct Conv {
    const uint16_t *w = nullptr;       // [phases][Cout][K][Cin]
    const float *bias = nullptr;
    // The Snake on this conv's input (exp(alpha), 1 / (exp(beta) + 1e-9)); applied by the conv
    // that produces the input, as its z output.
    const float *sa = nullptr, *sb = nullptr;
    int Cin = 0, Cout = 0, K = 1, dil = 1, phases = 1, H = 0;
    int S = 1;                         // input-channel splits (fixed at create: conv_splits)
    bool wide = false;                 // runs on k_conv_wide (fixed at create: conv_takes_wide)
    // the history pair: a chunk reads hbuf[parity] and writes the next chunk's into hbuf[parity ^ 1]
    float *hbuf[2] = {};
};

struct TLayer {
    const float *ln1, *ln2, *attn_scale, *mlp_scale;
    Conv qkv, o, gu, down;
    float *kc, *vc;
};

struct ConvNeXt {
    const uint16_t *dwt;               // depthwise weights, tap-major [7][C]
    const float *dw_b, *ln_w, *ln_b, *gamma;
    float *hbuf[2];                    // the depthwise conv's 6 history rows (pair, as Conv::hbuf)
    Conv pw1, pw2;
};

struct Unit { Conv c1, c2; };
struct Block { Conv up; Unit u[3]; int rate, Cin, Cout; };

} // namespace vc
} // namespace navi_amd

using namespace navi_amd;
using namespace navi_amd::vc;

struct navi_vocoder {
    navi_vocoder_params p{};
    int cmax = 0, ring = 0, VH = 0, HDT = 0, L = 0, CD = 0, DD = 0;
    int parity = 0;                    // which buffer of every history pair the next chunk reads
    int *d_pos0 = nullptr;             // the next chunk's first position (device)
    // what reset clears (every causal history buffer and the position): one fill kernel over
    // these spans instead of a memset per buffer
    ZeroSpan *d_spans = nullptr;
    int n_spans = 0;
    // each chunk size's launch sequence captured once per history parity and replayed
    std::vector<std::pair<std::pair<int, int>, hipGraphExec_t>> graphs;
    bool use_graphs = false;           // off by default: replays measured no faster than launches
    const uint16_t *cb_first = nullptr;
    uint16_t *cb_rest = nullptr;
    Conv rvq_proj, pre_conv, in_proj, out_proj, dec0;
    const float *final_norm = nullptr;
    std::vector<TLayer> layers;
    Conv up_conv[2];
    ConvNeXt cnx[2];
    Block blocks[4];
    Conv final_conv;                   // Cin -> 1 padded to 16 output channels
    float *pcm16 = nullptr;            // [rows][16] output of the padded final conv
    float *invf = nullptr;
    uint32_t *flag = nullptr;
    // Pinned, coherent host slots that the kernels read and write directly: a chunk's codes (read by
    // the RVQ front end) and its PCM (written by the last kernel), slot = the chunk's history
    // parity, so consecutive chunks alternate and one can be handed over while the next runs; the
    // f16-range flag word, copied there by a chunk's last kernel.
    // (h_*: the host's addresses, dh_*: the same memory as the kernels address it)
    int32_t *h_codes[2] = {}, *dh_codes[2] = {};
    float *h_pcm[2] = {}, *dh_pcm[2] = {};
    uint32_t *h_flag = nullptr, *dh_flag = nullptr;
    // The device flag is zero at the start of a call unless the previous call did not end with it
    // read back as zero (then this call clears it first): no clearing launch on the normal path.
    bool flag_dirty = false;
    void *h_buf = nullptr;
    hipEvent_t ev_slot[2] = {};
    // activations of one chunk (time-major rows)
    float *lat_in = nullptr;           // RVQ rows gathered from the codebooks [T][CD]
    float *lat = nullptr;              // RVQ latent [T][CD]
    float *pre = nullptr;              // pre_conv output [T][L]
    float *xs = nullptr, *xn = nullptr;   // transformer residual stream [T][lxs] and its RMSNorm [T][VH]
    float *qkv = nullptr, *att = nullptr, *gu = nullptr;   // att [T][latt], gu [T][lgu]
    // Row strides of the transformer's projection inputs: ROW_PAD floats past the row, since
    // strides that are multiples of 2-4 KB put the 16 rows of an MFMA operand load on the same
    // memory channels (the 16-row projections measured 12-19 % faster padded)
    int lxs = 0, latt = 0, lgu = 0;
    float *snapbuf = nullptr;          // compact copy of a padded stage for the stage hook
    float *post = nullptr;             // transformer output projection [T][L]
    float *upx[2] = {};                // upsampling stages' residual streams [R][L]
    float *lnx = nullptr;              // ConvNeXt depthwise + LayerNorm output [R][L]
    float *pwh = nullptr;              // ConvNeXt hidden [R][4L]
    float *dec_in = nullptr;           // Snake(dec0 output), block 0's input [R][DD]
    float *pcm = nullptr;
    // per decoder block: the residual stream, its Snake (the next conv's input) and the Snake of
    // each unit's first conv output
    float *res[4] = {}, *res_s[4] = {}, *mid_s[4] = {};
    float *dec_raw = nullptr;          // dec0's output before its Snake: written only for the stage hook
    navi_stage_fn hook = nullptr;      // debugging: called after every stage of a chunk
    void *hook_user = nullptr;
    float *part = nullptr;             // K-split partial sums (conv_splits)
    size_t part_floats = 0;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    double last_ms = 0;
    std::vector<void *> owned;

    template <class T>
    navi_status alloc(T *&ptr, size_t count, char *err, size_t errlen) {
        void *v = nullptr;
        NAVI_TRY_HIP(hipMalloc(&v, std::max<size_t>(count, 1) * sizeof(T)), err, errlen);
        owned.push_back(v);
        NAVI_TRY_HIP(hipMemsetAsync(v, 0, std::max<size_t>(count, 1) * sizeof(T), device_state().stream), err, errlen);
        ptr = static_cast<T *>(v);
        return NAVI_OK;
    }

    ~navi_vocoder() {
        for (auto &g : graphs) (void) hipGraphExecDestroy(g.second);
        if (ev0) (void) hipEventDestroy(ev0);
        if (ev1) (void) hipEventDestroy(ev1);
        for (hipEvent_t e : ev_slot)
            if (e) (void) hipEventDestroy(e);
        if (h_buf) (void) hipHostFree(h_buf);
        for (void *v : owned) (void) hipFree(v);
    }
};

namespace {

template <int MT, int K>
void launch_k(const ConvArgs &a, int pro, int epi, dim3 grid, hipStream_t s) {
#define NAVI_CONV(P_, E_)                                                                       \
    if (pro == P_ && epi == E_) {                                                               \
        hipLaunchKernelGGL((k_conv_mfma<MT, K, P_, E_>), grid, dim3(BT), 0, s, a);              \
        return;                                                                                 \
    }
    NAVI_CONV(PRO_NONE, EPI_BIAS)
    NAVI_CONV(PRO_NONE, EPI_GELU)
    NAVI_CONV(PRO_NONE, EPI_RESIDUAL)
    NAVI_CONV(PRO_NONE, EPI_SCALE_RESIDUAL)
    NAVI_CONV(PRO_NONE, EPI_CLAMP)
    NAVI_CONV(PRO_NONE, EPI_PARTIAL)
#undef NAVI_CONV
}

int conv_mt(int T) { return T <= 16 ? 1 : 4; }

// The final 96 -> 16 conv (one output channel padded to a 16-column tile) runs on k_conv_c96
// (input window and weights staged in LDS, every output channel in one block); the last block's
// own 96-channel convs take k_conv_wide / k_unit first. Chosen by the conv's shape only, so
// every chunking of the codes runs the same kernel.
bool conv_is_c96(const Conv &c) {
    return c.phases == 1 && c.S == 1 && c.dil <= 9 && (c.K == 7 || c.K == 1) && c.Cin == 96 && (c.Cout == 96 || c.Cout == 16);
}

bool launch_c96(const Conv &c, const ConvArgs &a, int pro, int epi, int T, hipStream_t s) {
    if (pro != PRO_NONE) return false;
    const dim3 grid((T + 127) / 128);
#define NAVI_C96(K_, NCT_, E_)                                                                  \
    if (c.K == K_ && c.Cout == 16 * NCT_ && epi == E_) {                                       \
        hipLaunchKernelGGL((k_conv_c96<K_, NCT_, 2, E_>), grid, dim3(BT), 0, s, a);             \
        return true;                                                                            \
    }
    NAVI_C96(7, 1, EPI_CLAMP)
#undef NAVI_C96
    return false;
}

// The decoder blocks' causal convs (K 7, 2 or 1, any phases, 32 | Cin, 64 | Cout or Cout = 96,
// at least 32 input rows per frame) run on k_conv_wide. Decided at create from the conv's shape and
// place, so every chunking of the codes runs the same kernel and sums in the same order.
bool conv_takes_wide(const Conv &c, int rows_per_frame) {
    return (c.K == 7 || c.K == 2 || c.K == 1) && c.dil <= 9 && c.Cin % 32 == 0 && (c.Cout % 64 == 0 || c.Cout == 96) &&
           rows_per_frame >= 32;
}

// Input-channel splits of a k_conv_wide conv (64-column tiles only), fixed at create: when the
// 64-row tiles of a 16-frame chunk (rows16 input rows) would leave the 256 CUs idle, the channels
// fall into S equal ranges of at least two 32-channel chunks each. A short chunk then runs S times
// the blocks (partials summed by k_conv_finish), a long one the same sums in one block per tile.
constexpr int WIDE_SPLIT_TILES = 256;
int wide_splits(const Conv &c, int rows16) {
    if (c.Cout % 64 != 0) return 1;
    const int tiles = (c.Cout / 64) * ((rows16 + 63) / 64) * c.phases, chunks = c.Cin / 32;
    int S = 1;
    while (tiles * S < WIDE_SPLIT_TILES && chunks % (2 * S) == 0 && chunks / (2 * S) >= 2) S *= 2;
    return S;
}

// Whether a launch over T rows runs the split blocks (fewer than WIDE_SPLIT_TILES 64-row tiles),
// and the largest such T (the rows the split workspace has to hold).
bool wide_split_run(const Conv &c, int T) {
    return c.S > 1 && (c.Cout / 64) * ((T + 63) / 64) * c.phases < WIDE_SPLIT_TILES;
}
int wide_split_max_rows(const Conv &c) {
    return c.S > 1 ? 64 * ((WIDE_SPLIT_TILES - 1) / ((c.Cout / 64) * c.phases)) : 0;
}

bool launch_wide_conv(const Conv &c, ConvArgs &a, int pro, int epi, int T, float *part, hipStream_t s) {
    if (pro != PRO_NONE) return false;
    const int P = c.phases;
    if (c.Cout == 96) {
        const dim3 g(1, (T + 127) / 128, P);
#define NAVI_W96(K_, E_)                                                                                           \
        if (c.K == K_ && epi == E_) {                                                                              \
            hipLaunchKernelGGL((k_conv_wide<K_, 128, 96, E_>), g, dim3(BT), 0, s, a);                             \
            return true;                                                                                           \
        }
        if (c.K == 7 && epi == EPI_BIAS) {
            hipLaunchKernelGGL((k_conv_wide<7, 128, 96, EPI_BIAS, 16>), g, dim3(BT), 0, s, a);
            return true;
        }
        NAVI_W96(2, EPI_BIAS)
        NAVI_W96(1, EPI_RESIDUAL)
#undef NAVI_W96
        return false;
    }
    const int nb = c.Cout / 64;
    a.cps = c.Cin / c.S;
    if (wide_split_run(c, T)) {
        const bool known = (c.K == 7 && epi == EPI_BIAS) || (c.K == 2 && epi == EPI_BIAS) || (c.K == 1 && epi == EPI_RESIDUAL);
        if (!known) return false;
        a.part = part;
        const dim3 g(nb, (T + 63) / 64, P * c.S);
        if (c.K == 7) hipLaunchKernelGGL((k_conv_wide<7, 64, 64, EPI_PARTIAL, 32, 1>), g, dim3(BT), 0, s, a);
        else if (c.K == 2) hipLaunchKernelGGL((k_conv_wide<2, 64, 64, EPI_PARTIAL, 32, 1>), g, dim3(BT), 0, s, a);
        else hipLaunchKernelGGL((k_conv_wide<1, 64, 64, EPI_PARTIAL, 32, 1>), g, dim3(BT), 0, s, a);
        const size_t n = static_cast<size_t>(T) * P * c.Cout;
        hipLaunchKernelGGL(k_conv_finish, dim3(static_cast<unsigned>((n + BT - 1) / BT)), dim3(BT), 0, s, a, c.S, epi);
        return true;
    }
    const bool big = static_cast<long>((T + 127) / 128) * nb * P >= 512;   // enough 128-row tiles to fill the chip twice
#define NAVI_WIDE(K_, E_, SM_)                                                                                           \
    if (big) hipLaunchKernelGGL((k_conv_wide<K_, 128, 64, E_, 32, SM_>), dim3(nb, (T + 127) / 128, P), dim3(BT), 0, s, a); \
    else hipLaunchKernelGGL((k_conv_wide<K_, 64, 64, E_, 32, SM_>), dim3(nb, (T + 63) / 64, P), dim3(BT), 0, s, a);
#define NAVI_WIDE_E(K_, E_)                          \
    if (c.K == K_ && epi == E_) {                    \
        if (c.S > 1) { NAVI_WIDE(K_, E_, 2) }        \
        else { NAVI_WIDE(K_, E_, 0) }                \
        return true;                                 \
    }
    NAVI_WIDE_E(7, EPI_BIAS)
    NAVI_WIDE_E(2, EPI_BIAS)
    NAVI_WIDE_E(1, EPI_RESIDUAL)
#undef NAVI_WIDE_E
#undef NAVI_WIDE
    return false;
}

// A residual unit of the last decoder block (96 channels: k7 then k1, one phase each) runs as one
// kernel, k_unit (conv.h): the k7's Snake'd output stays in LDS as the k1's input. (The 192-channel
// block's units on k_unit<192, 64> measured slower than its two k_conv_wide launches: 437-504 us
// against 295 + 153 us per unit for 240 frames, 64 against 47 us in 16-frame chunks.)
bool unit_fused(const Unit &u) {
    const int C = u.c1.Cout;
    return C == 96 && u.c1.Cin == C && u.c1.K == 7 && u.c1.phases == 1 && u.c1.dil <= 9 && u.c2.Cin == C && u.c2.Cout == C &&
           u.c2.K == 1 && u.c2.phases == 1;
}

void launch_unit(navi_vocoder &v, Unit &u, const float *x, int T, const float *res, float *y, float *z, const Conv &next) {
    UnitArgs a{};
    a.x = x; a.hist = u.c1.hbuf[v.parity]; a.hnext = u.c1.H > 0 ? u.c1.hbuf[v.parity ^ 1] : nullptr;
    a.w7 = u.c1.w; a.w1 = u.c2.w; a.b7 = u.c1.bias; a.b1 = u.c2.bias; a.za_mid = u.c2.sa; a.zb_mid = u.c2.sb;
    a.res = res; a.y = y; a.z = z; a.za = next.sa; a.zb = next.sb; a.flag = v.flag; a.T = T; a.dil = u.c1.dil;
    // 32-row tiles when 128-row ones would leave half the CUs idle (a short chunk): the same sums
    if (T < 128 * 128) hipLaunchKernelGGL((k_unit<96, 32, 16>), dim3((T + 31) / 32), dim3(BT), 0, device_state().stream, a);
    else hipLaunchKernelGGL((k_unit<96, 128, 16>), dim3((T + 127) / 128), dim3(BT), 0, device_state().stream, a);
}

// Input-channel splits of a conv over T rows: when the output tiles alone would leave most of the
// 256 CUs idle, the channel chunks are spread over up to S blocks per tile (at least 2 chunks each)
// and summed by k_conv_finish.
//
// The count is fixed per conv when the vocoder is created (from the rows of a 16-frame chunk, or
// of the largest chunk if smaller): the summation order, and so the PCM, then does not depend on
// how the codes are batched.
int conv_splits(const Conv &c, int T) {
    const int mt = conv_mt(T);
    const int blocks = ((c.Cout + 63) / 64) * ((T + 16 * mt - 1) / (16 * mt)) * c.phases;
    const int chunks = (c.Cin + CCH - 1) / CCH;
    int S = 1;
    while (blocks * S * 2 <= 384 && chunks >= S * 4) S *= 2;
    return S;
}


// k_conv_mfma over T rows (input-channel splits summed by k_conv_finish).
navi_status launch_generic(navi_vocoder &v, const Conv &c, ConvArgs &a, int pro, int epi, int T, char *err, size_t errlen) {
    hipStream_t s = device_state().stream;
    const int mt = conv_mt(T), S = c.S;
    const int chunks = (c.Cin + CCH - 1) / CCH;
    a.cps = (chunks + S - 1) / S * CCH;
    if (S > 1) {
        if (static_cast<size_t>(S) * T * c.phases * c.Cout > v.part_floats) {
            set_err(err, errlen, "vocoder: split workspace too small");
            return NAVI_ERR_INVALID;
        }
        a.part = v.part;
    }
    const int kepi = S > 1 ? static_cast<int>(EPI_PARTIAL) : epi;
    const dim3 grid((c.Cout + 63) / 64, (T + 16 * mt - 1) / (16 * mt), c.phases * S);
    switch (c.K * 10 + (mt == 1 ? 1 : 4)) {
    case 11: launch_k<1, 1>(a, pro, kepi, grid, s); break;
    case 14: launch_k<4, 1>(a, pro, kepi, grid, s); break;
    case 21: launch_k<1, 2>(a, pro, kepi, grid, s); break;
    case 24: launch_k<4, 2>(a, pro, kepi, grid, s); break;
    case 31: launch_k<1, 3>(a, pro, kepi, grid, s); break;
    case 34: launch_k<4, 3>(a, pro, kepi, grid, s); break;
    case 71: launch_k<1, 7>(a, pro, kepi, grid, s); break;
    case 74: launch_k<4, 7>(a, pro, kepi, grid, s); break;
    default:
        set_err(err, errlen, "vocoder: no conv kernel for K=%d", c.K);
        return NAVI_ERR_UNSUPPORTED;
    }
    if (S > 1) {
        const size_t n = static_cast<size_t>(T) * c.phases * c.Cout;
        hipLaunchKernelGGL(k_conv_finish, dim3(static_cast<unsigned>((n + BT - 1) / BT)), dim3(BT), 0, s, a, S, epi);
    }
    return NAVI_OK;
}

// Runs one conv over T input rows. A causal conv reads its history and writes the next chunk's
// into the other buffer of its pair (the pair then swaps). z (optional): also write Snake(y) with
// the Snake parameters of zc, the conv that consumes this output.
navi_status run_conv(navi_vocoder &v, Conv &c, int pro, int epi, const float *x, int T, int ldx, float *y, int ldy,
                     const float *res, const float *scale, char *err, size_t errlen, float *z = nullptr,
                     const Conv *zc = nullptr) {
    ConvArgs a{};
    a.x = x; a.hist = c.hbuf[v.parity]; a.w = c.w; a.bias = c.bias; a.res = res; a.scale = scale;
    a.y = y; a.z = z; a.flag = v.flag; a.ldx = ldx; a.ldy = ldy; a.T = T; a.Cin = c.Cin; a.Cout = c.Cout;
    a.dil = c.dil; a.phases = c.phases; a.lpad = (c.K - 1) * c.dil;   // causal
    a.hnext = c.H > 0 ? c.hbuf[v.parity ^ 1] : nullptr;
    if (z) {
        a.za = zc->sa;
        a.zb = zc->sb;
    }
    if (c.wide) {
        if (wide_split_run(c, T) && static_cast<size_t>(c.S) * T * c.phases * c.Cout > v.part_floats) {
            set_err(err, errlen, "vocoder: split workspace too small");
            return NAVI_ERR_INVALID;
        }
        if (!launch_wide_conv(c, a, pro, epi, T, v.part, device_state().stream)) {
            set_err(err, errlen, "vocoder: no wide conv kernel for K=%d epilogue %d", c.K, epi);
            return NAVI_ERR_UNSUPPORTED;
        }
    } else if (conv_is_c96(c)) {
        if (!launch_c96(c, a, pro, epi, T, device_state().stream)) {
            set_err(err, errlen, "vocoder: no 96-channel conv kernel for K=%d Cout=%d epilogue %d", c.K, c.Cout, epi);
            return NAVI_ERR_UNSUPPORTED;
        }
    } else {
        const navi_status st = launch_generic(v, c, a, pro, epi, T, err, errlen);
        if (st != NAVI_OK) return st;
    }
    return NAVI_OK;
}

size_t attention_lds(int window, int head_dim) {
    constexpr int RT = 16;
    return (static_cast<size_t>(window + RT - 1) * (2 * head_dim + 1) + static_cast<size_t>(RT) * head_dim) * sizeof(float);
}

#define VOC_TRY(expr)                         \
    do {                                      \
        const navi_status s_ = (expr);        \
        if (s_ != NAVI_OK) return s_;         \
    } while (0)

// The stage hook (Vocoder::set_stage_hook, vocoder.h:46-48): the device buffer of a finished stage,
// after the stream has drained. The stage names are the reference's (vocoder.hip:267-341), which
// its tools compare by.
navi_status snap(navi_vocoder &v, const std::string &name, const float *buf, int rows, int cols, char *err, size_t errlen,
                 int ld = 0) {
    if (!v.hook) return NAVI_OK;
    if (ld > cols) {                   // padded rows: the hook gets a compact copy
        NAVI_TRY_HIP(hipMemcpy2DAsync(v.snapbuf, static_cast<size_t>(cols) * 4, buf, static_cast<size_t>(ld) * 4,
                                      static_cast<size_t>(cols) * 4, rows, hipMemcpyDeviceToDevice, device_state().stream),
                     err, errlen);
        buf = v.snapbuf;
    }
    NAVI_TRY_HIP(hipStreamSynchronize(device_state().stream), err, errlen);
    v.hook(v.hook_user, name.c_str(), buf, rows, cols);
    return NAVI_OK;
}

// A transformer projection of the chunk on the row-projection kernels (rows.h): RMSNorm, SwiGLU
// and the layer-scaled residual add fused in, whole K per block, no split-K partials.
navi_status xf_rows(int epi, bool norm, const float *A, int lda, int M, int K, const float *ln, float eps, const uint16_t *w0,
                    int n0, const uint16_t *w1, int n1, float *y, int ldy, const float *rs, uint32_t *flag, char *err,
                    size_t errlen) {
    if (!rows::launch_rows_xf(epi, norm, A, lda, M, K, ln, eps, w0, n0, w1, n1, y, ldy, rs, flag, device_state().stream)) {
        set_err(err, errlen, "vocoder: no row-projection kernel for K=%d N=%d (epilogue %d)", K, n0 + n1, epi);
        return NAVI_ERR_UNSUPPORTED;
    }
    return NAVI_OK;
}

// One chunk of T frames: codes (already in the pinned slot of the history parity) -> T *
// samples_per_frame PCM samples in v.pcm and that pinned slot
// (the stage order of decode_chunk, vocoder.hip:261-343, which is the model's).
navi_status decode_chunk(navi_vocoder &v, int T, char *err, size_t errlen) {
    hipStream_t s = device_state().stream;
    const navi_vocoder_params &p = v.p;
    const int VH = v.VH, L = v.L, HDT = v.HDT, FF = p.xf.ff, CD = v.CD, nh = p.xf.n_head;
    // RVQ front end and its two output projections, one conv gathering its rows from the codebooks
    {
        ConvArgs ra{};
        ra.codes = v.dh_codes[v.parity]; ra.cb0 = v.cb_first; ra.cbr = v.cb_rest; ra.nq = p.n_q; ra.cbsize = p.codebook_size;
        ra.T = T; ra.Cin = CD;
        hipLaunchKernelGGL(k_rvq_rows, dim3((T * (CD / 4) + BT - 1) / BT), dim3(BT), 0, s, ra, v.lat_in);
    }
    VOC_TRY(run_conv(v, v.rvq_proj, PRO_NONE, EPI_BIAS, v.lat_in, T, CD, v.lat, CD, nullptr, nullptr, err, errlen));
    VOC_TRY(snap(v, "rvq", v.lat, T, CD, err, errlen));
    VOC_TRY(run_conv(v, v.pre_conv, PRO_NONE, EPI_BIAS, v.lat, T, CD, v.pre, L, nullptr, nullptr, err, errlen));
    VOC_TRY(snap(v, "pre_conv", v.pre, T, L, err, errlen));
    VOC_TRY(run_conv(v, v.in_proj, PRO_NONE, EPI_BIAS, v.pre, T, L, v.xs, v.lxs, nullptr, nullptr, err, errlen));
    VOC_TRY(snap(v, "in_proj", v.xs, T, VH, err, errlen, v.lxs));
    const size_t att_lds = attention_lds(p.sliding_window, p.xf.head_dim);
    for (size_t li = 0; li < v.layers.size(); ++li) {
        TLayer &ly = v.layers[li];
        const std::string ls = std::to_string(li);
        if (v.hook) {                 // the normed rows are a stage of their own only for the hook
            hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(BT), 0, s, v.xs, v.lxs, ly.ln1, VH, p.xf.rms_eps, v.xn);
            VOC_TRY(snap(v, "norm1_" + ls, v.xn, T, VH, err, errlen));
        }
        VOC_TRY(xf_rows(rows::EPI_PLAIN, true, v.xs, v.lxs, T, VH, ly.ln1, p.xf.rms_eps, ly.qkv.w, 3 * HDT, nullptr, 0, v.qkv,
                        3 * HDT, nullptr, v.flag, err, errlen));
        VOC_TRY(snap(v, "qkv_" + ls, v.qkv, T, 3 * HDT, err, errlen));
#define NAVI_ATT(HD_, RT_)                                                                                              \
        hipLaunchKernelGGL((k_window_attention<HD_, RT_>), dim3((T + RT_ - 1) / RT_, nh), dim3(BT), att_lds, s, v.qkv, nh, T, \
                           v.d_pos0, p.sliding_window, v.ring, v.invf, ly.kc, ly.vc, v.att, v.latt)
        if (p.xf.head_dim == 64) {
            if (T <= 32) NAVI_ATT(64, 4);
            else NAVI_ATT(64, 16);
        } else {
            if (T <= 32) NAVI_ATT(128, 4);
            else NAVI_ATT(128, 16);
        }
#undef NAVI_ATT
        VOC_TRY(snap(v, "attnraw" + ls, v.att, T, HDT, err, errlen, v.latt));
        VOC_TRY(xf_rows(rows::EPI_RESID, false, v.att, v.latt, T, HDT, nullptr, 0.f, ly.o.w, VH, nullptr, 0, v.xs, v.lxs,
                        ly.attn_scale, v.flag, err, errlen));
        VOC_TRY(snap(v, "xattn_" + ls, v.xs, T, VH, err, errlen, v.lxs));
        VOC_TRY(xf_rows(rows::EPI_SWIGLU, true, v.xs, v.lxs, T, VH, ly.ln2, p.xf.rms_eps, ly.gu.w, FF,
                        ly.gu.w + static_cast<size_t>(FF) * VH, FF, v.gu, v.lgu, nullptr, v.flag, err, errlen));
        VOC_TRY(xf_rows(rows::EPI_RESID, false, v.gu, v.lgu, T, FF, nullptr, 0.f, ly.down.w, VH, nullptr, 0, v.xs, v.lxs,
                        ly.mlp_scale, v.flag, err, errlen));
        VOC_TRY(snap(v, "layer" + ls, v.xs, T, VH, err, errlen, v.lxs));
    }
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(BT), 0, s, v.xs, v.lxs, v.final_norm, VH, p.xf.rms_eps, v.xn);
    VOC_TRY(run_conv(v, v.out_proj, PRO_NONE, EPI_BIAS, v.xn, T, VH, v.post, L, nullptr, nullptr, err, errlen));
    VOC_TRY(snap(v, "pre_transformer", v.post, T, L, err, errlen));
    // two upsampling stages: transposed conv, then the ConvNeXt block in place on its output
    int rows = T;
    const float *stage_in = v.post;
    for (int j = 0; j < 2; ++j) {
        float *up = v.upx[j];
        VOC_TRY(run_conv(v, v.up_conv[j], PRO_NONE, EPI_BIAS, stage_in, rows, L, up, L, nullptr, nullptr, err, errlen));
        rows *= p.upsampling_ratios[j];
        const std::string js = "up" + std::to_string(j);
        VOC_TRY(snap(v, js + "_t", up, rows, L, err, errlen));
        ConvNeXt &cx = v.cnx[j];
        hipLaunchKernelGGL(k_dw_ln<4>, dim3((rows + 3) / 4), dim3(BT), 0, s, up, cx.hbuf[v.parity], cx.dwt, cx.dw_b, cx.ln_w,
                           cx.ln_b, 1e-6f, rows, v.lnx, cx.hbuf[v.parity ^ 1]);
        VOC_TRY(snap(v, js + "_ln", v.lnx, rows, L, err, errlen));
        VOC_TRY(run_conv(v, cx.pw1, PRO_NONE, EPI_GELU, v.lnx, rows, L, v.pwh, 4 * L, nullptr, nullptr, err, errlen));
        VOC_TRY(run_conv(v, cx.pw2, PRO_NONE, EPI_SCALE_RESIDUAL, v.pwh, rows, 4 * L, up, L, up, cx.gamma, err, errlen));
        VOC_TRY(snap(v, js + "_cnx", up, rows, L, err, errlen));
        stage_in = up;
    }
    // The Snake that starts every conv of the decoder blocks is applied once per element by the
    // conv that produces its input (z output): dec0 -> block 0's transposed conv, that conv ->
    // unit 0's first conv, a first conv -> its second, a second conv -> the next unit's first /
    // the next block's transposed conv / the final conv. Only the Snake of a first conv's output
    // is kept (its raw output is not read again).
    VOC_TRY(run_conv(v, v.dec0, PRO_NONE, EPI_BIAS, stage_in, rows, L, v.hook ? v.dec_raw : nullptr, v.DD, nullptr, nullptr, err,
                     errlen, v.dec_in, &v.blocks[0].up));
    VOC_TRY(snap(v, "dec0", v.dec_raw, rows, v.DD, err, errlen));
    const float *blk_in = v.dec_in;
    int ch = v.DD;
    for (int b = 0; b < 4; ++b) {
        Block &bk = v.blocks[b];
        VOC_TRY(run_conv(v, bk.up, PRO_NONE, EPI_BIAS, blk_in, rows, ch, v.res[b], bk.Cout, nullptr, nullptr, err, errlen,
                         v.res_s[b], &bk.u[0].c1));
        rows *= bk.rate;
        ch = bk.Cout;
        const std::string bs = "dec" + std::to_string(b + 1) + "_b";
        VOC_TRY(snap(v, bs + "1", v.res[b], rows, ch, err, errlen));
        float *unit_in = v.res_s[b];           // the Snake'd residual stream a unit reads
        for (int k = 0; k < 3; ++k) {
            const Conv *next = k < 2 ? &bk.u[k + 1].c1 : b < 3 ? &v.blocks[b + 1].up : &v.final_conv;
            // the last unit's raw output is read by nothing but the stage hook (the next stage
            // takes its Snake'd copy)
            float *y = k < 2 || v.hook ? v.res[b] : nullptr;
            if (unit_fused(bk.u[k])) {
                // one launch reads unit_in (its k7 window reaches into the neighbouring blocks'
                // rows) while it writes the Snake'd output, so that goes to the other buffer
                float *unit_out = unit_in == v.res_s[b] ? v.mid_s[b] : v.res_s[b];
                launch_unit(v, bk.u[k], unit_in, rows, v.res[b], y, unit_out, *next);
                unit_in = unit_out;
            } else {
                VOC_TRY(run_conv(v, bk.u[k].c1, PRO_NONE, EPI_BIAS, v.res_s[b], rows, ch, nullptr, ch, nullptr, nullptr, err,
                                 errlen, v.mid_s[b], &bk.u[k].c2));
                VOC_TRY(run_conv(v, bk.u[k].c2, PRO_NONE, EPI_RESIDUAL, v.mid_s[b], rows, ch, y, ch, v.res[b], nullptr, err,
                                 errlen, v.res_s[b], next));
            }
            VOC_TRY(snap(v, bs + std::to_string(2 + k), v.res[b], rows, ch, err, errlen));
        }
        blk_in = unit_in;
    }
    VOC_TRY(run_conv(v, v.final_conv, PRO_NONE, EPI_CLAMP, blk_in, rows, ch, v.pcm16, 16, nullptr, nullptr, err, errlen));
    hipLaunchKernelGGL(k_take_col0, dim3((rows + BT - 1) / BT), dim3(BT), 0, s, v.pcm16, rows, 16, v.pcm, v.dh_pcm[v.parity],
                       v.d_pos0, T, v.flag, v.dh_flag);
    VOC_TRY(snap(v, "pcm", v.pcm, rows, 1, err, errlen));
    NAVI_TRY_HIP(hipGetLastError(), err, errlen);
    return NAVI_OK;
}

// A chunk: its launch sequence depends only on T and the history parity (every pointer and split
// count is fixed at create, the position lives on the device), so it can be captured once per
// (T, parity) as a HIP graph and replayed (navi_vocoder_set_graphs). Off by default: on MI355X the
// replays measured no faster than host launches (each kernel's own latency, not the launch gap,
// bounds a chunk). With the stage hook on, a chunk always runs eagerly.
navi_status run_chunk(navi_vocoder &v, int T, char *err, size_t errlen) {
    hipStream_t s = device_state().stream;
    if (!v.use_graphs || v.hook) {
        VOC_TRY(decode_chunk(v, T, err, errlen));
    } else {
        const std::pair<int, int> key{T, v.parity};
        hipGraphExec_t ex = nullptr;
        for (auto &g : v.graphs)
            if (g.first == key) ex = g.second;
        if (!ex) {
            NAVI_TRY_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), err, errlen);
            const navi_status st = decode_chunk(v, T, err, errlen);
            hipGraph_t graph = nullptr;
            const hipError_t ec = hipStreamEndCapture(s, &graph);
            if (st != NAVI_OK) {
                if (graph) (void) hipGraphDestroy(graph);
                return st;
            }
            NAVI_TRY_HIP(ec, err, errlen);
            const hipError_t ei = hipGraphInstantiateWithFlags(&ex, graph, 0);
            (void) hipGraphDestroy(graph);
            NAVI_TRY_HIP(ei, err, errlen);
            v.graphs.push_back({key, ex});
        }
        NAVI_TRY_HIP(hipGraphLaunch(ex, s), err, errlen);
    }
    v.parity ^= 1;
    return NAVI_OK;
}

// ---- create ----------------------------------------------------------------------------

struct Binder {
    const navi_tensor_ref *t;
    int n;
    char *err;
    size_t errlen;
    template <class T>
    navi_status get(const std::string &name, int dtype, uint64_t d0, uint64_t d1, uint64_t d2, const T *&out) const {
        const navi_tensor_ref *r = find_tensor(t, n, name);
        if (!r) {
            set_err(err, errlen, "vocoder: missing tensor '%s'", name.c_str());
            return NAVI_ERR_INVALID;
        }
        const int nd = d2 ? 3 : d1 ? 2 : 1;
        const bool ok = r->dtype == dtype && r->ndim == nd && r->dims[0] == d0 && (nd < 2 || r->dims[1] == d1) &&
                        (nd < 3 || r->dims[2] == d2);
        if (!ok) {
            set_err(err, errlen, "vocoder: tensor '%s' has an unexpected dtype or shape", name.c_str());
            return NAVI_ERR_INVALID;
        }
        if (reinterpret_cast<uintptr_t>(r->ptr) & 15u) {
            set_err(err, errlen, "vocoder: tensor '%s' is not 16-byte aligned", name.c_str());
            return NAVI_ERR_INVALID;
        }
        out = static_cast<const T *>(r->ptr);
        return NAVI_OK;
    }
};

const std::string DEC = "codec.decoder.";

} // namespace

extern "C" {

navi_status navi_vocoder_create(const navi_vocoder_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                                int32_t max_chunk_frames, navi_vocoder **out, char *err, size_t errlen) {
    if (!p || !tensors || !out) {
        set_err(err, errlen, "vocoder: null argument");
        return NAVI_ERR_INVALID;
    }
    *out = nullptr;
    navi_status st = ensure_device(err, errlen);
    if (st != NAVI_OK) return st;
    const navi_xformer_params &xf = p->xf;
    const int VH = xf.hidden, L = p->latent_dim, CD = p->codebook_dim, DD = p->decoder_dim, HDT = xf.n_head * xf.head_dim;
    int spf = p->upsampling_ratios[0] * p->upsampling_ratios[1];
    for (int b = 0; b < 4; ++b) spf *= p->upsample_rates[b];
    bool ok = xf.n_head == xf.n_kv_head && (xf.head_dim == 64 || xf.head_dim == 128) &&
              attention_lds(p->sliding_window, xf.head_dim) <= 64 * 1024 && p->n_q <= 16 && VH == 512 && HDT == 1024 &&
              xf.ff == 1024 && L == 4 * BT &&
              CD % 64 == 0 && DD % 64 == 0 && HDT % 64 == 0 && xf.ff % 64 == 0 && p->sliding_window >= 1 &&
              p->sliding_window <= 128 && spf == p->samples_per_frame && p->n_semantic == 1 && p->n_q >= 2 &&
              max_chunk_frames >= 1 && max_chunk_frames <= 4096;
    int width = DD;
    for (int b = 0; b < 4 && ok; ++b) {
        ok = width % 2 == 0 && (width / 2) % 32 == 0 && width % 32 == 0 && p->upsample_rates[b] >= 1;
        width /= 2;
    }
    for (int j = 0; j < 2 && ok; ++j) ok = p->upsampling_ratios[j] >= 1;
    if (!ok) {
        set_err(err, errlen, "vocoder: unsupported configuration");
        return NAVI_ERR_UNSUPPORTED;
    }
    auto v = new navi_vocoder();
    auto fail = [&](navi_status s_) { delete v; return s_; };
    v->p = *p;
    v->cmax = max_chunk_frames;
    v->VH = VH; v->L = L; v->CD = CD; v->DD = DD; v->HDT = HDT;
    v->ring = 8;
    while (v->ring < p->sliding_window + max_chunk_frames) v->ring *= 2;
    const Binder bd{tensors, n_tensors, err, errlen};
    hipStream_t s = device_state().stream;
    const uint64_t VQ = CD / 2;
#define VB(T, name, dt, d0, d1, d2, outp)                                                \
    do {                                                                                \
        if ((st = bd.get<T>((name), (dt), (d0), (d1), (d2), (outp))) != NAVI_OK) return fail(st); \
    } while (0)
#define VA(ptr, n_)                                                                     \
    do {                                                                                \
        if ((st = v->alloc(ptr, (n_), err, errlen)) != NAVI_OK) return fail(st);        \
    } while (0)
    auto relayout = [&](const uint16_t *w, int Cout, int Cin, int K, const uint16_t *&dst) -> navi_status {
        uint16_t *o = nullptr;
        navi_status s_ = v->alloc(o, static_cast<size_t>(Cout) * Cin * K, err, errlen);
        if (s_ != NAVI_OK) return s_;
        const size_t nn = static_cast<size_t>(Cout) * Cin * K;
        hipLaunchKernelGGL(k_relayout_conv, dim3(static_cast<unsigned>((nn + BT - 1) / BT)), dim3(BT), 0, s, w, Cout, Cin, K, o);
        dst = o;
        return NAVI_OK;
    };
    auto tconv = [&](const uint16_t *w, int Cin, int Cout, int k, int stride, const uint16_t *&dst) -> navi_status {
        uint16_t *o = nullptr;
        navi_status s_ = v->alloc(o, static_cast<size_t>(Cin) * Cout * k, err, errlen);
        if (s_ != NAVI_OK) return s_;
        const size_t nn = static_cast<size_t>(Cin) * Cout * k;
        hipLaunchKernelGGL(k_relayout_tconv, dim3(static_cast<unsigned>((nn + BT - 1) / BT)), dim3(BT), 0, s, w, Cin, Cout, k,
                           stride, o);
        dst = o;
        return NAVI_OK;
    };
    auto snake = [&](const std::string &prefix, int C, const float *&sa, const float *&sb) -> navi_status {
        const float *al = nullptr, *be = nullptr;
        navi_status s_ = bd.get<float>(prefix + ".alpha", NAVI_DT_F32, C, 0, 0, al);
        if (s_ == NAVI_OK) s_ = bd.get<float>(prefix + ".beta", NAVI_DT_F32, C, 0, 0, be);
        float *a_ = nullptr, *b_ = nullptr;
        if (s_ == NAVI_OK) s_ = v->alloc(a_, C, err, errlen);
        if (s_ == NAVI_OK) s_ = v->alloc(b_, C, err, errlen);
        if (s_ != NAVI_OK) return s_;
        hipLaunchKernelGGL(k_snake_prep, dim3((C + BT - 1) / BT), dim3(BT), 0, s, al, be, C, a_, b_);
        sa = a_;
        sb = b_;
        return NAVI_OK;
    };
    auto hist = [&](Conv &c) -> navi_status {
        c.H = (c.K - 1) * c.dil;
        if (c.H == 0) return NAVI_OK;
        navi_status s_ = v->alloc(c.hbuf[0], static_cast<size_t>(c.H) * c.Cin, err, errlen);
        if (s_ == NAVI_OK) s_ = v->alloc(c.hbuf[1], static_cast<size_t>(c.H) * c.Cin, err, errlen);
        return s_;
    };
    // RVQ front end: codebooks (rest concatenated) and the two output projections as one [CD][CD]
    VB(uint16_t, DEC + "quantizer.rvq_first.vq.layers.0._codebook.codebook", NAVI_DT_F16, p->codebook_size, VQ, 0, v->cb_first);
    VA(v->cb_rest, static_cast<size_t>(p->n_q - 1) * p->codebook_size * VQ);
    for (int q = 0; q < p->n_q - 1; ++q) {
        const uint16_t *cb = nullptr;
        VB(uint16_t, DEC + "quantizer.rvq_rest.vq.layers." + std::to_string(q) + "._codebook.codebook", NAVI_DT_F16,
           p->codebook_size, VQ, 0, cb);
        if (hipMemcpyAsync(v->cb_rest + static_cast<size_t>(q) * p->codebook_size * VQ, cb, p->codebook_size * VQ * 2,
                           hipMemcpyDeviceToDevice, s) != hipSuccess) {
            set_err(err, errlen, "vocoder: codebook copy failed");
            return fail(NAVI_ERR_HIP);
        }
    }
    {
        const uint16_t *pf = nullptr, *pr = nullptr;
        VB(uint16_t, DEC + "quantizer.rvq_first.output_proj.weight", NAVI_DT_F16, CD, VQ, 1, pf);
        VB(uint16_t, DEC + "quantizer.rvq_rest.output_proj.weight", NAVI_DT_F16, CD, VQ, 1, pr);
        uint16_t *w = nullptr;
        VA(w, static_cast<size_t>(CD) * CD);
        if (hipMemcpy2DAsync(w, CD * 2, pf, VQ * 2, VQ * 2, CD, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipMemcpy2DAsync(w + VQ, CD * 2, pr, VQ * 2, VQ * 2, CD, hipMemcpyDeviceToDevice, s) != hipSuccess) {
            set_err(err, errlen, "vocoder: projection copy failed");
            return fail(NAVI_ERR_HIP);
        }
        v->rvq_proj.w = w;
        v->rvq_proj.Cin = CD;
        v->rvq_proj.Cout = CD;
    }
    {
        const uint16_t *w = nullptr;
        VB(uint16_t, DEC + "pre_conv.conv.weight", NAVI_DT_F16, L, CD, 3, w);
        VB(float, DEC + "pre_conv.conv.bias", NAVI_DT_F32, L, 0, 0, v->pre_conv.bias);
        v->pre_conv.Cin = CD; v->pre_conv.Cout = L; v->pre_conv.K = 3;
        if ((st = relayout(w, L, CD, 3, v->pre_conv.w)) != NAVI_OK || (st = hist(v->pre_conv)) != NAVI_OK) return fail(st);
    }
    const std::string pt = DEC + "pre_transformer.";
    VB(uint16_t, pt + "input_proj.weight", NAVI_DT_F16, VH, L, 0, v->in_proj.w);
    VB(float, pt + "input_proj.bias", NAVI_DT_F32, VH, 0, 0, v->in_proj.bias);
    v->in_proj.Cin = L; v->in_proj.Cout = VH;
    VB(uint16_t, pt + "output_proj.weight", NAVI_DT_F16, L, VH, 0, v->out_proj.w);
    VB(float, pt + "output_proj.bias", NAVI_DT_F32, L, 0, 0, v->out_proj.bias);
    v->out_proj.Cin = VH; v->out_proj.Cout = L;
    VB(float, pt + "norm.weight", NAVI_DT_F32, VH, 0, 0, v->final_norm);
    v->layers.resize(xf.n_layer);
    for (int l = 0; l < xf.n_layer; ++l) {
        const std::string lp = pt + "layers." + std::to_string(l) + ".";
        TLayer &ly = v->layers[l];
        VB(float, lp + "input_layernorm.weight", NAVI_DT_F32, VH, 0, 0, ly.ln1);
        VB(float, lp + "post_attention_layernorm.weight", NAVI_DT_F32, VH, 0, 0, ly.ln2);
        VB(float, lp + "self_attn_layer_scale.scale", NAVI_DT_F32, VH, 0, 0, ly.attn_scale);
        VB(float, lp + "mlp_layer_scale.scale", NAVI_DT_F32, VH, 0, 0, ly.mlp_scale);
        const uint16_t *wq, *wk, *wv, *wg, *wu;
        VB(uint16_t, lp + "self_attn.q_proj.weight", NAVI_DT_F16, HDT, VH, 0, wq);
        VB(uint16_t, lp + "self_attn.k_proj.weight", NAVI_DT_F16, HDT, VH, 0, wk);
        VB(uint16_t, lp + "self_attn.v_proj.weight", NAVI_DT_F16, HDT, VH, 0, wv);
        VB(uint16_t, lp + "self_attn.o_proj.weight", NAVI_DT_F16, VH, HDT, 0, ly.o.w);
        VB(uint16_t, lp + "mlp.gate_proj.weight", NAVI_DT_F16, xf.ff, VH, 0, wg);
        VB(uint16_t, lp + "mlp.up_proj.weight", NAVI_DT_F16, xf.ff, VH, 0, wu);
        VB(uint16_t, lp + "mlp.down_proj.weight", NAVI_DT_F16, VH, xf.ff, 0, ly.down.w);
        uint16_t *qkv = nullptr, *gu = nullptr;
        VA(qkv, static_cast<size_t>(3) * HDT * VH);
        VA(gu, static_cast<size_t>(2) * xf.ff * VH);
        const size_t mq = static_cast<size_t>(HDT) * VH * 2, mg = static_cast<size_t>(xf.ff) * VH * 2;
        if (hipMemcpyAsync(qkv, wq, mq, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipMemcpyAsync(qkv + mq / 2, wk, mq, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipMemcpyAsync(qkv + mq, wv, mq, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipMemcpyAsync(gu, wg, mg, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipMemcpyAsync(gu + mg / 2, wu, mg, hipMemcpyDeviceToDevice, s) != hipSuccess) {
            set_err(err, errlen, "vocoder: weight copy failed");
            return fail(NAVI_ERR_HIP);
        }
        ly.qkv.w = qkv; ly.qkv.Cin = VH; ly.qkv.Cout = 3 * HDT;
        ly.gu.w = gu; ly.gu.Cin = VH; ly.gu.Cout = 2 * xf.ff;
        ly.o.Cin = HDT; ly.o.Cout = VH;
        ly.down.Cin = xf.ff; ly.down.Cout = VH;
        VA(ly.kc, static_cast<size_t>(v->ring) * HDT);
        VA(ly.vc, static_cast<size_t>(v->ring) * HDT);
    }
    for (int j = 0; j < 2; ++j) {
        const int r = p->upsampling_ratios[j];
        const std::string up = DEC + "upsample." + std::to_string(j) + ".";
        const uint16_t *w = nullptr;
        VB(uint16_t, up + "0.conv.weight", NAVI_DT_F16, L, L, r, w);
        VB(float, up + "0.conv.bias", NAVI_DT_F32, L, 0, 0, v->up_conv[j].bias);
        Conv &c = v->up_conv[j];
        c.Cin = L; c.Cout = L; c.K = 1; c.phases = r;
        if ((st = tconv(w, L, L, r, r, c.w)) != NAVI_OK) return fail(st);
        ConvNeXt &cx = v->cnx[j];
        const uint16_t *dw = nullptr;
        VB(uint16_t, up + "1.dwconv.conv.weight", NAVI_DT_F16, L, 1, 7, dw);
        {
            uint16_t *t_ = nullptr;
            VA(t_, static_cast<size_t>(7) * L);
            hipLaunchKernelGGL(k_tap_major, dim3((7 * L + BT - 1) / BT), dim3(BT), 0, s, dw, L, 7, t_);
            cx.dwt = t_;
        }
        VB(float, up + "1.dwconv.conv.bias", NAVI_DT_F32, L, 0, 0, cx.dw_b);
        VB(float, up + "1.norm.weight", NAVI_DT_F32, L, 0, 0, cx.ln_w);
        VB(float, up + "1.norm.bias", NAVI_DT_F32, L, 0, 0, cx.ln_b);
        VB(float, up + "1.gamma", NAVI_DT_F32, L, 0, 0, cx.gamma);
        VB(uint16_t, up + "1.pwconv1.weight", NAVI_DT_F16, 4 * L, L, 0, cx.pw1.w);
        VB(float, up + "1.pwconv1.bias", NAVI_DT_F32, 4 * L, 0, 0, cx.pw1.bias);
        VB(uint16_t, up + "1.pwconv2.weight", NAVI_DT_F16, L, 4 * L, 0, cx.pw2.w);
        VB(float, up + "1.pwconv2.bias", NAVI_DT_F32, L, 0, 0, cx.pw2.bias);
        cx.pw1.Cin = L; cx.pw1.Cout = 4 * L;
        cx.pw2.Cin = 4 * L; cx.pw2.Cout = L;
        VA(cx.hbuf[0], static_cast<size_t>(6) * L);
        VA(cx.hbuf[1], static_cast<size_t>(6) * L);
    }
    {
        const uint16_t *w = nullptr;
        VB(uint16_t, DEC + "decoder.0.conv.weight", NAVI_DT_F16, DD, L, 7, w);
        VB(float, DEC + "decoder.0.conv.bias", NAVI_DT_F32, DD, 0, 0, v->dec0.bias);
        v->dec0.Cin = L; v->dec0.Cout = DD; v->dec0.K = 7;
        if ((st = relayout(w, DD, L, 7, v->dec0.w)) != NAVI_OK || (st = hist(v->dec0)) != NAVI_OK) return fail(st);
    }
    const size_t C = static_cast<size_t>(max_chunk_frames);
    width = DD;
    size_t rows = static_cast<size_t>(p->upsampling_ratios[0]) * p->upsampling_ratios[1];
    const int dils[3] = {1, 3, 9};
    for (int b = 0; b < 4; ++b) {
        Block &bk = v->blocks[b];
        bk.rate = p->upsample_rates[b];
        bk.Cin = width;
        bk.Cout = width / 2;
        const std::string bp = DEC + "decoder." + std::to_string(b + 1) + ".block.";
        const uint16_t *w = nullptr;
        VB(uint16_t, bp + "1.conv.weight", NAVI_DT_F16, bk.Cin, bk.Cout, 2 * bk.rate, w);
        VB(float, bp + "1.conv.bias", NAVI_DT_F32, bk.Cout, 0, 0, bk.up.bias);
        bk.up.Cin = bk.Cin; bk.up.Cout = bk.Cout; bk.up.K = 2; bk.up.phases = bk.rate;
        if ((st = tconv(w, bk.Cin, bk.Cout, 2 * bk.rate, bk.rate, bk.up.w)) != NAVI_OK || (st = hist(bk.up)) != NAVI_OK ||
            (st = snake(bp + "0", bk.Cin, bk.up.sa, bk.up.sb)) != NAVI_OK)
            return fail(st);
        for (int k = 0; k < 3; ++k) {
            const std::string rp = bp + std::to_string(2 + k) + ".";
            Unit &un = bk.u[k];
            const uint16_t *w1 = nullptr, *w2 = nullptr;
            VB(uint16_t, rp + "conv1.conv.weight", NAVI_DT_F16, bk.Cout, bk.Cout, 7, w1);
            VB(float, rp + "conv1.conv.bias", NAVI_DT_F32, bk.Cout, 0, 0, un.c1.bias);
            VB(uint16_t, rp + "conv2.conv.weight", NAVI_DT_F16, bk.Cout, bk.Cout, 1, w2);
            VB(float, rp + "conv2.conv.bias", NAVI_DT_F32, bk.Cout, 0, 0, un.c2.bias);
            un.c1.Cin = un.c1.Cout = bk.Cout; un.c1.K = 7; un.c1.dil = dils[k];
            un.c2.Cin = un.c2.Cout = bk.Cout; un.c2.w = w2;
            if ((st = relayout(w1, bk.Cout, bk.Cout, 7, un.c1.w)) != NAVI_OK || (st = hist(un.c1)) != NAVI_OK ||
                (st = snake(rp + "act1", bk.Cout, un.c1.sa, un.c1.sb)) != NAVI_OK ||
                (st = snake(rp + "act2", bk.Cout, un.c2.sa, un.c2.sb)) != NAVI_OK)
                return fail(st);
        }
        rows *= bk.rate;
        VA(v->res[b], rows * C * bk.Cout);
        VA(v->res_s[b], rows * C * bk.Cout);
        VA(v->mid_s[b], rows * C * bk.Cout);
        width = bk.Cout;
    }
    {
        const uint16_t *w = nullptr, *w1 = nullptr;
        const float *b = nullptr;
        VB(uint16_t, DEC + "decoder.6.conv.weight", NAVI_DT_F16, 1, width, 7, w);
        VB(float, DEC + "decoder.6.conv.bias", NAVI_DT_F32, 1, 0, 0, b);
        Conv &c = v->final_conv;
        c.Cin = width; c.Cout = 16; c.K = 7;
        // tap-major [1][7][Cin] into row 0 of a zeroed [16][7][Cin]; bias 0 for the padding columns
        if ((st = relayout(w, 1, width, 7, w1)) != NAVI_OK) return fail(st);
        uint16_t *wp = nullptr;
        float *bp = nullptr;
        VA(wp, static_cast<size_t>(16) * 7 * width);
        VA(bp, 16);
        if (hipMemcpyAsync(wp, w1, static_cast<size_t>(7) * width * 2, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipMemcpyAsync(bp, b, 4, hipMemcpyDeviceToDevice, s) != hipSuccess) {
            set_err(err, errlen, "vocoder: final conv copy failed");
            return fail(NAVI_ERR_HIP);
        }
        c.w = wp;
        c.bias = bp;
        if ((st = hist(c)) != NAVI_OK || (st = snake(DEC + "decoder.5", width, c.sa, c.sb)) != NAVI_OK) return fail(st);
    }
    float invf[64] = {};
    for (int i = 0; i < xf.head_dim / 2; ++i) invf[i] = static_cast<float>(1.0 / std::pow(xf.rope_theta, (2.0 * i) / xf.head_dim));
    VA(v->invf, 64);
    VA(v->flag, 1);
    VA(v->d_pos0, 1);
    VA(v->lat_in, C * CD);
    VA(v->lat, C * CD);
    VA(v->pre, C * L);
    v->lxs = VH + ROW_PAD;
    v->latt = HDT + ROW_PAD;
    v->lgu = xf.ff + ROW_PAD;
    VA(v->xs, C * v->lxs);
    VA(v->xn, C * VH);
    VA(v->qkv, C * 3 * HDT);
    VA(v->att, C * v->latt);
    VA(v->gu, C * v->lgu);
    VA(v->snapbuf, C * std::max(VH, HDT));
    VA(v->post, C * L);
    const size_t up_rows = C * p->upsampling_ratios[0] * p->upsampling_ratios[1];
    VA(v->upx[0], C * p->upsampling_ratios[0] * L);
    VA(v->upx[1], up_rows * L);
    VA(v->lnx, up_rows * L);
    VA(v->pwh, up_rows * 4 * L);
    VA(v->dec_in, up_rows * DD);
    VA(v->dec_raw, up_rows * DD);
    VA(v->pcm, C * p->samples_per_frame);
    VA(v->pcm16, C * p->samples_per_frame * 16);
    {
        // split counts from the rows of a 16-frame chunk (or the largest chunk if smaller), and
        // the workspace the largest chunk then needs
        size_t need = 0;
        const int Cn = static_cast<int>(std::min<size_t>(C, 16)), Cf = static_cast<int>(C);
        auto upd = [&](Conv &c, int rows_per_frame) {
            c.wide = conv_takes_wide(c, rows_per_frame);
            c.S = c.wide ? wide_splits(c, Cn * rows_per_frame) : conv_splits(c, Cn * rows_per_frame);
            const size_t rows = c.wide ? std::min<size_t>(static_cast<size_t>(Cf) * rows_per_frame, wide_split_max_rows(c))
                                       : static_cast<size_t>(Cf) * rows_per_frame;
            if (c.S > 1) need = std::max(need, static_cast<size_t>(c.S) * rows * c.phases * c.Cout);
        };
        upd(v->rvq_proj, 1); upd(v->pre_conv, 1); upd(v->in_proj, 1); upd(v->out_proj, 1);
        for (TLayer &ly : v->layers) { upd(ly.qkv, 1); upd(ly.o, 1); upd(ly.gu, 1); upd(ly.down, 1); }
        int R = 1;
        for (int j = 0; j < 2; ++j) {
            upd(v->up_conv[j], R);
            R *= p->upsampling_ratios[j];
            upd(v->cnx[j].pw1, R); upd(v->cnx[j].pw2, R);
        }
        upd(v->dec0, R);
        for (Block &bk : v->blocks) {
            upd(bk.up, R);
            R *= bk.rate;
            for (Unit &u : bk.u) { upd(u.c1, R); upd(u.c2, R); }
        }
        upd(v->final_conv, R);
        v->part_floats = need;
        VA(v->part, need);
    }
    {
        std::vector<ZeroSpan> spans;
        auto add = [&](void *ptr, size_t words) {
            if (ptr && words) spans.push_back({static_cast<uint32_t *>(ptr), static_cast<uint32_t>(words)});
        };
        auto addc = [&](Conv &c) {
            add(c.hbuf[0], static_cast<size_t>(c.H) * c.Cin);
            add(c.hbuf[1], static_cast<size_t>(c.H) * c.Cin);
        };
        addc(v->pre_conv); addc(v->dec0); addc(v->final_conv);
        for (int j = 0; j < 2; ++j) {
            add(v->cnx[j].hbuf[0], 6 * static_cast<size_t>(v->L));
            add(v->cnx[j].hbuf[1], 6 * static_cast<size_t>(v->L));
        }
        for (Block &b : v->blocks) {
            addc(b.up);
            for (Unit &u : b.u) addc(u.c1);
        }
        add(v->d_pos0, 1);
        VA(v->d_spans, spans.size());
        v->n_spans = static_cast<int>(spans.size());
        if (hipMemcpyAsync(v->d_spans, spans.data(), spans.size() * sizeof(ZeroSpan), hipMemcpyHostToDevice, s) != hipSuccess) {
            set_err(err, errlen, "vocoder: span table copy failed");
            return fail(NAVI_ERR_HIP);
        }
    }
#undef VB
#undef VA
    if (hipMemcpyAsync(v->invf, invf, sizeof invf, hipMemcpyHostToDevice, s) != hipSuccess || hipEventCreate(&v->ev0) != hipSuccess ||
        hipEventCreate(&v->ev1) != hipSuccess || hipEventCreate(&v->ev_slot[0]) != hipSuccess ||
        hipEventCreate(&v->ev_slot[1]) != hipSuccess || hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess) {
        set_err(err, errlen, "vocoder: HIP setup failed");
        return fail(NAVI_ERR_HIP);
    }
    {
        // per slot: cmax frames of codes, then cmax frames of PCM (16-byte aligned), then the flag word
        const size_t codes_b = (static_cast<size_t>(C) * p->n_q * 4 + 15) / 16 * 16;
        const size_t pcm_b = (static_cast<size_t>(C) * p->samples_per_frame * 4 + 15) / 16 * 16;
        if (hipHostMalloc(&v->h_buf, 2 * (codes_b + pcm_b) + 64, hipHostMallocCoherent) != hipSuccess) {
            set_err(err, errlen, "vocoder: pinned staging allocation failed");
            return fail(NAVI_ERR_HIP);
        }
        void *dbuf = nullptr;
        if (hipHostGetDevicePointer(&dbuf, v->h_buf, 0) != hipSuccess) {
            set_err(err, errlen, "vocoder: no device address for the pinned staging");
            return fail(NAVI_ERR_HIP);
        }
        unsigned char *hb = static_cast<unsigned char *>(v->h_buf), *db = static_cast<unsigned char *>(dbuf);
        for (int b = 0; b < 2; ++b) {
            const size_t o = b * (codes_b + pcm_b);
            v->h_codes[b] = reinterpret_cast<int32_t *>(hb + o);
            v->dh_codes[b] = reinterpret_cast<int32_t *>(db + o);
            v->h_pcm[b] = reinterpret_cast<float *>(hb + o + codes_b);
            v->dh_pcm[b] = reinterpret_cast<float *>(db + o + codes_b);
        }
        v->h_flag = reinterpret_cast<uint32_t *>(hb + 2 * (codes_b + pcm_b));
        v->dh_flag = reinterpret_cast<uint32_t *>(db + 2 * (codes_b + pcm_b));
    }
    *out = v;
    return NAVI_OK;
}

void navi_vocoder_destroy(navi_vocoder *v) {
    if (!v) return;
    (void) hipStreamSynchronize(device_state().stream);
    delete v;
}

navi_status navi_vocoder_reset(navi_vocoder *v) {
    if (!v) return NAVI_ERR_INVALID;
    hipStream_t s = device_state().stream;
    // every causal history (conv, depthwise conv) and the position back to zero; the K/V rings need
    // no clearing: attention reads only positions already written this utterance
    // (asynchronous, as Vocoder::reset's memsets are: the next decode is queued behind it on the stream)
    hipLaunchKernelGGL(k_zero_spans, dim3(v->n_spans), dim3(BT), 0, s, v->d_spans);
    return hipGetLastError() == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

navi_status navi_vocoder_decode(navi_vocoder *v, const int32_t *codes, int32_t n_frames, float *pcm, char *err,
                                size_t errlen) {
    if (!v || (!codes && n_frames > 0) || (!pcm && n_frames > 0) || n_frames < 0) {
        set_err(err, errlen, "vocoder: null argument");
        return NAVI_ERR_INVALID;
    }
    const int nq = v->p.n_q, spf = v->p.samples_per_frame;
    for (int64_t i = 0; i < static_cast<int64_t>(n_frames) * nq; ++i)
        if (codes[i] < 0 || codes[i] >= v->p.codebook_size) {
            set_err(err, errlen, "vocoder: code %d at %lld outside the codebook", codes[i], static_cast<long long>(i));
            return NAVI_ERR_INVALID;
        }
    hipStream_t s = device_state().stream;
    if (v->flag_dirty) NAVI_TRY_HIP(hipMemsetAsync(v->flag, 0, 4, s), err, errlen);
    v->flag_dirty = true;                                  // until the call ends with the flag read as zero
    NAVI_TRY_HIP(hipEventRecord(v->ev0, s), err, errlen);
    // Chunk k reads its codes from, and writes its PCM into, the pinned slot of its history parity
    // (the parity alternates per chunk, so chunk k's slot is chunk k - 2's): before writing the
    // slot's codes, the chunk that used it last has finished and its PCM is handed over, while
    // chunk k - 1 still runs.
    const int cmax = v->cmax, nch = (n_frames + cmax - 1) / cmax, b0 = v->parity;
    auto hand_over = [&](int k) -> navi_status {
        const int b = (b0 + k) & 1, T = std::min(cmax, n_frames - k * cmax);
        NAVI_TRY_HIP(hipEventSynchronize(v->ev_slot[b]), err, errlen);
        std::memcpy(pcm + static_cast<size_t>(k) * cmax * spf, v->h_pcm[b], static_cast<size_t>(T) * spf * 4);
        return NAVI_OK;
    };
    *v->h_flag = 0;
    for (int k = 0; k < nch; ++k) {
        const int b = v->parity, f0 = k * cmax, T = std::min(cmax, n_frames - f0);
        if (k >= 2) VOC_TRY(hand_over(k - 2));
        std::memcpy(v->h_codes[b], codes + static_cast<size_t>(f0) * nq, static_cast<size_t>(T) * nq * 4);
        const navi_status st = run_chunk(*v, T, err, errlen);
        if (st != NAVI_OK) {
            (void) hipStreamSynchronize(s);
            return st;
        }
        NAVI_TRY_HIP(hipEventRecord(v->ev_slot[b], s), err, errlen);
    }
    NAVI_TRY_HIP(hipEventRecord(v->ev1, s), err, errlen);
    NAVI_TRY_HIP(hipStreamSynchronize(s), err, errlen);
    for (int k = std::max(0, nch - 2); k < nch; ++k) VOC_TRY(hand_over(k));
    float ms = 0.f;
    NAVI_TRY_HIP(hipEventElapsedTime(&ms, v->ev0, v->ev1), err, errlen);
    v->last_ms = ms;
    if (*v->h_flag) {
        set_err(err, errlen, "vocoder: an activation is outside the f16 range (|x| >= 65504 or NaN)");
        return NAVI_ERR_INVALID;
    }
    v->flag_dirty = false;
    return NAVI_OK;
}

navi_status navi_vocoder_set_graphs(navi_vocoder *v, int32_t enabled) {
    if (!v) return NAVI_ERR_INVALID;
    v->use_graphs = enabled != 0;
    return NAVI_OK;
}

navi_status navi_vocoder_set_stage_hook(navi_vocoder *v, navi_stage_fn fn, void *user) {
    if (!v) return NAVI_ERR_INVALID;
    v->hook = fn;
    v->hook_user = user;
    return NAVI_OK;
}

int32_t navi_vocoder_owns_tensor(const char *name) {
    (void) name;
    return 0;   // every codec tensor is read from the weight arena; the re-laid-out copies are made on the device
}

int32_t navi_vocoder_samples_per_frame(const navi_vocoder *v) { return v ? v->p.samples_per_frame : 0; }
int32_t navi_vocoder_max_chunk_frames(const navi_vocoder *v) { return v ? v->cmax : 0; }
double navi_vocoder_last_ms(const navi_vocoder *v) { return v ? v->last_ms : 0.0; }

} // extern "C"
