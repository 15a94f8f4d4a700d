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
//  * The last decoder block's 96-channel convs and the final conv run on k_conv_c96: a block
//    stages its whole input window and each tap's weights in LDS and covers every output
//    channel, reading the input ~1.4x instead of ~3.7x.
//  * Streaming state: each causal conv keeps its last (K-1)*dil input rows (the history the
//    next chunk's first rows read), the ConvNeXt depthwise conv its last 6, the attention its
//    K/V in a ring of >= window + chunk positions: chunked decoding equals one-shot decoding.
#include "conv.h"
#include "dev_common.h"
#include "host_util.h"

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

namespace navi_amd {
namespace vc {

using namespace cv;

// new[r] = row r of the last H rows of [old ; x] (the causal history for the next chunk).
__global__ void __launch_bounds__(BT) k_hist_update(const float *old, const float *x, int T, int H, int C, int ldx,
                                                    float *out) {
    const size_t i = static_cast<size_t>(blockIdx.x) * BT + threadIdx.x;
    if (i >= static_cast<size_t>(H) * C) return;
    const int r = static_cast<int>(i / C), c = static_cast<int>(i % C), src = r + T;
    gst(out + i, src < H ? gld(old + static_cast<size_t>(src) * C + c) : gld(x + static_cast<size_t>(src - H) * ldx + c));
}

// e[t] = [cb_first[c0] | sum_{q>=1} cb_rest[q-1][c_q]] (k_rvq, vocoder.hip:125-143).
__global__ void __launch_bounds__(BT) k_rvq(const int32_t *codes, int n_q, const uint16_t *cb_first, const uint16_t *cb_rest,
                                            int dim, int cb_size, float *e) {
    const int t = blockIdx.x;
    const int32_t *c = codes + static_cast<size_t>(t) * n_q;
    for (int i = threadIdx.x; i < 2 * dim; i += BT) {
        float v;
        if (i < dim) {
            v = h2f(gld(cb_first + static_cast<size_t>(gld(c)) * dim + i));
        } else {
            v = 0.f;
            for (int q = 1; q < n_q; ++q)
                v += h2f(gld(cb_rest + (static_cast<size_t>(q - 1) * cb_size + gld(c + q)) * dim + (i - dim)));
        }
        gst(e + static_cast<size_t>(t) * 2 * dim + i, v);
    }
}

// y[t] = RMSNorm(x[t]) * w over C channels.
__global__ void __launch_bounds__(BT) k_rmsnorm(const float *x, const float *w, int C, float eps, float *y) {
    __shared__ float red[4];
    const float *row = x + static_cast<size_t>(blockIdx.x) * C;
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

// ConvNeXt front: causal depthwise k7 conv + LayerNorm over channels (k_dwconv_ln, vocoder.hip:20-54).
// C = 4 * BT channels.
__global__ void __launch_bounds__(BT) k_dwconv_ln(const uint16_t *w, const float *bias, const float *x, const float *hist,
                                                  int C, const float *lw, const float *lb, float eps, float *y) {
    __shared__ float red[8];
    const int t = blockIdx.x;
    float v[4], s = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int c = threadIdx.x + k * BT;
        float acc = gld(bias + c);
        for (int j = 0; j < 7; ++j) {
            const int tt = t - 6 + j;
            const float xv = tt >= 0 ? gld(x + static_cast<size_t>(tt) * C + c) : gld(hist + static_cast<size_t>(6 + tt) * C + c);
            acc = fmaf(h2f(gld(w + c * 7 + j)), xv, acc);
        }
        v[k] = acc;
        s += acc;
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float mean = (red[0] + red[1] + red[2] + red[3]) / static_cast<float>(C);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float d = v[k] - mean;
        ss = fmaf(d, d, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = ss;
    __syncthreads();
    const float inv = rsqrtf((red[4] + red[5] + red[6] + red[7]) / static_cast<float>(C) + eps);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int c = threadIdx.x + k * BT;
        gst(y + static_cast<size_t>(t) * C + c, (v[k] - mean) * inv * gld(lw + c) + gld(lb + c));
    }
}

// RoPE on q and k of row t at position pos0 + t; k and v appended to the ring caches
// (k_rope_append, vocoder.hip:57-84). Row layout [q | k | v], nh heads of hd.
__global__ void __launch_bounds__(BT) k_rope_append(float *qkv, int nh, int hd, int pos0, int ring, const float *invf,
                                                    float *kc, float *vc) {
    const int t = blockIdx.x, pos = pos0 + t, slot = pos % ring, HDT = nh * hd, half = hd / 2;
    float *row = qkv + static_cast<size_t>(t) * 3 * HDT;
    for (int i = threadIdx.x; i < nh * half; i += BT) {
        const int h = i / half, p = i % half;
        float sn, cs;
        sincosf(static_cast<float>(pos) * gld(invf + p), &sn, &cs);
        float *q = row + h * hd, *k = row + HDT + h * hd;
        const float q0 = q[p], q1 = q[p + half], k0 = k[p], k1 = k[p + half];
        q[p] = q0 * cs - q1 * sn;
        q[p + half] = q1 * cs + q0 * sn;
        const float r0 = k0 * cs - k1 * sn, r1 = k1 * cs + k0 * sn;
        gst(kc + static_cast<size_t>(slot) * HDT + h * hd + p, r0);
        gst(kc + static_cast<size_t>(slot) * HDT + h * hd + p + half, r1);
    }
    for (int i = threadIdx.x; i < HDT; i += BT) gst(vc + static_cast<size_t>(slot) * HDT + i, row[2 * HDT + i]);
}

// Sliding-window causal attention: keys max(0, pos - window + 1) .. pos from the rings
// (k_attention, vocoder.hip:87-122). 128 threads, window <= 128, hd <= 128.
__global__ void __launch_bounds__(128) k_window_attn(const float *qkv, int nh, int hd, int pos0, int window, int ring,
                                                     const float *kc, const float *vc, float *out) {
    __shared__ float sc[128], red[4];
    const int t = blockIdx.x, h = blockIdx.y, pos = pos0 + t, HDT = nh * hd;
    const int k0 = max(0, pos - window + 1), n = pos - k0 + 1;
    const float *q = qkv + static_cast<size_t>(t) * 3 * HDT + h * hd;
    const int j = threadIdx.x, wv = j >> 6;
    float s = -INFINITY;
    if (j < n) {
        const float *k = kc + static_cast<size_t>((k0 + j) % ring) * HDT + h * hd;
        float d = 0.f;
        for (int i = 0; i < hd; ++i) d = fmaf(gld(q + i), gld(k + i), d);
        s = d * rsqrtf(static_cast<float>(hd));
    }
    float m = wave_max(s);
    if ((j & 63) == 0) red[wv] = m;
    __syncthreads();
    m = fmaxf(red[0], red[1]);
    const float e = j < n ? expf(s - m) : 0.f;
    float sum = wave_sum(e);
    __syncthreads();
    if ((j & 63) == 0) red[2 + wv] = sum;
    __syncthreads();
    sum = red[2] + red[3];
    sc[j] = e / sum;
    __syncthreads();
    if (j < hd) {
        float acc = 0.f;
        for (int i = 0; i < n; ++i) acc = fmaf(sc[i], gld(vc + static_cast<size_t>((k0 + i) % ring) * HDT + h * hd + j), acc);
        gst(out + static_cast<size_t>(t) * HDT + h * hd + j, acc);
    }
}

// pcm[t] = y[t][0]: the last conv runs on the matrix cores with its one output channel padded to
// a 16-column tile (15 zero weight rows); this keeps column 0.
__global__ void __launch_bounds__(BT) k_take_col0(const float *y, int T, int ld, float *pcm) {
    const int t = blockIdx.x * BT + threadIdx.x;
    if (t < T) gst(pcm + t, gld(y + static_cast<size_t>(t) * ld));
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
    float *hist = nullptr, *hist2 = nullptr;
};

struct TLayer {
    const float *ln1, *ln2, *attn_scale, *mlp_scale;
    Conv qkv, o, gu, down;
    float *kc, *vc;
};

struct ConvNeXt {
    const uint16_t *dw;
    const float *dw_b, *ln_w, *ln_b, *gamma;
    float *hist, *hist2;
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
    int cmax = 0, ring = 0, pos0 = 0, VH = 0, HDT = 0, L = 0, CD = 0, DD = 0;
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
    // buffers
    int32_t *d_codes = nullptr;
    float *e = nullptr, *h = nullptr, *a = nullptr, *x = nullptr, *n = nullptr, *qkv = nullptr, *att = nullptr,
          *gu = nullptr, *u = nullptr, *A = nullptr, *B = nullptr, *G = nullptr, *d = nullptr, *pcm = nullptr;
    float *P[4] = {}, *Q[4] = {}, *ZP[4] = {};
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
        if (ev0) (void) hipEventDestroy(ev0);
        if (ev1) (void) hipEventDestroy(ev1);
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
    NAVI_CONV(PRO_SILU_GATE, EPI_SCALE_RESIDUAL)
    NAVI_CONV(PRO_SILU_GATE, EPI_PARTIAL)
#undef NAVI_CONV
}

int conv_mt(int T) { return T <= 16 ? 1 : 4; }

// The 96-channel convs of the last decoder block (k7 and k1) and the final 96 -> 16 conv run on
// k_conv_c96 (input window and weights staged in LDS, every output channel in one block). Chosen
// by the conv's shape only, so every chunking of the codes runs the same kernel.
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
    NAVI_C96(7, 6, EPI_BIAS)
    NAVI_C96(1, 6, EPI_RESIDUAL)
    NAVI_C96(7, 1, EPI_CLAMP)
#undef NAVI_C96
    return false;
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

// Runs one conv over T input rows; updates its history afterwards. z (optional): also write
// Snake(y) with the Snake parameters of zc, the conv that consumes this output.
navi_status run_conv(navi_vocoder &v, Conv &c, int pro, int epi, const float *x, int T, int ldx, float *y, int ldy,
                     const float *res, const float *scale, char *err, size_t errlen, float *z = nullptr,
                     const Conv *zc = nullptr) {
    hipStream_t s = device_state().stream;
    ConvArgs a{};
    a.x = x; a.hist = c.hist; a.w = c.w; a.bias = c.bias; a.res = res; a.scale = scale;
    a.y = y; a.z = z; a.flag = v.flag; a.ldx = ldx; a.ldy = ldy; a.T = T; a.Cin = c.Cin; a.Cout = c.Cout;
    a.dil = c.dil; a.phases = c.phases; a.lpad = (c.K - 1) * c.dil;   // causal
    if (z) {
        a.za = zc->sa;
        a.zb = zc->sb;
    }
    if (conv_is_c96(c)) {
        if (!launch_c96(c, a, pro, epi, T, s)) {
            set_err(err, errlen, "vocoder: no 96-channel conv kernel for K=%d Cout=%d epilogue %d", c.K, c.Cout, epi);
            return NAVI_ERR_UNSUPPORTED;
        }
    } else {
        const navi_status st = launch_generic(v, c, a, pro, epi, T, err, errlen);
        if (st != NAVI_OK) return st;
    }
    if (c.H > 0) {
        const size_t nh = static_cast<size_t>(c.H) * c.Cin;
        hipLaunchKernelGGL(k_hist_update, dim3(static_cast<unsigned>((nh + BT - 1) / BT)), dim3(BT), 0, s, c.hist, x, T, c.H,
                           c.Cin, ldx, c.hist2);
        std::swap(c.hist, c.hist2);
    }
    return NAVI_OK;
}

#define VOC_TRY(expr)                         \
    do {                                      \
        const navi_status s_ = (expr);        \
        if (s_ != NAVI_OK) return s_;         \
    } while (0)

navi_status decode_chunk(navi_vocoder &v, int T, char *err, size_t errlen) {
    hipStream_t s = device_state().stream;
    const navi_vocoder_params &p = v.p;
    const int VH = v.VH, L = v.L, HDT = v.HDT, FF = p.xf.ff, CD = v.CD;
    hipLaunchKernelGGL(k_rvq, dim3(T), dim3(BT), 0, s, v.d_codes, p.n_q, v.cb_first, v.cb_rest, CD / 2, p.codebook_size, v.e);
    VOC_TRY(run_conv(v, v.rvq_proj, PRO_NONE, EPI_BIAS, v.e, T, CD, v.h, CD, nullptr, nullptr, err, errlen));
    VOC_TRY(run_conv(v, v.pre_conv, PRO_NONE, EPI_BIAS, v.h, T, CD, v.a, L, nullptr, nullptr, err, errlen));
    VOC_TRY(run_conv(v, v.in_proj, PRO_NONE, EPI_BIAS, v.a, T, L, v.x, VH, nullptr, nullptr, err, errlen));
    for (TLayer &ly : v.layers) {
        hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(BT), 0, s, v.x, ly.ln1, VH, p.xf.rms_eps, v.n);
        VOC_TRY(run_conv(v, ly.qkv, PRO_NONE, EPI_BIAS, v.n, T, VH, v.qkv, 3 * HDT, nullptr, nullptr, err, errlen));
        hipLaunchKernelGGL(k_rope_append, dim3(T), dim3(BT), 0, s, v.qkv, p.xf.n_head, p.xf.head_dim, v.pos0, v.ring, v.invf,
                           ly.kc, ly.vc);
        hipLaunchKernelGGL(k_window_attn, dim3(T, p.xf.n_head), dim3(128), 0, s, v.qkv, p.xf.n_head, p.xf.head_dim, v.pos0,
                           p.sliding_window, v.ring, ly.kc, ly.vc, v.att);
        VOC_TRY(run_conv(v, ly.o, PRO_NONE, EPI_SCALE_RESIDUAL, v.att, T, HDT, v.x, VH, v.x, ly.attn_scale, err, errlen));
        hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(BT), 0, s, v.x, ly.ln2, VH, p.xf.rms_eps, v.n);
        VOC_TRY(run_conv(v, ly.gu, PRO_NONE, EPI_BIAS, v.n, T, VH, v.gu, 2 * FF, nullptr, nullptr, err, errlen));
        VOC_TRY(run_conv(v, ly.down, PRO_SILU_GATE, EPI_SCALE_RESIDUAL, v.gu, T, 2 * FF, v.x, VH, v.x, ly.mlp_scale, err,
                         errlen));
    }
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(BT), 0, s, v.x, v.final_norm, VH, p.xf.rms_eps, v.n);
    VOC_TRY(run_conv(v, v.out_proj, PRO_NONE, EPI_BIAS, v.n, T, VH, v.u, L, nullptr, nullptr, err, errlen));
    int R = T;
    const float *src = v.u;
    for (int j = 0; j < 2; ++j) {
        float *dst = j == 0 ? v.A : v.B, *tmp = j == 0 ? v.B : v.A;
        VOC_TRY(run_conv(v, v.up_conv[j], PRO_NONE, EPI_BIAS, src, R, L, dst, L, nullptr, nullptr, err, errlen));
        R *= p.upsampling_ratios[j];
        ConvNeXt &cx = v.cnx[j];
        hipLaunchKernelGGL(k_dwconv_ln, dim3(R), dim3(BT), 0, s, cx.dw, cx.dw_b, dst, cx.hist, L, cx.ln_w, cx.ln_b, 1e-6f, tmp);
        const size_t nh = static_cast<size_t>(6) * L;
        hipLaunchKernelGGL(k_hist_update, dim3(static_cast<unsigned>((nh + BT - 1) / BT)), dim3(BT), 0, s, cx.hist, dst, R, 6,
                           L, L, cx.hist2);
        std::swap(cx.hist, cx.hist2);
        VOC_TRY(run_conv(v, cx.pw1, PRO_NONE, EPI_GELU, tmp, R, L, v.G, 4 * L, nullptr, nullptr, err, errlen));
        VOC_TRY(run_conv(v, cx.pw2, PRO_NONE, EPI_SCALE_RESIDUAL, v.G, R, 4 * L, dst, L, dst, cx.gamma, err, errlen));
        src = dst;
    }
    // The Snake that starts every conv of the decoder blocks is applied once per element by the
    // conv that produces its input (z output): dec0 -> block 0 up, up -> unit 0 conv1, conv1 ->
    // conv2, conv2 -> next conv1 / next block's up / the final conv. P holds the residual stream,
    // ZP its Snake for the next consumer, Q the Snake of conv1's output (conv1's raw output is not
    // needed).
    VOC_TRY(run_conv(v, v.dec0, PRO_NONE, EPI_BIAS, src, R, L, nullptr, v.DD, nullptr, nullptr, err, errlen, v.d,
                     &v.blocks[0].up));
    const float *in = v.d;
    int width = v.DD;
    for (int b = 0; b < 4; ++b) {
        Block &bk = v.blocks[b];
        VOC_TRY(run_conv(v, bk.up, PRO_NONE, EPI_BIAS, in, R, width, v.P[b], bk.Cout, nullptr, nullptr, err, errlen, v.ZP[b],
                         &bk.u[0].c1));
        R *= bk.rate;
        width = bk.Cout;
        for (int k = 0; k < 3; ++k) {
            const Conv *next = k < 2 ? &bk.u[k + 1].c1 : b < 3 ? &v.blocks[b + 1].up : &v.final_conv;
            VOC_TRY(run_conv(v, bk.u[k].c1, PRO_NONE, EPI_BIAS, v.ZP[b], R, width, nullptr, width, nullptr, nullptr, err,
                             errlen, v.Q[b], &bk.u[k].c2));
            VOC_TRY(run_conv(v, bk.u[k].c2, PRO_NONE, EPI_RESIDUAL, v.Q[b], R, width, v.P[b], width, v.P[b], nullptr, err,
                             errlen, v.ZP[b], next));
        }
        in = v.ZP[b];
    }
    VOC_TRY(run_conv(v, v.final_conv, PRO_NONE, EPI_CLAMP, in, R, width, v.pcm16, 16, nullptr, nullptr, err, errlen));
    hipLaunchKernelGGL(k_take_col0, dim3((R + BT - 1) / BT), dim3(BT), 0, s, v.pcm16, R, 16, v.pcm);
    v.pos0 += T;
    NAVI_TRY_HIP(hipGetLastError(), err, errlen);
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
    bool ok = xf.n_head == xf.n_kv_head && xf.head_dim <= 128 && xf.head_dim % 2 == 0 && VH % 64 == 0 && L == 4 * BT &&
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
        navi_status s_ = v->alloc(c.hist, static_cast<size_t>(c.H) * c.Cin, err, errlen);
        if (s_ == NAVI_OK) s_ = v->alloc(c.hist2, static_cast<size_t>(c.H) * c.Cin, err, errlen);
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
        VB(uint16_t, up + "1.dwconv.conv.weight", NAVI_DT_F16, L, 1, 7, cx.dw);
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
        VA(cx.hist, static_cast<size_t>(6) * L);
        VA(cx.hist2, static_cast<size_t>(6) * L);
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
        VA(v->P[b], rows * C * bk.Cout);
        VA(v->Q[b], rows * C * bk.Cout);
        VA(v->ZP[b], rows * C * bk.Cout);
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
    VA(v->d_codes, C * p->n_q);
    VA(v->e, C * CD);
    VA(v->h, C * CD);
    VA(v->a, C * L);
    VA(v->x, C * VH);
    VA(v->n, C * VH);
    VA(v->qkv, C * 3 * HDT);
    VA(v->att, C * HDT);
    VA(v->gu, C * 2 * xf.ff);
    VA(v->u, C * L);
    const size_t up_rows = C * p->upsampling_ratios[0] * p->upsampling_ratios[1];
    VA(v->A, up_rows * L);
    VA(v->B, up_rows * L);
    VA(v->G, up_rows * 4 * L);
    VA(v->d, up_rows * DD);
    VA(v->pcm, C * p->samples_per_frame);
    VA(v->pcm16, C * p->samples_per_frame * 16);
    {
        // split counts from the rows of a 16-frame chunk (or the largest chunk if smaller), and
        // the workspace the largest chunk then needs
        size_t need = 0;
        const int Cn = static_cast<int>(std::min<size_t>(C, 16)), Cf = static_cast<int>(C);
        auto upd = [&](Conv &c, int rows_per_frame) {
            c.S = conv_splits(c, Cn * rows_per_frame);
            if (c.S > 1) need = std::max(need, static_cast<size_t>(c.S) * Cf * rows_per_frame * c.phases * c.Cout);
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
#undef VB
#undef VA
    if (hipMemcpyAsync(v->invf, invf, sizeof invf, hipMemcpyHostToDevice, s) != hipSuccess || hipEventCreate(&v->ev0) != hipSuccess ||
        hipEventCreate(&v->ev1) != hipSuccess || hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess) {
        set_err(err, errlen, "vocoder: HIP setup failed");
        return fail(NAVI_ERR_HIP);
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
    v->pos0 = 0;
    auto zero = [&](float *ptr, size_t n) { return !ptr || hipMemsetAsync(ptr, 0, n * sizeof(float), s) == hipSuccess; };
    auto zc = [&](Conv &c) { return zero(c.hist, static_cast<size_t>(c.H) * c.Cin) && zero(c.hist2, static_cast<size_t>(c.H) * c.Cin); };
    bool ok = zc(v->pre_conv) && zc(v->dec0) && zc(v->final_conv);
    for (int j = 0; j < 2; ++j) ok = ok && zero(v->cnx[j].hist, 6 * static_cast<size_t>(v->L)) && zero(v->cnx[j].hist2, 6 * static_cast<size_t>(v->L));
    for (Block &b : v->blocks) {
        ok = ok && zc(b.up);
        for (Unit &u : b.u) ok = ok && zc(u.c1);
    }
    // the K/V rings need no clearing: attention reads only positions already written this utterance
    return ok && hipStreamSynchronize(s) == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
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
    NAVI_TRY_HIP(hipMemsetAsync(v->flag, 0, 4, s), err, errlen);
    NAVI_TRY_HIP(hipEventRecord(v->ev0, s), err, errlen);
    for (int f0 = 0; f0 < n_frames; f0 += v->cmax) {
        const int T = std::min(v->cmax, n_frames - f0);
        NAVI_TRY_HIP(hipMemcpyAsync(v->d_codes, codes + static_cast<size_t>(f0) * nq, static_cast<size_t>(T) * nq * 4,
                                    hipMemcpyHostToDevice, s), err, errlen);
        const navi_status st = decode_chunk(*v, T, err, errlen);
        if (st != NAVI_OK) return st;
        NAVI_TRY_HIP(hipMemcpyAsync(pcm + static_cast<size_t>(f0) * spf, v->pcm, static_cast<size_t>(T) * spf * 4,
                                    hipMemcpyDeviceToHost, s), err, errlen);
    }
    NAVI_TRY_HIP(hipEventRecord(v->ev1, s), err, errlen);
    NAVI_TRY_HIP(hipEventSynchronize(v->ev1), err, errlen);
    float ms = 0.f;
    NAVI_TRY_HIP(hipEventElapsedTime(&ms, v->ev0, v->ev1), err, errlen);
    v->last_ms = ms;
    uint32_t f = 0;
    NAVI_TRY_HIP(hipMemcpy(&f, v->flag, 4, hipMemcpyDeviceToHost), err, errlen);
    if (f) {
        set_err(err, errlen, "vocoder: an activation is outside the f16 range (|x| >= 65504 or NaN)");
        return NAVI_ERR_INVALID;
    }
    return NAVI_OK;
}

int32_t navi_vocoder_samples_per_frame(const navi_vocoder *v) { return v ? v->p.samples_per_frame : 0; }
int32_t navi_vocoder_max_chunk_frames(const navi_vocoder *v) { return v ? v->cmax : 0; }
double navi_vocoder_last_ms(const navi_vocoder *v) { return v ? v->last_ms : 0.0; }

} // extern "C"
