// The speaker encoder on gfx950: the C ABI's navi_speaker_*.
//
// Replaces SpeakerEncoder (model/qwen3tts/speaker.h, speaker.hip:20-331): 24 kHz audio -> 128-bin
// log-mel -> ECAPA-TDNN -> the 1024-d speaker embedding of a cloned voice. Runs once per clone,
// on the prompt's path only. MI355X design:
//
//  * Front end: reflect padding (n_fft - hop) / 2, periodic Hann, |X| = sqrt(re^2 + im^2 + 1e-9),
//    the slaney filterbank (librosa.filters.mel), log(max(., 1e-5)). navi_speaker_mel computes it
//    on the host (the reference's static SpeakerEncoder::mel, in double); navi_speaker_embed on
//    the device, one block per frame (k_logmel: FFT in LDS, also in double), so a clone uploads
//    audio, not a spectrogram, and no host loop sits on its path.
//  * Every conv (block 0 k5, the SE-Res2Net tdnn / dilated k3 / squeeze-excitation convs, MFA,
//    attentive pooling, fc) is conv.h's implicit GEMM on the matrix cores with "same" reflect
//    padding; ReLU, sigmoid and tanh(ReLU) are its epilogues, the Res2Net "slice + previous
//    output" input its ADD2 prologue. Each block writes its output straight into its slice of
//    the [T][1536] MFA input, which is also the next block's input (no copies).
//  * Attentive statistics pooling: in [x | mean | std] the mean and std columns are the same at
//    every time step, so their part of asp.tdnn is folded into a per-channel bias (one GEMV) and
//    the conv runs over the 1536 x channels only: the [T][4608] concatenation is never built.
//  * Time reductions (SE mean, pooling statistics, softmax over time) run 16 channels x 16 time
//    slices per block, summed in a fixed order: the same bits every run. k=1 convs with few
//    output tiles (the SE and fc GEMVs, attentive pooling's 128-channel conv) split their input
//    channels over blocks; the partial sums are added in split order.
#include "conv.h"
#include "dev_common.h"
#include "host_util.h"

#include <algorithm>
#include <cmath>
#include <complex>
#include <memory>
#include <string>
#include <vector>

namespace navi_amd {
namespace spk {

using namespace cv;

constexpr int C = 512, R = 64, SCALE = 8, SEC = 128, MFA = 1536, ASP = 128;
constexpr int NCH = 16, NPART = BT / NCH;     // time reductions: 16 channels x 16 time slices per block

// ---- time reductions ---------------------------------------------------------------------
// Thread (q, c) sums rows t = q, q + 16, ... of channel c; the 16 slice sums are added in slice
// order by one thread: fixed association, the same bits every run.

__device__ __forceinline__ float slice_total(float (&red)[NPART][NCH], int cl) {
    float s = red[0][cl];
#pragma unroll
    for (int q = 1; q < NPART; ++q) s += red[q][cl];
    return s;
}

// mean over time of x[t][c] (ld ldx), c < C_: out[c]
__global__ void __launch_bounds__(BT) k_time_mean(const float *x, int T, int C_, int ldx, float *out) {
    __shared__ float red[NPART][NCH];
    const int cl = threadIdx.x % NCH, c = blockIdx.x * NCH + cl, q = threadIdx.x / NCH;
    float s = 0.f;
    if (c < C_)
#pragma unroll 4
        for (int t = q; t < T; t += NPART) s += gld(x + static_cast<size_t>(t) * ldx + c);
    red[q][cl] = s;
    __syncthreads();
    if (q == 0 && c < C_) gst(out + c, slice_total(red, cl) / static_cast<float>(T));
}

// y[t][c] = b[t][c] * g[c] + r[t][c]   (squeeze-excitation scale + the block's residual)
__global__ void __launch_bounds__(BT) k_scale_add(const float *b, int ldb, const float *g, const float *r, int ldr, int T,
                                                  float *y, int ldy) {
    const size_t i = static_cast<size_t>(blockIdx.x) * BT + threadIdx.x;
    if (i >= static_cast<size_t>(T) * C) return;
    const int t = static_cast<int>(i / C), c = static_cast<int>(i % C);
    gst(y + static_cast<size_t>(t) * ldy + c, gld(b + static_cast<size_t>(t) * ldb + c) * gld(g + c) + gld(r + static_cast<size_t>(t) * ldr + c));
}

// Per channel c < C_: mean and std over time with weights w[t][c] (uniform 1/T when w is null):
// out[c] = sum w x, out[C_ + c] = sqrt(max(sum w (x - mean)^2, 1e-12)) (k_weighted_stats, speaker.hip:92-107).
__global__ void __launch_bounds__(BT) k_stats(const float *x, const float *w, int T, int C_, int ld, float *out) {
    __shared__ float red[NPART][NCH];
    __shared__ float mean[NCH];
    const int cl = threadIdx.x % NCH, c = blockIdx.x * NCH + cl, q = threadIdx.x / NCH;
    const float u = 1.f / static_cast<float>(T);
    float s = 0.f;
    if (c < C_)
#pragma unroll 4
        for (int t = q; t < T; t += NPART) {
            const size_t o = static_cast<size_t>(t) * ld + c;
            s = fmaf(w ? gld(w + o) : u, gld(x + o), s);
        }
    red[q][cl] = s;
    __syncthreads();
    if (q == 0) mean[cl] = slice_total(red, cl);
    __syncthreads();
    const float m = mean[cl];
    float v = 0.f;
    if (c < C_)
#pragma unroll 4
        for (int t = q; t < T; t += NPART) {
            const size_t o = static_cast<size_t>(t) * ld + c;
            const float d = gld(x + o) - m;
            v = fmaf(w ? gld(w + o) : u, d * d, v);
        }
    __syncthreads();
    red[q][cl] = v;
    __syncthreads();
    if (q == 0 && c < C_) {
        gst(out + c, m);
        gst(out + C_ + c, sqrtf(fmaxf(slice_total(red, cl), 1e-12f)));
    }
}

// softmax over time per channel, in place: a[t][c] (ld ld), c < C_
__global__ void __launch_bounds__(BT) k_time_softmax(float *a, int T, int C_, int ld) {
    __shared__ float red[NPART][NCH];
    __shared__ float tot[NCH];
    const int cl = threadIdx.x % NCH, c = blockIdx.x * NCH + cl, q = threadIdx.x / NCH;
    float m = -INFINITY;
    if (c < C_)
#pragma unroll 4
        for (int t = q; t < T; t += NPART) m = fmaxf(m, gld(a + static_cast<size_t>(t) * ld + c));
    red[q][cl] = m;
    __syncthreads();
    if (q == 0) {
        float mx = red[0][cl];
#pragma unroll
        for (int i = 1; i < NPART; ++i) mx = fmaxf(mx, red[i][cl]);
        tot[cl] = mx;
    }
    __syncthreads();
    const float mx = tot[cl];
    float s = 0.f;
    if (c < C_)
#pragma unroll 4
        for (int t = q; t < T; t += NPART) s += expf(gld(a + static_cast<size_t>(t) * ld + c) - mx);
    __syncthreads();
    red[q][cl] = s;
    __syncthreads();
    if (q == 0) tot[cl] = slice_total(red, cl);
    __syncthreads();
    const float inv = 1.f / tot[cl];
    // in place: four rows' loads go out before their stores (a load after a store to the same
    // array would wait for it)
    if (c < C_)
        for (int t0 = q; t0 < T; t0 += 4 * NPART) {
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int t = t0 + k * NPART;
                v[k] = t < T ? gld(a + static_cast<size_t>(t) * ld + c) : 0.f;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int t = t0 + k * NPART;
                if (t < T) gst(a + static_cast<size_t>(t) * ld + c, expf(v[k] - mx) * inv);
            }
        }
}

// The attentive pooling's constant columns folded into a bias: out[co] = b[co] + sum_i
// W[co][MFA + i] mean[i] + W[co][2 MFA + i] std[i], W the stored asp.tdnn weight [ASP][3 MFA].
__global__ void __launch_bounds__(BT) k_asp_bias(const uint16_t *W, const float *b, const float *stats, float *out) {
    __shared__ float red[BT / WAVE];
    const int co = blockIdx.x;
    const uint16_t *row = W + static_cast<size_t>(co) * 3 * MFA + MFA;
    float s = 0.f;
    for (int i = threadIdx.x; i < 2 * MFA; i += BT) s = fmaf(h2f(gld(row + i)), gld(stats + i), s);
    s = wave_sum(s);
    if ((threadIdx.x & (WAVE - 1)) == 0) red[threadIdx.x / WAVE] = s;
    __syncthreads();
    if (threadIdx.x == 0) gst(out + co, gld(b + co) + ((red[0] + red[1]) + red[2]) + red[3]);
}

// dst[co][ci] = src[co][ci] for ci < n (the first n of ld input channels of a k=1 conv)
__global__ void k_take_cols(const uint16_t *src, int rows, int ld, int n, uint16_t *dst) {
    const size_t i = static_cast<size_t>(blockIdx.x) * BT + threadIdx.x;
    if (i >= static_cast<size_t>(rows) * n) return;
    const size_t r = i / n, c = i % n;
    gst(dst + i, gld(src + r * ld + c));
}

// ---- device mel front end ------------------------------------------------------------------
// The host front end's arithmetic in the same double precision, one block per frame
// (SpeakerEncoder::mel, speaker.hip:269-303, computes it in f32 on one host thread; f32 leaves
// low-energy bins of tonal audio with ~1e-2 relative error). The 1024-point real FFT is a
// 512-point complex FFT of z[m] = x[2m] + i x[2m+1] (Stockham radix-2, naturally ordered, in
// LDS) followed by the real-input split X[k] = E[k] + e^{-2 pi i k / 1024} O[k],
// E = (Z[k] + conj Z[512-k]) / 2, O = (Z[k] - conj Z[512-k]) / 2i. Each filter sums only its
// nonzero bins, in bin order as the host does.

constexpr int NFFT = 1024, NH = NFFT / 2, NBIN = NH + 1, MELS = 128;

struct MelTables {                       // built once at create
    double2 tw[NH / 2];                  // e^{-2 pi i q / NH}: the half-length FFT's twiddles
    double2 post[NBIN];                  // e^{-2 pi i k / NFFT}
    double hann[NFFT];                   // periodic
    int lo[MELS], hi[MELS];              // filter m's nonzero bins [lo, hi)
    float fb[MELS][NBIN];                // librosa's f32 filterbank, as the host uses it
};

__device__ __forceinline__ double2 cmul(double2 a, double2 b) { return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x); }

// mel[t][m] (time-major, the layout block 0's conv reads) for frame t = blockIdx.x
__global__ void __launch_bounds__(BT) k_logmel(const float *wav, int64_t n, int pad, int hop, const MelTables *tb, float *mel) {
    static_assert(NH / 2 == BT, "one butterfly per thread per stage");
    __shared__ double2 buf[2][NH];
    __shared__ double mag[NBIN];
    const int t = blockIdx.x, j = threadIdx.x;
    const int64_t base = static_cast<int64_t>(t) * hop - pad;
    auto sample = [&](int i) {
        int64_t q = base + i;
        if (q < 0) q = -q;                                  // reflect padding (n > pad is checked)
        if (q >= n) q = 2 * (n - 1) - q;
        return static_cast<double>(gld(wav + q)) * tb->hann[i];
    };
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int m = j + r * BT;
        buf[0][m] = make_double2(sample(2 * m), sample(2 * m + 1));
    }
    __syncthreads();
    int cur = 0;
    for (int ns = 1; ns < NH; ns <<= 1) {
        const int k = j & (ns - 1);
        const double2 a = buf[cur][j], b = cmul(buf[cur][j + NH / 2], tb->tw[k * (NH / (2 * ns))]);
        const int o = 2 * (j - k) + k;
        buf[cur ^ 1][o] = make_double2(a.x + b.x, a.y + b.y);
        buf[cur ^ 1][o + ns] = make_double2(a.x - b.x, a.y - b.y);
        cur ^= 1;
        __syncthreads();
    }
    const double2 *Z = buf[cur];
    for (int k = j; k < NBIN; k += BT) {
        const double2 zk = Z[k & (NH - 1)], zr = Z[(NH - k) & (NH - 1)];
        const double2 e = make_double2(0.5 * (zk.x + zr.x), 0.5 * (zk.y - zr.y));
        const double2 o = make_double2(0.5 * (zk.y + zr.y), -0.5 * (zk.x - zr.x));
        const double2 x = cmul(tb->post[k], o);
        const double re = e.x + x.x, im = e.y + x.y;
        mag[k] = sqrt(re * re + im * im + 1e-9);
    }
    __syncthreads();
    if (j < MELS) {
        const float *row = tb->fb[j];
        double s = 0.0;
        for (int k = gld(tb->lo + j), e = gld(tb->hi + j); k < e; ++k) s += static_cast<double>(gld(row + k)) * mag[k];
        gst(mel + static_cast<size_t>(t) * MELS + j, static_cast<float>(log(fmax(s, 1e-5))));
    }
}

// ---- host mel front end (SpeakerEncoder::mel, speaker.hip:269-303) -------------------------

// librosa.filters.mel(sr, n_fft, n_mels, fmin, fmax): slaney mel scale and norm (speaker.hip:45-71)
std::vector<float> mel_filterbank(int sr, int n_fft, int n_mels, double fmin, double fmax) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp, logstep = std::log(6.4) / 27.0;
    auto hz_to_mel = [&](double f) { return f >= min_log_hz ? min_log_mel + std::log(f / min_log_hz) / logstep : f / f_sp; };
    auto mel_to_hz = [&](double m) { return m >= min_log_mel ? min_log_hz * std::exp(logstep * (m - min_log_mel)) : f_sp * m; };
    const int nb = n_fft / 2 + 1;
    std::vector<double> mel_f(n_mels + 2);
    const double m0 = hz_to_mel(fmin), m1 = hz_to_mel(fmax);
    for (int i = 0; i < n_mels + 2; ++i) mel_f[i] = mel_to_hz(m0 + (m1 - m0) * i / (n_mels + 1));
    std::vector<float> w(static_cast<size_t>(n_mels) * nb);
    for (int i = 0; i < n_mels; ++i) {
        const double enorm = 2.0 / (mel_f[i + 2] - mel_f[i]);
        for (int k = 0; k < nb; ++k) {
            const double f = static_cast<double>(sr) / 2.0 * k / (nb - 1);
            const double lo = (f - mel_f[i]) / (mel_f[i + 1] - mel_f[i]), hi = (mel_f[i + 2] - f) / (mel_f[i + 2] - mel_f[i + 1]);
            w[static_cast<size_t>(i) * nb + k] = static_cast<float>(std::max(0.0, std::min(lo, hi)) * enorm);
        }
    }
    return w;
}

// In-place radix-2 FFT of n = 2^k points (double), twiddles from one table.
void fft(std::vector<std::complex<double>> &a, const std::vector<std::complex<double>> &tw) {
    const size_t n = a.size();
    for (size_t i = 1, j = 0; i < n; ++i) {
        size_t bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) std::swap(a[i], a[j]);
    }
    for (size_t len = 2; len <= n; len <<= 1) {
        const size_t step = n / len;
        for (size_t i = 0; i < n; i += len)
            for (size_t k = 0; k < len / 2; ++k) {
                const std::complex<double> u = a[i + k], v = a[i + k + len / 2] * tw[k * step];
                a[i + k] = u + v;
                a[i + k + len / 2] = u - v;
            }
    }
}

} // namespace spk
} // namespace navi_amd

using namespace navi_amd;
using namespace navi_amd::spk;

namespace {

struct SConv {
    const uint16_t *w = nullptr;   // [Cout][K][Cin]
    const float *bias = nullptr;
    int Cin = 0, Cout = 0, K = 1, dil = 1;
};

template <int MT, int K>
void launch_spk(const ConvArgs &a, int pro, int epi, dim3 grid, hipStream_t s) {
#define NAVI_SPK(P_, E_)                                                                        \
    if (pro == P_ && epi == E_) {                                                               \
        hipLaunchKernelGGL((k_conv_mfma<MT, K, P_, E_>), grid, dim3(BT), 0, s, a);              \
        return;                                                                                 \
    }
    if constexpr (K == 3) NAVI_SPK(PRO_ADD2, EPI_RELU)
    NAVI_SPK(PRO_NONE, EPI_RELU)
    if constexpr (K == 1) {
        NAVI_SPK(PRO_NONE, EPI_PARTIAL)
        NAVI_SPK(PRO_NONE, EPI_BIAS)
        NAVI_SPK(PRO_NONE, EPI_SIGMOID)
        NAVI_SPK(PRO_NONE, EPI_RELU_TANH)
    }
#undef NAVI_SPK
}

} // namespace

struct navi_speaker {
    navi_speaker_params p{};
    int max_frames = 0;
    SConv block0, mfa, asp_x, asp_conv, fc;
    struct Block {
        SConv tdnn1, res[SCALE - 1], tdnn2, se1, se2;
    } blocks[3];
    const uint16_t *asp_w = nullptr;          // asp.tdnn as stored [ASP][3 MFA][1] (its mean/std columns)
    const float *asp_b = nullptr;
    float *mel = nullptr, *a = nullptr, *b = nullptr, *c = nullptr, *cat3 = nullptr, *att = nullptr, *attw = nullptr;
    float *g2 = nullptr, *mean = nullptr, *g = nullptr, *gse = nullptr, *stats = nullptr, *pooled = nullptr, *bias2 = nullptr;
    float *emb = nullptr;
    uint32_t *flag = nullptr;
    MelTables *tables = nullptr;              // the device front end's constants
    float *part = nullptr;                    // split-K partial sums
    size_t part_cap = 0;
    float *wav = nullptr;                     // audio of the last navi_speaker_embed
    int64_t wav_cap = 0;
    int last_frames = 0;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    double last_ms = 0;
    std::vector<void *> owned;

    template <class T>
    navi_status alloc(T *&ptr, size_t n, char *err, size_t errlen) {
        void *v = nullptr;
        NAVI_TRY_HIP(hipMalloc(&v, std::max<size_t>(n, 1) * sizeof(T)), err, errlen);
        owned.push_back(v);
        NAVI_TRY_HIP(hipMemsetAsync(v, 0, std::max<size_t>(n, 1) * sizeof(T), device_state().stream), err, errlen);
        ptr = static_cast<T *>(v);
        return NAVI_OK;
    }

    ~navi_speaker() {
        if (ev0) (void) hipEventDestroy(ev0);
        if (ev1) (void) hipEventDestroy(ev1);
        for (void *v : owned) (void) hipFree(v);
    }

    // "same" reflect-padded conv over T rows: x [T][ldx] -> y [T][ldy] (x2: the ADD2 input, ld ldx)
    navi_status conv(const SConv &cv, int pro, int epi, const float *x, int T, int ldx, float *y, int ldy, char *err,
                     size_t errlen, const float *x2 = nullptr, const float *bias = nullptr) {
        ConvArgs ca{};
        ca.x = x; ca.x2 = x2; ca.w = cv.w; ca.bias = bias ? bias : cv.bias; ca.y = y; ca.flag = flag;
        ca.ldx = ldx; ca.ldy = ldy; ca.T = T; ca.Cin = cv.Cin; ca.Cout = cv.Cout; ca.dil = cv.dil; ca.phases = 1;
        ca.cps = cv.Cin; ca.lpad = (cv.K - 1) * cv.dil / 2; ca.reflect = 1;
        // 16-row tiles unless that already gives the chip two blocks per CU
        const int mt = ((cv.Cout + 63) / 64) * ((T + 63) / 64) >= 512 ? 4 : 1;
        dim3 grid((cv.Cout + 63) / 64, (T + 16 * mt - 1) / (16 * mt), 1);
        hipStream_t s = device_state().stream;
        // under 192 blocks: split the input channels (>= 128 per split) so about 256 blocks run
        const int blocks = static_cast<int>(grid.x * grid.y);
        if (cv.K == 1 && pro == PRO_NONE && blocks < 192 && cv.Cin >= 256) {
            int sp = std::min((256 + blocks - 1) / blocks, cv.Cin / 128);
            while (sp > 1 && static_cast<size_t>(sp) * T * cv.Cout > part_cap) --sp;
            if (sp > 1) {
                ca.cps = ((cv.Cin + sp - 1) / sp + CCH - 1) / CCH * CCH;
                sp = (cv.Cin + ca.cps - 1) / ca.cps;
                ca.part = part;
                grid.z = static_cast<unsigned>(sp);
                launch_spk<1, 1>(ca, PRO_NONE, EPI_PARTIAL, grid, s);
                const size_t n = static_cast<size_t>(T) * cv.Cout;
                hipLaunchKernelGGL(k_conv_finish, dim3(static_cast<unsigned>((n + BT - 1) / BT)), dim3(BT), 0, s, ca, sp, epi);
                NAVI_TRY_HIP(hipGetLastError(), err, errlen);
                return NAVI_OK;
            }
        }
        switch (cv.K * 10 + mt) {
        case 11: launch_spk<1, 1>(ca, pro, epi, grid, s); break;
        case 14: launch_spk<4, 1>(ca, pro, epi, grid, s); break;
        case 31: launch_spk<1, 3>(ca, pro, epi, grid, s); break;
        case 34: launch_spk<4, 3>(ca, pro, epi, grid, s); break;
        case 51: launch_spk<1, 5>(ca, pro, epi, grid, s); break;
        case 54: launch_spk<4, 5>(ca, pro, epi, grid, s); break;
        default:
            set_err(err, errlen, "speaker: no conv kernel for K=%d", cv.K);
            return NAVI_ERR_UNSUPPORTED;
        }
        NAVI_TRY_HIP(hipGetLastError(), err, errlen);
        return NAVI_OK;
    }

    // SpeakerEncoder::Impl::run (speaker.hip:175-220) over the T mel rows in `mel`.
    navi_status run(int T, char *err, size_t errlen) {
        hipStream_t s = device_state().stream;
        const unsigned tb = static_cast<unsigned>((C + NCH - 1) / NCH), tm = static_cast<unsigned>((MFA + NCH - 1) / NCH);
#define SP_TRY(x)                                                                               \
        do {                                                                                    \
            const navi_status st_ = (x);                                                        \
            if (st_ != NAVI_OK) return st_;                                                     \
        } while (0)
        SP_TRY(conv(block0, PRO_NONE, EPI_RELU, mel, T, p.num_mels, a, C, err, errlen));
        const float *in = a;
        int ldin = C;
        for (int bi = 0; bi < 3; ++bi) {
            Block &bk = blocks[bi];
            SP_TRY(conv(bk.tdnn1, PRO_NONE, EPI_RELU, in, T, ldin, b, C, err, errlen));
            // Res2Net: slice 0 passes, slice 1 = conv(slice 1), slice i = conv(slice i + out i-1)
            NAVI_TRY_HIP(hipMemcpy2DAsync(c, C * sizeof(float), b, C * sizeof(float), R * sizeof(float), T,
                                          hipMemcpyDeviceToDevice, s), err, errlen);
            for (int i = 1; i < SCALE; ++i)
                SP_TRY(conv(bk.res[i - 1], i == 1 ? PRO_NONE : PRO_ADD2, EPI_RELU, b + i * R, T, C, c + i * R, C, err, errlen,
                            i == 1 ? nullptr : c + (i - 1) * R));
            SP_TRY(conv(bk.tdnn2, PRO_NONE, EPI_RELU, c, T, C, b, C, err, errlen));
            // squeeze-excitation on the time mean, then out = b * gate + the block input, written
            // into this block's slice of the MFA input (which is also the next block's input)
            hipLaunchKernelGGL(k_time_mean, dim3(tb), dim3(BT), 0, s, b, T, C, C, mean);
            SP_TRY(conv(bk.se1, PRO_NONE, EPI_RELU, mean, 1, C, g, SEC, err, errlen));
            SP_TRY(conv(bk.se2, PRO_NONE, EPI_SIGMOID, g, 1, SEC, gse, C, err, errlen));
            float *out = cat3 + bi * C;
            const size_t n = static_cast<size_t>(T) * C;
            hipLaunchKernelGGL(k_scale_add, dim3(static_cast<unsigned>((n + BT - 1) / BT)), dim3(BT), 0, s, b, C, gse, in, ldin, T,
                               out, MFA);
            in = out;
            ldin = MFA;
        }
        SP_TRY(conv(mfa, PRO_NONE, EPI_RELU, cat3, T, MFA, att, MFA, err, errlen));
        // attentive statistics pooling
        hipLaunchKernelGGL(k_stats, dim3(tm), dim3(BT), 0, s, att, nullptr, T, MFA, MFA, stats);
        hipLaunchKernelGGL(k_asp_bias, dim3(ASP), dim3(BT), 0, s, asp_w, asp_b, stats, bias2);
        SP_TRY(conv(asp_x, PRO_NONE, EPI_RELU_TANH, att, T, MFA, g2, ASP, err, errlen, nullptr, bias2));
        SP_TRY(conv(asp_conv, PRO_NONE, EPI_BIAS, g2, T, ASP, attw, MFA, err, errlen));
        hipLaunchKernelGGL(k_time_softmax, dim3(tm), dim3(BT), 0, s, attw, T, MFA, MFA);
        hipLaunchKernelGGL(k_stats, dim3(tm), dim3(BT), 0, s, att, attw, T, MFA, MFA, pooled);
        SP_TRY(conv(fc, PRO_NONE, EPI_BIAS, pooled, 1, 2 * MFA, emb, p.enc_dim, err, errlen));
#undef SP_TRY
        NAVI_TRY_HIP(hipGetLastError(), err, errlen);
        return NAVI_OK;
    }
};

namespace {

// device: the front end of navi_speaker_embed (k_logmel) is built for the model's 1024-point FFT
navi_status check_params(const navi_speaker_params *p, char *err, size_t errlen, bool device = false) {
    if (!p) {
        set_err(err, errlen, "speaker: null params");
        return NAVI_ERR_INVALID;
    }
    const bool pow2 = p->n_fft >= 16 && (p->n_fft & (p->n_fft - 1)) == 0;
    if (!pow2 || p->win != p->n_fft || p->hop < 1 || p->hop > p->n_fft || p->num_mels != 128 || p->sample_rate < 1 ||
        p->enc_dim < 16 || p->enc_dim % 16 != 0 || !(p->fmax > p->fmin) || p->fmin < 0.f || (device && p->n_fft != NFFT)) {
        set_err(err, errlen, "speaker: unsupported front end (n_fft %d, win %d, hop %d, mels %d, dim %d)", p->n_fft, p->win, p->hop,
                p->num_mels, p->enc_dim);
        return NAVI_ERR_UNSUPPORTED;
    }
    return NAVI_OK;
}

// reflect padding mirrors once: the widest pad (k3, dilation 4: 4 rows) must stay below T
navi_status check_frames(const navi_speaker *h, int32_t T, char *err, size_t errlen) {
    if (T < 5 || T > h->max_frames) {
        set_err(err, errlen, "speaker: %d mel frames, this encoder takes 5..%d (raise max_seconds)", T, h->max_frames);
        return NAVI_ERR_INVALID;
    }
    return NAVI_OK;
}

// The device part of an embed: (wav_n > 0) the front end from h->wav into h->mel, the network,
// the embedding back to the host. Device time of both in last_ms.
navi_status embed_device(navi_speaker *h, int T, int64_t wav_n, float *emb, char *err, size_t errlen) {
    hipStream_t s = device_state().stream;
    NAVI_TRY_HIP(hipMemsetAsync(h->flag, 0, 4, s), err, errlen);
    NAVI_TRY_HIP(hipEventRecord(h->ev0, s), err, errlen);
    if (wav_n > 0)
        hipLaunchKernelGGL(k_logmel, dim3(static_cast<unsigned>(T)), dim3(BT), 0, s, h->wav, wav_n, (NFFT - h->p.hop) / 2, h->p.hop,
                           h->tables, h->mel);
    const navi_status st = h->run(T, err, errlen);
    if (st != NAVI_OK) return st;
    NAVI_TRY_HIP(hipEventRecord(h->ev1, s), err, errlen);
    uint32_t bad = 0;
    NAVI_TRY_HIP(hipMemcpyAsync(emb, h->emb, static_cast<size_t>(h->p.enc_dim) * sizeof(float), hipMemcpyDeviceToHost, s), err,
                 errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(&bad, h->flag, 4, hipMemcpyDeviceToHost, s), err, errlen);
    NAVI_TRY_HIP(hipStreamSynchronize(s), err, errlen);
    float ms = 0.f;
    (void) hipEventElapsedTime(&ms, h->ev0, h->ev1);
    h->last_ms = ms;
    h->last_frames = T;
    if (bad) {
        set_err(err, errlen, "speaker: an activation is outside the f16 range (|x| >= 65504 or NaN)");
        return NAVI_ERR_INVALID;
    }
    return NAVI_OK;
}

} // namespace

extern "C" {

navi_status navi_speaker_mel(const navi_speaker_params *p, const float *wav, int64_t n, float *mel_out, int64_t capacity,
                             int32_t *n_frames, char *err, size_t errlen) {
    navi_status st = check_params(p, err, errlen);
    if (st != NAVI_OK) return st;
    if (!wav || !n_frames) {
        set_err(err, errlen, "speaker: null argument");
        return NAVI_ERR_INVALID;
    }
    const int nf = p->n_fft, hop = p->hop, nm = p->num_mels, nb = nf / 2 + 1, pad = (nf - hop) / 2;
    if (n < static_cast<int64_t>(pad) + 1) {
        set_err(err, errlen, "speaker: reference audio too short (%lld samples)", static_cast<long long>(n));
        return NAVI_ERR_INVALID;
    }
    const int64_t len = n + 2 * pad;
    if (len < nf) {
        set_err(err, errlen, "speaker: reference audio shorter than one window");
        return NAVI_ERR_INVALID;
    }
    const int64_t T = (len - nf) / hop + 1;
    if (T > (1 << 24)) {
        set_err(err, errlen, "speaker: reference audio too long");
        return NAVI_ERR_INVALID;
    }
    *n_frames = static_cast<int32_t>(T);
    if (!mel_out) return NAVI_OK;                                      // size query
    if (capacity < T * nm) {
        set_err(err, errlen, "speaker: mel buffer holds %lld values, %lld needed", static_cast<long long>(capacity),
                static_cast<long long>(T * nm));
        return NAVI_ERR_INVALID;
    }
    // reflect padding (index -i and 2(n-1) - i), periodic Hann, |FFT|, filterbank, log
    auto sample = [&](int64_t i) {
        i -= pad;
        if (i < 0) i = -i;
        if (i >= n) i = 2 * (n - 1) - i;
        return static_cast<double>(wav[i]);
    };
    std::vector<double> hann(nf);
    for (int i = 0; i < nf; ++i) hann[i] = 0.5 - 0.5 * std::cos(2.0 * M_PI * i / nf);
    std::vector<std::complex<double>> tw(nf / 2), fr(nf);
    for (int k = 0; k < nf / 2; ++k) tw[k] = std::polar(1.0, -2.0 * M_PI * k / nf);
    const std::vector<float> fb = mel_filterbank(p->sample_rate, nf, nm, p->fmin, p->fmax);
    std::vector<double> mag(nb);
    for (int64_t t = 0; t < T; ++t) {
        for (int i = 0; i < nf; ++i) fr[i] = std::complex<double>(sample(t * hop + i) * hann[i], 0.0);
        fft(fr, tw);
        for (int k = 0; k < nb; ++k) mag[k] = std::sqrt(std::norm(fr[k]) + 1e-9);
        for (int m = 0; m < nm; ++m) {
            const float *row = &fb[static_cast<size_t>(m) * nb];
            double s = 0.0;
            for (int k = 0; k < nb; ++k) s += static_cast<double>(row[k]) * mag[k];
            mel_out[static_cast<size_t>(m) * T + t] = static_cast<float>(std::log(std::max(s, 1e-5)));
        }
    }
    return NAVI_OK;
}

navi_status navi_speaker_create(const navi_speaker_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                                double max_seconds, navi_speaker **out, char *err, size_t errlen) {
    navi_status st = check_params(p, err, errlen, true);
    if (st != NAVI_OK) return st;
    if (!tensors || !out || !(max_seconds > 0.0) || max_seconds > 600.0) {
        set_err(err, errlen, "speaker: bad argument (max_seconds %.1f)", max_seconds);
        return NAVI_ERR_INVALID;
    }
    *out = nullptr;
    if ((st = ensure_device(err, errlen)) != NAVI_OK) return st;
    auto h = new navi_speaker();
    auto fail = [&](navi_status s_) { delete h; return s_; };
    h->p = *p;
    h->max_frames = static_cast<int>(max_seconds * p->sample_rate / p->hop) + 2;
    hipStream_t s = device_state().stream;
    const std::string S = "speaker_encoder.";
    auto tensor = [&](const std::string &name, int dtype, uint64_t d0, uint64_t d1, uint64_t d2, const void *&ptr) {
        const navi_tensor_ref *r = find_tensor(tensors, n_tensors, name);
        if (!r) {
            set_err(err, errlen, "speaker: missing tensor '%s'", name.c_str());
            return NAVI_ERR_INVALID;
        }
        const int nd = d2 ? 3 : 1;
        if (r->dtype != dtype || r->ndim != nd || r->dims[0] != d0 || (nd == 3 && (r->dims[1] != d1 || r->dims[2] != d2)) ||
            (reinterpret_cast<uintptr_t>(r->ptr) & 15u)) {
            set_err(err, errlen, "speaker: tensor '%s' has an unexpected dtype, shape or alignment", name.c_str());
            return NAVI_ERR_INVALID;
        }
        ptr = r->ptr;
        return NAVI_OK;
    };
    // bind a conv: weight [Cout][Cin][K] f16 -> relaid [Cout][K][Cin], bias [Cout] f32
    auto bind = [&](const std::string &name, int cin, int cout, int k, int dil, SConv &cv) -> navi_status {
        const void *w = nullptr, *b = nullptr;
        navi_status s_;
        if ((s_ = tensor(name + ".weight", NAVI_DT_F16, cout, cin, k, w)) != NAVI_OK ||
            (s_ = tensor(name + ".bias", NAVI_DT_F32, cout, 0, 0, b)) != NAVI_OK)
            return s_;
        uint16_t *o = nullptr;
        if ((s_ = h->alloc(o, static_cast<size_t>(cout) * cin * k, err, errlen)) != NAVI_OK) return s_;
        const size_t nn = static_cast<size_t>(cout) * cin * k;
        hipLaunchKernelGGL(k_relayout_conv, dim3(static_cast<unsigned>((nn + BT - 1) / BT)), dim3(BT), 0, s,
                           static_cast<const uint16_t *>(w), cout, cin, k, o);
        cv = SConv{o, static_cast<const float *>(b), cin, cout, k, dil};
        return NAVI_OK;
    };
#define SB(...)                                                                                 \
    do {                                                                                        \
        if ((st = bind(__VA_ARGS__)) != NAVI_OK) return fail(st);                               \
    } while (0)
    SB(S + "blocks.0.conv", p->num_mels, C, 5, 1, h->block0);
    const int dils[3] = {2, 3, 4};
    for (int b = 0; b < 3; ++b) {
        const std::string bp = S + "blocks." + std::to_string(b + 1) + ".";
        navi_speaker::Block &bk = h->blocks[b];
        SB(bp + "tdnn1.conv", C, C, 1, 1, bk.tdnn1);
        for (int r = 0; r < SCALE - 1; ++r) SB(bp + "res2net_block.blocks." + std::to_string(r) + ".conv", R, R, 3, dils[b], bk.res[r]);
        SB(bp + "tdnn2.conv", C, C, 1, 1, bk.tdnn2);
        SB(bp + "se_block.conv1", C, SEC, 1, 1, bk.se1);
        SB(bp + "se_block.conv2", SEC, C, 1, 1, bk.se2);
    }
    SB(S + "mfa.conv", MFA, MFA, 1, 1, h->mfa);
    SB(S + "asp.conv", ASP, MFA, 1, 1, h->asp_conv);
    SB(S + "fc", 2 * MFA, p->enc_dim, 1, 1, h->fc);
#undef SB
    {   // asp.tdnn: the x columns as a 1536-input conv; the stored weight for the folded bias
        const void *w = nullptr, *b = nullptr;
        if ((st = tensor(S + "asp.tdnn.conv.weight", NAVI_DT_F16, ASP, 3 * MFA, 1, w)) != NAVI_OK ||
            (st = tensor(S + "asp.tdnn.conv.bias", NAVI_DT_F32, ASP, 0, 0, b)) != NAVI_OK)
            return fail(st);
        h->asp_w = static_cast<const uint16_t *>(w);
        h->asp_b = static_cast<const float *>(b);
        uint16_t *o = nullptr;
        if ((st = h->alloc(o, static_cast<size_t>(ASP) * MFA, err, errlen)) != NAVI_OK) return fail(st);
        const size_t nn = static_cast<size_t>(ASP) * MFA;
        hipLaunchKernelGGL(k_take_cols, dim3(static_cast<unsigned>((nn + BT - 1) / BT)), dim3(BT), 0, s, h->asp_w, ASP, 3 * MFA,
                           MFA, o);
        h->asp_x = SConv{o, nullptr, MFA, ASP, 1, 1};
    }
    const size_t T = static_cast<size_t>(h->max_frames);
#define SA(ptr, n_)                                                                             \
    do {                                                                                        \
        if ((st = h->alloc(ptr, (n_), err, errlen)) != NAVI_OK) return fail(st);                \
    } while (0)
    SA(h->mel, T * p->num_mels);
    SA(h->a, T * C);
    SA(h->b, T * C);
    SA(h->c, T * C);
    SA(h->cat3, T * MFA);
    SA(h->att, T * MFA);
    SA(h->attw, T * MFA);
    SA(h->g2, T * ASP);
    SA(h->mean, C);
    SA(h->g, SEC);
    SA(h->gse, C);
    SA(h->stats, 2 * MFA);
    SA(h->pooled, 2 * MFA);
    SA(h->bias2, ASP);
    SA(h->emb, p->enc_dim);
    SA(h->flag, 1);
    h->wav_cap = static_cast<int64_t>(h->max_frames + 2) * p->hop + NFFT;
    SA(h->wav, static_cast<size_t>(h->wav_cap));
    SA(h->tables, 1);
    h->part_cap = size_t(2) << 20;
    SA(h->part, h->part_cap);
#undef SA
    {   // the front end's tables, copied synchronously
        auto tb = std::make_unique<MelTables>();
        for (int q = 0; q < NH / 2; ++q)
            tb->tw[q] = make_double2(std::cos(-2.0 * M_PI * q / NH), std::sin(-2.0 * M_PI * q / NH));
        for (int k = 0; k < NBIN; ++k)
            tb->post[k] = make_double2(std::cos(-2.0 * M_PI * k / NFFT), std::sin(-2.0 * M_PI * k / NFFT));
        for (int i = 0; i < NFFT; ++i) tb->hann[i] = 0.5 - 0.5 * std::cos(2.0 * M_PI * i / NFFT);
        const std::vector<float> fb = mel_filterbank(p->sample_rate, NFFT, MELS, p->fmin, p->fmax);
        for (int m = 0; m < MELS; ++m) {
            int lo = NBIN, hi = 0;
            for (int k = 0; k < NBIN; ++k) {
                tb->fb[m][k] = fb[static_cast<size_t>(m) * NBIN + k];
                if (tb->fb[m][k] != 0.f) lo = std::min(lo, k), hi = k + 1;
            }
            tb->lo[m] = std::min(lo, hi);
            tb->hi[m] = hi;
        }
        if (hipMemcpy(h->tables, tb.get(), sizeof(MelTables), hipMemcpyHostToDevice) != hipSuccess) {
            set_err(err, errlen, "speaker: table upload failed");
            return fail(NAVI_ERR_HIP);
        }
    }
    if (hipEventCreate(&h->ev0) != hipSuccess || hipEventCreate(&h->ev1) != hipSuccess || hipGetLastError() != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        set_err(err, errlen, "speaker: HIP setup failed");
        return fail(NAVI_ERR_HIP);
    }
    *out = h;
    return NAVI_OK;
}

void navi_speaker_destroy(navi_speaker *h) {
    if (!h) return;
    (void) hipStreamSynchronize(device_state().stream);
    delete h;
}

navi_status navi_speaker_embed_mel(navi_speaker *h, const float *mel, int32_t n_frames, float *emb, char *err, size_t errlen) {
    if (!h || !mel || !emb) {
        set_err(err, errlen, "speaker: null argument");
        return NAVI_ERR_INVALID;
    }
    navi_status st = check_frames(h, n_frames, err, errlen);
    if (st != NAVI_OK) return st;
    const int T = n_frames, nm = h->p.num_mels;
    // [n_mels][T] -> time-major [T][n_mels]
    std::vector<float> tm(static_cast<size_t>(T) * nm);
    for (int m = 0; m < nm; ++m)
        for (int t = 0; t < T; ++t) tm[static_cast<size_t>(t) * nm + m] = mel[static_cast<size_t>(m) * T + t];
    NAVI_TRY_HIP(hipMemcpyAsync(h->mel, tm.data(), tm.size() * sizeof(float), hipMemcpyHostToDevice, device_state().stream), err,
                 errlen);
    return embed_device(h, T, 0, emb, err, errlen);
}

navi_status navi_speaker_embed(navi_speaker *h, const float *wav, int64_t n, float *emb, char *err, size_t errlen) {
    if (!h || !wav || !emb) {
        set_err(err, errlen, "speaker: null argument");
        return NAVI_ERR_INVALID;
    }
    int32_t T = 0;
    navi_status st = navi_speaker_mel(&h->p, wav, n, nullptr, 0, &T, err, errlen);   // length checks and the frame count
    if (st != NAVI_OK) return st;
    if (T > h->max_frames || n > h->wav_cap) {
        set_err(err, errlen, "speaker: reference audio longer than the encoder's max_seconds (%d frames > %d)", T, h->max_frames);
        return NAVI_ERR_INVALID;
    }
    if ((st = check_frames(h, T, err, errlen)) != NAVI_OK) return st;
    NAVI_TRY_HIP(hipMemcpyAsync(h->wav, wav, static_cast<size_t>(n) * sizeof(float), hipMemcpyHostToDevice, device_state().stream),
                 err, errlen);
    return embed_device(h, T, n, emb, err, errlen);
}

const float *navi_speaker_tap_mel(const navi_speaker *h, int32_t *n_frames) {
    if (n_frames) *n_frames = h ? h->last_frames : 0;
    return h ? h->mel : nullptr;
}

int32_t navi_speaker_dim(const navi_speaker *h) { return h ? h->p.enc_dim : 0; }

double navi_speaker_last_ms(const navi_speaker *h) { return h ? h->last_ms : 0.0; }

} // extern "C"
