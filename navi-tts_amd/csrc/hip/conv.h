// The implicit-GEMM convolution on the matrix cores (v_mfma_f32_16x16x32_f16), shared by the
// codec decoder (vocoder.hip: causal convs, transposed-conv phases) and the speaker encoder
// (speaker.hip: "same" convs with reflect padding). Rows = output time steps, columns = output
// channels, the reduction over (tap, input channel); weights laid out [phase][Cout][tap][Cin]
// (k_relayout_conv), activations staged per channel chunk as f16 hi + lo pairs.
#pragma once

#include "dev_common.h"

namespace navi_amd {
namespace cv {

constexpr int BT = 256;
constexpr int CCH = 64;                  // input channels staged per step
constexpr int LDW = CCH + 8;             // padded LDS row (halves)

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

// Prologues (applied to the input as it is staged): SILU_GATE silu(x[ci]) * x[Cin + ci]; ADD2 x + x2.
enum Pro { PRO_NONE = 0, PRO_SILU_GATE = 2, PRO_ADD2 = 3 };
// Epilogues after the bias: RELU_TANH is tanh(max(v, 0)); PARTIAL stores split-K partial sums.
enum Epi { EPI_BIAS = 0, EPI_GELU = 1, EPI_RESIDUAL = 2, EPI_SCALE_RESIDUAL = 3, EPI_CLAMP = 4, EPI_PARTIAL = 5,
           EPI_RELU = 6, EPI_SIGMOID = 7, EPI_RELU_TANH = 8 };

struct ConvArgs {
    const float *x;        // input rows [T][ldx]; PRO_SILU_GATE: gate at [ci], up at [Cin + ci]
    const float *hist;     // [(K-1)*dil][Cin] rows before t = 0, or null (zeros)
    const uint16_t *w;     // [phases][Cout][K][Cin] f16
    const float *bias;     // [Cout] or null
    const float *res;      // EPI_RESIDUAL / EPI_SCALE_RESIDUAL: rows like y (stride ldy)
    const float *scale;    // EPI_SCALE_RESIDUAL: [Cout]
    float *y;              // output row t * phases + phase, stride ldy (may be null when z is set)
    // Optional second output z = Snake(y) = y + sin^2(y * za) * zb per output channel (za = exp(alpha),
    // zb = 1 / (exp(beta) + 1e-9)): the prologue of the conv that consumes y, applied once per
    // element by its producer. Same layout as y.
    float *z;
    const float *za, *zb;
    float *part;           // EPI_PARTIAL: [splits][T * phases][Cout] partial sums, no bias
    uint32_t *flag;        // set when a (prologue-applied) activation is outside the f16 range
    const float *x2;       // PRO_ADD2: second input, same layout as x
    int ldx, ldy, T, Cin, Cout, dil, phases, cps;   // cps: input channels per K split
    // Output t reads input rows t - lpad + j * dil (j < K): lpad = (K-1) dil is the causal conv,
    // (K-1) dil / 2 the "same" one. Rows outside [0, T) read hist / zero, or with reflect their
    // mirror (-t, 2 (T-1) - t: PyTorch padding_mode="reflect").
    int lpad, reflect;
};

__device__ __forceinline__ float silu(float g) { return g / (1.f + expf(-g)); }

__device__ __forceinline__ float snake(float v, float za, float zb) {
    const float sn = sinf(v * za);
    return v + sn * sn * zb;
}

// y (and z) at output (row, co) from the accumulated sum (EPI_PARTIAL excluded).
__device__ __forceinline__ void conv_epilogue(const ConvArgs &a, int epi, size_t o, int co, float v) {
    if (a.bias) v += gld(a.bias + co);
    if (epi == EPI_GELU) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    else if (epi == EPI_RESIDUAL) v += gld(a.res + o);
    else if (epi == EPI_SCALE_RESIDUAL) v = v * gld(a.scale + co) + gld(a.res + o);
    else if (epi == EPI_CLAMP) v = fminf(fmaxf(v, -1.f), 1.f);
    else if (epi == EPI_RELU) v = fmaxf(v, 0.f);
    else if (epi == EPI_SIGMOID) v = 1.f / (1.f + expf(-v));
    else if (epi == EPI_RELU_TANH) v = tanhf(fmaxf(v, 0.f));
    if (a.y) gst(a.y + o, v);
    if (a.z) gst(a.z + o, snake(v, gld(a.za + co), gld(a.zb + co)));
}

namespace {

// Output lane layout of v_mfma_f32_16x16x32_f16: lane l holds column l % 16 of rows
// 4 * (l / 16) + r, r = 0..3; A and B use the same lane -> k mapping. blockIdx.z = split *
// phases + phase: a block reduces input channels [split * cps, (split + 1) * cps).
template <int MT, int K, int PRO, int EPI>
__global__ void __launch_bounds__(BT) k_conv_mfma(ConvArgs a) {
    constexpr int MAXH = (K - 1) * 9;                       // dilation <= 9
    constexpr int WROWS = MT * 16 + MAXH;
    __shared__ __align__(16) _Float16 whi[WROWS][LDW];
    __shared__ __align__(16) _Float16 wlo[WROWS][LDW];
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int n0 = blockIdx.x * 64 + wv * 16;
    const int t0 = blockIdx.y * (MT * 16);
    const int phase = blockIdx.z % a.phases, split = blockIdx.z / a.phases;
    const int cb = split * a.cps, ce = min(a.Cin, cb + a.cps);
    const int H = (K - 1) * a.dil, rows = MT * 16 + H;
    const bool live = n0 < a.Cout;                          // Cout % 16 == 0: whole waves are in or out
    const uint16_t *wbase = a.w + (static_cast<size_t>(phase) * a.Cout + (live ? n0 + (l & 15) : 0)) * K * a.Cin + (l >> 4) * 8;
    f32x4_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // Staging of the time window of one channel chunk: a thread owns IT float4s of it, always
    // the same 4 channels (BT is a multiple of the chunk's float4 count, 8 or 16). A chunk's
    // loads (inputs, weights) are all issued at once, and the next chunk's go out before this
    // chunk's MFMAs, so no load waits on another.
    constexpr int IT = (WROWS * (CCH / 4) + BT - 1) / BT;
    constexpr bool TWO = PRO == PRO_SILU_GATE || PRO == PRO_ADD2;   // a second operand per element
    f32x4_t av[IT], au[TWO ? IT : 1];
    u32x4_t bq[K][CCH / 32];
    auto load_tap = [&](int j, int ci0) {
        const int cc = min(CCH, ce - ci0);
#pragma unroll
        for (int s = 0; s < CCH / 32; ++s)
            if (s * 32 < cc)
                bq[j][s] = __builtin_nontemporal_load((const NAVI_GLOBAL u32x4_t *) (wbase + static_cast<size_t>(j) * a.Cin + ci0 + s * 32));
    };
    auto load_a = [&](int ci0) {
        const int q4 = min(CCH, ce - ci0) >> 2;
        const int ci = ci0 + (threadIdx.x % q4) * 4;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int r = (threadIdx.x + it * BT) / q4;
            int t = t0 - a.lpad + r;
            if (a.reflect) t = t < 0 ? -t : t >= a.T ? 2 * (a.T - 1) - t : t;
            av[it] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (TWO) au[it] = av[it];
            if (r < rows) {
                if (t >= 0 && t < a.T) {
                    const float *row = a.x + static_cast<size_t>(t) * a.ldx;
                    av[it] = *(const NAVI_GLOBAL f32x4_t *) (row + ci);
                    if (PRO == PRO_SILU_GATE) au[it] = *(const NAVI_GLOBAL f32x4_t *) (row + a.Cin + ci);
                    if (PRO == PRO_ADD2) au[it] = *(const NAVI_GLOBAL f32x4_t *) (a.x2 + static_cast<size_t>(t) * a.ldx + ci);
                } else if (t < 0 && a.hist) {
                    av[it] = *(const NAVI_GLOBAL f32x4_t *) (a.hist + static_cast<size_t>(H + t) * a.Cin + ci);
                }
            }
        }
    };
    bool bad = false;
    if (cb < ce) {
        if (live)
#pragma unroll
            for (int j = 0; j < K; ++j) load_tap(j, cb);
        load_a(cb);
    }
    for (int ci0 = cb; ci0 < ce; ci0 += CCH) {
        const int cc = min(CCH, ce - ci0);                  // multiple of 32
        const bool more = ci0 + CCH < ce;
        __syncthreads();                                    // the previous chunk's readers are done
        {
            const int q4 = cc >> 2, c = (threadIdx.x % q4) * 4;
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int r = (threadIdx.x + it * BT) / q4;
                int t = t0 - a.lpad + r;
                if (a.reflect) t = t < 0 ? -t : t >= a.T ? 2 * (a.T - 1) - t : t;
                if (r >= rows) continue;
                f32x4_t v = av[it];
                if (PRO == PRO_SILU_GATE && t >= 0 && t < a.T) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = silu(v[e]) * au[it][e];
                }
                if (PRO == PRO_ADD2) v += au[it];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    bad |= !(fabsf(v[e]) < 65504.f);
                    const _Float16 h = static_cast<_Float16>(v[e]);
                    whi[r][c + e] = h;
                    wlo[r][c + e] = static_cast<_Float16>(v[e] - static_cast<float>(h));
                }
            }
        }
        __syncthreads();
        if (more) load_a(ci0 + CCH);
        if (live) {
#pragma unroll
            for (int j = 0; j < K; ++j) {
#pragma unroll
                for (int s = 0; s < CCH / 32; ++s) {
                    if (s * 32 < cc) {
                        half8v b;
                        __builtin_memcpy(&b, &bq[j][s], 16);
#pragma unroll
                        for (int i = 0; i < MT; ++i) {
                            const int wr = i * 16 + (l & 15) + j * a.dil;
                            const half8v h = *reinterpret_cast<const half8v *>(&whi[wr][s * 32 + (l >> 4) * 8]);
                            const half8v o = *reinterpret_cast<const half8v *>(&wlo[wr][s * 32 + (l >> 4) * 8]);
                            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, b, acc[i], 0, 0, 0);
                            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o, b, acc[i], 0, 0, 0);
                        }
                    }
                }
                if (more) load_tap(j, ci0 + CCH);           // tap j's registers are free again
            }
        }
    }
    if (bad) gst(a.flag, 1u);
    if (!live) return;
    const int co = n0 + (l & 15);
    float *part = a.part + static_cast<size_t>(split) * a.T * a.phases * a.Cout;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + i * 16 + (l >> 4) * 4 + r;
            if (t >= a.T) continue;
            const size_t row = static_cast<size_t>(t) * a.phases + phase;
            if (EPI == EPI_PARTIAL) gst(part + row * a.Cout + co, acc[i][r]);
            else conv_epilogue(a, EPI, row * a.ldy + co, co, acc[i][r]);
        }
}

// Sum of the K-split partials in split order, then the epilogue (EPI_PARTIAL's second half).
// (kernels in an unnamed namespace: every including file gets its own)
__global__ void __launch_bounds__(BT) k_conv_finish(ConvArgs a, int splits, int epi) {
    const size_t rows = static_cast<size_t>(a.T) * a.phases, n = rows * a.Cout;
    const size_t i = static_cast<size_t>(blockIdx.x) * BT + threadIdx.x;
    if (i >= n) return;
    const size_t row = i / a.Cout;
    const int co = static_cast<int>(i - row * a.Cout);
    float v = 0.f;
    for (int s0 = 0; s0 < splits; s0 += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (s0 + j < splits) t[j] = gld(a.part + (s0 + j) * n + i);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (s0 + j < splits) v = s0 + j == 0 ? t[j] : v + t[j];
    }
    conv_epilogue(a, epi, row * a.ldy + co, co, v);
}

// [Cout][Cin][K] -> [Cout][K][Cin]
__global__ void k_relayout_conv(const uint16_t *w, int Cout, int Cin, int K, uint16_t *out) {
    const size_t i = static_cast<size_t>(blockIdx.x) * BT + threadIdx.x, n = static_cast<size_t>(Cout) * Cin * K;
    if (i >= n) return;
    const int j = static_cast<int>(i % K), ci = static_cast<int>((i / K) % Cin), co = static_cast<int>(i / (static_cast<size_t>(K) * Cin));
    gst(out + (static_cast<size_t>(co) * K + j) * Cin + ci, gld(w + i));
}


} // namespace

} // namespace cv
} // namespace navi_amd
