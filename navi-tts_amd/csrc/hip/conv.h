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
typedef _Float16 half4v __attribute__((ext_vector_type(4)));

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
    // When set: the causal history the next chunk reads (the last (K-1) dil rows of [hist ; x]),
    // written by this launch into the other buffer of the conv's history pair.
    float *hnext;
    // RVQ rows (rvq_row4): codes [T][nq]; input channel ci < Cin/2 of frame t is cb0[code 0][ci],
    // channel Cin/2 + c the sum over q = 1..nq-1 of cbr[q-1][code q][c] (codebooks [cbsize][Cin/2] f16).
    const int32_t *codes;
    const uint16_t *cb0, *cbr;
    int nq, cbsize;
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

// The per-output-channel operands of the epilogue, loaded once per thread (a thread's outputs
// share their channel).
struct EpiCol {
    float bias, scale, za, zb;
};
__device__ __forceinline__ EpiCol epi_col(const ConvArgs &a, int epi, int co) {
    EpiCol c{0.f, 1.f, 0.f, 0.f};
    if (a.bias) c.bias = gld(a.bias + co);
    if (epi == EPI_SCALE_RESIDUAL) c.scale = gld(a.scale + co);
    if (a.z) {
        c.za = gld(a.za + co);
        c.zb = gld(a.zb + co);
    }
    return c;
}
__device__ __forceinline__ bool epi_has_res(int epi) { return epi == EPI_RESIDUAL || epi == EPI_SCALE_RESIDUAL; }

// y (and z) at output offset o from the accumulated sum v (EPI_PARTIAL excluded); res: the
// residual at o, loaded by the caller before any of its stores (the residual stream is usually
// y itself, so a load after a store could not be hoisted and every output would wait a memory
// round trip).
__device__ __forceinline__ void conv_store(const ConvArgs &a, int epi, size_t o, const EpiCol &c, float v, float res) {
    if (a.bias) v += c.bias;
    if (epi == EPI_GELU) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    else if (epi == EPI_RESIDUAL) v += res;
    else if (epi == EPI_SCALE_RESIDUAL) v = v * c.scale + res;
    else if (epi == EPI_CLAMP) v = fminf(fmaxf(v, -1.f), 1.f);
    else if (epi == EPI_RELU) v = fmaxf(v, 0.f);
    else if (epi == EPI_SIGMOID) v = 1.f / (1.f + expf(-v));
    else if (epi == EPI_RELU_TANH) v = tanhf(fmaxf(v, 0.f));
    if (a.y) gst(a.y + o, v);
    if (a.z) gst(a.z + o, snake(v, c.za, c.zb));
}

// rows [0, H) of out = the last H rows of [hist ; x] (C channels; hist [H][C], x rows of stride
// ldx): the causal history a conv (or the ConvNeXt depthwise conv) reads in the next chunk. out is
// the other buffer of the history pair, which the running launch does not read, so every block of
// the launch can copy an equal share of it, each with its loads issued before its stores.
__device__ __forceinline__ void carry_rows(const float *hist, const float *x, int ldx, int T, int H, int C, float *out) {
    const int q = C >> 2, n = H * q;
    const int nb = gridDim.x * gridDim.y * gridDim.z;
    const int b = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const int per = (n + nb - 1) / nb, i0 = b * per, i1 = min(n, i0 + per);
    constexpr int U = 4;
    for (int i = i0 + static_cast<int>(threadIdx.x); i < i1; i += U * BT) {
        f32x4_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = i + u * BT;
            if (k < i1) {
                const int r = k / q, c = (k - r * q) * 4, src = r + T - H;   // row of x, or of hist if < 0
                v[u] = src >= 0 ? ld4(x + static_cast<size_t>(src) * ldx + c) : ld4(hist + static_cast<size_t>(src + H) * C + c);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = i + u * BT;
            if (k < i1) {
                const int r = k / q, c = (k - r * q) * 4;
                st4(out + static_cast<size_t>(r) * C + c, v[u]);
            }
        }
    }
}

// The (column block, row tile) of this block in a gridDim.x x gridDim.y tile grid, remapped for
// the round-robin dispatch of block ids over the 8 XCDs (block x + gridDim.x y goes to XCD
// (x + gridDim.x y) % 8): XCD k's blocks take a contiguous run of the tiles in row-major order, so
// the column blocks of a row tile, which read the same input window, share one L2.
__device__ __forceinline__ void xcd_tile(int &col, int &row) {
    const int ncol = static_cast<int>(gridDim.x), n = ncol * static_cast<int>(gridDim.y);
    const int id = static_cast<int>(blockIdx.x) + ncol * static_cast<int>(blockIdx.y);
    const int k = id & 7, slot = id >> 3, q = n >> 3, r = n & 7;
    const int tile = k * q + min(k, r) + slot;           // XCD k holds q + (k < r) ids
    col = tile % ncol;
    row = tile / ncol;
}

// Four input channels ci..ci+3 of the RVQ front end at frame t: the semantic codebook's row, or
// the rest codebooks' rows summed in f32 in codebook order (k_rvq, vocoder.hip:125-143).
// Every code load first (indices clamped into the frame's row, so all of them run at once), then
// every row load, then the sum: two memory latencies.
__device__ __forceinline__ f32x4_t rvq_row4(const ConvArgs &a, int t, int ci) {
    const int half = a.Cin >> 1;
    const int32_t *code = a.codes + static_cast<size_t>(t) * a.nq;
    auto unpack = [](u32x2_t w) {
        return f32x4_t{h2f(static_cast<uint16_t>(w.x)), h2f(static_cast<uint16_t>(w.x >> 16)), h2f(static_cast<uint16_t>(w.y)),
                       h2f(static_cast<uint16_t>(w.y >> 16))};
    };
    if (ci < half) return unpack(gld(reinterpret_cast<const u32x2_t *>(a.cb0 + static_cast<size_t>(gld(code)) * half + ci)));
    constexpr int MAXQ = 16;
    int cq[MAXQ - 1];
#pragma unroll
    for (int q = 1; q < MAXQ; ++q) cq[q - 1] = gld(code + min(q, a.nq - 1));
    u32x2_t w[MAXQ - 1];
#pragma unroll
    for (int q = 1; q < MAXQ; ++q)
        if (q < a.nq)
            w[q - 1] = gld(reinterpret_cast<const u32x2_t *>(a.cbr + (static_cast<size_t>(q - 1) * a.cbsize + cq[q - 1]) * half +
                                                            (ci - half)));
    f32x4_t v = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 1; q < MAXQ; ++q)
        if (q < a.nq) v += unpack(w[q - 1]);
    return v;
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
    int tcol, trow;
    xcd_tile(tcol, trow);
    const int n0 = tcol * 64 + wv * 16;
    const int t0 = trow * (MT * 16);
    const int phase = blockIdx.z % a.phases, split = blockIdx.z / a.phases;
    const int cb = split * a.cps, ce = min(a.Cin, cb + a.cps);
    const int H = (K - 1) * a.dil, rows = MT * 16 + H;
    const bool live = n0 < a.Cout;                          // Cout % 16 == 0: whole waves are in or out
    const uint16_t *wbase = a.w + (static_cast<size_t>(phase) * a.Cout + (live ? n0 + (l & 15) : 0)) * K * a.Cin + (l >> 4) * 8;
    f32x4_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // Staging of the time window of one channel chunk: a thread owns the same 4 channels c4 of every
    // chunk and rows rr0 + 16 it of the window (IT of them). Where each of those rows comes from (a
    // row of x, of the history, or zeros) is the same for every chunk, so it is worked out once:
    // off[it] is the element offset of the row's channel 0 in x (bit it of xm) or in hist (hm). A
    // chunk's loads (inputs, weights) are all issued at once,
    // and the next chunk's go out before this chunk's MFMAs, so no load waits on another.
    constexpr int Q4 = CCH / 4, RPI = BT / Q4;               // float4s per staged row, rows per item step
    constexpr int IT = (WROWS + RPI - 1) / RPI;
    constexpr bool TWO = PRO == PRO_SILU_GATE || PRO == PRO_ADD2;   // a second operand per element
    static_assert(BT % Q4 == 0, "every item step covers whole rows");
    const int c4 = (static_cast<int>(threadIdx.x) % Q4) * 4, rr0 = static_cast<int>(threadIdx.x) / Q4;
    int off[IT];
    uint32_t xm = 0, hm = 0;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int r = rr0 + RPI * it;
        int t = t0 - a.lpad + r;
        if (a.reflect) t = t < 0 ? -t : t >= a.T ? 2 * (a.T - 1) - t : t;
        off[it] = 0;
        if (r < rows) {
            if (t >= 0 && t < a.T) {
                off[it] = t * a.ldx;
                xm |= 1u << it;
            } else if (t < 0 && a.hist) {
                off[it] = (H + t) * a.Cin;
                hm |= 1u << it;
            }
        }
    }
    f32x4_t av[IT], au[TWO ? IT : 1];
    u32x4_t bq[K][CCH / 32];
    auto load_tap = [&](int j, int ci0) {
        const int cc = min(CCH, ce - ci0);
#pragma unroll
        for (int s = 0; s < CCH / 32; ++s)   // past the chunk's channels: zeros (the staged A is zero there too)
            bq[j][s] = s * 32 < cc ? *((const NAVI_GLOBAL u32x4_t *) (wbase + static_cast<size_t>(j) * a.Cin + ci0 + s * 32))
                                   : u32x4_t{0u, 0u, 0u, 0u};
    };
    auto load_a = [&](int ci0) {
        const bool in = c4 < ce - ci0;                      // this thread's channels are inside the chunk
        const int ci = ci0 + c4;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            av[it] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (TWO) au[it] = av[it];
            if (!in) continue;
            if ((xm >> it) & 1u) {
                const float *row = a.x + off[it];
                av[it] = *(const NAVI_GLOBAL f32x4_t *) (row + ci);
                if (PRO == PRO_SILU_GATE) au[it] = *(const NAVI_GLOBAL f32x4_t *) (row + a.Cin + ci);
                if (PRO == PRO_ADD2) au[it] = *(const NAVI_GLOBAL f32x4_t *) (a.x2 + off[it] + ci);
            } else if ((hm >> it) & 1u) {
                av[it] = *(const NAVI_GLOBAL f32x4_t *) (a.hist + off[it] + ci);
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
        const bool more = ci0 + CCH < ce;
        __syncthreads();                                    // the previous chunk's readers are done
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int r = rr0 + RPI * it;
            if (r >= rows) continue;
            f32x4_t v = av[it];
            if (PRO == PRO_SILU_GATE && ((xm >> it) & 1u)) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = silu(v[e]) * au[it][e];
            }
            if (PRO == PRO_ADD2) v += au[it];
            half4v h, o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bad |= !(fabsf(v[e]) < 65504.f);
                h[e] = static_cast<_Float16>(v[e]);
                o[e] = static_cast<_Float16>(v[e] - static_cast<float>(h[e]));
            }
            *reinterpret_cast<half4v *>(&whi[r][c4]) = h;
            *reinterpret_cast<half4v *>(&wlo[r][c4]) = o;
        }
        __syncthreads();
        if (more) load_a(ci0 + CCH);
        if (live) {
#pragma unroll
            for (int j = 0; j < K; ++j) {
                // a partial chunk's missing channels hold zeros in A and B: no branch here, so the
                // accumulators stay in place across the unrolled steps
#pragma unroll
                for (int s = 0; s < CCH / 32; ++s) {
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
                if (more) load_tap(j, ci0 + CCH);           // tap j's registers are free again
            }
        }
    }
    if (bad) gst(a.flag, 1u);
    // the next chunk's history last: its stores wait for its loads, which nothing else needs
    if (!live) {
        if (a.hnext) carry_rows(a.hist, a.x, a.ldx, a.T, H, a.Cin, a.hnext);
        return;
    }
    const int co = n0 + (l & 15);
    float *part = a.part + static_cast<size_t>(split) * a.T * a.phases * a.Cout;
    if constexpr (EPI == EPI_PARTIAL) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + i * 16 + (l >> 4) * 4 + r;
                if (t < a.T) gst(part + (static_cast<size_t>(t) * a.phases + phase) * a.Cout + co, acc[i][r]);
            }
    } else {
        // every load of the epilogue first, then the stores
        const EpiCol cc = epi_col(a, EPI, co);
        float res[MT][4];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + i * 16 + (l >> 4) * 4 + r;
                res[i][r] = epi_has_res(EPI) && t < a.T ? gld(a.res + (static_cast<size_t>(t) * a.phases + phase) * a.ldy + co) : 0.f;
            }
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + i * 16 + (l >> 4) * 4 + r;
                if (t < a.T) conv_store(a, EPI, (static_cast<size_t>(t) * a.phases + phase) * a.ldy + co, cc, acc[i][r], res[i][r]);
            }
    }
    if (a.hnext) carry_rows(a.hist, a.x, a.ldx, a.T, H, a.Cin, a.hnext);
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// The wide implicit-GEMM conv for the decoder blocks' causal convs (K = 7, 2 or 1, any number of
// transposed-conv phases, no prologue): v_mfma_f32_32x32x16_f16, whose operands cover
// twice the products of a 16x16x32 step per LDS read. A block computes BM rows x BN output channels
// of one phase (blockIdx.z); per chunk of 32 input channels it stages in LDS the time window
// (BM + (K-1) dil rows, f16 hi + lo) and the weights of every tap for its BN channels, so each
// operand is read from memory once per block and from LDS by the waves that use it. BM = 128:
// wave w owns rows 32w..32w+31 and all BN / 32 column tiles (every A read feeds BN / 32 MFMAs);
// BM = 64: waves in 2 x 2, BN / 2 columns each (twice the blocks for short chunks). Per output the
// sum runs over chunks, taps, 16-channel steps, hi then lo, in an order that does not depend on BM,
// BN or T. The next chunk's loads are in flight during this chunk's MFMAs.
// Lane layout of the 32x32x16 step (checked on the device): lane l holds A[l % 32][8 (l / 32) ..]
// and B[8 (l / 32) ..][l % 32]; accumulator r of lane l is row 8 (r / 4) + 4 (l / 32) + r % 4,
// column l % 32.
// Input-channel splits (a conv whose output tiles alone leave the CUs idle in short chunks): the
// channels fall into S equal ranges of a.cps. SM = 1: block z = phase * S + s sums range s only and
// writes it to a.part[s] (k_conv_finish adds the ranges in order and applies the epilogue);
// SM = 2: one block sums every range, each from zero, and adds the range sums in the same order
// itself, so a launch without partials gives the same bits as the split launch (the split count is
// the conv's, whatever the chunk; only how it runs depends on the chunk's size). SM = 0: no split.
template <int K, int BM, int BN, int EPI, int CC = 32, int SM = 0>
__global__ void __launch_bounds__(BT) k_conv_wide(ConvArgs a) {
    constexpr int LDA = CC + 8;                             // LDS row (halves)
    static_assert(CC == 32 || CC == 16, "channels per chunk");
    constexpr int MAXWR = BM + (K - 1) * 9;                 // window rows at dilation <= 9
    constexpr int NCT = BM == 128 ? BN / 32 : BN / 64;      // 32-column tiles per wave
    static_assert(BN % 32 == 0 && (BM == 128 || (BM == 64 && BN % 64 == 0)), "tile shape");
    __shared__ __align__(16) _Float16 ahi[MAXWR * LDA];
    __shared__ __align__(16) _Float16 alo[MAXWR * LDA];
    __shared__ __align__(16) _Float16 bw[K * BN * LDA];
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int wr = BM == 128 ? 32 * wv : 32 * (wv >> 1), wc = BM == 128 ? 0 : (BN / 2) * (wv & 1);
    const int S = SM == 1 ? static_cast<int>(gridDim.z) / a.phases : 1, sp = SM == 1 ? static_cast<int>(blockIdx.z) % S : 0;
    int tcol, trow;
    xcd_tile(tcol, trow);
    const int n0 = tcol * BN, t0 = trow * BM, phase = SM == 1 ? static_cast<int>(blockIdx.z) / S : blockIdx.z;
    const int cbeg = SM == 1 ? sp * a.cps : 0, cend = SM == 1 ? min(a.Cin, cbeg + a.cps) : a.Cin;
    const int H = (K - 1) * a.dil, rows = BM + H;
    // A staging: 8 float4 per window row, thread -> rows (tid / 8) + 32 it, channels 4 (tid % 8);
    // each row's source (x, history or zeros) fixed for the launch
    constexpr int RPI = BT / (CC / 4), ITA = (MAXWR + RPI - 1) / RPI;
    const int c4 = (static_cast<int>(threadIdx.x) % (CC / 4)) * 4, rr0 = static_cast<int>(threadIdx.x) / (CC / 4);
    int aoff[ITA];
    uint32_t xm = 0, hm = 0;
#pragma unroll
    for (int it = 0; it < ITA; ++it) {
        const int r = rr0 + RPI * it, t = t0 - a.lpad + r;
        aoff[it] = 0;
        if (r < rows) {
            if (t >= 0 && t < a.T) {
                aoff[it] = t * a.ldx + c4;
                xm |= 1u << it;
            } else if (t < 0 && a.hist) {
                aoff[it] = (H + t) * a.Cin + c4;
                hm |= 1u << it;
            }
        }
    }
    // B staging: channels [ci0, ci0 + CC) of (column, tap), in CC / 8 pieces of 16 B
    constexpr int QB = CC / 8, NBI = BN * K * QB, ITB = (NBI + BT - 1) / BT;
    int boff[ITB], bl[ITB];
#pragma unroll
    for (int it = 0; it < ITB; ++it) {
        const int e = static_cast<int>(threadIdx.x) + BT * it, q = e % QB, ct = e / QB, col = ct / K, tap = ct - col * K;
        boff[it] = ((phase * a.Cout + n0 + col) * K + tap) * a.Cin + 8 * q;
        bl[it] = (tap * BN + col) * LDA + 8 * q;
    }
    f32x4_t av[ITA];
    u32x4_t bv[ITB];
    auto load = [&](int ci0) {
#pragma unroll
        for (int it = 0; it < ITA; ++it) {
            av[it] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if ((xm >> it) & 1u) av[it] = *(const NAVI_GLOBAL f32x4_t *) (a.x + aoff[it] + ci0);
            else if ((hm >> it) & 1u) av[it] = *(const NAVI_GLOBAL f32x4_t *) (a.hist + aoff[it] + ci0);
        }
#pragma unroll
        for (int it = 0; it < ITB; ++it)
            if (ITB * BT == NBI || static_cast<int>(threadIdx.x) + BT * it < NBI)
                bv[it] = *((const NAVI_GLOBAL u32x4_t *) (a.w + boff[it] + ci0));
    };
    f32x16_t acc[NCT], racc[SM == 2 ? NCT : 1];
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
    bool bad = false, rfirst = true;
    load(cbeg);
    for (int ci0 = cbeg; ci0 < cend; ci0 += CC) {
        if constexpr (SM == 2) {
            if (ci0 > 0 && ci0 % a.cps == 0) {              // a range ends: fold its sum in, restart from zero
#pragma unroll
                for (int c = 0; c < NCT; ++c)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        racc[c][r] = rfirst ? acc[c][r] : racc[c][r] + acc[c][r];
                        acc[c][r] = 0.f;
                    }
                rfirst = false;
            }
        }
        __syncthreads();                                    // the previous chunk's readers are done
#pragma unroll
        for (int it = 0; it < ITA; ++it) {
            const int r = rr0 + RPI * it;
            if (r >= rows) continue;
            half4v h, o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bad |= !(fabsf(av[it][e]) < 65504.f);
                h[e] = static_cast<_Float16>(av[it][e]);
                o[e] = static_cast<_Float16>(av[it][e] - static_cast<float>(h[e]));
            }
            *reinterpret_cast<half4v *>(&ahi[r * LDA + c4]) = h;
            *reinterpret_cast<half4v *>(&alo[r * LDA + c4]) = o;
        }
#pragma unroll
        for (int it = 0; it < ITB; ++it)
            if (ITB * BT == NBI || static_cast<int>(threadIdx.x) + BT * it < NBI)
                *reinterpret_cast<u32x4_t *>(&bw[bl[it]]) = bv[it];
        __syncthreads();
        if (ci0 + CC < cend) load(ci0 + CC);
#pragma unroll
        for (int j = 0; j < K; ++j) {
#pragma unroll
            for (int ks = 0; ks < CC / 16; ++ks) {
                const int ar = (wr + (l & 31) + j * a.dil) * LDA + 16 * ks + 8 * (l >> 5);
                const half8v h = *reinterpret_cast<const half8v *>(&ahi[ar]);
                const half8v o = *reinterpret_cast<const half8v *>(&alo[ar]);
#pragma unroll
                for (int c = 0; c < NCT; ++c) {
                    const half8v b = *reinterpret_cast<const half8v *>(&bw[(j * BN + wc + 32 * c + (l & 31)) * LDA + 16 * ks + 8 * (l >> 5)]);
                    acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h, b, acc[c], 0, 0, 0);
                    acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(o, b, acc[c], 0, 0, 0);
                }
            }
        }
    }
    if (bad) gst(a.flag, 1u);
    if constexpr (SM == 2) {
        if (!rfirst) {
#pragma unroll
            for (int c = 0; c < NCT; ++c)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[c][r] = racc[c][r] + acc[c][r];
        }
    }
    if constexpr (SM == 1) {
        float *part = a.part + static_cast<size_t>(sp) * a.T * a.phases * a.Cout;
#pragma unroll
        for (int c = 0; c < NCT; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t0 + wr + 8 * (r / 4) + 4 * (l >> 5) + (r & 3), co = n0 + wc + 32 * c + (l & 31);
                if (t < a.T) gst(part + (static_cast<size_t>(t) * a.phases + phase) * a.Cout + co, acc[c][r]);
            }
        if (a.hnext) carry_rows(a.hist, a.x, a.ldx, a.T, H, a.Cin, a.hnext);
        return;
    }
    // every load of the epilogue first (column operands, residuals), then the stores
    EpiCol cc[NCT];
#pragma unroll
    for (int c = 0; c < NCT; ++c) cc[c] = epi_col(a, EPI, n0 + wc + 32 * c + (l & 31));
    float res[NCT][16];
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + wr + 8 * (r / 4) + 4 * (l >> 5) + (r & 3), co = n0 + wc + 32 * c + (l & 31);
            res[c][r] = epi_has_res(EPI) && t < a.T
                            ? gld(a.res + (static_cast<size_t>(t) * a.phases + phase) * a.ldy + co) : 0.f;
        }
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + wr + 8 * (r / 4) + 4 * (l >> 5) + (r & 3), co = n0 + wc + 32 * c + (l & 31);
            if (t < a.T) conv_store(a, EPI, (static_cast<size_t>(t) * a.phases + phase) * a.ldy + co, cc[c], acc[c][r], res[c][r]);
        }
    if (a.hnext) carry_rows(a.hist, a.x, a.ldx, a.T, H, a.Cin, a.hnext);
}

// The 96-channel convs (the codec decoder's last block and its final conv): a block covers
// RB = 64 MT rows and every output channel (Cout = 16 NCT). The whole input window (the rows plus
// the (K-1) dil causal halo, all 96 channels, f16 hi + lo) is staged in LDS once, and so is each
// tap's weight slice [Cout][96], one tap ahead of its MFMAs: the four waves (16 MT rows each)
// read both operands from LDS, and the input is read ~1.4x instead of the 64-column blocks'
// ~3.7x. Per output the sum runs over taps, then 32-channel steps, in an order that does not
// depend on T. Causal (rows before 0 from hist), no K split, no prologue, phases 1, dil <= 9.
template <int K, int NCT, int MT, int EPI>
__global__ void __launch_bounds__(BT) k_conv_c96(ConvArgs a) {
    constexpr int CIN = 96, LD = CIN + 8, RB = 64 * MT, MAXROWS = RB + (K - 1) * 9, CO = 16 * NCT;
    constexpr int WCH = CO * (CIN / 8), WIT = (WCH + BT - 1) / BT;   // 16-byte chunks of a tap's weights
    __shared__ __align__(16) _Float16 xhi[MAXROWS * LD];
    __shared__ __align__(16) _Float16 xlo[MAXROWS * LD];
    __shared__ __align__(16) _Float16 wt[2][CO * LD];
    const int H = (K - 1) * a.dil, rows = RB + H;
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int t0 = blockIdx.x * RB;
    auto load_w = [&](int j, u32x4_t (&r)[WIT]) {
#pragma unroll
        for (int k = 0; k < WIT; ++k) {
            const int i = threadIdx.x + k * BT, co = i / (CIN / 8), c8 = i - co * (CIN / 8);
            if (i < WCH) r[k] = *(const NAVI_GLOBAL u32x4_t *) (a.w + (static_cast<size_t>(co) * K + j) * CIN + c8 * 8);
        }
    };
    auto store_w = [&](int buf, const u32x4_t (&r)[WIT]) {
#pragma unroll
        for (int k = 0; k < WIT; ++k) {
            const int i = threadIdx.x + k * BT, co = i / (CIN / 8), c8 = i - co * (CIN / 8);
            if (i < WCH) *reinterpret_cast<u32x4_t *>(&wt[buf][co * LD + c8 * 8]) = r[k];
        }
    };
    u32x4_t wr[WIT];
    load_w(0, wr);
    // the input window: all of its loads go out IB float4 per thread at a time before any is used
    bool bad = false;
    {
        constexpr int q4 = CIN / 4, IT = (MAXROWS * q4 + BT - 1) / BT, IB = IT < 12 ? IT : 12;
#pragma unroll
        for (int b0 = 0; b0 < IT; b0 += IB) {
            f32x4_t sv[IB];
#pragma unroll
            for (int k = 0; k < IB; ++k) {
                const int i = threadIdx.x + (b0 + k) * BT, r = i / q4, c = (i - r * q4) * 4, t = t0 - a.lpad + r;
                sv[k] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                if (b0 + k < IT && r < rows) {
                    if (t >= 0 && t < a.T) sv[k] = *(const NAVI_GLOBAL f32x4_t *) (a.x + static_cast<size_t>(t) * a.ldx + c);
                    else if (t < 0 && a.hist) sv[k] = *(const NAVI_GLOBAL f32x4_t *) (a.hist + static_cast<size_t>(H + t) * CIN + c);
                }
            }
#pragma unroll
            for (int k = 0; k < IB; ++k) {
                const int i = threadIdx.x + (b0 + k) * BT, r = i / q4, c = (i - r * q4) * 4;
                if (b0 + k >= IT || r >= rows) continue;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    bad |= !(fabsf(sv[k][e]) < 65504.f);
                    const _Float16 h = static_cast<_Float16>(sv[k][e]);
                    xhi[r * LD + c + e] = h;
                    xlo[r * LD + c + e] = static_cast<_Float16>(sv[k][e] - static_cast<float>(h));
                }
            }
        }
    }
    if (bad) gst(a.flag, 1u);
    store_w(0, wr);
    __syncthreads();
    f32x4_t acc[MT][NCT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int n = 0; n < NCT; ++n) acc[i][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const int buf = j & 1;
        if (j + 1 < K) load_w(j + 1, wr);                   // next tap's weights, in flight meanwhile
#pragma unroll
        for (int ks = 0; ks < CIN / 32; ++ks) {
            half8v b[NCT];
#pragma unroll
            for (int n = 0; n < NCT; ++n)
                b[n] = *reinterpret_cast<const half8v *>(&wt[buf][(n * 16 + (l & 15)) * LD + ks * 32 + (l >> 4) * 8]);
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int r = wv * (16 * MT) + i * 16 + (l & 15) + j * a.dil;
                const half8v h = *reinterpret_cast<const half8v *>(&xhi[r * LD + ks * 32 + (l >> 4) * 8]);
                const half8v o = *reinterpret_cast<const half8v *>(&xlo[r * LD + ks * 32 + (l >> 4) * 8]);
#pragma unroll
                for (int n = 0; n < NCT; ++n) {
                    acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, b[n], acc[i][n], 0, 0, 0);
                    acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o, b[n], acc[i][n], 0, 0, 0);
                }
            }
        }
        if (j + 1 < K) {
            store_w(buf ^ 1, wr);                           // last read in tap j - 1, before the barrier below it
            __syncthreads();
        }
    }
    // every load of the epilogue first (column operands, residuals), then the stores
    EpiCol cc[NCT];
#pragma unroll
    for (int n = 0; n < NCT; ++n) cc[n] = epi_col(a, EPI, n * 16 + (l & 15));
    float res[MT][4][NCT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + wv * (16 * MT) + i * 16 + (l >> 4) * 4 + r;
#pragma unroll
            for (int n = 0; n < NCT; ++n)
                res[i][r][n] = epi_has_res(EPI) && t < a.T ? gld(a.res + static_cast<size_t>(t) * a.ldy + n * 16 + (l & 15)) : 0.f;
        }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + wv * (16 * MT) + i * 16 + (l >> 4) * 4 + r;
            if (t >= a.T) continue;
#pragma unroll
            for (int n = 0; n < NCT; ++n) {
                const int co = n * 16 + (l & 15);
                conv_store(a, EPI, static_cast<size_t>(t) * a.ldy + co, cc[n], acc[i][n][r], res[i][r][n]);
            }
        }
    if (a.hnext) carry_rows(a.hist, a.x, a.ldx, a.T, H, CIN, a.hnext);
}

// One residual unit of the codec decoder's narrow blocks (C = 96 or 192 channels) in one kernel:
// the Snake'd residual stream x -> k7 conv (dilation dil) + bias -> Snake with the k1's parameters
// -> k1 conv + bias + the residual -> y, and y's Snake with the next conv's parameters -> z. A block
// owns BM rows and all C output channels (C = 96: 128 rows, waves 4 x 1, each wave 32 rows x 96
// columns, or 32 rows, waves 1 x 3, each wave 32 rows x 32 columns and the fourth wave staging only;
// C = 192: 64 rows, waves 2 x 2, each wave 32 rows x 96 columns). An output's sums run the same
// MFMA chain whatever BM. The k7 stages its time window and every tap's weights per
// CC7-channel chunk as k_conv_wide does; its output tile goes through the Snake into LDS as f16 hi
// + lo, where the k1 reads it as its A operand while the k1's weights are staged 32 channels at a
// time, the next piece in flight during the MFMAs: the intermediate never goes to memory and the
// unit is one launch. Per output the k7 sums chunks, taps, 16-channel steps, hi then lo, and the
// k1 16-channel steps in channel order, hi then lo, whatever the chunk's row count.
struct UnitArgs {
    const float *x, *hist;              // k7 input rows [T][C] and its history [6 dil][C]
    float *hnext;                       // the next chunk's k7 history (the other buffer of its pair)
    const uint16_t *w7, *w1;            // [C][7][C] and [C][C] f16
    const float *b7, *b1;               // [C]
    const float *za_mid, *zb_mid;       // the Snake on the k1's input
    const float *res;                   // the residual stream [T][C]
    float *y;                           // the unit's output [T][C] (may be res itself), or null
    float *z;                           // Snake(y) with (za, zb): the next conv's input; not x
    const float *za, *zb;
    uint32_t *flag;
    int T, dil;
};

template <int C, int BM, int CC7>
__global__ void __launch_bounds__(BT) k_unit(UnitArgs u) {
    constexpr int K = 7, LDA = CC7 + 8;
    constexpr int WRW = BM / 32;                            // waves along rows
    constexpr int WCW = 4 / WRW < C / 32 ? 4 / WRW : C / 32;   // waves along columns
    constexpr int NCT = C / (WCW * 32);                     // 32-column tiles per wave
    static_assert(WRW * WCW <= 4 && C == WCW * 32 * NCT, "each computing wave 32 rows x 32 NCT columns");
    constexpr int MAXWR = BM + (K - 1) * 9, LDM = C + 8, CC1 = 32, LDW = CC1 + 8;
    constexpr int A_BYTES = MAXWR * LDA * 2 * 2, B_BYTES = K * C * LDA * 2;           // k7 staging
    constexpr int M_BYTES = BM * LDM * 2 * 2, W_BYTES = C * LDW * 2;                  // k1 operands
    constexpr int SMEM = (A_BYTES + B_BYTES > M_BYTES + W_BYTES ? A_BYTES + B_BYTES : M_BYTES + W_BYTES);
    __shared__ __align__(16) unsigned char smem[SMEM];
    _Float16 *ahi = reinterpret_cast<_Float16 *>(smem), *alo = ahi + MAXWR * LDA, *bw = alo + MAXWR * LDA;
    _Float16 *mhi = reinterpret_cast<_Float16 *>(smem), *mlo = mhi + BM * LDM, *w1s = mlo + BM * LDM;
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int wr = 32 * (wv % WRW), wc = 32 * NCT * (wv / WRW);
    const bool mma = wv < WRW * WCW;                        // a computing wave (the rest stage only)
    const int t0 = blockIdx.x * BM;
    const int H = (K - 1) * u.dil, rows = BM + H, lpad = H;
    // ---- k7: the staging and step order of k_conv_wide ----
    constexpr int RPI = BT / (CC7 / 4), ITA = (MAXWR + RPI - 1) / RPI;
    const int c4 = (static_cast<int>(threadIdx.x) % (CC7 / 4)) * 4, rr0 = static_cast<int>(threadIdx.x) / (CC7 / 4);
    int aoff[ITA];
    uint32_t xm = 0, hm = 0;
#pragma unroll
    for (int it = 0; it < ITA; ++it) {
        const int r = rr0 + RPI * it, t = t0 - lpad + r;
        aoff[it] = 0;
        if (r < rows) {
            if (t >= 0 && t < u.T) {
                aoff[it] = t * C + c4;
                xm |= 1u << it;
            } else if (t < 0 && u.hist) {
                aoff[it] = (H + t) * C + c4;
                hm |= 1u << it;
            }
        }
    }
    constexpr int QB = CC7 / 8, NBI = C * K * QB, ITB = (NBI + BT - 1) / BT;
    int boff[ITB], bl[ITB];
#pragma unroll
    for (int it = 0; it < ITB; ++it) {
        const int e = static_cast<int>(threadIdx.x) + BT * it, q = e % QB, ct = e / QB, col = ct / K, tap = ct - col * K;
        boff[it] = (col * K + tap) * C + 8 * q;
        bl[it] = (tap * C + col) * LDA + 8 * q;
    }
    f32x4_t av[ITA];
    u32x4_t bv[ITB];
    auto load = [&](int ci0) {
#pragma unroll
        for (int it = 0; it < ITA; ++it) {
            av[it] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if ((xm >> it) & 1u) av[it] = *(const NAVI_GLOBAL f32x4_t *) (u.x + aoff[it] + ci0);
            else if ((hm >> it) & 1u) av[it] = *(const NAVI_GLOBAL f32x4_t *) (u.hist + aoff[it] + ci0);
        }
#pragma unroll
        for (int it = 0; it < ITB; ++it)
            if (ITB * BT == NBI || static_cast<int>(threadIdx.x) + BT * it < NBI)
                bv[it] = *((const NAVI_GLOBAL u32x4_t *) (u.w7 + boff[it] + ci0));
    };
    // the k1's weights, 32 input channels (CC1) at a time: [C][CC1] in 16-byte pieces
    constexpr int W1Q = C * CC1 / 8, ITW = (W1Q + BT - 1) / BT;
    u32x4_t w1r[ITW];
    auto load_w1 = [&](int ci0) {
#pragma unroll
        for (int it = 0; it < ITW; ++it) {
            const int e = static_cast<int>(threadIdx.x) + BT * it, col = e / (CC1 / 8), q = e - col * (CC1 / 8);
            if (ITW * BT == W1Q || e < W1Q) w1r[it] = *(const NAVI_GLOBAL u32x4_t *) (u.w1 + static_cast<size_t>(col) * C + ci0 + 8 * q);
        }
    };
    f32x16_t acc[NCT];
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
    bool bad = false;
    load(0);
    for (int ci0 = 0; ci0 < C; ci0 += CC7) {
        __syncthreads();
#pragma unroll
        for (int it = 0; it < ITA; ++it) {
            const int r = rr0 + RPI * it;
            if (r >= rows) continue;
            half4v h, o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bad |= !(fabsf(av[it][e]) < 65504.f);
                h[e] = static_cast<_Float16>(av[it][e]);
                o[e] = static_cast<_Float16>(av[it][e] - static_cast<float>(h[e]));
            }
            *reinterpret_cast<half4v *>(&ahi[r * LDA + c4]) = h;
            *reinterpret_cast<half4v *>(&alo[r * LDA + c4]) = o;
        }
#pragma unroll
        for (int it = 0; it < ITB; ++it)
            if (ITB * BT == NBI || static_cast<int>(threadIdx.x) + BT * it < NBI)
                *reinterpret_cast<u32x4_t *>(&bw[bl[it]]) = bv[it];
        __syncthreads();
        if (ci0 + CC7 < C) load(ci0 + CC7);
        else load_w1(0);                                    // the k1's first weight piece, during the last MFMAs
        if (!mma) continue;
#pragma unroll
        for (int j = 0; j < K; ++j) {
#pragma unroll
            for (int ks = 0; ks < CC7 / 16; ++ks) {
                const int ar = (wr + (l & 31) + j * u.dil) * LDA + 16 * ks + 8 * (l >> 5);
                const half8v h = *reinterpret_cast<const half8v *>(&ahi[ar]);
                const half8v o = *reinterpret_cast<const half8v *>(&alo[ar]);
#pragma unroll
                for (int c = 0; c < NCT; ++c) {
                    const half8v b = *reinterpret_cast<const half8v *>(&bw[(j * C + wc + 32 * c + (l & 31)) * LDA + 16 * ks + 8 * (l >> 5)]);
                    acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h, b, acc[c], 0, 0, 0);
                    acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(o, b, acc[c], 0, 0, 0);
                }
            }
        }
    }
    // ---- the k7's output through the k1's Snake into LDS as f16 hi + lo ----
    float b7c[NCT], zam[NCT], zbm[NCT];
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
        const int co = wc + 32 * c + (l & 31);
        b7c[c] = gld(u.b7 + co);
        zam[c] = gld(u.za_mid + co);
        zbm[c] = gld(u.zb_mid + co);
    }
    __syncthreads();                                        // every wave is done with the k7 staging
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if (!mma) break;
            const int row = wr + 8 * (r / 4) + 4 * (l >> 5) + (r & 3), co = wc + 32 * c + (l & 31);
            const float m = snake(acc[c][r] + b7c[c], zam[c], zbm[c]);
            if (t0 + row < u.T) bad |= !(fabsf(m) < 65504.f);
            const _Float16 h = static_cast<_Float16>(m);
            mhi[row * LDM + co] = h;
            mlo[row * LDM + co] = static_cast<_Float16>(m - static_cast<float>(h));
        }
    if (bad) gst(u.flag, 1u);
    // ---- k1: 32-channel weight pieces, 16-channel steps in channel order, hi then lo ----
    f32x16_t acc1[NCT];
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc1[c][r] = 0.f;
    for (int ci0 = 0; ci0 < C; ci0 += CC1) {
        if (ci0 > 0) __syncthreads();                       // the previous piece's readers are done
#pragma unroll
        for (int it = 0; it < ITW; ++it) {
            const int e = static_cast<int>(threadIdx.x) + BT * it, col = e / (CC1 / 8), q = e - col * (CC1 / 8);
            if (ITW * BT == W1Q || e < W1Q) *reinterpret_cast<u32x4_t *>(&w1s[col * LDW + 8 * q]) = w1r[it];
        }
        __syncthreads();                                    // the piece (and, first time, the tile) in LDS
        if (ci0 + CC1 < C) load_w1(ci0 + CC1);
        if (!mma) continue;
#pragma unroll
        for (int ks = 0; ks < CC1 / 16; ++ks) {
            const int ar = (wr + (l & 31)) * LDM + ci0 + 16 * ks + 8 * (l >> 5);
            const half8v h = *reinterpret_cast<const half8v *>(&mhi[ar]);
            const half8v o = *reinterpret_cast<const half8v *>(&mlo[ar]);
#pragma unroll
            for (int c = 0; c < NCT; ++c) {
                const half8v b = *reinterpret_cast<const half8v *>(&w1s[(wc + 32 * c + (l & 31)) * LDW + 16 * ks + 8 * (l >> 5)]);
                acc1[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h, b, acc1[c], 0, 0, 0);
                acc1[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(o, b, acc1[c], 0, 0, 0);
            }
        }
    }
    // ---- epilogue: every load first (column operands, residuals), then the stores ----
    if (!mma) {
        if (u.hnext) carry_rows(u.hist, u.x, C, u.T, H, C, u.hnext);
        return;
    }
    float b1c[NCT], zac[NCT], zbc[NCT], rs[NCT][16];
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
        const int co = wc + 32 * c + (l & 31);
        b1c[c] = gld(u.b1 + co);
        zac[c] = gld(u.za + co);
        zbc[c] = gld(u.zb + co);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + wr + 8 * (r / 4) + 4 * (l >> 5) + (r & 3);
            rs[c][r] = t < u.T ? gld(u.res + static_cast<size_t>(t) * C + co) : 0.f;
        }
    }
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + wr + 8 * (r / 4) + 4 * (l >> 5) + (r & 3), co = wc + 32 * c + (l & 31);
            if (t >= u.T) continue;
            const float v = (acc1[c][r] + b1c[c]) + rs[c][r];
            const size_t o = static_cast<size_t>(t) * C + co;
            if (u.y) gst(u.y + o, v);
            gst(u.z + o, snake(v, zac[c], zbc[c]));
        }
    if (u.hnext) carry_rows(u.hist, u.x, C, u.T, H, C, u.hnext);
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
    conv_store(a, epi, row * a.ldy + co, epi_col(a, epi, co), v, epi_has_res(epi) ? gld(a.res + row * a.ldy + co) : 0.f);
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
