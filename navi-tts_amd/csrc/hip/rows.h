// Row projections on the matrix cores, whole K in one block: Y = X W^T for up to a few hundred
// rows (the multi-stream decode's n streams, the prefill's prompt rows), with the RMSNorm of the
// input, SwiGLU and the residual add fused in. Shared by streams.hip and prefill.hip; the kernels
// sit in an unnamed namespace, so every including file gets its own.
#pragma once

#include "dev_common.h"

namespace navi_amd {
namespace rows {

// A block owns 16 output columns (SwiGLU: 16 gate and the matching 16 up columns; above 64 rows,
// several such groups) for up to 64 rows (more rows: more blocks along y); its NWV waves take a
// slice of K each, loading their A
// rows (f32, split into f16 hi + lo for two v_mfma_f32_16x16x32_f16 each) and W rows (f16)
// straight from global memory, all KS MFMA steps' loads in flight at once, no LDS staging. The
// waves' tiles are summed in LDS in wave order. With NORM the rows are the residual stream: A is multiplied by the RMSNorm weight as it
// is loaded, every lane sums the squares of its elements, and the row scale rsqrt(mean(x^2) + eps)
// (sums taken in a fixed order, the same in every block) multiplies the results. Epilogues:
// plain store, SiLU(gate) * up, or an add into the residual stream. No split-K partials and no
// finish kernels: at these sizes the launch count is what bounds a layer.
enum { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_RESID = 2, EPI_QKV = 3 };

// EPI_QKV: the q|k|v projection of a prompt with the per-head work of the attention's input in its
// epilogue: q and k heads RMSNorm'd (qn / kn) and rotated (rotate-half RoPE at position pos0 + m),
// q kept f32 in q [M][nq 128], k and v rounded to f16 into the cache rows kc / vc [pos][nkv 128].
// A block owns one 128-wide head of 16 rows (talker.hip:46-82's k_qk_norm_rope).
struct HeadOut {
    const float *qn, *kn, *invf;
    float *q;
    uint16_t *kc, *vc;
    int nq, nkv, pos0;
};

struct RowArgs {
    const float *a;                   // A [M][lda] f32
    const float *ln;                  // NORM: RMSNorm weight [K]
    const uint16_t *w0, *w1, *w2;     // W rows [0, n1) of w0, [n1, n2) of w1, [n2, ..) of w2, each [rows][K]
    float *y;                         // PLAIN / SWIGLU: [M][ldy] output; RESID: the residual stream, added to
    uint32_t *flag;                   // set when an activation is outside the f16 range
    int lda, M, K, n1, n2, F, ldy;    // F: SWIGLU gate rows [0, F), up rows [F, 2F) of the combined W
    float eps;
    const float *rs;                  // RESID: per-column scale of the added product (a layer scale), or null
    int ypk;                          // packed kernels: y's width for a SWIGLU / RESID output in the tile layout
    HeadOut ho;                       // EPI_QKV
    int ars = 1, aoff = 0;            // packed kernels: row m of the product reads row m * ars + aoff of A
};

// Tile layouts of the packed kernels (the prompt prefill): every operand load of a wave is one
// contiguous 1 KB instead of 16 rows x 64 B. Reads of L2-resident data run about twice as fast that
// way (16 rows x 64 B touch 16 cache lines per instruction, 1 KB touches 8).
// f32 activations [M][K] (K % 32 == 0): element (m, k) of 16-row tile m / 16 and 32-column step
// k / 32 sits where lane (m % 16) + 16 ((k / 8) % 4) of the MFMA A operand loads it, as two 1 KB
// halves (k % 8 < 4, then >= 4) of 64 lanes x 4 floats.
__host__ __device__ inline size_t pk_a(int m, int k, int K) {
    return ((static_cast<size_t>(m >> 4) * (K >> 5) + (k >> 5)) * 2 + ((k >> 2) & 1)) * 256 +
           static_cast<size_t>((m & 15) + 16 * ((k >> 3) & 3)) * 4 + (k & 3);
}
// f16 weights [N][K]: element (n, k) where lane (n % 16) + 16 ((k / 8) % 4) of the MFMA B operand
// loads it, 64 lanes x 8 halves per 16-row tile and 32-column step.
__host__ __device__ inline size_t pk_w(int n, int k, int K) {
    return (static_cast<size_t>(n >> 4) * (K >> 5) + (k >> 5)) * 512 + static_cast<size_t>((n & 15) + 16 * ((k >> 3) & 3)) * 8 +
           (k & 7);
}

namespace {

typedef _Float16 rhalf8 __attribute__((ext_vector_type(8)));

// NWV waves per block, each one batch of KS MFMA steps (32 k each): K = 32 KS NWV. Every load of
// a wave is issued before its first MFMA (the whole chain is one memory latency), and the kernels
// stay small (no unrolled K loop, so the decode's few kernels stay in the instruction cache).
// CG column groups: the block owns 16 CG output columns and every wave applies its A registers to
// all of them, so A (f32, the bulk of a block's reads once the rows pass a few dozen) is read
// N / (16 CG) times per launch instead of N / 16. A column's sums are the same at any CG.
// PK: A, W and a SWIGLU / RESID y in the tile layouts above (W one [N][K] matrix in w0, y of width
// a.ypk); the same products in the same order, so the same bits as the row-major kernel.
template <int MT, int EPI, bool NORM, int NWV, int KS, int CG = 1, bool PK = false>
__global__ void __launch_bounds__(NWV * WAVE) k_rows(RowArgs a) {
    constexpr int NT = EPI == EPI_SWIGLU ? 2 : 1, K = 32 * KS * NWV;
    static_assert(CG * MT <= NWV, "one finishing wave per output tile");
    static_assert(EPI != EPI_QKV || (MT == 1 && CG == 8 && NWV >= 8), "EPI_QKV: one 128-wide head of 16 rows per block");
    __shared__ f32x4_t red[NWV][NT][CG][MT][WAVE];
    __shared__ float hs[EPI == EPI_QKV ? 16 : 1][EPI == EPI_QKV ? 128 : 1];
    __shared__ float ssq[NWV][MT][WAVE];
    __shared__ float rscale[MT * 16];
    const int w = static_cast<int>(threadIdx.x) / WAVE, l = static_cast<int>(threadIdx.x) & (WAVE - 1);
    const int c = l & 15, kq = l >> 4, m0 = blockIdx.y * (MT * 16);
    const int nb0 = blockIdx.x * (16 * CG) + c;        // column of group 0; group g: nb0 + 16 g
    auto wrow = [&](int n) {
        return n < a.n1 ? a.w0 + static_cast<size_t>(n) * K
             : n < a.n2 ? a.w1 + static_cast<size_t>(n - a.n1) * K : a.w2 + static_cast<size_t>(n - a.n2) * K;
    };
    const int kbeg = w * (K / NWV) + 8 * kq;
    u32x4_t bv[NT][CG][KS];
    f32x4_t av[KS][MT][2], lv[KS][2];
    {
        const uint16_t *wr[NT][CG];
#pragma unroll
        for (int g = 0; g < CG; ++g) {
            wr[0][g] = wrow(nb0 + 16 * g);
            if constexpr (NT == 2) wr[NT - 1][g] = wrow(a.F + nb0 + 16 * g);
        }
#pragma unroll
        for (int st = 0; st < KS; ++st) {
            const int k = kbeg + 32 * st;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int g = 0; g < CG; ++g) {
                    if constexpr (PK) {
                        const int n = (t ? a.F : 0) + blockIdx.x * (16 * CG) + 16 * g;
                        bv[t][g][st] = *(const NAVI_GLOBAL u32x4_t *) (a.w0 + (static_cast<size_t>(n >> 4) * (K / 32) + w * KS + st) * 512 + l * 8);
                    } else {
                        bv[t][g][st] = *(const NAVI_GLOBAL u32x4_t *) (wr[t][g] + k);
                    }
                }
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int m = m0 + 16 * i + c;
                if (PK && m < a.M) {
                    // lanes of a 16-row tile read one contiguous 1 KB when ars == 1 and aoff == 0
                    const int r = m * a.ars + a.aoff;
                    const NAVI_GLOBAL f32x4_t *p = (const NAVI_GLOBAL f32x4_t *) (a.a + (static_cast<size_t>(r >> 4) * (K / 32) + w * KS + st) * 512 + ((r & 15) + 16 * kq) * 4);
                    av[st][i][0] = p[0];
                    av[st][i][1] = p[64];
                } else if (m < a.M) {
                    const NAVI_GLOBAL f32x4_t *p = (const NAVI_GLOBAL f32x4_t *) (a.a + static_cast<size_t>(m) * a.lda + k);
                    av[st][i][0] = p[0];
                    av[st][i][1] = p[1];
                } else {
                    av[st][i][0] = av[st][i][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                }
            }
            if constexpr (NORM) {
                const NAVI_GLOBAL f32x4_t *p = (const NAVI_GLOBAL f32x4_t *) (a.ln + k);
                lv[st][0] = p[0];
                lv[st][1] = p[1];
            }
        }
    }
    f32x4_t acc[NT][CG][MT];
    float ss[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        ss[i] = 0.f;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int g = 0; g < CG; ++g) acc[t][g][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    bool bad = false;
#pragma unroll
    for (int st = 0; st < KS; ++st) {
        rhalf8 b[NT][CG];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int g = 0; g < CG; ++g) __builtin_memcpy(&b[t][g], &bv[t][g][st], 16);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            rhalf8 hi, lo;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float v = av[st][i][j >> 2][j & 3];
                if constexpr (NORM) {
                    ss[i] = fmaf(v, v, ss[i]);
                    v *= lv[st][j >> 2][j & 3];
                }
                bad |= !(fabsf(v) < 65504.f);
                const _Float16 h = static_cast<_Float16>(v);
                hi[j] = h;
                lo[j] = static_cast<_Float16>(v - static_cast<float>(h));
            }
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int g = 0; g < CG; ++g) {
                    acc[t][g][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, b[t][g], acc[t][g][i], 0, 0, 0);
                    acc[t][g][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo, b[t][g], acc[t][g][i], 0, 0, 0);
                }
        }
    }
    if (bad) gst(a.flag, 1u);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int g = 0; g < CG; ++g) red[w][t][g][i][l] = acc[t][g][i];
        if constexpr (NORM) ssq[w][i][l] = ss[i];
    }
    __syncthreads();
    if constexpr (NORM) {
        // row r of the tile: lanes r % 16 + 16 q of every wave hold its sums of squares
        if (threadIdx.x < MT * 16) {
            const int i = threadIdx.x / 16, r = threadIdx.x % 16;
            float t = 0.f;
#pragma unroll
            for (int ww = 0; ww < NWV; ++ww)
#pragma unroll
                for (int q = 0; q < 4; ++q) t += ssq[ww][i][r + 16 * q];
            rscale[threadIdx.x] = rsqrtf(t / static_cast<float>(K) + a.eps);
        }
        __syncthreads();
    }
    // wave g MT + i finishes column group g of M-tile i: lane l holds column c of rows
    // 4 (l / 16) + r, r = 0..3
    if (w < CG * MT) {
        const int g = w / MT, i = w % MT, nb = nb0 + 16 * g;
        f32x4_t v[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            v[t] = red[0][t][g][i][l];
#pragma unroll
            for (int ww = 1; ww < NWV; ++ww) v[t] += red[ww][t][g][i][l];
        }
        // RESID: the four residual values are loaded before the first store (a load after a
        // store to the same buffer would wait for it: four memory round trips instead of one)
        float old[4] = {0.f, 0.f, 0.f, 0.f}, rsc = 1.f;
        if constexpr (EPI == EPI_RESID) {
            if (a.rs) rsc = a.rs[nb];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 16 * i + 4 * kq + r;
                if (m < a.M) old[r] = a.y[PK ? pk_a(m, nb, a.ypk) : static_cast<size_t>(m) * a.ldy + nb];
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int mr = 16 * i + 4 * kq + r, m = m0 + mr;
            if (m >= a.M) continue;
            const float sc = NORM ? rscale[mr] : 1.f;
            if constexpr (EPI == EPI_QKV) {
                hs[mr][16 * g + c] = v[0][r] * sc;
                continue;
            }
            float *dst = a.y + (PK && EPI != EPI_PLAIN ? pk_a(m, nb, a.ypk) : static_cast<size_t>(m) * a.ldy + nb);
            if constexpr (EPI == EPI_PLAIN) {
                *dst = v[0][r] * sc;
            } else if constexpr (EPI == EPI_SWIGLU) {
                const float g = v[0][r] * sc, u = v[NT - 1][r] * sc;
                *dst = g / (1.f + expf(-g)) * u;
            } else {
                *dst = a.rs ? v[0][r] * rsc + old[r] : old[r] + v[0][r];
            }
        }
    }
    if constexpr (EPI == EPI_QKV) {
        // one wave per (row, head): lane l holds dims l and l + 64 (the values 0 + x, so a -0 sum
        // is stored as +0), the same arithmetic as a separate norm/RoPE pass over the stored rows
        __syncthreads();
        const HeadOut &o = a.ho;
        const int hh = blockIdx.x, QD = o.nq * 128, KVD = o.nkv * 128;
        for (int r2 = 2 * w; r2 < 2 * w + 2 && w < 8; ++r2) {
            const int m = m0 + r2, pos = o.pos0 + m;
            if (m >= a.M) break;
            const float a0 = 0.f + hs[r2][l], a1 = 0.f + hs[r2][l + 64];
            if (hh >= o.nq + o.nkv) {
                uint16_t *vd = o.vc + static_cast<size_t>(pos) * KVD + (hh - o.nq - o.nkv) * 128;
                gst(vd + l, f2h(a0));
                gst(vd + l + 64, f2h(a1));
                continue;
            }
            float sn, cs;
            sincosf(static_cast<float>(pos) * gld(o.invf + l), &sn, &cs);
            const float *nw = hh < o.nq ? o.qn : o.kn;
            const float sc = rsqrtf(wave_sum(fmaf(a0, a0, a1 * a1)) / 128.f + a.eps);
            const float x0 = a0 * sc * gld(nw + l), x1 = a1 * sc * gld(nw + l + 64);
            const float y0 = x0 * cs - x1 * sn;
            const float y1 = x1 * cs + x0 * sn;
            if (hh < o.nq) {
                float *qd = o.q + static_cast<size_t>(m) * QD + hh * 128;
                gst(qd + l, y0);
                gst(qd + l + 64, y1);
            } else {
                uint16_t *kd = o.kc + static_cast<size_t>(pos) * KVD + (hh - o.nq) * 128;
                gst(kd + l, f2h(y0));
                gst(kd + l + 64, f2h(y1));
            }
        }
    }
}

template <int MT>
void launch_rows_mt(int epi, bool norm, const dim3 &grid, const RowArgs &ra, hipStream_t s) {
    // K = hidden (1024) for q|k|v, gate|up and the heads: 8 waves x 4 steps; the residual adds
    // (K = 2048 for o, 3072 for down) one 16-row tile per block: 16 waves x 4 or 6 steps
    if (epi == EPI_SWIGLU) hipLaunchKernelGGL((k_rows<MT, EPI_SWIGLU, true, 8, 4>), grid, dim3(8 * WAVE), 0, s, ra);
    else if (epi == EPI_RESID) {
        if constexpr (MT == 1) {
            if (ra.K == 2048) hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 4>), grid, dim3(16 * WAVE), 0, s, ra);
            else hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 6>), grid, dim3(16 * WAVE), 0, s, ra);
        }
    } else if (norm) hipLaunchKernelGGL((k_rows<MT, EPI_PLAIN, true, 8, 4>), grid, dim3(8 * WAVE), 0, s, ra);
    else hipLaunchKernelGGL((k_rows<MT, EPI_PLAIN, false, 8, 4>), grid, dim3(8 * WAVE), 0, s, ra);
}

template <int MT, int EPI, bool NORM, int NWV, int KS, int CG>
bool launch_wide(int M, int N, const RowArgs &ra, hipStream_t s) {
    if (N % (16 * CG) != 0) return false;
    const dim3 grid(N / (16 * CG), (M + 16 * MT - 1) / (16 * MT));
    hipLaunchKernelGGL((k_rows<MT, EPI, NORM, NWV, KS, CG>), grid, dim3(NWV * WAVE), 0, s, ra);
    return true;
}

// More than 64 rows (a prefill's prompt): blocks over several column groups. false: N does not
// split into the groups, the caller takes the one-group kernels.
bool launch_rows_wide(int epi, bool norm, int M, int N, const RowArgs &ra, hipStream_t s) {
    // gate|up: 48-row tiles up to 96 rows (two row tiles instead of three: 65 rows 1.70 -> 1.60 ms,
    // 96 rows 1.90 -> 1.74 ms per prefill), 32-row tiles above (130 rows: 2.40 against 2.46 ms)
    if (epi == EPI_SWIGLU)
        return M <= 96 ? launch_wide<3, EPI_SWIGLU, true, 8, 4, 2>(M, N, ra, s)
                       : launch_wide<2, EPI_SWIGLU, true, 8, 4, 2>(M, N, ra, s);
    if (epi == EPI_RESID)
        return ra.K == 2048 ? launch_wide<2, EPI_RESID, false, 16, 4, 2>(M, N, ra, s)
                            : launch_wide<1, EPI_RESID, false, 16, 6, 2>(M, N, ra, s);
    return norm ? launch_wide<2, EPI_PLAIN, true, 8, 4, 4>(M, N, ra, s)
                : launch_wide<2, EPI_PLAIN, false, 8, 4, 4>(M, N, ra, s);
}

// Y = A W^T over M rows (K: 1024 for PLAIN and SWIGLU, 2048 or 3072 for RESID; N a multiple of
// 16). SWIGLU: W = gate (w0, F rows) | up (w1, F rows), y [M][F]; RESID: y (the residual stream)
// += A W^T; norm (SWIGLU always): A is the residual stream, RMSNorm'd with ln and eps on the way in.
void launch_rows(int epi, bool norm, const float *A, int lda, int M, int K, const float *ln, float eps, const uint16_t *w0,
                 int n0, const uint16_t *w1, int n1, const uint16_t *w2, int n2, float *y, int ldy, uint32_t *flag,
                 hipStream_t s) {
    const int F = epi == EPI_SWIGLU ? n0 : 0, N = epi == EPI_SWIGLU ? n0 : n0 + n1 + n2;
    const RowArgs ra{A, ln, w0, w1, w2, y, flag, lda, M, K, n0, n0 + n1, F, ldy, eps};
    if (M > 64 && launch_rows_wide(epi, norm, M, N, ra, s)) return;
    const int mt = epi == EPI_RESID ? 1 : M <= 16 ? 1 : M <= 32 ? 2 : M <= 48 ? 3 : 4;
    const dim3 grid(N / 16, (M + 16 * mt - 1) / (16 * mt));
    switch (mt) {
    case 1: launch_rows_mt<1>(epi, norm, grid, ra, s); break;
    case 2: launch_rows_mt<2>(epi, norm, grid, ra, s); break;
    case 3: launch_rows_mt<3>(epi, norm, grid, ra, s); break;
    default: launch_rows_mt<4>(epi, norm, grid, ra, s); break;
    }
}

// dst (tile layout pk_w) = the row-major f16 matrix src [n][K]: one thread per 16-byte lane slot.
__global__ void __launch_bounds__(256) k_tile_w(const uint16_t *src, int n, int K, uint16_t *dst) {
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x, slots = static_cast<size_t>(n) * K / 8;
    if (i >= slots) return;
    const int ln = static_cast<int>(i & 63), steps = K / 32;
    const size_t tile = i / 64;
    const int row = static_cast<int>(tile / steps) * 16 + (ln & 15), k = static_cast<int>(tile % steps) * 32 + 8 * (ln >> 4);
    *reinterpret_cast<u32x4_t *>(dst + i * 8) = *reinterpret_cast<const u32x4_t *>(src + static_cast<size_t>(row) * K + k);
}

void tile_weights(const uint16_t *src, int n, int K, uint16_t *dst, hipStream_t s) {
    const size_t slots = static_cast<size_t>(n) * K / 8;
    hipLaunchKernelGGL(k_tile_w, dim3(static_cast<unsigned>((slots + 255) / 256)), dim3(256), 0, s, src, n, K, dst);
}

// x (tile layout pk_a of width H) = the rows src [T][H]: one thread per 4 floats. clear (optional):
// a word set to 0 by the first thread, for a sequence that starts with this launch (its flag).
__global__ void __launch_bounds__(256) k_tile_rows(const float *src, int T, int H, float *x, uint32_t *clear) {
    const int i = blockIdx.x * 256 + threadIdx.x, m = i / (H / 4), k = 4 * (i % (H / 4));
    if (clear && i == 0) *(NAVI_GLOBAL uint32_t *) clear = 0u;
    if (m >= T) return;
    *(NAVI_GLOBAL f32x4_t *) (x + pk_a(m, k, H)) = *(const NAVI_GLOBAL f32x4_t *) (src + static_cast<size_t>(m) * H + k);
}

void tile_rows(const float *src, int T, int H, float *x, hipStream_t s, uint32_t *clear = nullptr) {
    hipLaunchKernelGGL(k_tile_rows, dim3((T * (H / 4) + 255) / 256), dim3(256), 0, s, src, T, H, x, clear);
}

template <int MT, int EPI, bool NORM, int NWV, int KS, int CG>
void launch_pk(int M, int N, const RowArgs &ra, hipStream_t s) {
    const dim3 grid(N / (16 * CG), (M + 16 * MT - 1) / (16 * MT));
    hipLaunchKernelGGL((k_rows<MT, EPI, NORM, NWV, KS, CG, true>), grid, dim3(NWV * WAVE), 0, s, ra);
}

// The prompt prefill's projections on the tile layouts (talker shapes: K 1024 into q|k|v and gate|up,
// 2048 into o, 3072 into down). A: [M][K] tiled; W: one [N][K] tiled matrix (q|k|v and gate|up
// stacked); y: PLAIN row-major [M][ldy], SWIGLU ([M][F]) and RESID ([M][N]) tiled. Tile shapes from a
// sweep at 10 and 130 rows (weights streamed from HBM): above 64 rows 16-row tiles with 8 (q|k|v),
// 4 (gate|up, o) or 2 (down) column groups per block; up to 64 rows the one-group kernels. Every
// shape keeps the row-major kernels' split of K over the waves, so the outputs are theirs bit for
// bit (gate|up over 16 waves x 2 steps measured 0.7 us faster at 130 rows, with other bits).
// false: a shape these kernels do not take.
// EPI_QKV (above 64 rows, talker heads of 128 with ho): the q|k|v projection with the head norms,
// RoPE and the K/V store in its epilogue; y is not written.
bool launch_rows_pk(int epi, bool norm, const float *A, int M, int K, const float *ln, float eps, const uint16_t *w, int N,
                    float *y, int ldy, uint32_t *flag, hipStream_t s, const HeadOut &ho = {}, int ars = 1, int aoff = 0) {
    const int F = epi == EPI_SWIGLU ? N : 0;
    const RowArgs ra{A, ln, w, nullptr, nullptr, y, flag, 0, M, K, epi == EPI_SWIGLU ? 2 * N : N, epi == EPI_SWIGLU ? 2 * N : N,
                     F, ldy, eps, nullptr, N, ho, ars, aoff};
    if (M < 1 || N % 128 != 0 || (epi == EPI_SWIGLU && !norm) || ars < 1 || aoff < 0) return false;
    const bool wide = M > 64;
    if (epi == EPI_QKV) {
        if (!wide || !norm || K != 1024 || N != 128 * (ho.nq + 2 * ho.nkv)) return false;
        launch_pk<1, EPI_QKV, true, 8, 4, 8>(M, N, ra, s);
        return true;
    }
    // up to 64 rows: 16-row tiles up to 32 rows (faster than 32-row tiles there), 32-row tiles for
    // q|k|v and a whole-M tile for gate|up above (the sweep's best at 64 rows)
    if (epi == EPI_PLAIN && norm && K == 1024) {
        if (wide) launch_pk<1, EPI_PLAIN, true, 8, 4, 8>(M, N, ra, s);
        else if (M <= 32) launch_pk<1, EPI_PLAIN, true, 8, 4, 1>(M, N, ra, s);
        else launch_pk<2, EPI_PLAIN, true, 8, 4, 1>(M, N, ra, s);
        return true;
    }
    if (epi == EPI_SWIGLU && K == 1024) {
        if (wide) launch_pk<1, EPI_SWIGLU, true, 8, 4, 4>(M, N, ra, s);
        else if (M <= 32) launch_pk<1, EPI_SWIGLU, true, 8, 4, 1>(M, N, ra, s);
        else if (M <= 48) launch_pk<3, EPI_SWIGLU, true, 8, 4, 1>(M, N, ra, s);
        else launch_pk<4, EPI_SWIGLU, true, 8, 4, 1>(M, N, ra, s);
        return true;
    }
    if (epi == EPI_RESID && K == 2048) {
        if (wide && M <= 96) launch_pk<1, EPI_RESID, false, 16, 4, 2>(M, N, ra, s);   // more blocks where they are few
        else if (wide) launch_pk<1, EPI_RESID, false, 16, 4, 4>(M, N, ra, s);
        else launch_pk<1, EPI_RESID, false, 16, 4, 1>(M, N, ra, s);
        return true;
    }
    if (epi == EPI_RESID && K == 3072) {
        if (wide) launch_pk<1, EPI_RESID, false, 16, 6, 2>(M, N, ra, s);
        else launch_pk<1, EPI_RESID, false, 16, 6, 1>(M, N, ra, s);
        return true;
    }
    return false;
}

// The codec decoder's transformer layers (vocoder.hip): q|k|v and gate|up over K = 512 with the
// RMSNorm fused (SwiGLU on gate|up), o and down over K = 1024 adding into the residual stream with
// the per-column layer scale rs. One split of K over the waves per shape, whatever the row count
// (MT and the column groups do not change a column's sums), so the output of a row does not
// depend on how many rows a chunk has. false: a shape these kernels do not take.
bool launch_rows_xf(int epi, bool norm, const float *A, int lda, int M, int K, const float *ln, float eps, const uint16_t *w0,
                    int n0, const uint16_t *w1, int n1, float *y, int ldy, const float *rs, uint32_t *flag, hipStream_t s) {
    const int F = epi == EPI_SWIGLU ? n0 : 0, N = epi == EPI_SWIGLU ? n0 : n0 + n1;
    RowArgs ra{A, ln, w0, w1, nullptr, y, flag, lda, M, K, n0, n0 + n1, F, ldy, eps, rs};
    if (M < 1 || N % 16 != 0) return false;
    const int mt = M <= 16 ? 1 : M <= 32 ? 2 : M <= 48 ? 3 : 4;
    const dim3 g1(N / 16, (M + 16 * mt - 1) / (16 * mt));
    if (K == 512 && norm && (epi == EPI_PLAIN || epi == EPI_SWIGLU)) {
        if (M > 64) {
            if (epi == EPI_PLAIN && N % 64 == 0) return launch_wide<2, EPI_PLAIN, true, 8, 2, 4>(M, N, ra, s);
            if (epi == EPI_SWIGLU && N % 32 == 0) return launch_wide<2, EPI_SWIGLU, true, 8, 2, 2>(M, N, ra, s);
        }
#define NAVI_XF(MT_)                                                                                      \
        if (mt == MT_) {                                                                                  \
            if (epi == EPI_PLAIN) hipLaunchKernelGGL((k_rows<MT_, EPI_PLAIN, true, 8, 2>), g1, dim3(8 * WAVE), 0, s, ra); \
            else hipLaunchKernelGGL((k_rows<MT_, EPI_SWIGLU, true, 8, 2>), g1, dim3(8 * WAVE), 0, s, ra); \
            return true;                                                                                  \
        }
        NAVI_XF(1) NAVI_XF(2) NAVI_XF(3) NAVI_XF(4)
#undef NAVI_XF
    }
    if (K == 1024 && !norm && epi == EPI_RESID) {
        if (M > 64 && N % 32 == 0) return launch_wide<1, EPI_RESID, false, 16, 2, 2>(M, N, ra, s);
        hipLaunchKernelGGL((k_rows<1, EPI_RESID, false, 16, 2>), dim3(N / 16, (M + 15) / 16), dim3(16 * WAVE), 0, s, ra);
        return true;
    }
    return false;
}

} // namespace

} // namespace rows
} // namespace navi_amd
