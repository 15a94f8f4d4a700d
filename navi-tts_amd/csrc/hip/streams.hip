// Multi-stream batched decode on gfx950 (the C ABI's navi_streams_*): n independent requests
// ("streams"), each with its own KV cache, repetition set and seeds, advanced by one frame per
// call, with the talker and the code predictor run as GEMMs over the streams on the matrix cores.
//
// The reference has no batched decode. Each stream's frame follows the batch-1 frame row by row
// (k_frame, model/qwen3tts/frame.hip:517-579, and the host side of Frame, frame.hip:653-810):
// same seeds, same sampling rules, same step assembly, so stream i computes what navi_frame_run
// computes for it alone, up to the summation order of the projections. MI355X design:
//
//  * Projections: the whole-K MFMA row kernels of rows.h (activations as f16 hi + lo pairs, f16
//    weights) with M = n streams (code-predictor positions 0 and 1: 2n rows), the RMSNorm, SwiGLU
//    and residual add fused in, on the MFMA tile layouts (rows.h pk_a / pk_w: a tiled copy of the
//    weights made at create; the residual stream, attention output and MLP hidden stored tiled), so
//    every operand load of a wave is one contiguous 1 KB. Every weight byte streams from HBM once
//    per step for all streams (twice for the residual projections above 16 rows), so the weights
//    cost ~3.3 GB per step whatever n. The step (582 launches) is captured once as a HIP graph and
//    replayed.
//  * Talker attention: split-KV decode attention, one block per (stream, kv head, key range), with
//    the q/k head norms, RoPE and the step's f16 K/V store folded in (the range holding the new key
//    stores it); the two q heads of a GQA group share the K/V loads (16 lanes per key for the
//    scores, the same keys' V rows in flight); a combine kernel merges the ranges' (max, sum,
//    vector).
//  * Code-predictor attention: one block per (stream, kv head) fuses the q/k head norms, RoPE, the
//    f16 K/V store into the stream's cp cache and the attention over its <= 16 positions.
//  * Sampling: block_sample (sampler.h, the frame kernel's sampler) with one block per stream.
#include "dev_common.h"
#include "host_util.h"
#include "linear.h"
#include "rows.h"
#include "sampler.h"

#include <algorithm>
#include <cstring>
#include <cmath>
#include <string>
#include <vector>

namespace navi_amd {
namespace ms {

using namespace rows;

constexpr int BT = 256, NW = BT / WAVE;
constexpr int HD = 128, NCB = 16, CPH = NCB - 1;
constexpr int MAX_TL = 32, MAX_CL = 8;
constexpr int KPS = 256;               // keys per attention split (one per thread)
constexpr float ATT_SCALE = 0.08838834764831845f;   // 1/sqrt(128)

// Per-stream state the kernels read: position, frame index, seeds, cache pointers.
struct StreamMeta {
    int n_past, frame_index;
    uint64_t talker_seed, cp_seed;
};

// ---- talker: split-KV decode attention ----------------------------------------------------

// Block (m, g, s): keys [s * KPS, min(n, (s + 1) * KPS)) of stream m, n = n_past + 1, for the two
// q heads of kv group g, from the raw q|k|v row of the stream (part, the projection's output).
// Waves 0 and 1 take q heads 2g and 2g + 1: per-head RMSNorm and RoPE at the stream's position
// (norm_rope_store, frame.hip:311-346). The block whose range holds the step's own key (n_past)
// also normalises and ropes its k (wave 2), rounds k and v (wave 3) to f16, stores them into the
// stream's cache at n_past and uses those values for that key; every other key comes from the
// cache. Writes per head (max, sum of e^(score - max), unnormalised vector) to
// out[m][g][s][h] = {m, l, o[HD]}.
__global__ void __launch_bounds__(BT, 4) k_st_attn(const float *part, const StreamMeta *meta, uint16_t *const *kcache,
                                                uint16_t *const *vcache, int nq, int nkv, int splits, const float *qn,
                                                const float *kn, float eps, const float *invf, float *partials) {
    __shared__ float qs[2][HD], nkv_[2][HD], sc[2][KPS], red[2][NW], opart[NW][4][2][HD];
    const int m = blockIdx.x, g = blockIdx.y, s = blockIdx.z;
    const int pos = meta[m].n_past, n = pos + 1, j0 = s * KPS, j1 = min(n, j0 + KPS), cnt = max(0, j1 - j0);
    const bool own = pos >= j0 && pos < j0 + KPS;       // this range holds the step's own key
    const int QD = nq * HD, KVD = nkv * HD, W = QD + 2 * KVD;
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    float *out = partials + ((static_cast<size_t>(m) * nkv + g) * splits + s) * 2 * (HD + 2);
    const uint16_t *kb = kcache[m] + g * HD, *vb = vcache[m] + g * HD;
    u32x4_t vr[KPS / NW / 4];
    // Scores, 16 lanes per key: wave w takes keys 64w .. 64w + 63 of the range, four per load
    // instruction (lane 16r + c reads 16-byte chunk c of key 4i + r, so each instruction reads
    // four whole 256-byte rows), summed by DPP within the 16-lane row; lane 16r keeps the two
    // heads' scores in sc.
    {
        const int c = l & 15, r = l >> 4;
        constexpr int KI = KPS / NW / 4;
        u32x4_t kr[KI];
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int jl = wv * (KPS / NW) + 4 * i + r;
            kr[i] = jl < cnt && j0 + jl != pos ? *(const NAVI_GLOBAL u32x4_t *) (kb + static_cast<size_t>(j0 + jl) * KVD + c * 8)
                                               : u32x4_t{0u, 0u, 0u, 0u};
        }
        // while those loads are in flight: q heads 2g, 2g + 1 and (own range) the step's k and v,
        // lane l holding dims l and l + 64
        if (wv < 2 || own) {
            const float *row = part + static_cast<size_t>(m) * W;
            const float *hp = wv < 2 ? row + (2 * g + wv) * HD : row + QD + (wv - 2) * KVD + g * HD;
            const float a0 = gld(hp + l), a1 = gld(hp + l + HD / 2);
            if (wv < 3) {
                float sn, cs;
                sincosf(static_cast<float>(pos) * gld(invf + l), &sn, &cs);
                const float *nw = wv < 2 ? qn : kn;
                const float scl = rsqrtf(wave_sum(fmaf(a0, a0, a1 * a1)) / static_cast<float>(HD) + eps);
                const float x0 = a0 * scl * gld(nw + l), x1 = a1 * scl * gld(nw + l + HD / 2);
                const float y0 = x0 * cs - x1 * sn, y1 = x0 * sn + x1 * cs;
                if (wv < 2) {
                    qs[wv][l] = y0;
                    qs[wv][l + HD / 2] = y1;
                } else {
                    const uint16_t h0 = f2h(y0), h1 = f2h(y1);
                    uint16_t *kd = kcache[m] + static_cast<size_t>(pos) * KVD + g * HD;
                    gst(kd + l, h0);
                    gst(kd + l + HD / 2, h1);
                    nkv_[0][l] = h2f(h0);
                    nkv_[0][l + HD / 2] = h2f(h1);
                }
            } else {
                const uint16_t h0 = f2h(a0), h1 = f2h(a1);
                uint16_t *vd = vcache[m] + static_cast<size_t>(pos) * KVD + g * HD;
                gst(vd + l, h0);
                gst(vd + l + HD / 2, h1);
                nkv_[1][l] = h2f(h0);
                nkv_[1][l + HD / 2] = h2f(h1);
            }
        }
        __syncthreads();
        float q0[8], q1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            q0[e] = qs[0][c * 8 + e];
            q1[e] = qs[1][c * 8 + e];
        }
        if (own) {                         // the step's own key: its chunk from LDS
#pragma unroll
            for (int i = 0; i < KI; ++i) {
                const int jl = wv * (KPS / NW) + 4 * i + r;
                if (j0 + jl == pos) {
                    half8_t hk;
#pragma unroll
                    for (int e = 0; e < 8; ++e) hk[e] = static_cast<_Float16>(nkv_[0][c * 8 + e]);
                    __builtin_memcpy(&kr[i], &hk, 16);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int jl = wv * (KPS / NW) + 4 * i + r;
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
                sc[0][jl] = a0 * ATT_SCALE;
                sc[1][jl] = a1 * ATT_SCALE;
            }
        }
        // the same keys' V chunks go out after the scores and fly during the softmax, so K and V
        // are never in registers together (about 110 VGPRs instead of 168: the whole grid of a
        // 32-stream step resident at once, four blocks per CU instead of three; the sums are
        // unchanged); the step's own value from LDS
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int jl = wv * (KPS / NW) + 4 * i + r;
            if (own && j0 + jl == pos) {
                half8_t hv;
#pragma unroll
                for (int e = 0; e < 8; ++e) hv[e] = static_cast<_Float16>(nkv_[1][c * 8 + e]);
                __builtin_memcpy(&vr[i], &hv, 16);
            } else {
                vr[i] = jl < cnt && j0 + jl != pos ? *(const NAVI_GLOBAL u32x4_t *) (vb + static_cast<size_t>(j0 + jl) * KVD + c * 8)
                                                   : u32x4_t{0u, 0u, 0u, 0u};
            }
        }
    }
    __syncthreads();
    const bool mine = static_cast<int>(threadIdx.x) < cnt;
    const float d0 = mine ? sc[0][threadIdx.x] : -INFINITY, d1 = mine ? sc[1][threadIdx.x] : -INFINITY;
    float mx0 = wave_max(d0), mx1 = wave_max(d1);
    if (l == 0) { red[0][wv] = mx0; red[1][wv] = mx1; }
    __syncthreads();
    mx0 = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    mx1 = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    const float e0 = static_cast<int>(threadIdx.x) < cnt ? expf(d0 - mx0) : 0.f;
    const float e1 = static_cast<int>(threadIdx.x) < cnt ? expf(d1 - mx1) : 0.f;
    sc[0][threadIdx.x] = e0;
    sc[1][threadIdx.x] = e1;
    const float s0 = wave_sum(e0), s1 = wave_sum(e1);
    __syncthreads();                                      // red reads done, probabilities published
    if (l == 0) { red[0][wv] = s0; red[1][wv] = s1; }
    // V: wave w sums keys w * 64 .. w * 64 + 63 of the range; lane 16r + c holds 16-byte chunk c
    // (dims 8c .. 8c + 7) of keys 4i + r, i = 0..15 (loaded with the K chunks above), for both
    // heads; the 4 x 4 partials per dim are summed in LDS below.
    {
        constexpr int KI = KPS / NW / 4;
        const int c = l & 15, r = l >> 4, jw = wv * (KPS / NW);
        float o0[8], o1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o0[e] = o1[e] = 0.f;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int jl = jw + 4 * i + r;
            const float p0 = sc[0][jl], p1 = sc[1][jl];      // 0 past cnt
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
    float *o = out + hh * (HD + 2);
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc += opart[w][r][hh][d];
    gst(o + 2 + d, acc);
    if (d == 0) {
        gst(o, hh ? mx1 : mx0);
        gst(o + 1, red[hh][0] + red[hh][1] + red[hh][2] + red[hh][3]);
    }
}

// att[m][(2g + h) * HD + d] = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M) over the key ranges
// (att in the tile layout of width nq * HD).
__global__ void __launch_bounds__(BT) k_st_attn_combine(const float *part, const StreamMeta *meta, int nq, int nkv, int splits,
                                                        float *att) {
    const int m = blockIdx.x, g = blockIdx.y, hh = threadIdx.x >> 7, d = threadIdx.x & (HD - 1);
    const int used = (meta[m].n_past + 1 + KPS - 1) / KPS;
    const float *p = part + (static_cast<size_t>(m) * nkv + g) * splits * 2 * (HD + 2) + hh * (HD + 2);
    // the ranges' (max, sum, value) loads in batches of CB, every load of a batch in flight at
    // once; the first batch (contexts up to CB * KPS keys) stays in registers for both passes
    constexpr int CB = 8;
    float mv[CB], lv[CB], ov[CB];
#pragma unroll
    for (int s = 0; s < CB; ++s) {
        const float *ps = p + s * 2 * (HD + 2);
        mv[s] = s < used ? gld(ps) : -INFINITY;
        lv[s] = s < used ? gld(ps + 1) : 0.f;
        ov[s] = s < used ? gld(ps + 2 + d) : 0.f;
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < CB; ++s)
        if (s < used) M = fmaxf(M, mv[s]);
    for (int s0 = CB; s0 < used; s0 += CB) {
        float mb[CB];
#pragma unroll
        for (int s = 0; s < CB; ++s) mb[s] = s0 + s < used ? gld(p + (s0 + s) * 2 * (HD + 2)) : -INFINITY;
#pragma unroll
        for (int s = 0; s < CB; ++s)
            if (s0 + s < used) M = fmaxf(M, mb[s]);
    }
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int s = 0; s < CB; ++s)
        if (s < used) {
            const float w = expf(mv[s] - M);
            den = fmaf(lv[s], w, den);
            num = fmaf(ov[s], w, num);
        }
    for (int s0 = CB; s0 < used; s0 += CB) {
        float mb[CB], lb[CB], ob[CB];
#pragma unroll
        for (int s = 0; s < CB; ++s) {
            const float *ps = p + (s0 + s) * 2 * (HD + 2);
            mb[s] = s0 + s < used ? gld(ps) : -INFINITY;
            lb[s] = s0 + s < used ? gld(ps + 1) : 0.f;
            ob[s] = s0 + s < used ? gld(ps + 2 + d) : 0.f;
        }
#pragma unroll
        for (int s = 0; s < CB; ++s)
            if (s0 + s < used) {
                const float w = expf(mb[s] - M);
                den = fmaf(lb[s], w, den);
                num = fmaf(ob[s], w, num);
            }
    }
    gst(att + pk_a(m, (g * 2 + hh) * HD + d, nq * HD), num / den);
}

// ---- code predictor: norms + RoPE + K/V store + attention, per (stream, kv head) -----------

// Rows m * T + t (t < T <= 2) at cp positions p0 + t of stream m, per (stream, kv group g). Wave
// w < 2 T takes row t = w / 2 and q head 2g + (w & 1) on its own, with no block barrier: it loads
// its q row, the k and v rows of the launch's T rows and the cached keys and values of positions
// 0..p0 - 1 straight into the layouts its loops use (every load in flight at once), normalises and
// ropes q and the new keys per head, rounds the new keys and values to f16 (the head-2g wave of
// row t stores row t's into cpk/cpv [stream][layer][pos][kvd]), moves them through its own LDS
// slice into the score and value layouts, and attends row t over positions 0..p0 + t with the
// f16-rounded keys (the frame kernel's cp attention reads the same f16 values). Scores: lanes
// 4j..4j+3 take key j, lane 4j + s dims 32s..32s+31 in one FMA chain, summed by two DPP steps.
// Value sum: lane l owns dims 2l, 2l+1 over all NCB rows (rows past the keys are zero with
// weight 0), even and odd keys in two chains.
__global__ void __launch_bounds__(BT) k_st_cp_attn(const float *part, int T, int p0, int nq, int nkv, const float *qn,
                                                   const float *kn, float eps, const float *invf, int layer, int n_layer,
                                                   uint16_t *cpk, uint16_t *cpv, float *att) {
    __shared__ __align__(16) float lq[NW][HD], lk[NW][2][HD], lv[NW][2][HD];
    const int m = blockIdx.x, g = blockIdx.y, w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (w >= 2 * T) return;
    const int t = w >> 1, hh = w & 1, n = p0 + t + 1, j = l >> 2, sq = l & 3;
    const int QD = nq * HD, KVD = nkv * HD, W = QD + 2 * KVD;
    const size_t base = (static_cast<size_t>(m) * n_layer + layer) * NCB * KVD + g * HD;
    // every load first: q, the T new k / v rows (lane l: dims l, l + 64), the cached keys (lane
    // 4j + s: 32 dims of key j) and values (lane l: dims 2l, 2l+1 of every row), weights, RoPE.
    // The q|k|v values are taken as 0 + x (a -0 becomes +0), the value a sum over one partial
    // gives, so the stored keys and values keep the bits they had when the rows were summed here.
    const float *qr = part + static_cast<size_t>(m * T + t) * W + (g * 2 + hh) * HD;
    const float qa = 0.f + gld(qr + l), qb = 0.f + gld(qr + l + HD / 2);
    float ka[2] = {}, kb[2] = {}, va[2] = {}, vb[2] = {};
#pragma unroll
    for (int u = 0; u < 2; ++u)
        if (u < T) {
            const float *r = part + static_cast<size_t>(m * T + u) * W + QD + g * HD;
            ka[u] = 0.f + gld(r + l);
            kb[u] = 0.f + gld(r + l + HD / 2);
            va[u] = 0.f + gld(r + KVD + l);
            vb[u] = 0.f + gld(r + KVD + l + HD / 2);
        }
    u32x4_t kc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        kc[c] = j < p0 ? *(const NAVI_GLOBAL u32x4_t *) (cpk + base + static_cast<size_t>(j) * KVD + 32 * sq + 8 * c)
                       : u32x4_t{0u, 0u, 0u, 0u};
    uint32_t vcw[NCB];
#pragma unroll
    for (int r = 0; r < NCB; ++r)
        vcw[r] = r < p0 ? *(const NAVI_GLOBAL uint32_t *) (cpv + base + static_cast<size_t>(r) * KVD + 2 * l) : 0u;
    const float qn0 = gld(qn + l), qn1 = gld(qn + l + HD / 2), kn0 = gld(kn + l), kn1 = gld(kn + l + HD / 2);
    const float inv_f = gld(invf + l);
    // q of row t, then the new keys and values of rows 0..T-1, into this wave's LDS slice
    {
        float sn, cs;
        sincosf(static_cast<float>(p0 + t) * inv_f, &sn, &cs);
        const float scl = rsqrtf(wave_sum(fmaf(qa, qa, qb * qb)) / static_cast<float>(HD) + eps);
        const float x0 = qa * scl * qn0, x1 = qb * scl * qn1;
        lq[w][l] = x0 * cs - x1 * sn;
        lq[w][l + HD / 2] = x0 * sn + x1 * cs;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
        if (u < T) {
            float sn, cs;
            sincosf(static_cast<float>(p0 + u) * inv_f, &sn, &cs);
            const float scl = rsqrtf(wave_sum(fmaf(ka[u], ka[u], kb[u] * kb[u])) / static_cast<float>(HD) + eps);
            const float x0 = ka[u] * scl * kn0, x1 = kb[u] * scl * kn1;
            const uint16_t k0 = f2h(x0 * cs - x1 * sn), k1 = f2h(x0 * sn + x1 * cs), v0 = f2h(va[u]), v1 = f2h(vb[u]);
            if (hh == 0 && u == t) {
                const size_t o = base + static_cast<size_t>(p0 + u) * KVD;
                gst(cpk + o + l, k0);
                gst(cpk + o + l + HD / 2, k1);
                gst(cpv + o + l, v0);
                gst(cpv + o + l + HD / 2, v1);
            }
            lk[w][u][l] = h2f(k0);
            lk[w][u][l + HD / 2] = h2f(k1);
            lv[w][u][l] = h2f(v0);
            lv[w][u][l + HD / 2] = h2f(v1);
        }
    // scores (this wave's LDS writes above are visible to its own later reads)
    float acc = 0.f;
    {
        const f32x4_t *qv = reinterpret_cast<const f32x4_t *>(&lq[w][sq * 32]);
        const int u = j - p0;
        const f32x4_t *kn4 = reinterpret_cast<const f32x4_t *>(&lk[w][u >= 0 && u < T ? u : 0][sq * 32]);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            f32x4_t kk;
            if (j < p0) {
                const uint32_t wd0 = kc[c >> 1][2 * (c & 1)], wd1 = kc[c >> 1][2 * (c & 1) + 1];
                kk = f32x4_t{h2f(static_cast<uint16_t>(wd0)), h2f(static_cast<uint16_t>(wd0 >> 16)),
                             h2f(static_cast<uint16_t>(wd1)), h2f(static_cast<uint16_t>(wd1 >> 16))};
            } else if (u < T) {
                kk = kn4[c];
            } else {
                kk = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
            const f32x4_t qq = qv[c];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = fmaf(kk[e], qq[e], acc);
        }
    }
    acc += dpp_mov<0xB1>(acc);       // quad_perm [1,0,3,2]
    acc += dpp_mov<0x4E>(acc);       // quad_perm [2,3,0,1]: the 4 lanes of key j hold its dot
    const float sl = j < n ? acc * ATT_SCALE : -INFINITY;
    const float mx = wave_max(sl);
    const float e = j < n ? expf(sl - mx) : 0.f;
    const float inv = 1.f / wave_sum(sq == 0 ? e : 0.f);
    float o0 = 0.f, o1 = 0.f, q0 = 0.f, q1 = 0.f;
    auto vrow = [&](int r, float &a, float &b) {
        if (r < p0) {
            a = h2f(static_cast<uint16_t>(vcw[r]));
            b = h2f(static_cast<uint16_t>(vcw[r] >> 16));
        } else if (r - p0 < T) {
            a = lv[w][r - p0][2 * l];
            b = lv[w][r - p0][2 * l + 1];
        } else {
            a = 0.f;
            b = 0.f;
        }
    };
#pragma unroll
    for (int r = 0; r < NCB; r += 2) {
        const float pa = lane_value(e, 4 * r), pb = lane_value(e, 4 * r + 4);
        float a0, a1, b0, b1;
        vrow(r, a0, a1);
        vrow(r + 1, b0, b1);
        o0 = fmaf(pa, a0, o0);
        o1 = fmaf(pa, a1, o1);
        q0 = fmaf(pb, b0, q0);
        q1 = fmaf(pb, b1, q1);
    }
    float *dst = att + pk_a(m * T + t, (g * 2 + hh) * HD + 2 * l, QD);   // dims 2l, 2l + 1: adjacent in the tile layout
    gst(dst, (o0 + q0) * inv);
    gst(dst + 1, (o1 + q1) * inv);
}

// ---- sampling, one block per stream --------------------------------------------------------

struct SampleArgs {
    float temperature, rep_penalty, cp_temperature;
    int top_k, cp_top_k, min_frames, eos_id, suppress_from;
};

// Talker codebook 0 of stream m (tl_modified_logit + tl_sample, frame.hip:413-454): control range
// suppressed except EOS, EOS suppressed before min_frames, repetition penalty over the stream's
// set; then the cp input rows of the stream: x[2m] = post-norm hidden, x[2m + 1] = codec_emb[cb0]
// (x in the tile layout of width H).
__global__ void __launch_bounds__(BT) k_st_talker_sample(const float *logits, int V, const StreamMeta *meta, uint8_t *seen,
                                                         SampleArgs sa, const float *hidden, const uint16_t *codec_emb, int H,
                                                         float *cp_x, int32_t *codes) {
    constexpr int VT = 3072;
    __shared__ float lg[VT];
    __shared__ __align__(16) unsigned hist[SAMPLE_LDS_WORDS];
    __shared__ float sred[2 * NW];
    __shared__ int sidx[NW], sel;
    const int m = blockIdx.x;
    const StreamMeta me = meta[m];
    const float *lp = logits + static_cast<size_t>(m) * V;
    uint8_t *sn = seen + static_cast<size_t>(m) * V;
    for (int i = threadIdx.x; i < VT; i += BT) {
        float v = gld(lp + i);
        if (i >= sa.suppress_from && i != sa.eos_id) v = -INFINITY;
        else if (i == sa.eos_id && me.frame_index < sa.min_frames) v = -INFINITY;
        else if (sa.rep_penalty > 0.f && gld(sn + i)) v = v > 0.f ? v / sa.rep_penalty : v * sa.rep_penalty;
        lg[i] = v;
    }
    __syncthreads();
    const int cb0 = block_sample<VT, BT>(sa.temperature, sa.top_k, me.talker_seed, SampleLds{lg, hist, sred, sidx, &sel});
    if (threadIdx.x == 0) {
        gst(codes + static_cast<size_t>(m) * NCB, cb0);
        if (cb0 != sa.eos_id) gst(sn + cb0, static_cast<uint8_t>(1u));
    }
    const float *hr = hidden + static_cast<size_t>(m) * H;
    const uint16_t *er = codec_emb + static_cast<size_t>(cb0) * H;
    for (int i = threadIdx.x; i < H; i += BT) {
        gst(cp_x + pk_a(2 * m, i, H), gld(hr + i));
        gst(cp_x + pk_a(2 * m + 1, i, H), h2f(gld(er + i)));
    }
}

// Code pos of stream m from lm_head[pos - 1]'s logits (cp_sample, frame.hip:483-500: no
// suppression, penalty or EOS gate; seed cp_seed + pos * 0xD1B54A32D192ED03); then, if next_emb,
// the next cp input row x[m] = next_emb[code] (x in the tile layout of width H).
__global__ void __launch_bounds__(BT) k_st_cp_sample(const float *logits, const StreamMeta *meta, SampleArgs sa, int pos,
                                                     const uint16_t *next_emb, int H, float *x, int32_t *codes) {
    constexpr int VC = 2048;
    __shared__ float lg[VC];
    __shared__ __align__(16) unsigned hist[SAMPLE_LDS_WORDS];
    __shared__ float sred[2 * NW];
    __shared__ int sidx[NW], sel;
    const int m = blockIdx.x;
    const float *lp = logits + static_cast<size_t>(m) * VC;
    for (int i = threadIdx.x; i < VC; i += BT) lg[i] = gld(lp + i);
    __syncthreads();
    const uint64_t seed = meta[m].cp_seed + static_cast<uint64_t>(pos) * 0xD1B54A32D192ED03ull;
    const int code = block_sample<VC, BT>(sa.cp_temperature, sa.cp_top_k, seed, SampleLds{lg, hist, sred, sidx, &sel});
    if (threadIdx.x == 0) gst(codes + static_cast<size_t>(m) * NCB + pos, code);
    if (next_emb) {
        const uint16_t *er = next_emb + static_cast<size_t>(code) * H;
        for (int i = threadIdx.x; i < H; i += BT) gst(x + pk_a(m, i, H), h2f(gld(er + i)));
    }
}

// xn[m] = RMSNorm(x[m]) * w for the residual rows x (tile layout of width H) into xn (row stride
// H): the talker's final norm (k_rmsnorm, kernels.h:342-350); H == 4 * BT.
__global__ void __launch_bounds__(BT) k_st_final_norm(const float *x, const float *w, float eps, float *xn, int H) {
    __shared__ float red[NW];
    const int m = blockIdx.x, i = threadIdx.x * 4;
    const f32x4_t v = ld4(x + pk_a(m, i, H)), wv = ld4(w + i);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) ss = fmaf(v[j], v[j], ss);
    ss = wave_sum(ss);
    if ((threadIdx.x & (WAVE - 1)) == 0) red[threadIdx.x / WAVE] = ss;
    __syncthreads();
    const float scale = rsqrtf((red[0] + red[1] + red[2] + red[3]) / static_cast<float>(H) + eps);
    f32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = v[j] * scale * wv[j];
    st4(xn + static_cast<size_t>(m) * H + i, o);
}

struct EmbTable {
    const uint16_t *cp_emb[CPH];
};

// step_out[m] = codec_emb[c0] + sum_cb cp_emb[cb][c_{cb+1}] + trailing[m], f32 adds in that order
// (assemble_step, frame.hip:504-513).
__global__ void __launch_bounds__(BT) k_st_assemble(const int32_t *codes, const uint16_t *codec_emb, EmbTable et,
                                                    const float *trailing, int H, float *step_out) {
    const int m = blockIdx.x;
    const int32_t *c = codes + static_cast<size_t>(m) * NCB;
    int cs[NCB];
#pragma unroll
    for (int k = 0; k < NCB; ++k) cs[k] = gld(c + k);
    for (int i = threadIdx.x; i < H; i += BT) {
        float v = h2f(gld(codec_emb + static_cast<size_t>(cs[0]) * H + i));
#pragma unroll
        for (int cb = 0; cb < CPH; ++cb) v += h2f(gld(et.cp_emb[cb] + static_cast<size_t>(cs[cb + 1]) * H + i));
        gst(step_out + static_cast<size_t>(m) * H + i, v + gld(trailing + static_cast<size_t>(m) * H + i));
    }
}

struct LayerW {
    const float *ln1, *ln2, *qn, *kn;
    const uint16_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    uint16_t *qkv_t, *o_t, *gu_t, *d_t;   // the tiled copies: [q; k; v], o, [gate; up], down
};

} // namespace ms
} // namespace navi_amd

using namespace navi_amd;
using namespace navi_amd::ms;

// The step's activations and split-K workspace, and the HIP stream it runs on.
// x (the residual stream), att and h in the tile layout (rows.h pk_a), the rest row-major.
struct StreamWork {
    float *x = nullptr, *xn = nullptr, *att = nullptr, *h = nullptr, *part = nullptr, *apart = nullptr;
    float *lg = nullptr;
    hipStream_t st = nullptr;
};

struct navi_streams {
    navi_model_params p{};
    int H = 0, NQ = 0, NKV = 0, QD = 0, KVD = 0, F = 0, VT = 0, VC = 0, TL = 0, CL = 0;
    int ms = 0, max_pos = 0, splits = 0;
    // weights
    std::vector<LayerW> tl, cl;
    const float *tl_norm = nullptr, *cp_norm = nullptr;
    const uint16_t *codec_head = nullptr, *codec_emb = nullptr;
    EmbTable cp_emb{};
    const uint16_t *lm_head[CPH] = {};
    uint16_t *lm_head_t[CPH] = {};                  // tiled copies of lm_head
    uint16_t *tiled = nullptr;                      // every tiled weight copy, one allocation
    StreamWork work;
    float *step = nullptr, *invf_t = nullptr, *invf_c = nullptr;
    size_t part_floats = 0;
    uint16_t *cpk = nullptr, *cpv = nullptr;
    uint8_t *seen = nullptr;
    int32_t *codes = nullptr;
    uint32_t *flag = nullptr;
    StreamMeta *meta = nullptr;
    uint16_t **ktab = nullptr, **vtab = nullptr;   // device [TL][ms]: stream caches per layer
    std::vector<uint16_t *> kh, vh;                 // host copy of the tables
    std::vector<StreamMeta> hmeta;
    float *tap = nullptr;                           // taps: hidden [ms][H] | logits [ms][VT] | cp logits [ms][15][VC]
    bool taps_on = false;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    double last_ms = 0;
    std::vector<void *> owned;
    // The step as one HIP graph (about 950 launches), captured again when what the kernels take by
    // value changes: stream count, key ranges, input pointers, sampling arguments.
    bool use_graphs = true;
    hipGraphExec_t gexec = nullptr;
    std::vector<int> gkey;

    float *tap_hidden() const { return tap; }
    float *tap_logits() const { return tap ? tap + static_cast<size_t>(ms) * H : nullptr; }
    float *tap_cp() const { return tap ? tap + static_cast<size_t>(ms) * (H + VT) : nullptr; }

    template <class T>
    navi_status alloc(T *&ptr, size_t n, char *err, size_t errlen) {
        void *v = nullptr;
        NAVI_TRY_HIP(hipMalloc(&v, std::max<size_t>(n, 1) * sizeof(T)), err, errlen);
        owned.push_back(v);
        NAVI_TRY_HIP(hipMemsetAsync(v, 0, std::max<size_t>(n, 1) * sizeof(T), device_state().stream), err, errlen);
        ptr = static_cast<T *>(v);
        return NAVI_OK;
    }

    ~navi_streams() {
        if (gexec) (void) hipGraphExecDestroy(gexec);
        if (ev0) (void) hipEventDestroy(ev0);
        if (ev1) (void) hipEventDestroy(ev1);
        for (void *v : owned) (void) hipFree(v);
    }
};

namespace {

uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

navi_status bind_layers(const char *who, const navi_tensor_ref *t, int n, const std::string &prefix, int L, int H, int QD,
                        int KVD, int F, std::vector<LayerW> &out, char *err, size_t errlen) {
    out.resize(L);
    for (int l = 0; l < L; ++l) {
        const std::string p = prefix + ".layers." + std::to_string(l) + ".";
        LayerW &w = out[l];
        navi_status st;
#define SB(T, name, dt, d0, d1, dst) \
        if ((st = bind_tensor<T>(who, t, n, p + name, dt, d0, d1, dst, err, errlen)) != NAVI_OK) return st
        SB(float, "input_layernorm.weight", NAVI_DT_F32, H, 0, w.ln1);
        SB(float, "post_attention_layernorm.weight", NAVI_DT_F32, H, 0, w.ln2);
        SB(float, "self_attn.q_norm.weight", NAVI_DT_F32, HD, 0, w.qn);
        SB(float, "self_attn.k_norm.weight", NAVI_DT_F32, HD, 0, w.kn);
        SB(uint16_t, "self_attn.q_proj.weight", NAVI_DT_F16, QD, H, w.wq);
        SB(uint16_t, "self_attn.k_proj.weight", NAVI_DT_F16, KVD, H, w.wk);
        SB(uint16_t, "self_attn.v_proj.weight", NAVI_DT_F16, KVD, H, w.wv);
        SB(uint16_t, "self_attn.o_proj.weight", NAVI_DT_F16, H, QD, w.wo);
        SB(uint16_t, "mlp.gate_proj.weight", NAVI_DT_F16, F, H, w.wg);
        SB(uint16_t, "mlp.up_proj.weight", NAVI_DT_F16, F, H, w.wu);
        SB(uint16_t, "mlp.down_proj.weight", NAVI_DT_F16, H, F, w.wd);
#undef SB
    }
    return NAVI_OK;
}

// One decoder layer over `rows` rows: x (the residual stream) in and out. attend() turns the
// q|k|v rows in g.part into the attention output rows in g.att.
// false: a projection shape the tiled kernels do not take (the shapes checked at create all are).
template <class Attend>
bool layer(navi_streams &h, StreamWork &g, const LayerW &w, float eps, int rows, Attend attend) {
    const int H = h.H, QKVW = h.QD + 2 * h.KVD;
    hipStream_t s = g.st;
    if (!launch_rows_pk(EPI_PLAIN, true, g.x, rows, H, w.ln1, eps, w.qkv_t, QKVW, g.part, QKVW, h.flag, s)) return false;
    attend();
    return launch_rows_pk(EPI_RESID, false, g.att, rows, h.QD, nullptr, 0.f, w.o_t, H, g.x, 0, h.flag, s) &&
           launch_rows_pk(EPI_SWIGLU, true, g.x, rows, H, w.ln2, eps, w.gu_t, h.F, g.h, 0, h.flag, s) &&
           launch_rows_pk(EPI_RESID, false, g.h, rows, h.F, nullptr, 0.f, w.d_t, H, g.x, 0, h.flag, s);
}

navi_status unsupported(char *err, size_t errlen) {
    set_err(err, errlen, "streams: a projection shape the tiled row kernels do not take");
    return NAVI_ERR_UNSUPPORTED;
}

// The frame of streams i0 .. i0 + n - 1 (per-stream state at those offsets), on g.st.
navi_status run_group(navi_streams *h, StreamWork &g, int i0, int n, int zsplits, const float *step_in,
                      const float *d_trailing, const SampleArgs &sa, char *err, size_t errlen) {
    hipStream_t s = g.st;
    const int H = h->H;
    const float et = h->p.talker.rms_eps, ec = h->p.cp.rms_eps;
    const StreamMeta *meta = h->meta + i0;
    uint8_t *seen = h->seen + static_cast<size_t>(i0) * h->VT;
    int32_t *codes = h->codes + static_cast<size_t>(i0) * NCB;
    uint16_t *cpk = h->cpk + static_cast<size_t>(i0) * h->CL * NCB * h->KVD;
    uint16_t *cpv = h->cpv + static_cast<size_t>(i0) * h->CL * NCB * h->KVD;

    // talker step over the group's streams
    tile_rows(step_in, n, H, g.x, s);
    for (int l = 0; l < h->TL; ++l) {
        uint16_t *const *kt = h->ktab + static_cast<size_t>(l) * h->ms + i0;
        uint16_t *const *vt = h->vtab + static_cast<size_t>(l) * h->ms + i0;
        const bool ok = layer(*h, g, h->tl[l], et, n, [&]() {
            hipLaunchKernelGGL(k_st_attn, dim3(n, h->NKV, zsplits), dim3(BT), 0, s, g.part, meta, kt, vt, h->NQ, h->NKV,
                               h->splits, h->tl[l].qn, h->tl[l].kn, et, h->invf_t, g.apart);
            hipLaunchKernelGGL(k_st_attn_combine, dim3(n, h->NKV), dim3(BT), 0, s, g.apart, meta, h->NQ, h->NKV, h->splits,
                               g.att);
        });
        if (!ok) return unsupported(err, errlen);
    }
    // final norm (the post-norm hidden rows are the cp's first input rows), head, codebook 0
    hipLaunchKernelGGL(k_st_final_norm, dim3(n), dim3(BT), 0, s, g.x, h->tl_norm, et, g.xn, H);
    launch_rows(EPI_PLAIN, false, g.xn, H, n, H, nullptr, 0.f, h->codec_head, h->VT, nullptr, 0, nullptr, 0, g.lg, h->VT,
                h->flag, s);
    if (h->taps_on) {
        NAVI_TRY_HIP(hipMemcpyAsync(h->tap_hidden() + static_cast<size_t>(i0) * H, g.xn, static_cast<size_t>(n) * H * 4,
                                    hipMemcpyDeviceToDevice, s), err, errlen);
        NAVI_TRY_HIP(hipMemcpyAsync(h->tap_logits() + static_cast<size_t>(i0) * h->VT, g.lg, static_cast<size_t>(n) * h->VT * 4,
                                    hipMemcpyDeviceToDevice, s), err, errlen);
    }
    hipLaunchKernelGGL(k_st_talker_sample, dim3(n), dim3(BT), 0, s, g.lg, h->VT, meta, seen, sa, g.xn, h->codec_emb, H, g.x,
                       codes);

    // code predictor: positions 0 and 1 as one 2-row pass per stream, then one row per position
    for (int pos = 1; pos < NCB; ++pos) {
        const int T = pos == 1 ? 2 : 1, p0 = pos == 1 ? 0 : pos, rows = n * T;
        for (int l = 0; l < h->CL; ++l) {
            const bool ok = layer(*h, g, h->cl[l], ec, rows, [&]() {
                hipLaunchKernelGGL(k_st_cp_attn, dim3(n, h->NKV), dim3(2 * T * WAVE), 0, s, g.part, T, p0, h->NQ, h->NKV,
                                   h->cl[l].qn, h->cl[l].kn, ec, h->invf_c, l, h->CL, cpk, cpv, g.att);
            });
            if (!ok) return unsupported(err, errlen);
        }
        // the cp norm and lm_head[pos - 1] on the last row of each stream (row m T + T - 1 of x)
        if (!launch_rows_pk(EPI_PLAIN, true, g.x, n, H, h->cp_norm, ec, h->lm_head_t[pos - 1], h->VC, g.lg, h->VC, h->flag, s, {},
                            T, T - 1))
            return unsupported(err, errlen);
        if (h->taps_on)
            NAVI_TRY_HIP(hipMemcpy2DAsync(h->tap_cp() + (static_cast<size_t>(i0) * CPH + (pos - 1)) * h->VC,
                                          static_cast<size_t>(CPH) * h->VC * 4, g.lg, static_cast<size_t>(h->VC) * 4,
                                          static_cast<size_t>(h->VC) * 4, n, hipMemcpyDeviceToDevice, s),
                         err, errlen);
        hipLaunchKernelGGL(k_st_cp_sample, dim3(n), dim3(BT), 0, s, g.lg, meta, sa, pos,
                           pos < CPH ? h->cp_emb.cp_emb[pos - 1] : nullptr, H, g.x, codes);
    }
    hipLaunchKernelGGL(k_st_assemble, dim3(n), dim3(BT), 0, s, codes, h->codec_emb, h->cp_emb,
                       d_trailing + static_cast<size_t>(i0) * H, H, h->step + static_cast<size_t>(i0) * H);
    NAVI_TRY_HIP(hipGetLastError(), err, errlen);
    return NAVI_OK;
}

} // namespace

extern "C" {

navi_status navi_streams_create(const navi_model_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                                int32_t max_streams, int32_t max_positions, navi_streams **out, char *err, size_t errlen) {
    if (!p || !tensors || !out) {
        set_err(err, errlen, "streams: null argument");
        return NAVI_ERR_INVALID;
    }
    *out = nullptr;
    navi_status st = ensure_device(err, errlen);
    if (st != NAVI_OK) return st;
    const navi_xformer_params &t = p->talker, &c = p->cp;
    if (t.hidden != 1024 || c.hidden != t.hidden || t.head_dim != HD || c.head_dim != HD || t.n_head != 2 * t.n_kv_head ||
        c.n_head != t.n_head || c.n_kv_head != t.n_kv_head || t.ff != 3072 || t.n_head != 16 || c.ff != t.ff || t.vocab != 3072 ||
        c.vocab != 2048 || p->n_code_groups != NCB || t.n_layer < 1 || t.n_layer > MAX_TL || c.n_layer < 1 ||
        c.n_layer > MAX_CL) {
        set_err(err, errlen, "streams: unsupported shape");
        return NAVI_ERR_UNSUPPORTED;
    }
    if (max_streams < 1 || max_streams > 64 || max_positions < 1 || max_positions > 32768) {
        set_err(err, errlen, "streams: max_streams %d / max_positions %d out of range (1..64 / 1..32768)", max_streams,
                max_positions);
        return NAVI_ERR_INVALID;
    }
    auto h = new navi_streams();
    auto fail = [&](navi_status s_) { delete h; return s_; };
    h->p = *p;
    h->H = t.hidden; h->NQ = t.n_head; h->NKV = t.n_kv_head; h->QD = t.n_head * HD; h->KVD = t.n_kv_head * HD;
    h->F = t.ff; h->VT = t.vocab; h->VC = c.vocab; h->TL = t.n_layer; h->CL = c.n_layer;
    h->ms = max_streams;
    h->max_pos = max_positions;
    h->splits = (max_positions + KPS - 1) / KPS;
    const int H = h->H;
    if ((st = bind_layers("streams", tensors, n_tensors, "talker.model", h->TL, H, h->QD, h->KVD, h->F, h->tl, err, errlen)) != NAVI_OK ||
        (st = bind_layers("streams", tensors, n_tensors, "talker.code_predictor.model", h->CL, H, h->QD, h->KVD, h->F, h->cl, err,
                          errlen)) != NAVI_OK ||
        (st = bind_tensor<float>("streams", tensors, n_tensors, "talker.model.norm.weight", NAVI_DT_F32, H, 0, h->tl_norm, err,
                                 errlen)) != NAVI_OK ||
        (st = bind_tensor<float>("streams", tensors, n_tensors, "talker.code_predictor.model.norm.weight", NAVI_DT_F32, H, 0,
                                 h->cp_norm, err, errlen)) != NAVI_OK ||
        (st = bind_tensor<uint16_t>("streams", tensors, n_tensors, "talker.codec_head.weight", NAVI_DT_F16, h->VT, H,
                                    h->codec_head, err, errlen)) != NAVI_OK ||
        (st = bind_tensor<uint16_t>("streams", tensors, n_tensors, "talker.model.codec_embedding.weight", NAVI_DT_F16, h->VT, H,
                                    h->codec_emb, err, errlen)) != NAVI_OK)
        return fail(st);
    for (int i = 0; i < CPH; ++i) {
        if ((st = bind_tensor<uint16_t>("streams", tensors, n_tensors,
                                        "talker.code_predictor.model.codec_embedding." + std::to_string(i) + ".weight",
                                        NAVI_DT_F16, h->VC, H, h->cp_emb.cp_emb[i], err, errlen)) != NAVI_OK ||
            (st = bind_tensor<uint16_t>("streams", tensors, n_tensors, "talker.code_predictor.lm_head." + std::to_string(i) + ".weight",
                                        NAVI_DT_F16, h->VC, H, h->lm_head[i], err, errlen)) != NAVI_OK)
            return fail(st);
    }
    const size_t R = static_cast<size_t>(2) * max_streams;   // rows of the first cp pass
    const int QKVW = h->QD + 2 * h->KVD;
    size_t pf_need = 0;
    for (int M = 1; M <= static_cast<int>(R); ++M) {
        const int shapes[][2] = {{H, QKVW}, {h->QD, H}, {H, 2 * h->F}, {h->F, H}, {H, h->VT}, {H, h->VC}};
        for (const auto &s : shapes) pf_need = std::max(pf_need, pf::splits_floats(M, s[0], s[1]));
    }
    h->part_floats = pf_need;
#define SA(ptr, n_) \
    if ((st = h->alloc(ptr, (n_), err, errlen)) != NAVI_OK) return fail(st)
    StreamWork &g = h->work;
    const size_t R16 = (R + 15) / 16 * 16;          // x, att and h (tile layout) hold whole 16-row tiles
    SA(g.x, R16 * H);
    SA(g.xn, R * H);
    SA(g.att, R16 * h->QD);
    SA(g.h, R16 * h->F);
    const size_t per_layer = static_cast<size_t>(QKVW) * H + static_cast<size_t>(H) * h->QD + static_cast<size_t>(2 * h->F) * H +
                             static_cast<size_t>(H) * h->F;
    SA(h->tiled, per_layer * (h->TL + h->CL) + static_cast<size_t>(CPH) * h->VC * H);
    SA(g.part, pf_need);
    SA(g.apart, static_cast<size_t>(max_streams) * h->NKV * h->splits * 2 * (HD + 2));
    SA(g.lg, static_cast<size_t>(max_streams) * h->VT);
    g.st = device_state().stream;
    SA(h->step, static_cast<size_t>(max_streams) * H);
    SA(h->invf_t, HD / 2);
    SA(h->invf_c, HD / 2);
    SA(h->cpk, static_cast<size_t>(max_streams) * h->CL * NCB * h->KVD);
    SA(h->cpv, static_cast<size_t>(max_streams) * h->CL * NCB * h->KVD);
    SA(h->seen, static_cast<size_t>(max_streams) * h->VT);
    SA(h->codes, static_cast<size_t>(max_streams) * NCB);
    SA(h->flag, 1);
    SA(h->meta, max_streams);
    SA(h->ktab, static_cast<size_t>(MAX_TL) * max_streams);
    SA(h->vtab, static_cast<size_t>(MAX_TL) * max_streams);
#undef SA
    h->kh.assign(static_cast<size_t>(MAX_TL) * max_streams, nullptr);
    h->vh.assign(static_cast<size_t>(MAX_TL) * max_streams, nullptr);
    h->hmeta.resize(max_streams);
    float it[HD / 2], ic[HD / 2];
    for (int i = 0; i < HD / 2; ++i) {
        it[i] = static_cast<float>(1.0 / std::pow(t.rope_theta, 2.0 * i / HD));
        ic[i] = static_cast<float>(1.0 / std::pow(c.rope_theta, 2.0 * i / HD));
    }
    hipStream_t s = device_state().stream;
    {
        // the tiled copies the row projections read
        uint16_t *q = h->tiled;
        auto put = [&](const uint16_t *src, int rows_, int K) {
            tile_weights(src, rows_, K, q, s);
            q += static_cast<size_t>(rows_) * K;
        };
        for (std::vector<LayerW> *ls : {&h->tl, &h->cl})
            for (LayerW &w : *ls) {
                w.qkv_t = q;
                put(w.wq, h->QD, H);
                put(w.wk, h->KVD, H);
                put(w.wv, h->KVD, H);
                w.o_t = q;
                put(w.wo, H, h->QD);
                w.gu_t = q;
                put(w.wg, h->F, H);
                put(w.wu, h->F, H);
                w.d_t = q;
                put(w.wd, H, h->F);
            }
        for (int i = 0; i < CPH; ++i) {
            h->lm_head_t[i] = q;
            put(h->lm_head[i], h->VC, H);
        }
    }
    if (hipMemcpyAsync(h->invf_t, it, sizeof it, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(h->invf_c, ic, sizeof ic, hipMemcpyHostToDevice, s) != hipSuccess || hipEventCreate(&h->ev0) != hipSuccess ||
        hipEventCreate(&h->ev1) != hipSuccess || hipStreamSynchronize(s) != hipSuccess) {
        set_err(err, errlen, "streams: HIP setup failed");
        return fail(NAVI_ERR_HIP);
    }
    *out = h;
    return NAVI_OK;
}

void navi_streams_destroy(navi_streams *h) {
    if (!h) return;
    (void) hipStreamSynchronize(device_state().stream);
    delete h;
}

navi_status navi_streams_reset(navi_streams *h, int32_t stream) {
    if (!h || stream >= h->ms) return NAVI_ERR_INVALID;
    hipStream_t s = device_state().stream;
    const size_t off = stream < 0 ? 0 : static_cast<size_t>(stream) * h->VT;
    const size_t n = stream < 0 ? static_cast<size_t>(h->ms) * h->VT : h->VT;
    return hipMemsetAsync(h->seen + off, 0, n, s) == hipSuccess && hipStreamSynchronize(s) == hipSuccess ? NAVI_OK : NAVI_ERR_HIP;
}

navi_status navi_streams_set_graphs(navi_streams *h, int32_t on) {
    if (!h) return NAVI_ERR_INVALID;
    h->use_graphs = on != 0;
    return NAVI_OK;
}

navi_status navi_streams_set_taps(navi_streams *h, int32_t on) {
    if (!h) return NAVI_ERR_INVALID;
    h->taps_on = on != 0;
    if (!on || h->tap) return NAVI_OK;
    char err[8];
    const navi_status st = h->alloc(h->tap, static_cast<size_t>(h->ms) * (h->H + h->VT + CPH * h->VC), err, sizeof err);
    if (st != NAVI_OK) h->taps_on = false;
    return st;
}

const float *navi_streams_tap_hidden(const navi_streams *h) { return h ? h->tap_hidden() : nullptr; }
const float *navi_streams_tap_logits(const navi_streams *h) { return h ? h->tap_logits() : nullptr; }
const float *navi_streams_tap_cp_logits(const navi_streams *h) { return h ? h->tap_cp() : nullptr; }

float *navi_streams_step_out(navi_streams *h) { return h ? h->step : nullptr; }
int32_t navi_streams_max_streams(const navi_streams *h) { return h ? h->ms : 0; }
double navi_streams_last_ms(const navi_streams *h) { return h ? h->last_ms : 0.0; }

navi_status navi_streams_run(navi_streams *h, int32_t n, const navi_kv_view *kv, const int32_t *n_past, const float *d_step_in,
                             const float *d_trailing, const navi_sampling *smp, const uint64_t *seeds,
                             const int32_t *frame_index, int32_t *codes_out, char *err, size_t errlen) {
    if (!h || !kv || !n_past || !d_trailing || !smp || !seeds || !frame_index || !codes_out) {
        set_err(err, errlen, "streams: null argument");
        return NAVI_ERR_INVALID;
    }
    if (n < 1 || n > h->ms) {
        set_err(err, errlen, "streams: %d streams, this handle takes 1..%d", n, h->ms);
        return NAVI_ERR_INVALID;
    }
    bool tab_changed = false;
    for (int i = 0; i < n; ++i) {
        if (kv[i].n_layer != h->TL || kv[i].kv_dim != h->KVD || !kv[i].k || !kv[i].v) {
            set_err(err, errlen, "streams: stream %d: KV cache layer count or width mismatch", i);
            return NAVI_ERR_INVALID;
        }
        if (n_past[i] < 0 || n_past[i] >= kv[i].max_pos || n_past[i] >= h->max_pos) {
            set_err(err, errlen, "stream %d: KV cache full", i);
            return NAVI_ERR_KV_FULL;
        }
        for (int l = 0; l < h->TL; ++l) {
            uint16_t *&kd = h->kh[static_cast<size_t>(l) * h->ms + i], *&vd = h->vh[static_cast<size_t>(l) * h->ms + i];
            if (kd != kv[i].k[l] || vd != kv[i].v[l]) {
                kd = kv[i].k[l];
                vd = kv[i].v[l];
                tab_changed = true;
            }
        }
        StreamMeta &m = h->hmeta[i];
        m.n_past = n_past[i];
        m.frame_index = frame_index[i];
        m.talker_seed = splitmix64(seeds[i] ^ (static_cast<uint64_t>(frame_index[i]) * 0xA24BAED4963EE407ull));
        m.cp_seed = splitmix64(m.talker_seed ^ 0x9FB21C651E98DF25ull);
    }
    hipStream_t s = device_state().stream;
    if (tab_changed) {
        NAVI_TRY_HIP(hipMemcpyAsync(h->ktab, h->kh.data(), h->kh.size() * sizeof(uint16_t *), hipMemcpyHostToDevice, s), err, errlen);
        NAVI_TRY_HIP(hipMemcpyAsync(h->vtab, h->vh.data(), h->vh.size() * sizeof(uint16_t *), hipMemcpyHostToDevice, s), err, errlen);
    }
    NAVI_TRY_HIP(hipMemcpyAsync(h->meta, h->hmeta.data(), n * sizeof(StreamMeta), hipMemcpyHostToDevice, s), err, errlen);
    NAVI_TRY_HIP(hipMemsetAsync(h->flag, 0, 4, s), err, errlen);
    NAVI_TRY_HIP(hipEventRecord(h->ev0, s), err, errlen);
    SampleArgs sa{smp->temperature, smp->repetition_penalty, smp->cp_temperature, smp->top_k, smp->cp_top_k, smp->min_frames,
                  h->p.codec_eos_id, h->VT - 1024};
    // the step after the uploads above, replayed from a graph unless taps are on or graphs are off
    int zs = 1;                                             // key ranges of the longest context
    for (int i = 0; i < n; ++i) zs = std::max(zs, (n_past[i] + 1 + KPS - 1) / KPS);
    const float *step_base = d_step_in ? d_step_in : h->step;
    auto enqueue = [&]() { return run_group(h, h->work, 0, n, zs, step_base, d_trailing, sa, err, errlen); };
    if (h->use_graphs && !h->taps_on) {
        std::vector<int> key{n, zs};
        for (const void *ptr : {static_cast<const void *>(step_base), static_cast<const void *>(d_trailing)}) {
            const uint64_t u = reinterpret_cast<uint64_t>(ptr);
            key.push_back(static_cast<int>(u & 0xFFFFFFFFu));
            key.push_back(static_cast<int>(u >> 32));
        }
        int sw[sizeof(SampleArgs) / sizeof(int)];
        static_assert(sizeof(SampleArgs) % sizeof(int) == 0, "sampling args as words");
        std::memcpy(sw, &sa, sizeof sa);
        key.insert(key.end(), sw, sw + sizeof sw / sizeof sw[0]);
        if (!h->gexec || key != h->gkey) {
            if (h->gexec) {
                (void) hipGraphExecDestroy(h->gexec);
                h->gexec = nullptr;
            }
            NAVI_TRY_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), err, errlen);
            const navi_status st = enqueue();
            hipGraph_t graph = nullptr;
            const hipError_t ec = hipStreamEndCapture(s, &graph);
            if (st != NAVI_OK) {
                if (graph) (void) hipGraphDestroy(graph);
                return st;
            }
            NAVI_TRY_HIP(ec, err, errlen);
            const hipError_t ei = hipGraphInstantiateWithFlags(&h->gexec, graph, 0);
            (void) hipGraphDestroy(graph);
            NAVI_TRY_HIP(ei, err, errlen);
            h->gkey = key;
        }
        NAVI_TRY_HIP(hipGraphLaunch(h->gexec, s), err, errlen);
    } else {
        const navi_status st = enqueue();
        if (st != NAVI_OK) return st;
    }
    NAVI_TRY_HIP(hipEventRecord(h->ev1, s), err, errlen);
    uint32_t bad = 0;
    NAVI_TRY_HIP(hipMemcpyAsync(codes_out, h->codes, static_cast<size_t>(n) * NCB * sizeof(int32_t), hipMemcpyDeviceToHost, s), err,
                 errlen);
    NAVI_TRY_HIP(hipMemcpyAsync(&bad, h->flag, 4, hipMemcpyDeviceToHost, s), err, errlen);
    NAVI_TRY_HIP(hipStreamSynchronize(s), err, errlen);
    float ms_ = 0.f;
    (void) hipEventElapsedTime(&ms_, h->ev0, h->ev1);
    h->last_ms = ms_;
    if (bad) {
        set_err(err, errlen, "streams: an activation is outside the f16 range (|x| >= 65504 or NaN)");
        return NAVI_ERR_INVALID;
    }
    return NAVI_OK;
}

} // extern "C"
