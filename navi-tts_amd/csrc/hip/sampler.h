// Block-wide seeded sampling of one index (the reference's tl_sample / cp_sample path): greedy
// argmax, or temperature -> exact top-k threshold -> e^(v - max) -> PCG32 draw. Shared by the
// frame kernel (every block samples redundantly) and the multi-stream sampler (one block per
// stream); identical inputs give identical picks in both.
#pragma once

#include "dev_common.h"

namespace navi_amd {

__device__ __forceinline__ unsigned float_key(float f) {
    const unsigned u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(unsigned u) {
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

// PCG-XSH-RR 64/32 step with the reference's increment (frame.hip:169-175).
__device__ __forceinline__ uint32_t pcg32_next(uint64_t &s) {
    const uint64_t old = s;
    s = old * 6364136223846793005ull + 1442695040888963407ull;
    const uint32_t xs = static_cast<uint32_t>(((old >> 18u) ^ old) >> 27u);
    const uint32_t rot = static_cast<uint32_t>(old >> 59u);
    return (xs >> rot) | (xs << ((0u - rot) & 31u));
}

// Radix-select counters: pass 0 keeps 4 copies of each of its 256 bins ([digit][lane & 3], so the
// lanes of one atomic instruction that share a top byte, nearly all of them, spread over 4 banks);
// passes 1-3 one 256-bin histogram each.
constexpr int SAMPLE_HIST_WORDS = 4 * 256 + 3 * 256;
// The sampler's LDS counters plus one 64-bit candidate mask per 64-index chunk (V <= 4096).
constexpr int SAMPLE_LDS_WORDS = SAMPLE_HIST_WORDS + 2 * 64;

// LDS the sampler works in (all block-shared): lg[V] holds the (already modified) logits on entry
// and is overwritten; hist: SAMPLE_LDS_WORDS words, 16-byte aligned; sred: 2 * NW floats;
// sidx: NW ints; sel: 1 int.
struct SampleLds {
    float *lg;
    unsigned *hist;
    float *sred;
    int *sidx;
    int *sel;
};

// Sampling of one index from the V values in L.lg with BT threads (NW = BT / 64 waves).
// Thread layout: element i = k * BT + tid, so index order is (k, wave, lane). Greedy: argmax,
// lowest index on ties (frame.hip:178-203). Else (frame.hip:421-454, 212-296): /temperature,
// exact top-k threshold (the k-th largest by a 4-pass 8-bit radix select over monotone keys,
// values >= it survive), e^(v - max), and wave 0 draws with the PCG32 u over the survivors in
// index order with the fused running sum of the reference (`cum += p * inv_sum` compiles to an
// FMA under hipcc's default contraction). Each radix pass costs one barrier: the histograms are
// cleared up front, and every wave finds the digit itself from the shared histogram with a DPP
// prefix sum. The select stops early once the chosen bin lies wholly inside the top k (its count
// is the number still needed): the bin's lowest value then admits exactly the same survivors as
// the k-th largest value would. The draw compacts the candidates in index order and runs the
// fused running sum as a lane-to-lane DPP chain (below). The result is the same in every thread.
template <int V, int BT>
__device__ __forceinline__ int block_sample(float temperature, int top_k, uint64_t seed, const SampleLds &L) {
    constexpr int PER = V / BT, NW = BT / WAVE;
    static_assert(V % BT == 0 && BT == 256, "4 waves, V a multiple of the block");
    const int tid = static_cast<int>(threadIdx.x), lane = tid & (WAVE - 1), wave = tid / WAVE;
    float x[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) x[k] = L.lg[k * BT + tid];
    if (temperature <= 0.f) {
        float bv = x[0];
        int bi = tid;
#pragma unroll
        for (int k = 1; k < PER; ++k)
            if (x[k] > bv) { bv = x[k]; bi = k * BT + tid; }   // k ascending: the first maximum of this thread
        const float m = wave_max(bv);
        const int wi = wave_min_int(bv == m ? bi : V);
        if (lane == 0) { L.sred[wave] = m; L.sidx[wave] = wi; }
        __syncthreads();
        float v = L.sred[0];
        int i0 = L.sidx[0];
#pragma unroll
        for (int w = 1; w < NW; ++w)
            if (L.sred[w] > v || (L.sred[w] == v && L.sidx[w] < i0)) { v = L.sred[w]; i0 = L.sidx[w]; }
        return i0;
    }
    unsigned *const hist = L.hist;
    const bool topk = top_k > 0 && top_k < V;
    if (topk) {
        static_assert(SAMPLE_HIST_WORDS % BT == 0, "histogram clear");
#pragma unroll
        for (int p = 0; p < SAMPLE_HIST_WORDS / BT; ++p) hist[p * BT + tid] = 0u;
    }
    float lmx = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; ++k) { x[k] = x[k] / temperature; lmx = fmaxf(lmx, x[k]); }
    lmx = wave_max(lmx);
    if (lane == 0) L.sred[wave] = lmx;
    __syncthreads();
    float mx = L.sred[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, L.sred[w]);
    float thr = -INFINITY;
    if (topk) {
        unsigned prefix = 0, mask = 0;
        int need = top_k;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int shift = 24 - 8 * p;
            unsigned *const hp = hist + (p == 0 ? 0 : 1024 + (p - 1) * 256);
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const unsigned key = float_key(x[k]);
                if (p == 0) atomicAdd(&hp[(key >> 24) * 4 + (lane & 3)], 1u);
                else if ((key & mask) == prefix) atomicAdd(&hp[(key >> shift) & 0xFFu], 1u);
            }
            __syncthreads();
            // lane l owns digits 255-4l .. 252-4l (descending); every wave finds the digit itself
            int c[4], tot = 0;
            if (p == 0) {
                // digits 252-4l+q, q = 0..3: four replicas each, 16 consecutive words
                const u32x4_t *h4 = reinterpret_cast<const u32x4_t *>(hp + (252 - 4 * lane) * 4);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4_t r = h4[q];
                    c[3 - q] = static_cast<int>((r.x + r.y) + (r.z + r.w));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) c[j] = static_cast<int>(hp[255 - 4 * lane - j]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) tot += c[j];
            int above = wave_incl_scan(tot) - tot;
            int dsel = -1, nsel = 0, csel = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (dsel < 0 && above < need && above + c[j] >= need) { dsel = 255 - 4 * lane - j; nsel = need - above; csel = c[j]; }
                above += c[j];
            }
            const uint64_t hit = __ballot(dsel >= 0);
            const int src = hit ? static_cast<int>(__builtin_ctzll(hit)) : 0;   // exactly one lane finds it
            const int digit = __builtin_amdgcn_readlane(dsel, src);
            need = __builtin_amdgcn_readlane(nsel, src);
            const int cnt = __builtin_amdgcn_readlane(csel, src);
            prefix |= static_cast<unsigned>(digit) << shift;
            mask |= 0xFFu << shift;
            // The whole bin survives: its lowest float admits exactly the same values as the k-th
            // largest. Not for the bin that starts at +0 (-0 compares equal to it but keys below
            // it) nor for one whose lowest key is a NaN pattern.
            if (need == cnt && prefix >= 0x00800000u && prefix != 0x80000000u) break;
        }
        thr = key_float(prefix);
    }
    // e = e^(x - max) for the survivors; chunk c = k * NW + wave (indices 64c .. 64c + 63) records
    // which of its lanes hold a candidate (e != 0)
    constexpr int NCH = V / WAVE;
    static_assert(NCH <= WAVE, "one chunk per lane in the prefix");
    uint64_t *const cmask = reinterpret_cast<uint64_t *>(hist + SAMPLE_HIST_WORDS);
    float e[PER];
    float ls = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        e[k] = x[k] >= thr ? expf(x[k] - mx) : 0.f;
        ls += e[k];
        const uint64_t bm = __ballot(e[k] != 0.f);
        if (lane == 0) cmask[k * NW + wave] = bm;
    }
    ls = wave_sum(ls);
    if (lane == 0) L.sred[NW + wave] = ls;
    __syncthreads();
    // the candidates compacted in index order into lg (the logits are in registers by now): chunk
    // c starts after the candidates of chunks 0..c-1, a DPP prefix sum with one chunk per lane
    const uint64_t lm = lane < NCH ? cmask[lane] : 0ull;
    const int lc = __builtin_popcountll(lm);
    const int incl = wave_incl_scan(lc), excl = incl - lc;
    const int ncand = __builtin_amdgcn_readlane(incl, WAVE - 1);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint64_t bm = __ballot(e[k] != 0.f);
        const int below = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bm >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bm), 0u)));
        if (e[k] != 0.f) L.lg[__builtin_amdgcn_readlane(excl, k * NW + wave) + below] = e[k];
    }
    __syncthreads();
    if (wave == 0) {
        float ssum = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) ssum += L.sred[NW + w];
        const float inv = 1.f / ssum;
        uint64_t st = seed * 0x9E3779B97F4A7C15ull + 0xBF58476D1CE4E5B9ull + 1ull;
        (void) pcg32_next(st); (void) pcg32_next(st); (void) pcg32_next(st);
        const float u = static_cast<float>(pcg32_next(st) >> 8) * (1.0f / 16777216.0f);
        int chosen = V - 1;
        float carry = 0.f;
        // The running sum over the candidates, 64 at a time: lane j takes candidate g + j, and
        // every step lane j recomputes fma(p_j, inv, value of lane j - 1) (lane 0: the carry),
        // DPP wave_shr:1 moving the values one lane up. After s steps lanes 0..s-1 hold exactly
        // the sequential sums, so m steps give the reference's chain for the group. The sums
        // never decrease, so the lanes below u are a prefix and their count is the pick.
        for (int g = 0; g < ncand; g += WAVE) {
            const int m = min(WAVE, ncand - g);
            const float pc = lane < m ? L.lg[g + lane] : 0.f;
            float cum = carry;
            // steps past m recompute the same values (lane j - 1 is final by then): 8 per trip
            for (int step = 0; step < m; step += 8) {
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float sh = __int_as_float(
                        __builtin_amdgcn_update_dpp(__float_as_int(carry), __float_as_int(cum), 0x138, 0xF, 0xF, false));
                    cum = fmaf(pc, inv, sh);
                }
            }
            const int nb = __builtin_popcountll(__ballot(lane < m && cum < u));
            if (nb < m) {
                // candidate pos = g + nb: its chunk is the first whose inclusive count exceeds pos,
                // and it is the (pos - start)-th set lane of that chunk's mask
                const int pos = g + nb;
                const int cs = __builtin_popcountll(__ballot(lane < NCH && incl <= pos));
                const int r = pos - __builtin_amdgcn_readlane(excl, cs);
                const uint32_t mlo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(lm)), cs));
                const uint32_t mhi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(lm >> 32)), cs));
                const uint64_t mk = (static_cast<uint64_t>(mhi) << 32) | mlo;
                const int rank = static_cast<int>(__builtin_amdgcn_mbcnt_hi(mhi, __builtin_amdgcn_mbcnt_lo(mlo, 0u)));
                const uint64_t hit = __ballot(((mk >> lane) & 1ull) && rank == r);
                chosen = cs * WAVE + static_cast<int>(__builtin_ctzll(hit));
                break;
            }
            carry = lane_value(cum, m - 1);
        }
        if (lane == 0) *L.sel = chosen;
    }
    __syncthreads();
    return *L.sel;
}

} // namespace navi_amd
