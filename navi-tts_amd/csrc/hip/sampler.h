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

// LDS the sampler works in (all block-shared): lg[V] holds the (already modified) logits on entry
// and is overwritten; hist: 4 x 256 counters; sred: 2 * NW floats; sidx: NW ints; sel: 1 int.
struct SampleLds {
    float *lg;
    unsigned (*hist)[256];
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
// FMA under hipcc's default contraction). Each radix pass costs one barrier: the four histograms
// are cleared up front, and every wave finds the digit itself from the shared histogram with a
// DPP prefix sum. The result is the same in every thread.
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
    unsigned (*hist)[256] = L.hist;
    const bool topk = top_k > 0 && top_k < V;
    if (topk) {
#pragma unroll
        for (int p = 0; p < 4; ++p) hist[p][tid] = 0u;
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
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const unsigned key = float_key(x[k]);
                if ((key & mask) == prefix) atomicAdd(&hist[p][(key >> shift) & 0xFFu], 1u);
            }
            __syncthreads();
            // lane l owns digits 255-4l .. 252-4l (descending); every wave finds the digit itself
            int c[4], tot = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) { c[j] = static_cast<int>(hist[p][255 - 4 * lane - j]); tot += c[j]; }
            int above = wave_incl_scan(tot) - tot;
            int dsel = -1, nsel = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (dsel < 0 && above < need && above + c[j] >= need) { dsel = 255 - 4 * lane - j; nsel = need - above; }
                above += c[j];
            }
            const uint64_t hit = __ballot(dsel >= 0);
            const int src = hit ? static_cast<int>(__builtin_ctzll(hit)) : 0;   // exactly one lane finds it
            const int digit = __builtin_amdgcn_readlane(dsel, src);
            need = __builtin_amdgcn_readlane(nsel, src);
            prefix |= static_cast<unsigned>(digit) << shift;
            mask |= 0xFFu << shift;
        }
        thr = key_float(prefix);
    }
    float ls = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const float e = x[k] >= thr ? expf(x[k] - mx) : 0.f;
        L.lg[k * BT + tid] = e;
        ls += e;
    }
    ls = wave_sum(ls);
    if (lane == 0) L.sred[NW + wave] = ls;
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
        float cum = 0.f;
        bool found = false;
        for (int k = 0; k < PER && !found; ++k) {
            for (int w = 0; w < NW && !found; ++w) {
                const int base = k * BT + w * WAVE;
                const float ev = L.lg[base + lane];
                uint64_t nz = __ballot(ev != 0.f);
                while (nz && !found) {
                    const int b = static_cast<int>(__builtin_ctzll(nz));
                    nz &= nz - 1;
                    cum = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), b)), inv, cum);
                    if (cum >= u) { chosen = base + b; found = true; }
                }
            }
        }
        if (lane == 0) *L.sel = chosen;
    }
    __syncthreads();
    return *L.sel;
}

} // namespace navi_amd
