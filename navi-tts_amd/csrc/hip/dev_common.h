// Device helpers shared by the gfx950 kernels: wave64 reductions, f16 unpacking
// and the tagged-word mailboxes the persistent frame kernel communicates through.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace navi_amd {

constexpr int WAVE = 64;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Wave64 reductions without the LDS crossbar (a __shfl_xor butterfly compiles to six dependent
// ds_bpermute round trips): DPP quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and
// row_mirror reduce each 16-lane row in registers, then the four row results are read as
// scalars. Every lane gets the result. Call with all 64 lanes active (readlane reads inactive
// lanes' stale registers).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_value(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// A DPP read of v for a reduction step; with bound_ctrl the compiler fuses it into the
// consuming v_add/v_max (one instruction per step).
template <int CTRL>
__device__ __forceinline__ float dpp_red(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_rows(float v, float old) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWS, 0xF, false));
}

// Sum over the 64 lanes, the same value in every lane: quad_perm, row_half_mirror and row_mirror
// make each 16-lane row hold its row sum r_k; row_bcast:15 into rows 1 and 3 and row_bcast:31 into
// rows 2 and 3 leave (r3 + r2) + (r1 + r0) in lane 63.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_red<0xB1>(v);      // quad_perm [1,0,3,2]
    v += dpp_red<0x4E>(v);      // quad_perm [2,3,0,1]
    v += dpp_red<0x141>(v);     // row_half_mirror
    v += dpp_red<0x140>(v);     // row_mirror
    v += dpp_rows<0x142, 0xA>(v, 0.f);
    v += dpp_rows<0x143, 0xC>(v, 0.f);
    return lane_value(v, 63);
}

// wave_sum of N values at once, one DPP stage for all of them before the next (the N chains
// interleave instead of waiting out each step's hazard); each result as wave_sum's.
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_red<0xB1>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_red<0x4E>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_red<0x141>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_red<0x140>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_rows<0x142, 0xA>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_rows<0x143, 0xC>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = lane_value(v[i], 63);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_red<0xB1>(v));
    v = fmaxf(v, dpp_red<0x4E>(v));
    v = fmaxf(v, dpp_red<0x141>(v));
    v = fmaxf(v, dpp_red<0x140>(v));
    v = fmaxf(v, dpp_rows<0x142, 0xA>(v, v));
    v = fmaxf(v, dpp_rows<0x143, 0xC>(v, v));
    return lane_value(v, 63);
}

// Inclusive prefix sum over the 64 lanes: row_shr 1/2/4/8 within each 16-lane row, then
// row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2 and 3. All lanes active.
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_shift(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, false); }
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += dpp_shift<0x111, 0xF>(v);
    v += dpp_shift<0x112, 0xF>(v);
    v += dpp_shift<0x114, 0xF>(v);
    v += dpp_shift<0x118, 0xF>(v);
    v += dpp_shift<0x142, 0xA>(v);
    v += dpp_shift<0x143, 0xC>(v);
    return v;
}

__device__ __forceinline__ int wave_min_int(int v) {
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xA, 0xF, false));
    v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xC, 0xF, false));
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 f;
    __builtin_memcpy(&f, &h, 2);
    return static_cast<float>(f);
}

__device__ __forceinline__ uint16_t f2h(float v) {
    const _Float16 h = static_cast<_Float16>(v);
    uint16_t u;
    __builtin_memcpy(&u, &h, 2);
    return u;
}

// f32 -> f16 -> f32: the value a K/V cache entry holds.
__device__ __forceinline__ float round_f16(float v) { return static_cast<float>(static_cast<_Float16>(v)); }

// acc + sum_i w[i] * x[i] over one 16-byte weight fragment (8 f16), left to right.
__device__ __forceinline__ float dot8(const uint4 w, const float *x, float acc) {
    half8_t h;
    __builtin_memcpy(&h, &w, 16);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = fmaf(static_cast<float>(h[i]), x[i], acc);
    return acc;
}

// acc[r] = this lane's 16 weights of row r (two 16-byte fragments) times xf, accumulated in
// dot8(w[r][1], xf[1], dot8(w[r][0], xf[0], 0))'s order; element-major so the R chains interleave.
template <int R>
__device__ __forceinline__ void dot16_rows(const uint4 (&w)[R][2], const float (&xf)[2][8], float (&acc)[R]) {
    half8_t h[R][2];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        __builtin_memcpy(&h[r][0], &w[r][0], 16);
        __builtin_memcpy(&h[r][1], &w[r][1], 16);
        acc[r] = 0.f;
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = fmaf(static_cast<float>(h[r][c][i]), xf[c][i], acc[r]);
}

// Global memory accessed through address space 1, so the compiler emits global_* (counted by
// vmcnt only) instead of flat_* instructions, which also count in lgkmcnt and would make every
// LDS wait also wait for the in-flight weight stream.
#define NAVI_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ T gld(const T *p) { return *(const NAVI_GLOBAL T *) p; }
template <class T>
__device__ __forceinline__ void gst(T *p, T v) { *(NAVI_GLOBAL T *) p = v; }

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// 16-byte global load as a native vector (a HIP uint4 struct copy through an address-space-1
// pointer still lowers to flat_load).
__device__ __forceinline__ uint4 ldg16(const uint16_t *p) {
    const u32x4_t v = *(const NAVI_GLOBAL u32x4_t *) p;
    uint4 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// Streaming (non-temporal) 16-byte load for data read once per pass: the weight stream must
// not evict the kernel's code and mailboxes from L2.
__device__ __forceinline__ uint4 ldg16_stream(const uint16_t *p) {
    const u32x4_t v = __builtin_nontemporal_load((const NAVI_GLOBAL u32x4_t *) p);
    uint4 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// A wave-uniform pointer moved to SGPRs, so accesses address it as saddr + a shared
// per-lane VGPR offset instead of one 64-bit VGPR pair per call site.
template <class T>
__device__ __forceinline__ T *sgpr_ptr(T *p) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return reinterpret_cast<T *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// ---------------------------------------------------------------------------
// Tagged mailboxes. A 64-bit word holds {f32 value (low), u32 tag (high)} and
// is written and read with device-scope relaxed atomics, which compile to
// plain global stores/loads with the sc1 bit on gfx950: coherent across the
// eight XCDs' L2s without any fence or cache flush. A consumer accepts a word
// only when its tag is the tag of the phase it waits for, so the data and its
// readiness travel in one store and one load.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void mb_put(uint64_t *p, float v, uint32_t tag) {
    const uint64_t w = (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v);
    __hip_atomic_store((NAVI_GLOBAL uint64_t *) p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t mb_peek(uint64_t *p) {
    return __hip_atomic_load((NAVI_GLOBAL uint64_t *) p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t ctl_peek(uint32_t *p) {
    return __hip_atomic_load((NAVI_GLOBAL uint32_t *) p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void ctl_put(uint32_t *p, uint32_t v) {
    __hip_atomic_store((NAVI_GLOBAL uint32_t *) p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t tag_of(uint64_t w) { return static_cast<uint32_t>(w >> 32); }
__device__ __forceinline__ float val_of(uint64_t w) { return __uint_as_float(static_cast<uint32_t>(w)); }

// part[0] + part[1] + ... + part[S-1] at four consecutive columns, in that order (deterministic);
// the loads go out eight partials at a time instead of one after another.
__device__ __forceinline__ f32x4_t sum_parts4(const float *part, int S, size_t stride, size_t idx) {
    f32x4_t v = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < S; s0 += 8) {
        f32x4_t t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (s0 + j < S) t[j] = *(const NAVI_GLOBAL f32x4_t *) (part + (s0 + j) * stride + idx);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (s0 + j < S) v = s0 + j == 0 ? t[j] : v + t[j];
    }
    return v;
}

__device__ __forceinline__ f32x4_t ld4(const float *p) { return *(const NAVI_GLOBAL f32x4_t *) p; }
__device__ __forceinline__ void st4(float *p, f32x4_t v) { *(NAVI_GLOBAL f32x4_t *) p = v; }

} // namespace navi_amd
