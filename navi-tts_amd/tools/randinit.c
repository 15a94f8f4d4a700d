/*
 * Deterministic random-init weight filler for synthetic `.navi` blobs.
 *
 * Every element is a pure function of (seed, tensor name, element index), so
 * a blob can be regenerated bit-identically on any machine, in any tensor
 * order, with any number of threads. The reference has no random-init mode
 * (its converter only re-encodes an HF checkpoint, tools/convert.py:271-315);
 * this fills the same tensor table with N(0, sigma) values instead.
 *
 * Generator: elements 2p and 2p+1 come from two SplitMix64 outputs
 *   r_a = mix64(key + (2p+1)*GAMMA), r_b = mix64(key + (2p+2)*GAMMA)
 * (Steele, Lea & Flood 2014, "Fast splittable pseudorandom number
 * generators"), turned into two standard normals by the Box-Muller transform
 * (Box & Muller 1958). key = mix64(seed) ^ fnv1a64(name).
 *
 * f16 output is round-to-nearest-even from the f32 value, the conversion
 * numpy's astype(float16) performs (gcc 11 has no _Float16 on x86).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define GAMMA 0x9E3779B97F4A7C15ull

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t fnv1a64(const char *s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (; *s; ++s) { h ^= (unsigned char)*s; h *= 0x100000001b3ull; }
    return h;
}

uint64_t navi_rand_key(uint64_t seed, const char *name) { return mix64(seed + GAMMA) ^ fnv1a64(name); }

/* Standard normals for elements 2p and 2p+1 of the stream `key`. */
static inline void normal_pair(uint64_t key, uint64_t p, double *z0, double *z1) {
    const uint64_t ra = mix64(key + (2 * p + 1) * GAMMA);
    const uint64_t rb = mix64(key + (2 * p + 2) * GAMMA);
    const double u1 = ((double)(ra >> 11) + 1.0) * (1.0 / 9007199254740992.0);   /* (0, 1] */
    const double u2 = (double)(rb >> 11) * (1.0 / 9007199254740992.0);           /* [0, 1) */
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586476925286766559 * u2;
    *z0 = r * cos(t);
    *z1 = r * sin(t);
}

/* IEEE binary32 -> binary16, round to nearest even, with subnormals, inf and nan. */
uint16_t navi_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {                                            /* below 2^-14: f16 subnormal */
        if (ax < 0x33000000u) return (uint16_t)sign;                   /* below 2^-25: zero */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;                               /* 14..24 */
        uint32_t v = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (v & 1u))) ++v;
        return (uint16_t)(sign | v);
    }
    uint32_t v = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) ++v;
    return (uint16_t)(sign | v);
}

void navi_fill_normal_f16(uint64_t seed, const char *name, double sigma, uint16_t *out, uint64_t n) {
    const uint64_t key = navi_rand_key(seed, name);
    const int64_t np_ = (int64_t)((n + 1) / 2);
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < np_; ++p) {
        double z0, z1;
        normal_pair(key, (uint64_t)p, &z0, &z1);
        out[2 * p] = navi_f32_to_f16((float)(sigma * z0));
        if ((uint64_t)(2 * p + 1) < n) out[2 * p + 1] = navi_f32_to_f16((float)(sigma * z1));
    }
}

void navi_fill_normal_f32(uint64_t seed, const char *name, double sigma, float *out, uint64_t n) {
    const uint64_t key = navi_rand_key(seed, name);
    const int64_t np_ = (int64_t)((n + 1) / 2);
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < np_; ++p) {
        double z0, z1;
        normal_pair(key, (uint64_t)p, &z0, &z1);
        out[2 * p] = (float)(sigma * z0);
        if ((uint64_t)(2 * p + 1) < n) out[2 * p + 1] = (float)(sigma * z1);
    }
}

/* f32 array -> f16 bits, the conversion used for every >=2-D tensor of a blob. */
void navi_f32_to_f16_array(const float *in, uint16_t *out, uint64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) out[i] = navi_f32_to_f16(in[i]);
}
