/*
 * C restatement of the reference sampler's integer and f32 arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): compiled by oracle/csrc/Makefile
 * into oracle/lib/liboracle_sampler.so and loaded by tests/ to cross-check the Python
 * oracle (oracle/rng.py, oracle/sampler.py) with a second, independent restatement.
 *
 * Follows model/qwen3tts/frame.hip of the reference:
 *   ora_splitmix64     - splitmix64, frame.hip:581-586 (Steele/Vigna SplitMix64 finalizer)
 *   ora_pcg32_next     - pcg32_next, frame.hip:169-175 (O'Neill PCG-XSH-RR 64/32, fixed increment)
 *   ora_draw_uniform   - block_draw's seeding and u, frame.hip:284-286
 *   ora_frame_seeds    - Frame::Impl::launch, frame.hip:658-659
 *   ora_cp_pos_seed    - cp_sample, frame.hip:497
 *   ora_kth_largest    - block_kth_largest, frame.hip:212-256: monotone float->u32 key and four
 *                        8-bit radix passes, here serial
 *   ora_draw           - block_draw, frame.hip:263-296: nonzero entries in index order, running
 *                        sum cum = fma(p, inv_sum, cum) (the contraction hipcc applies to the
 *                        reference's `cum += p[i] * inv_sum`), first cum >= u, else V-1
 *   ora_argmax         - block_argmax, frame.hip:178-203: lowest index wins ties
 *
 * Built with -ffp-contract=off so that the only fused operation is the explicit fmaf.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

uint64_t ora_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint32_t ora_pcg32_next_inc(uint64_t *state, uint64_t inc) {
    const uint64_t old = *state;
    *state = old * 6364136223846793005ull + inc;
    const uint32_t xs = (uint32_t) (((old >> 18) ^ old) >> 27);
    const uint32_t rot = (uint32_t) (old >> 59);
    return (xs >> rot) | (xs << ((0u - rot) & 31u));
}

uint32_t ora_pcg32_next(uint64_t *state) { return ora_pcg32_next_inc(state, 1442695040888963407ull); }

float ora_draw_uniform(uint64_t seed) {
    uint64_t st = seed * 0x9E3779B97F4A7C15ull + 0xBF58476D1CE4E5B9ull + 1ull;
    (void) ora_pcg32_next(&st);
    (void) ora_pcg32_next(&st);
    (void) ora_pcg32_next(&st);
    return (float) (ora_pcg32_next(&st) >> 8) * (1.0f / 16777216.0f);
}

void ora_frame_seeds(uint64_t seed, int32_t frame_index, uint64_t *talker, uint64_t *cp) {
    *talker = ora_splitmix64(seed ^ ((uint64_t) (int64_t) frame_index * 0xA24BAED4963EE407ull));
    *cp = ora_splitmix64(*talker ^ 0x9FB21C651E98DF25ull);
}

uint64_t ora_cp_pos_seed(uint64_t cp_seed, int32_t pos) {
    return cp_seed + (uint64_t) (int64_t) pos * 0xD1B54A32D192ED03ull;
}

static uint32_t float_key(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static float key_float(uint32_t u) {
    const uint32_t b = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* k-th largest of xs[0..V), 1 <= k <= V. Walks each 256-bin histogram from the top digit down
 * and keeps the digit where the count of larger keys first reaches k. */
float ora_kth_largest(const float *xs, int32_t V, int32_t k) {
    uint32_t prefix = 0, mask = 0;
    int32_t need = k;
    uint32_t hist[256];
    for (int pass = 3; pass >= 0; --pass) {
        const int shift = pass * 8;
        memset(hist, 0, sizeof hist);
        for (int32_t i = 0; i < V; ++i) {
            const uint32_t key = float_key(xs[i]);
            if ((key & mask) == prefix) hist[(key >> shift) & 0xFFu]++;
        }
        int32_t above = 0;
        int d = 255;
        for (; d >= 0; --d) {
            const int32_t c = (int32_t) hist[d];
            if (above < need && above + c >= need) break;
            above += c;
        }
        if (d < 0) d = 0;   /* unreachable for 1 <= k <= V */
        need -= above;
        prefix |= (uint32_t) d << shift;
        mask |= 0xFFu << shift;
    }
    return key_float(prefix);
}

int32_t ora_draw(const float *p, int32_t V, float inv_sum, uint64_t seed) {
    const float u = ora_draw_uniform(seed);
    float cum = 0.f;
    for (int32_t i = 0; i < V; ++i) {
        if (p[i] == 0.f) continue;
        cum = fmaf(p[i], inv_sum, cum);
        if (cum >= u) return i;
    }
    return V - 1;
}

int32_t ora_argmax(const float *v, int32_t n) {
    float bv = -INFINITY;
    int32_t bi = 0;
    for (int32_t i = 0; i < n; ++i)
        if (v[i] > bv) { bv = v[i]; bi = i; }
    return bi;
}
