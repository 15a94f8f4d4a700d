"""Seeding and the PCG32 stream of the reference sampler, in exact 64-bit integers.

Test infrastructure. Restates model/qwen3tts/frame.hip:
* `splitmix64`            - frame.hip:581-586 (Steele/Vigna SplitMix64 finalizer);
* `pcg32_next`            - frame.hip:169-175 (O'Neill 2014 PCG-XSH-RR 64/32, fixed increment);
* `draw_uniform`          - frame.hip:284-286 (state = seed*phi + c + 1, 3 discards, top 24 bits);
* `frame_seeds`, `cp_pos_seed` - frame.hip:658-659 and 497.
"""
M64 = (1 << 64) - 1

PCG_MULT = 6364136223846793005
PCG_INC = 1442695040888963407


def splitmix64(x: int) -> int:
    x = (x + 0x9E3779B97F4A7C15) & M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def pcg32_output(old: int) -> int:
    xs = (((old >> 18) ^ old) >> 27) & 0xFFFFFFFF
    rot = old >> 59
    return ((xs >> rot) | (xs << ((-rot) & 31))) & 0xFFFFFFFF


def pcg32_next(state: int, inc: int = PCG_INC) -> tuple[int, int]:
    """(output, new_state): output from the old state, LCG advance."""
    return pcg32_output(state), (state * PCG_MULT + inc) & M64


def draw_uniform(seed: int) -> float:
    """The u in [0, 1) the draw compares against (exactly representable in f32)."""
    st = (seed * 0x9E3779B97F4A7C15 + 0xBF58476D1CE4E5B9 + 1) & M64
    for _ in range(3):
        _, st = pcg32_next(st)
    out, _ = pcg32_next(st)
    return (out >> 8) * (1.0 / 16777216.0)


def frame_seeds(seed: int, frame_index: int) -> tuple[int, int]:
    talker = splitmix64(seed ^ ((frame_index * 0xA24BAED4963EE407) & M64))
    cp = splitmix64(talker ^ 0x9FB21C651E98DF25)
    return talker, cp


def cp_pos_seed(cp_seed: int, pos: int) -> int:
    return (cp_seed + pos * 0xD1B54A32D192ED03) & M64
