"""Pins the oracle's seeding and PCG32 stream (oracle/rng.py).

Checks: textbook known answers (SplitMix64 seeded with 0; the PCG32 reference demo
stream), agreement of the Python restatement with the independent C restatement
(oracle/csrc/sampler.c) on many seeds, and the draw's output lattice.
"""
import numpy as np
import pytest

from oracle import csampler, rng

M64 = (1 << 64) - 1


def test_splitmix64_known_answers():
    # Vigna's splitmix64.c seeded with x = 0: next() returns splitmix64 of 0, then of 0 + phi, ...
    assert rng.splitmix64(0) == 0xE220A8397B1DCDAF
    assert rng.splitmix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4
    assert rng.splitmix64((2 * 0x9E3779B97F4A7C15) & M64) == 0x06C45D188009454F


def test_pcg32_reference_demo_stream():
    # pcg32-demo (O'Neill): pcg32_srandom_r(&rng, 42u, 54u), then six pcg32_random_r outputs.
    inc = (54 << 1) | 1
    st = 0
    _, st = rng.pcg32_next(st, inc)
    st = (st + 42) & M64
    _, st = rng.pcg32_next(st, inc)
    out = []
    for _ in range(6):
        o, st = rng.pcg32_next(st, inc)
        out.append(o)
    assert out == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_pcg32_python_matches_c():
    r = np.random.default_rng(5)
    for seed in r.integers(0, 2 ** 63, 50, dtype=np.int64).tolist() + [0, M64]:
        py, st = [], seed
        for _ in range(8):
            o, st = rng.pcg32_next(st)
            py.append(o)
        assert py == csampler.pcg32_stream(seed, 8)


def test_seeding_python_matches_c():
    r = np.random.default_rng(6)
    seeds = [0, 1, 2, M64, 0xDEADBEEF] + r.integers(0, 2 ** 63, 200, dtype=np.int64).tolist()
    for s in seeds:
        assert rng.splitmix64(s) == csampler.splitmix64(s)
        assert np.float32(rng.draw_uniform(s)) == np.float32(csampler.draw_uniform(s))
        for fi in (0, 1, 2, 31, 239, 100000):
            assert rng.frame_seeds(s, fi) == csampler.frame_seeds(s, fi)
        for pos in range(1, 16):
            assert rng.cp_pos_seed(s, pos) == csampler.cp_pos_seed(s, pos)


def test_draw_uniform_lattice_and_spread():
    us = np.array([rng.draw_uniform(s) for s in range(4000)])
    assert np.all((us >= 0) & (us < 1))
    assert np.all(us * 16777216.0 == np.floor(us * 16777216.0))   # top 24 bits of a pcg32 output
    assert abs(us.mean() - 0.5) < 0.02 and abs(us.var() - 1 / 12) < 0.01


def test_frame_seeds_distinct_per_frame_and_seed():
    got = {rng.frame_seeds(s, f) for s in range(4) for f in range(64)}
    assert len(got) == 4 * 64
    t, c = rng.frame_seeds(2, 0)
    assert t == rng.splitmix64(2) and c == rng.splitmix64(t ^ 0x9FB21C651E98DF25)


@pytest.mark.parametrize("pos", [1, 2, 15])
def test_cp_pos_seed_is_affine(pos):
    base = 0x123456789ABCDEF
    assert rng.cp_pos_seed(base, pos) == (base + pos * 0xD1B54A32D192ED03) & M64
    assert rng.cp_pos_seed(base, 0) == base
