"""Pins the oracle's sampler (oracle/sampler.py).

* kth_largest: the Python sort, the C restatement of the reference's 4-pass radix select and
  the definition (count of larger entries < k <= count of entries >= t) agree, with ties, -inf
  and signed zeros;
* fma_f32 (the draw's fused running sum) against C fmaf;
* draw: Python against C on random candidate sets, one-hot and hand-worked cases, and the
  empirical distribution against the softmax weights;
* modified logits: suppression range, EOS gate, repetition penalty sign rule (special cases
  written out by hand);
* greedy: lowest index on ties.
"""
import numpy as np
import pytest

from oracle import csampler, rng, sampler

F32 = np.float32


def _kth_by_definition(xs, k):
    vals = np.unique(xs)[::-1]
    for t in vals:
        if np.sum(xs > t) < k <= np.sum(xs >= t):
            return t
    raise AssertionError("no threshold")


def _cases():
    r = np.random.default_rng(11)
    for V in (2048, 3072):
        x = r.standard_normal(V).astype(F32) * 3
        yield x, [1, 2, 50, V // 2, V]
        t = np.round(x).astype(F32)                         # heavy ties
        yield t, [1, 7, 50, 51, V - 1, V]
        m = x.copy()
        m[r.integers(0, V, V // 3)] = -np.inf                # suppressed entries
        m[5] = 0.0
        m[6] = -0.0
        yield m, [1, 50, V // 2, V]
    yield np.zeros(64, F32), [1, 64]
    yield np.full(64, -np.inf, F32), [1, 64]


@pytest.mark.parametrize("case", list(range(8)))
def test_kth_largest_three_ways(case):
    xs, ks = list(_cases())[case]
    for k in ks:
        want = _kth_by_definition(xs, k)
        assert sampler.kth_largest(xs, k) == want
        assert F32(csampler.kth_largest(xs, k)) == want


def test_fma_matches_c_fmaf():
    r = np.random.default_rng(3)
    a = r.random(3000).astype(F32)
    b = (r.random(3000) * 1e-3).astype(F32)
    c = np.cumsum(r.random(3000)).astype(F32) / F32(3000)
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.fmaf.argtypes = [ctypes.c_float] * 3
    libm.fmaf.restype = ctypes.c_float
    diff_from_unfused = 0
    for x, y, z in zip(a, b, c):
        got = sampler.fma_f32(x, y, z)
        assert got == F32(libm.fmaf(float(x), float(y), float(z)))
        diff_from_unfused += got != F32(F32(x * y) + z)
    assert diff_from_unfused > 0   # the fused and unfused sums really differ on these inputs


def test_draw_python_matches_c():
    r = np.random.default_rng(4)
    for trial in range(300):
        V = int(r.choice([16, 2048, 3072]))
        xs = (r.standard_normal(V) * 2).astype(F32)
        e, inv, _ = sampler.softmax_weights(xs, int(r.choice([1, 5, 50, V])))
        seed = int(r.integers(0, 2 ** 63))
        assert sampler.draw(e, inv, seed)[0] == csampler.draw(e, inv, seed)


def test_draw_hand_cases():
    e = np.zeros(100, F32)
    e[42] = 1.0
    for s in range(20):
        assert sampler.draw(e, F32(1.0), s)[0] == 42
    # all mass on nonzero entries but a total below u: falls through to V-1
    e = np.zeros(10, F32)
    e[3] = 1e-9
    assert sampler.draw(e, F32(1.0), 1)[0] == (3 if rng.draw_uniform(1) <= 1e-9 else 9)
    # two equal halves: index 0 exactly when u <= 0.5
    e = np.zeros(8, F32)
    e[[2, 5]] = 1.0
    for s in range(50):
        want = 2 if rng.draw_uniform(s) <= 0.5 else 5
        assert sampler.draw(e, F32(0.5), s)[0] == want


def test_draw_distribution_follows_softmax():
    xs = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -3.0], F32)
    e, inv, _ = sampler.softmax_weights(xs, 0)
    p = e.astype(np.float64) * float(inv)
    n = 20000
    counts = np.bincount([sampler.draw(e, inv, s)[0] for s in range(n)], minlength=6)
    chi2 = np.sum((counts - n * p) ** 2 / (n * p))
    assert chi2 < 30, (counts, n * p)   # 5 degrees of freedom; p ~ 1e-5 at 30


def test_softmax_weights_topk_keeps_ties():
    xs = np.array([3, 1, 3, 2, 3, 0], F32)
    e, inv, thr = sampler.softmax_weights(xs, 2)
    assert thr == 3 and np.count_nonzero(e) == 3          # v >= k-th largest keeps every tie
    assert np.all(e[[0, 2, 4]] == 1.0)
    assert inv == F32(1.0) / F32(3.0)


def test_modified_logits_special_cases():
    V, eos, sup = 3072, 2050, 2048
    lg = np.full(V, 2.0, F32)
    lg[10], lg[11] = -2.0, 0.0
    seen = np.zeros(V, bool)
    seen[[10, 11, 12, eos, 3000]] = True
    v = sampler.talker_modified_logits(lg, seen, eos, sup, frame_index=0, min_frames=2, repetition_penalty=1.05)
    assert np.all(np.isneginf(v[sup:]))                    # control range suppressed, EOS too before min_frames
    assert v[10] == F32(-2.0) * F32(1.05)                  # negative: multiplied
    assert v[11] == F32(0.0) * F32(1.05)                   # zero is "not > 0": multiplied
    assert v[12] == F32(2.0) / F32(1.05)                   # positive: divided
    assert v[13] == 2.0                                    # unseen untouched
    v = sampler.talker_modified_logits(lg, seen, eos, sup, frame_index=2, min_frames=2, repetition_penalty=1.05)
    assert v[eos] == F32(2.0) / F32(1.05)                  # allowed from frame min_frames on, penalised if seen
    assert np.isneginf(v[sup]) and np.isneginf(v[eos + 1])
    v = sampler.talker_modified_logits(lg, seen, eos, sup, frame_index=5, min_frames=2, repetition_penalty=0.0)
    assert v[12] == 2.0 and v[eos] == 2.0                  # penalty <= 0: off


def test_greedy_lowest_index_on_ties():
    v = np.array([1, 5, 2, 5, 5], F32)
    assert sampler.greedy(v) == 1 == csampler.argmax(v)
    v = np.full(7, -np.inf, F32)
    assert sampler.greedy(v) == 0 == csampler.argmax(v)


def test_sample_cp_greedy_is_argmax_of_raw_logits():
    r = np.random.default_rng(9)
    lg = r.standard_normal(2048).astype(F32)
    s = sampler.Sampling(cp_temperature=0.0)
    assert sampler.sample_cp(lg, s, 123, 4) == int(np.argmax(lg))
