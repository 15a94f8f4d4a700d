"""Prompt rows, prefill and the linear layer on the GPU vs the CPU oracle (through the C ABI).

* navi_linear (split-f16 MFMA GEMM) against numpy in f64 over shapes that exercise 1-4 row
  tiles, partial K steps and split-K, with bias, SiLU and residual; an activation outside the
  f16 range is an error, not an infinity;
* build_prompt against Oracle.build_prompt (the reference's layout, talker.hip:283-352);
* prefill against Oracle.prefill at T = 1, T = 10 (the reference's layout), T = 32 and 48 (the
  2- and 3-tile single-group row projections), T = 65, T = 130 (BASELINE's streaming
  configuration), T = 256, 257 and 264 (the most a 256-token handle takes; above 256 rows the
  attention walks 256-key chunks), and on a handle sized as the reference's (max_prompt_tokens
  1024, talker.h:37; MAX_KEYS 1024, talker.hip:86) at T = 300, 512, 513, 1024 and 1032 (its
  maximum): post-norm hidden and logits within 2e-2 max abs and cosine > 0.9995
  (the north star's bar), K/V cache rows within a few f16 ulps;
* device prompt + device prefill + device frames == oracle codes (greedy).
"""
import numpy as np
import pytest

from gpu_util import compare, log, top2_margin

pytestmark = pytest.mark.gpu

TOL_ABS, TOL_COS = 2e-2, 0.9995


@pytest.fixture(scope="module")
def abi():
    from navi_amd import abi as a
    a.device_open()
    return a


def _f16(rng, shape, sigma):
    return (rng.standard_normal(shape) * sigma).astype(np.float16)


@pytest.mark.parametrize("M,K,N,act,bias,resid", [
    (1, 1024, 3072, 0, False, False),
    (7, 1024, 1024, 1, True, False),
    (16, 2048, 1024, 0, False, True),
    (33, 3072, 1024, 0, True, True),
    (64, 1024, 4096, 1, False, False),
    (130, 2048, 2048, 0, True, False),
    (200, 1024, 64, 0, False, True),
])
def test_linear_matches_numpy(abi, M, K, N, act, bias, resid):
    rng = np.random.default_rng(M * 7 + K + N)
    x = rng.standard_normal((M, K)).astype(np.float32) * 3
    w = _f16(rng, (N, K), 0.05)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    r = rng.standard_normal((M, N)).astype(np.float32) if resid else None
    want = x.astype(np.float64) @ w.astype(np.float64).T
    if b is not None:
        want += b
    if act:
        want = want / (1 + np.exp(-want))
    if r is not None:
        want += r
    dx, dw, dy = abi.DeviceBuffer(x.nbytes), abi.DeviceBuffer(w.nbytes), abi.DeviceBuffer(4 * M * N)
    dx.upload(x)
    dw.upload(w.view(np.uint16))
    db = dr = None
    if b is not None:
        db = abi.DeviceBuffer(b.nbytes)
        db.upload(b)
    if r is not None:
        dy.upload(r)                                         # residual aliases the output
        dr = dy
    log(f"linear M={M} K={K} N={N} act={act} bias={bias} resid={resid}")
    abi.linear(dx.ptr, K, M, dw.ptr, K, N, dy.ptr, N, bias=db.ptr if db else None, residual=dr.ptr if dr else None, act=act)
    got = dy.download(np.float32, M * N).reshape(M, N)
    scale = np.abs(x).astype(np.float64) @ np.abs(w.astype(np.float64)).T
    err = np.abs(got - want) / (scale + 1.0)
    log(f"  max scaled err {err.max():.3e}")
    assert err.max() < 2e-6


def test_linear_rejects_values_outside_f16(abi):
    x = np.ones((4, 64), np.float32)
    x[2, 5] = 1e5
    w = np.ones((64, 64), np.float16)
    dx, dw, dy = abi.DeviceBuffer(x.nbytes), abi.DeviceBuffer(w.nbytes), abi.DeviceBuffer(4 * 4 * 64)
    dx.upload(x)
    dw.upload(w.view(np.uint16))
    with pytest.raises(abi.NaviError) as e:
        abi.linear(dx.ptr, 64, 4, dw.ptr, 64, 64, dy.ptr, 64)
    assert e.value.status == abi.NAVI_ERR_INVALID and "f16 range" in str(e.value)


def test_linear_rejects_bad_shapes(abi):
    d = abi.DeviceBuffer(4096)
    with pytest.raises(abi.NaviError):
        abi.linear(d.ptr, 48, 1, d.ptr, 48, 64, d.ptr, 64)   # K not a multiple of 32
    with pytest.raises(abi.NaviError):
        abi.linear(d.ptr, 64, 1, d.ptr, 64, 32, d.ptr, 32)   # N not a multiple of 64


class Side:
    def __init__(self, abi, path, max_prompt_tokens=256, max_positions=512):
        from oracle.model import Oracle
        self.ora = Oracle(path)
        self.W = abi.DeviceWeights(path, select=lambda t: t.name.startswith("talker."))
        self.talker = abi.Talker(self.W, max_prompt_tokens=max_prompt_tokens, max_positions=max_positions)
        self.frame = abi.Frame(self.W)


@pytest.fixture(scope="module")
def side(abi, small_blob):
    return Side(abi, small_blob)


def _ids(kv, n_text, seed):
    rng = np.random.default_rng(seed)
    head = [kv["text.im_start_id"], kv["text.assistant_id"], 198]
    tail = [kv["text.im_end_id"], 198, kv["text.im_start_id"], kv["text.assistant_id"], 198]
    return head + rng.integers(0, 151643, n_text).tolist() + tail


@pytest.mark.parametrize("language", ["english", "auto"])
def test_prompt_matches_oracle(side, language):
    ids = _ids(side.ora.kv, 17, 3)
    spk = np.random.default_rng(4).standard_normal(1024).astype(np.float32)
    pr = side.talker.build_prompt(ids, language, spk)
    pre, trail, pad = side.talker.prompt_arrays(pr)
    opre, otrail, opad = side.ora.build_prompt(ids, language, spk)
    log(f"prompt {language}: prefill {pre.shape} trailing {trail.shape}")
    assert pre.shape == opre.shape and trail.shape == otrail.shape
    for got, want in ((pre, opre), (trail, otrail), (pad, opad)):
        assert np.abs(got - want).max() < 1e-4


# 65: the first row count on the column-group row projections; 256: the most keys the
# short-context attention takes (every thread owns a key); 257: one key into the long-prompt
# attention's second 256-key chunk; 264: the handle's maximum (max_prompt_tokens 256 + 8)
@pytest.mark.parametrize("T", [1, 10, 32, 48, 65, 130, 256, 257, 264])
def test_prefill_matches_oracle(abi, side, T):
    _check_prefill(abi, side, T)


@pytest.fixture(scope="module")
def side_long(abi, small_blob):
    s = Side(abi, small_blob, max_prompt_tokens=1024, max_positions=2048)
    yield s
    s.talker.close()


# 300: a ragged last 16-row tile and a partial second key chunk; 513: one key into the third chunk
@pytest.mark.parametrize("T", [300, 512, 513, 1024, 1032])
def test_long_prefill_matches_oracle(abi, side_long, T):
    _check_prefill(abi, side_long, T)


def _check_prefill(abi, side, T):
    rng = np.random.default_rng(T)
    rows = rng.standard_normal((T, 1024)).astype(np.float32)
    d = abi.DeviceBuffer(rows.nbytes)
    d.upload(rows)
    log(f"prefill T={T}")
    side.talker.prefill(d.ptr, T)
    hid, lg = side.talker.hidden_logits()
    kvo = side.ora.new_kv(T + 1)
    ohid, olg = side.ora.prefill(rows, kvo)
    for name, got, want in (("hidden", hid, ohid), ("logits", lg, olg)):
        mx, cos = compare(got, want)
        log(f"  {name}: max abs {mx:.3e} cosine {cos:.7f}")
        assert mx < TOL_ABS and cos > TOL_COS
    for l in range(side.ora.tp.n_layer):
        k, v = side.talker.kv.read(l, T)
        for got, want in ((k, kvo[l][0][:T].numpy()), (v, kvo[l][1][:T].numpy())):
            assert np.allclose(got, want, rtol=4e-3, atol=2e-3)
            assert np.mean(got != want) < 0.05
    log(f"  device {side.talker.last_ms():.3f} ms")


def test_device_prompt_prefill_frames_match_oracle(abi, side):
    """The whole front end on the device: prompt rows -> prefill -> frame 0 -> talker frames."""
    from oracle import sampler as osamp
    ids = _ids(side.ora.kv, 24, 5)
    spk = np.random.default_rng(6).standard_normal(1024).astype(np.float32)
    n = 5
    pr = side.talker.build_prompt(ids, "english", spk)
    side.talker.prefill(pr.prefill, pr.n_prefill)
    opre, otrail, opad = side.ora.build_prompt(ids, "english", spk)
    kvo = side.ora.new_kv(64)
    ohid, olg = side.ora.prefill(opre, kvo)
    log(f"end to end: prefill {pr.n_prefill} rows, top-2 margin of frame-0 logits {top2_margin(olg):.4f}")
    s = abi.Sampling.greedy(min_frames=n)
    so = osamp.Sampling(temperature=0.0, cp_temperature=0.0, min_frames=n)
    side.frame.reset()
    side.ora.reset()
    step = None
    for i in range(n):
        trail_d = pr.trailing + 4 * 1024 * i if i < pr.n_trailing else pr.tts_pad
        trail_h = otrail[i] if i < otrail.shape[0] else opad
        if i == 0:
            r = side.frame.run_first(side.talker.d_hidden, side.talker.d_logits, trail_d, s, 0, 0)
            c, step = side.ora.frame(so, 0, 0, trail_h, hidden=ohid, logits=olg)
        else:
            r = side.frame.run(side.talker.kv, pr.n_prefill + i - 1, trail_d, s, 0, i)
            c, step = side.ora.frame(so, 0, i, trail_h, kv=kvo, n_past=pr.n_prefill + i - 1, step_in=step)
        assert r.ok, r.error
        log(f"  frame {i}: gpu {list(r.codes)[:6]}... oracle {c[:6]}...")
        assert list(r.codes) == c


@pytest.mark.parametrize("T", [10, 130])
def test_prefill_graph_replays_match_eager(abi, side, T):
    """Prefills replayed from the captured graph (navi_talker_set_graphs) give bit for bit the hidden, logits
    and K/V rows of prefills whose kernels the host launches one by one; three replays, each
    with an eager prefill of other rows and a synchronisation in between."""
    rng = np.random.default_rng(100 + T)
    rows = rng.standard_normal((T, 1024)).astype(np.float32)
    other = rng.standard_normal((T, 1024)).astype(np.float32)
    d, d2 = abi.DeviceBuffer(rows.nbytes), abi.DeviceBuffer(other.nbytes)
    d.upload(rows)
    d2.upload(other)

    def run(graphs, buf):
        side.talker.set_graphs(graphs)
        side.talker.prefill(buf.ptr, T)
        hid, lg = side.talker.hidden_logits()
        kv = [side.talker.kv.read(l, T) for l in range(side.ora.tp.n_layer)]
        return hid.copy(), lg.copy(), kv
    want = run(False, d)
    for rep in range(3):
        got = run(True, d)
        np.testing.assert_array_equal(got[0], want[0])
        np.testing.assert_array_equal(got[1], want[1])
        for (gk, gv), (wk, wv) in zip(got[2], want[2]):
            np.testing.assert_array_equal(gk, wk)
            np.testing.assert_array_equal(gv, wv)
        run(False, d2)                                   # eager work between the replays
    side.talker.set_graphs(False)
    log(f"prefill T={T}: 3 graph replays == eager")
