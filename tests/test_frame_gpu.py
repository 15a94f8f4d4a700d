"""Frame parity on the GPU: the gfx950 frame kernel vs the CPU oracle.

Mirrors the reference's frame gate (tests/test_frame.cpp:20-130): greedy frames
code-for-code, sampled determinism (same seed identical, other seed differs) and
a forced wait timeout that fails cleanly with a working frame afterwards. Parity
bar (north star): greedy codes bit-exact; talker hidden/logits and cp logits
within 2e-2 max abs and cosine > 0.9995; the next-step embedding bit-exact.
"""
import numpy as np
import pytest

from gpu_util import compare, device_from_oracle_prefill, log, top2_margin

pytestmark = pytest.mark.gpu

TOL_ABS, TOL_COS = 2e-2, 0.9995


def prompt_ids(n_text, seed, kv):
    rng = np.random.default_rng(seed)
    text = rng.integers(0, 151643, size=n_text).tolist()
    head = [kv["text.im_start_id"], kv["text.assistant_id"], 198]
    tail = [kv["text.im_end_id"], 198, kv["text.im_start_id"], kv["text.assistant_id"], 198]
    return head + text + tail


class Session:
    """Oracle prefill mirrored onto the device; frames run on both sides."""

    def __init__(self, path, n_text=32, seed=0, max_pos=512):
        from navi_amd import abi
        from oracle.model import Oracle
        self.abi = abi
        self.ora = Oracle(path)
        kv = self.ora.kv
        ids = prompt_ids(n_text, seed, kv)
        spk = np.random.default_rng(seed).standard_normal(1024).astype(np.float32)
        self.pre, self.trail, self.pad = self.ora.build_prompt(ids, "english", spk)
        self.kv_o = self.ora.new_kv(max_pos)
        self.hidden, self.logits = self.ora.prefill(self.pre, self.kv_o)
        self.n_prefill = self.pre.shape[0]
        abi.device_open()
        self.W = abi.DeviceWeights(path, select=lambda t: t.name.startswith("talker."))
        self.frame = abi.Frame(self.W)
        self.kv = abi.KvCache(self.ora.tp.n_layer, max_pos, 1024)
        device_from_oracle_prefill(self.ora, self.kv_o, self.n_prefill, self.kv)
        self.d_hidden = abi.DeviceBuffer(4 * 1024)
        self.d_hidden.upload(self.hidden)
        self.d_logits = abi.DeviceBuffer(4 * self.logits.size)
        self.d_logits.upload(self.logits)
        rows = np.concatenate([self.trail, self.pad[None]], 0).astype(np.float32)
        self.d_trail = abi.DeviceBuffer(rows.nbytes)
        self.d_trail.upload(rows)
        self.n_trail = self.trail.shape[0]

    def trailing(self, i):
        return self.d_trail.ptr + 4 * 1024 * min(i, self.n_trail)

    def trailing_host(self, i):
        return self.trail[i] if i < self.n_trail else self.pad

    def gpu_frame(self, i, s, seed):
        if i == 0:
            return self.frame.run_first(self.d_hidden.ptr, self.d_logits.ptr, self.trailing(0), s, seed, 0)
        return self.frame.run(self.kv, self.n_prefill + i - 1, self.trailing(i), s, seed, i)


@pytest.fixture(scope="module")
def sess(small_blob):
    return Session(small_blob)


def test_greedy_frames_match_oracle(sess):
    from oracle import sampler as osamp
    n = 6
    s_gpu = sess.abi.Sampling.greedy(min_frames=n)
    s_ora = osamp.Sampling(temperature=0.0, top_k=50, repetition_penalty=1.05, cp_temperature=0.0, cp_top_k=50, min_frames=n)
    sess.frame.reset()
    sess.ora.reset()
    sess.frame.set_taps(True)
    step = None
    for i in range(n):
        log(f"greedy frame {i}")
        r = sess.gpu_frame(i, s_gpu, 0)
        assert r.ok, r.error
        dbg = {}
        if i == 0:
            codes, step_o = sess.ora.frame(s_ora, 0, 0, sess.trailing_host(0), hidden=sess.hidden, logits=sess.logits, debug=dbg)
        else:
            codes, step_o = sess.ora.frame(s_ora, 0, i, sess.trailing_host(i), kv=sess.kv_o, n_past=sess.n_prefill + i - 1,
                                           step_in=step, debug=dbg)
        step = step_o
        hid, lg, cpl = sess.frame.taps()
        if i > 0:
            e_h, c_h = compare(hid, dbg["hidden"])
            e_l, c_l = compare(lg, dbg["logits"])
            log(f"  hidden max|d| {e_h:.2e} cos {c_h:.7f}; logits max|d| {e_l:.2e} cos {c_l:.7f}")
            assert e_h < TOL_ABS and c_h > TOL_COS
            assert e_l < TOL_ABS and c_l > TOL_COS
        for p in range(15):
            e, c = compare(cpl[p], dbg["cp_logits"][p])
            assert e < TOL_ABS and c > TOL_COS, (i, p, e, c)
        margins = [top2_margin(dbg["cp_logits"][p]) for p in range(15)]
        log(f"  gpu {list(r.codes)}\n  ora {codes}  min cp top-2 margin {min(margins):.2e}")
        assert list(r.codes) == codes, f"frame {i}: codes differ"
        np.testing.assert_array_equal(sess.frame.step_out(), step_o)


def test_sampled_determinism(sess):
    s = sess.abi.Sampling.make(min_frames=8)

    def run(seed, n=8):
        sess.frame.reset()
        out = []
        for i in range(n):
            r = sess.gpu_frame(i, s, seed)
            assert r.ok, r.error
            out.append(list(r.codes))
        return out

    a, b, c = run(2), run(2), run(3)
    log(f"seed 2: {a[0]} ... seed 3: {c[0]} ...")
    assert a == b, "same seed must be bit-identical run to run"
    assert a != c, "a different seed must differ"


def test_sampler_matches_oracle_on_device_logits(sess):
    """Given the device's own logits (taps), the device sampler chooses what the
    oracle's restatement of tl_sample / cp_sample chooses (frame.hip:421-500)."""
    from oracle import rng, sampler as osamp
    s_gpu = sess.abi.Sampling.make(min_frames=2)
    s_ora = osamp.Sampling(min_frames=2)
    sess.frame.reset()
    sess.frame.set_taps(True)
    seen = np.zeros(3072, bool)
    seed = 7
    for i in range(6):
        r = sess.gpu_frame(i, s_gpu, seed)
        assert r.ok, r.error
        _, lg, cpl = sess.frame.taps()
        tseed, cseed = rng.frame_seeds(seed, i)
        cb0 = osamp.sample_talker(lg, seen, s_ora, tseed, i, 2050, 2048)
        cps = [osamp.sample_cp(cpl[p - 1], s_ora, cseed, p) for p in range(1, 16)]
        log(f"frame {i}: gpu {list(r.codes)} oracle {[cb0] + cps}")
        assert r.codes[0] == cb0
        assert list(r.codes[1:]) == cps
        if cb0 != 2050:
            seen[cb0] = True


def edge_logits():
    """Codebook-0 logits shaped to reach the sampler's corner cases (indices >= 2048 other than
    EOS are suppressed, and EOS is gated at frame 0, so only the first 2048 entries count):
    (name, logits, temperature, top_k)."""
    rng = np.random.default_rng(5)
    V, A = 3072, 2048
    out = []
    base = np.clip(rng.normal(0.0, 1.0, V), -6.0, 3.5).astype(np.float32)
    ties = base.copy()                      # 20 above, 100 tied at the top-50 threshold
    idx = rng.choice(A, 120, replace=False)
    ties[idx[:20]] = rng.uniform(5.0, 6.0, 20)
    ties[idx[20:]] = 4.0
    out.append(("ties", ties, 0.9, 50))
    out.append(("ties-greedy", ties, 0.0, 50))
    narrow = (1.0 + 1e-4 * rng.random(V)).astype(np.float32)    # one top byte, deep radix passes
    out.append(("narrow", narrow, 0.9, 50))
    zeros = -rng.uniform(0.5, 4.0, V).astype(np.float32)         # threshold at 0 with +0 and -0 tied
    idx = rng.choice(A, 110, replace=False)
    zeros[idx[:30]] = rng.uniform(1.0, 3.0, 30)
    zeros[idx[30:70]] = 0.0
    zeros[idx[70:]] = -0.0
    out.append(("zeros", zeros, 0.9, 50))
    tiny = -rng.uniform(0.5, 4.0, V).astype(np.float32)          # k-th value in the bin that starts at +0
    idx = rng.choice(A, 110, replace=False)
    tiny[idx[:49]] = rng.uniform(1.0, 3.0, 49)
    tiny[idx[49]] = np.float32(1.5e-38)
    tiny[idx[50:]] = -0.0
    out.append(("tiny", tiny, 1.0, 50))
    wide = (rng.normal(0.0, 40.0, V)).astype(np.float32)
    out.append(("wide", wide, 0.9, 50))
    out.append(("k-beyond-finite", base, 0.9, 3000))   # k-th largest is -inf: all finite values survive
    out.append(("k1", base, 0.9, 1))
    out.append(("k0", base, 0.9, 0))
    out.append(("kV", base, 0.9, V))
    return out


def test_sampler_edge_cases_match_oracle(sess):
    """Codebook-0 sampling of crafted logits (frame 0 takes them as the prefill's output) picks
    what the oracle's sample_talker picks: threshold ties, one shared top byte, +0/-0 at the
    threshold, a threshold bin that starts at +0 with -0 below it, top_k past the finite values,
    top_k 1, 0 and V."""
    from oracle import rng, sampler as osamp
    d_lg = sess.abi.DeviceBuffer(4 * 3072)
    for name, lg, temp, k in edge_logits():
        d_lg.upload(np.ascontiguousarray(lg, dtype=np.float32))
        for seed in (1, 2, 3):
            s_gpu = sess.abi.Sampling.make(temperature=temp, top_k=k)
            s_ora = osamp.Sampling(temperature=temp, top_k=k)
            sess.frame.reset()
            r = sess.frame.run_first(sess.d_hidden.ptr, d_lg.ptr, sess.trailing(0), s_gpu, seed, 0)
            assert r.ok, r.error
            tseed, _ = rng.frame_seeds(seed, 0)
            want = osamp.sample_talker(lg, np.zeros(3072, bool), s_ora, tseed, 0, 2050, 2048)
            log(f"{name} T {temp} k {k} seed {seed}: gpu {r.codes[0]} oracle {want}")
            assert r.codes[0] == want, name


def test_timeout_fails_cleanly_then_recovers(sess):
    """frame.h:33-36 spin cap: a cap of 1 fails the frame with 'timed out' (test_frame.cpp:99-119)."""
    import time
    tight = sess.abi.Frame(sess.W, spin_cap=1)
    s = sess.abi.Sampling.greedy()
    t0 = time.time()
    r = tight.run_first(sess.d_hidden.ptr, sess.d_logits.ptr, sess.trailing(0), s, 0, 0)
    ms = (time.time() - t0) * 1e3
    log(f"spin cap 1: ok={r.ok} status={r.status} '{r.error.decode()}' in {ms:.1f} ms")
    assert not r.ok and r.status == sess.abi.NAVI_ERR_TIMEOUT and b"timed out" in r.error and ms < 2000
    tight.close()
    sess.frame.reset()
    r = sess.gpu_frame(0, s, 0)
    assert r.ok, r.error


def test_timeout_stamp_does_not_survive_the_epoch_wrap(sess):
    """Nothing is latched (frame.hip:78-99): a timed-out launch stamps its epoch into the abort word;
    epochs repeat after 2^20 launches, so the wrap clears that word (and the mailboxes). Here the
    epoch is moved to just below the wrap, one launch times out (spin cap 1) at the last epoch
    before it, frames then run across the wrap, and a launch that reuses the timed-out epoch, and a
    frame loop that wraps midway, must both succeed with the codes of an undisturbed frame."""
    last = (1 << 32) - 4096
    s = sess.abi.Sampling.greedy(min_frames=8)
    fr = sess.abi.Frame(sess.W)
    fr.reset()
    want = list(fr.run_first(sess.d_hidden.ptr, sess.d_logits.ptr, sess.trailing(0), s, 0, 0).codes)
    fr.set_epoch(last - 4096)
    fr.set_spin_cap(1)
    r = fr.run_first(sess.d_hidden.ptr, sess.d_logits.ptr, sess.trailing(0), s, 0, 0)
    log(f"timeout at epoch {fr.epoch:#x}: ok={r.ok} '{r.error.decode()}'")
    assert not r.ok and r.status == sess.abi.NAVI_ERR_TIMEOUT and fr.epoch == last
    fr.set_spin_cap(0)
    for k in range(3):                                    # across the wrap: epochs 4096, 8192, ...
        fr.reset()
        r = fr.run_first(sess.d_hidden.ptr, sess.d_logits.ptr, sess.trailing(0), s, 0, 0)
        assert r.ok, (k, fr.epoch, r.error)
        assert list(r.codes) == want
    assert fr.epoch == 3 * 4096
    fr.set_epoch(last - 4096)                            # the next launch reuses the timed-out epoch
    fr.reset()
    r = fr.run_first(sess.d_hidden.ptr, sess.d_logits.ptr, sess.trailing(0), s, 0, 0)
    assert r.ok and fr.epoch == last, r.error
    assert list(r.codes) == want
    fr.set_epoch(last - 2 * 4096)                        # a loop of 4 frames that wraps after its second
    fr.reset()
    pad = sess.d_trail.ptr + 4 * 1024 * sess.n_trail
    codes, eos, _ = fr.run_many(sess.kv, sess.n_prefill - 1, sess.d_trail.ptr, sess.n_trail, pad, s, 0, 0, 4,
                                skip_first=True, d_hidden=sess.d_hidden.ptr, d_logits=sess.d_logits.ptr)
    assert codes.shape == (4, 16) and fr.epoch == 2 * 4096
    sess.frame.reset()
    single = [list(sess.gpu_frame(i, s, 0).codes) for i in range(4)]
    assert [list(c) for c in codes] == single
    fr.close()


def test_kv_full_is_an_error(sess):
    s = sess.abi.Sampling.greedy()
    r = sess.frame.run(sess.kv, sess.kv.max_pos, sess.trailing(0), s, 0, 1)
    assert not r.ok and r.status == sess.abi.NAVI_ERR_KV_FULL and b"KV cache full" in r.error


def test_frame_loop_matches_single_frames(sess):
    """navi_frame_run_many: the frames of an on-device loop are the frames navi_frame_run gives
    one call at a time (same kernel, same inputs, same seeds: bit-identical codes)."""
    s = sess.abi.Sampling.make(min_frames=12)
    n = 12
    sess.frame.reset()
    single = []
    for i in range(n):
        r = sess.gpu_frame(i, s, 5)
        assert r.ok, r.error
        single.append(list(r.codes))
    step_single = sess.frame.step_out()
    sess.frame.reset()
    pad = sess.d_trail.ptr + 4 * 1024 * sess.n_trail
    codes, eos, us = sess.frame.run_many(sess.kv, sess.n_prefill - 1, sess.d_trail.ptr, sess.n_trail, pad, s, 5, 0, n,
                                         skip_first=True, d_hidden=sess.d_hidden.ptr, d_logits=sess.d_logits.ptr)
    log(f"loop of {n} frames: {us / n:.1f} us/frame device, eos={eos}")
    assert not eos and codes.shape == (n, 16)
    assert [list(c) for c in codes] == single
    np.testing.assert_array_equal(sess.frame.step_out(), step_single)


def test_frame_loop_matches_oracle_greedy(sess):
    """navi_frame_run_many against the oracle directly (not only against single device frames):
    8 greedy frames from the prefill, run as one on-device loop, give the oracle's codes frame for
    frame, and the last step embedding is the oracle's bit for bit."""
    import torch
    from oracle import sampler as osamp
    n = 8
    s = sess.abi.Sampling.greedy(min_frames=n)
    so = osamp.Sampling(temperature=0.0, cp_temperature=0.0, repetition_penalty=1.05, min_frames=n)
    sess.frame.reset()
    pad = sess.d_trail.ptr + 4 * 1024 * sess.n_trail
    codes, eos, _ = sess.frame.run_many(sess.kv, sess.n_prefill - 1, sess.d_trail.ptr, sess.n_trail, pad, s, 4, 0, n,
                                        skip_first=True, d_hidden=sess.d_hidden.ptr, d_logits=sess.d_logits.ptr)
    assert not eos and codes.shape == (n, 16)
    kvo = [(k.clone(), v.clone()) for k, v in sess.kv_o]
    sess.ora.reset()
    want, step = [], None
    with torch.no_grad():
        for i in range(n):
            if i == 0:
                c, step = sess.ora.frame(so, 4, 0, sess.trailing_host(0), hidden=sess.hidden, logits=sess.logits)
            else:
                c, step = sess.ora.frame(so, 4, i, sess.trailing_host(i), kv=kvo, n_past=sess.n_prefill + i - 1,
                                         step_in=step)
            want.append(c)
    log(f"loop vs oracle: {n} frames, first {want[0][:4]}, last {want[-1][:4]}")
    assert [list(c) for c in codes] == want
    np.testing.assert_array_equal(sess.frame.step_out(), step)


def test_frame_loop_stops_at_eos(sess):
    """A frame that samples EOS ends the loop on the device; it is the last row returned."""
    s = sess.abi.Sampling.greedy(min_frames=0)
    lg = sess.logits.copy()
    lg[2050] = 1e4                                     # EOS wins the greedy pick of frame 0
    d_lg = sess.abi.DeviceBuffer(4 * lg.size)
    d_lg.upload(lg.astype(np.float32))
    sess.frame.reset()
    pad = sess.d_trail.ptr + 4 * 1024 * sess.n_trail
    codes, eos, _ = sess.frame.run_many(sess.kv, sess.n_prefill - 1, sess.d_trail.ptr, sess.n_trail, pad, s, 0, 0, 8,
                                        skip_first=True, d_hidden=sess.d_hidden.ptr, d_logits=d_lg.ptr)
    log(f"eos loop: {len(codes)} frame(s), first code {codes[0][0] if len(codes) else None}")
    assert eos and codes.shape == (1, 16) and codes[0][0] == 2050


def test_frame_loop_timeout_is_an_error(sess):
    """A wait past its spin cap ends the loop with NAVI_ERR_TIMEOUT; the next loop runs normally."""
    tight = sess.abi.Frame(sess.W, spin_cap=1)
    s = sess.abi.Sampling.greedy(min_frames=4)
    pad = sess.d_trail.ptr + 4 * 1024 * sess.n_trail
    with pytest.raises(sess.abi.NaviError) as e:
        tight.run_many(sess.kv, sess.n_prefill - 1, sess.d_trail.ptr, sess.n_trail, pad, s, 0, 0, 4,
                       skip_first=True, d_hidden=sess.d_hidden.ptr, d_logits=sess.d_logits.ptr)
    assert e.value.status == sess.abi.NAVI_ERR_TIMEOUT and "timed out" in str(e.value)
    tight.close()
    sess.frame.reset()
    codes, eos, _ = sess.frame.run_many(sess.kv, sess.n_prefill - 1, sess.d_trail.ptr, sess.n_trail, pad, s, 0, 0, 4,
                                        skip_first=True, d_hidden=sess.d_hidden.ptr, d_logits=sess.d_logits.ptr)
    assert codes.shape == (4, 16)


@pytest.mark.parametrize("n_past", [700, 2500])
def test_long_context_frames_match_oracle(small_blob, n_past):
    """Talker attention over long cached contexts on random f16 K/V rows: 44 and 157 keys per
    key range (several score passes per wave, several value groups per wave). Two greedy frames,
    teacher-forced: talker hidden/logits and cp logits within tolerance, codes through the greedy
    gate (gpu_util.check_greedy_frame), the next step input bit-exact."""
    import torch
    from navi_amd import abi
    from oracle import sampler as osamp
    from oracle.model import Oracle
    from gpu_util import check_greedy_frame, summarize_decisions
    ora = Oracle(small_blob)
    abi.device_open()
    W = abi.DeviceWeights(small_blob, select=lambda t: t.name.startswith("talker."))
    fr = abi.Frame(W)
    max_pos = n_past + 4
    L = ora.tp.n_layer
    kv_o = ora.new_kv(max_pos)
    kv_d = abi.KvCache(L, max_pos, 1024)
    rng = np.random.default_rng(n_past)
    for l in range(L):
        k = rng.standard_normal((n_past, 1024)).astype(np.float16)
        v = rng.standard_normal((n_past, 1024)).astype(np.float16)
        kv_o[l][0][:n_past] = torch.from_numpy(k.astype(np.float32))
        kv_o[l][1][:n_past] = torch.from_numpy(v.astype(np.float32))
        kv_d.fill(l, k, v, 0)
    step = rng.standard_normal(1024).astype(np.float32)
    trail = rng.standard_normal(1024).astype(np.float32)
    d_trail = abi.DeviceBuffer(trail.nbytes)
    d_trail.upload(trail)
    abi.upload(fr.d_step_out, step)
    s_gpu = abi.Sampling.greedy(min_frames=4)
    s_ora = osamp.Sampling(temperature=0.0, top_k=50, repetition_penalty=1.05, cp_temperature=0.0, cp_top_k=50,
                           min_frames=4)
    fr.reset()
    fr.set_taps(True)
    ora.reset()
    record = []
    for f in range(2):
        r = fr.run(kv_d, n_past + f, d_trail.ptr, s_gpu, 9, f)
        assert r.ok, r.error
        hid, lg, cpl = fr.taps()
        dbg = {}
        codes = list(r.codes)
        _, step = ora.frame(s_ora, 9, f, trail, kv=kv_o, n_past=n_past + f, step_in=step, debug=dbg, force=codes)
        e_h, c_h = compare(hid, dbg["hidden"])
        e_l, c_l = compare(lg, dbg["logits"])
        e_c = max(compare(cpl[p], dbg["cp_logits"][p])[0] for p in range(15))
        c_c = min(compare(cpl[p], dbg["cp_logits"][p])[1] for p in range(15))
        log(f"n_past {n_past + f}: hidden {e_h:.2e}/{c_h:.7f} logits {e_l:.2e}/{c_l:.7f} cp {e_c:.2e}/{c_c:.7f} codes {codes}")
        assert e_h < TOL_ABS and c_h > TOL_COS
        assert e_l < TOL_ABS and c_l > TOL_COS
        assert e_c < TOL_ABS and c_c > TOL_COS
        check_greedy_frame(f, codes, dbg, record, lg, cpl)
        np.testing.assert_array_equal(abi.download(fr.d_step_out, np.float32, 1024), step)
    summarize_decisions(f"frame_long_context_{n_past}", record, max_flips=1)
    fr.close()
