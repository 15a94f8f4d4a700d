"""BASELINE configs[1] at its exact workload, the one bench.py times: the full 0.6B random-init
model (weights N(0, 0.02) seed 1), 256 cached positions of f16 K/V from N(0, 1), the step input
from N(0, 1), drawn in bench.py's order from numpy's default_rng(1); a zero trailing row.

Two frames at n_past 256 and 257 through the C ABI, compared with the oracle on the same inputs:
* greedy, teacher-forced: talker hidden/logits and cp logits within 2e-2 max abs and cosine
  > 0.9995; every decision through gpu_util.check_greedy_frame; the next step input bit-exact;
* sampled as the bench samples (top-k 50, T 0.9, rep 1.05, seed 2, frame index i): the oracle's
  sampler, given the device's own logits, picks every device code (reference: k_frame,
  frame.hip:517-579; tl_sample / cp_sample, frame.hip:413-500).
"""
import numpy as np
import pytest
import torch

from gpu_util import check_greedy_frame, compare, log, summarize_decisions

pytestmark = pytest.mark.gpu

N_PAST, SEED, TOL_ABS, TOL_COS = 256, 1, 2e-2, 0.9995


@pytest.fixture(scope="module")
def w1(scratch_dir):
    from navi_amd import blob
    path = scratch_dir / "full_seed1.navi"
    if not path.exists():
        blob.write_random_blob(path, SEED, parts=("talker", "cp"))
    yield path
    path.unlink()


class Config1:
    def __init__(self, path):
        from navi_amd import abi
        from oracle.model import Oracle
        self.abi = abi
        self.ora = Oracle(path)
        abi.device_open()
        self.W = abi.DeviceWeights(path, select=lambda t: t.name.startswith("talker."))
        self.frame = abi.Frame(self.W)
        L = self.ora.tp.n_layer
        self.kv = abi.KvCache(L, 300, 1024)
        self.kv_o = self.ora.new_kv(300)
        rng = np.random.default_rng(SEED)                     # bench.py's draw order
        for l in range(L):
            k = rng.standard_normal((N_PAST, 1024)).astype(np.float16)
            v = rng.standard_normal((N_PAST, 1024)).astype(np.float16)
            self.kv.fill(l, k, v)
            self.kv_o[l][0][:N_PAST] = torch.from_numpy(k.astype(np.float32))
            self.kv_o[l][1][:N_PAST] = torch.from_numpy(v.astype(np.float32))
        self.step = rng.standard_normal(1024).astype(np.float32)
        self.trail = np.zeros(1024, np.float32)
        self.d_trail = abi.DeviceBuffer(4 * 1024)
        self.d_trail.upload(self.trail)


@pytest.fixture(scope="module")
def c1(w1):
    return Config1(w1)


def test_config1_greedy_frames_match_oracle(c1):
    from oracle import sampler as osamp
    abi = c1.abi
    s = abi.Sampling.greedy(min_frames=10 ** 6)
    so = osamp.Sampling(temperature=0.0, cp_temperature=0.0, repetition_penalty=1.05, min_frames=10 ** 6)
    c1.frame.reset()
    c1.frame.set_taps(True)
    c1.ora.reset()
    abi.upload(c1.frame.d_step_out, c1.step)
    step = c1.step
    record = []
    for f in range(2):
        r = c1.frame.run(c1.kv, N_PAST + f, c1.d_trail.ptr, s, 2, f)
        assert r.ok, r.error
        codes = list(r.codes)
        hid, lg, cpl = c1.frame.taps()
        dbg = {}
        _, step = c1.ora.frame(so, 2, f, c1.trail, kv=c1.kv_o, n_past=N_PAST + f, step_in=step, debug=dbg, force=codes)
        e_h, c_h = compare(hid, dbg["hidden"])
        e_l, c_l = compare(lg, dbg["logits"])
        e_c = max(compare(cpl[p], dbg["cp_logits"][p])[0] for p in range(15))
        c_c = min(compare(cpl[p], dbg["cp_logits"][p])[1] for p in range(15))
        log(f"configs[1] frame at n_past {N_PAST + f}: hidden {e_h:.2e}/{c_h:.7f} logits {e_l:.2e}/{c_l:.7f} "
            f"cp {e_c:.2e}/{c_c:.7f}; codes {codes}; {r.us:.0f} us")
        assert e_h < TOL_ABS and c_h > TOL_COS
        assert e_l < TOL_ABS and c_l > TOL_COS
        assert e_c < TOL_ABS and c_c > TOL_COS
        check_greedy_frame(f, codes, dbg, record, lg, cpl)
        np.testing.assert_array_equal(c1.frame.step_out(), step)
    summarize_decisions("config1_greedy_2_frames", record)


def test_config1_sampled_frames_match_oracle_on_device_logits(c1):
    from oracle import rng, sampler as osamp
    abi = c1.abi
    s = abi.Sampling.make(min_frames=10 ** 6)
    so = osamp.Sampling(min_frames=10 ** 6)
    c1.frame.reset()
    c1.frame.set_taps(True)
    abi.upload(c1.frame.d_step_out, c1.step)
    seen = np.zeros(3072, bool)
    for f in range(2):
        r = c1.frame.run(c1.kv, N_PAST + f, c1.d_trail.ptr, s, 2, f)
        assert r.ok, r.error
        _, lg, cpl = c1.frame.taps()
        tseed, cseed = rng.frame_seeds(2, f)
        cb0 = osamp.sample_talker(lg, seen, so, tseed, f, 2050, 2048)
        cps = [osamp.sample_cp(cpl[p - 1], so, cseed, p) for p in range(1, 16)]
        log(f"configs[1] sampled frame {f}: gpu {list(r.codes)} oracle sampler {[cb0] + cps}")
        assert [cb0] + cps == list(r.codes)
        if cb0 != 2050:
            seen[cb0] = True
