"""BASELINE configs[4] at its own size: 32 independent streams at context ~1024 (f16 N(0,1) KV),
on the 2-layer random-init model so the CPU oracle stays cheap (the kernels, tiles and launch
shapes depend on the stream count and the context, not on the layer count).

This reaches what the 5-stream test does not: the projections at M = 32 rows (talker, cp positions
2..15) and M = 64 rows (cp positions 0 and 1 as one pass), the split-KV talker attention over
four 256-key ranges and its combine, and the sampler over 32 blocks. Stream i must compute the
batch-1 frame (k_frame, frame.hip:517-579) of the oracle for itself:
* greedy, two steps, teacher-forced: every decision through gpu_util.check_greedy_frame; talker
  hidden/logits and cp logits within 2e-2 max abs and cosine > 0.9995; next step input bit-exact;
* sampled (top-k 50, T 0.9, rep 1.05, seeds 0..31 as in configs[4]): the oracle's sampler, given
  the device's logits, picks every device code.
"""
import numpy as np
import pytest

from gpu_util import check_greedy_frame, compare, log, summarize_decisions
from test_streams_gpu import Batch, TOL_ABS, TOL_COS

pytestmark = pytest.mark.gpu

N = 32
MAX_POS = 1040


@pytest.fixture(scope="module")
def batch32(small_blob):
    b = Batch(small_blob, [1024 - (i % 4) for i in range(N)], seed=4, max_pos=MAX_POS, max_streams=N)
    b.seeds = list(range(N))
    return b


def test_greedy_32_streams_at_context_1024(batch32):
    from oracle import sampler as osamp
    b = batch32
    steps = 2
    s_gpu = b.abi.Sampling.greedy(min_frames=steps)
    s_ora = osamp.Sampling(temperature=0.0, top_k=50, repetition_penalty=1.05, cp_temperature=0.0, cp_top_k=50,
                           min_frames=steps)
    b.st.reset()
    b.st.set_taps(True)
    step_o = [b.step[i].copy() for i in range(N)]
    seen = [np.zeros(b.ora.tp.vocab, bool) for _ in range(N)]
    n_past = list(b.n_past)
    record = []
    for f in range(steps):
        log(f"32-stream greedy step {f}: n_past {n_past[:4]}...")
        codes = b.st.run(b.kv_d, n_past, b.d_trail.ptr, s_gpu, b.seeds, [f] * N,
                         d_step_in=b.d_step.ptr if f == 0 else None)
        hid, lg, cpl = b.st.taps(N)
        dev_step = b.st.step_out(N)
        worst = [0.0, 1.0, 0.0, 1.0, 0.0, 1.0]
        for i in range(N):
            b.ora.seen = seen[i]
            dbg = {}
            _, so = b.ora.frame(s_ora, b.seeds[i], f, b.trail[i], kv=b.kv_o[i], n_past=n_past[i], step_in=step_o[i],
                                debug=dbg, force=codes[i])
            e_h, c_h = compare(hid[i], dbg["hidden"])
            e_l, c_l = compare(lg[i], dbg["logits"])
            e_c = max(compare(cpl[i][p], dbg["cp_logits"][p])[0] for p in range(15))
            c_c = min(compare(cpl[i][p], dbg["cp_logits"][p])[1] for p in range(15))
            worst = [max(worst[0], e_h), min(worst[1], c_h), max(worst[2], e_l), min(worst[3], c_l),
                     max(worst[4], e_c), min(worst[5], c_c)]
            assert e_h < TOL_ABS and c_h > TOL_COS, (i, e_h, c_h)
            assert e_l < TOL_ABS and c_l > TOL_COS, (i, e_l, c_l)
            assert e_c < TOL_ABS and c_c > TOL_COS, (i, e_c, c_c)
            check_greedy_frame(f, codes[i], dbg, record, lg[i], cpl[i])
            np.testing.assert_array_equal(dev_step[i], so)
            step_o[i] = so
            n_past[i] += 1
        log(f"  worst over streams: hidden {worst[0]:.2e}/{worst[1]:.7f} logits {worst[2]:.2e}/{worst[3]:.7f} "
            f"cp {worst[4]:.2e}/{worst[5]:.7f}")
    summarize_decisions("streams_32_ctx1024_greedy", record, max_flips=2)


def test_sampled_32_streams_match_oracle_on_device_logits(batch32):
    from oracle import rng, sampler as osamp
    b = batch32
    s_gpu = b.abi.Sampling.make(min_frames=2)
    s_ora = osamp.Sampling(min_frames=2)
    b.st.reset()
    b.st.set_taps(True)
    seen = [np.zeros(3072, bool) for _ in range(N)]
    n_past = list(b.n_past)
    for f in range(2):
        codes = b.st.run(b.kv_d, n_past, b.d_trail.ptr, s_gpu, b.seeds, [f] * N,
                         d_step_in=b.d_step.ptr if f == 0 else None)
        _, lg, cpl = b.st.taps(N)
        for i in range(N):
            tseed, cseed = rng.frame_seeds(b.seeds[i], f)
            cb0 = osamp.sample_talker(lg[i], seen[i], s_ora, tseed, f, 2050, 2048)
            cps = [osamp.sample_cp(cpl[i][p - 1], s_ora, cseed, p) for p in range(1, 16)]
            assert [cb0] + cps == list(codes[i]), (f, i, list(codes[i]), [cb0] + cps)
            if cb0 != 2050:
                seen[i][cb0] = True
            n_past[i] += 1
        log(f"sampled step {f}: 32 streams match the oracle sampler on device logits; stream 0 {list(codes[0][:6])}")
