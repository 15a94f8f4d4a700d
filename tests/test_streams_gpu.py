"""Multi-stream batched decode (navi_streams_*) on the GPU against the CPU oracle.

Each stream is an independent request: its own KV cache (random f16 N(0,1) rows, different
context lengths), step input, trailing row, seed and repetition set. Stream i of a batched run
must compute the batch-1 frame of the oracle (oracle/model.py Oracle.frame, which restates
k_frame, frame.hip:517-579) for that stream alone:

* greedy: codes through the greedy gate (gpu_util.check_greedy_frame) with teacher forcing;
  talker hidden/logits and cp logits within 2e-2 max abs and cosine > 0.9995; the next step
  input bit-exact (same codes, same f32 adds);
* sampled: given the device's own logits (taps), the oracle sampler picks the device's codes;
* errors: a stream past its cache fails with "KV cache full"; a bad stream count is invalid.
"""
import numpy as np
import pytest

from gpu_util import check_greedy_frame, compare, log, summarize_decisions

pytestmark = pytest.mark.gpu

TOL_ABS, TOL_COS = 2e-2, 0.9995
N_STREAMS = 5
MAX_POS = 600


class Batch:
    def __init__(self, path, contexts, seed=11, max_pos=MAX_POS, max_streams=8):
        import torch
        from navi_amd import abi
        from oracle.model import Oracle
        self.abi = abi
        self.ora = Oracle(path)
        abi.device_open()
        self.W = abi.DeviceWeights(path, select=lambda t: t.name.startswith("talker."))
        self.st = abi.Streams(self.W, max_streams=max_streams, max_positions=max_pos)
        rng = np.random.default_rng(seed)
        L, kvd = self.ora.tp.n_layer, 1024
        self.kv_o, self.kv_d, self.n_past = [], [], list(contexts)
        for n in contexts:
            kvo = self.ora.new_kv(max_pos)
            kvd_ = abi.KvCache(L, max_pos, kvd)
            for l in range(L):
                k = rng.standard_normal((n, kvd)).astype(np.float16)
                v = rng.standard_normal((n, kvd)).astype(np.float16)
                kvo[l][0][:n] = torch.from_numpy(k.astype(np.float32))
                kvo[l][1][:n] = torch.from_numpy(v.astype(np.float32))
                if n:
                    kvd_.fill(l, k, v, 0)
            self.kv_o.append(kvo)
            self.kv_d.append(kvd_)
        n = len(contexts)
        self.step = rng.standard_normal((n, 1024)).astype(np.float32)
        self.trail = rng.standard_normal((n, 1024)).astype(np.float32)
        self.d_step = abi.DeviceBuffer(self.step.nbytes)
        self.d_step.upload(self.step)
        self.d_trail = abi.DeviceBuffer(self.trail.nbytes)
        self.d_trail.upload(self.trail)
        self.seeds = [3 + 7 * i for i in range(n)]
        self.seen = [np.zeros(self.ora.tp.vocab, bool) for _ in range(n)]


@pytest.fixture(scope="module")
def batch(small_blob):
    return Batch(small_blob, [37, 300, 1, 129, 256][:N_STREAMS])


def greedy_steps(b, steps, name):
    """`steps` batched greedy steps of every stream of `b`, each checked against the oracle's
    frame for that stream alone (teacher-forced on the device codes): taps within tolerance,
    codes through the greedy gate, next step input bit-exact."""
    from oracle import sampler as osamp
    n = len(b.n_past)
    s_gpu = b.abi.Sampling.greedy(min_frames=steps)
    s_ora = osamp.Sampling(temperature=0.0, top_k=50, repetition_penalty=1.05, cp_temperature=0.0, cp_top_k=50,
                           min_frames=steps)
    b.st.reset()
    b.st.set_taps(True)
    step_o = [b.step[i].copy() for i in range(n)]
    seen = [np.zeros(b.ora.tp.vocab, bool) for _ in range(n)]
    n_past = list(b.n_past)
    record = []
    for f in range(steps):
        log(f"batched greedy step {f}: n_past {n_past}")
        codes = b.st.run(b.kv_d, n_past, b.d_trail.ptr, s_gpu, b.seeds, [f] * n,
                         d_step_in=b.d_step.ptr if f == 0 else None)
        hid, lg, cpl = b.st.taps(n)
        dev_step = b.st.step_out(n)
        for i in range(n):
            b.ora.seen = seen[i]
            dbg = {}
            oc, so = b.ora.frame(s_ora, b.seeds[i], f, b.trail[i], kv=b.kv_o[i], n_past=n_past[i], step_in=step_o[i],
                                 debug=dbg, force=codes[i])
            e_h, c_h = compare(hid[i], dbg["hidden"])
            e_l, c_l = compare(lg[i], dbg["logits"])
            e_c = max(compare(cpl[i][p], dbg["cp_logits"][p])[0] for p in range(15))
            c_c = min(compare(cpl[i][p], dbg["cp_logits"][p])[1] for p in range(15))
            log(f"  stream {i}: hidden {e_h:.2e}/{c_h:.7f} logits {e_l:.2e}/{c_l:.7f} cp {e_c:.2e}/{c_c:.7f} codes {list(codes[i])}")
            assert e_h < TOL_ABS and c_h > TOL_COS
            assert e_l < TOL_ABS and c_l > TOL_COS
            assert e_c < TOL_ABS and c_c > TOL_COS
            check_greedy_frame(f, codes[i], dbg, record, lg[i], cpl[i])
            np.testing.assert_array_equal(dev_step[i], so)
            step_o[i] = so
            n_past[i] += 1
    summarize_decisions(name, record, max_flips=1)


def test_greedy_streams_match_oracle(batch):
    greedy_steps(batch, 3, "streams_5_greedy")


def test_greedy_streams_from_an_empty_cache(small_blob):
    """Streams whose caches start empty (n_past 0: the key range that holds the step's own key has
    no cached key at all) beside short ones, stepped past the first cached keys."""
    greedy_steps(Batch(small_blob, [0, 1, 2], seed=13), 3, "streams_ctx0_greedy")


def test_sampled_streams_match_oracle_on_device_logits(batch):
    """top-k 50, T 0.9, rep 1.05 with a different seed per stream: given the device logits, the
    oracle's sampler (tl_sample / cp_sample restated) picks every device code."""
    from oracle import rng, sampler as osamp
    b = batch
    n = len(b.n_past)
    s_gpu = b.abi.Sampling.make(min_frames=2)
    s_ora = osamp.Sampling(min_frames=2)
    b.st.reset()
    b.st.set_taps(True)
    seen = [np.zeros(3072, bool) for _ in range(n)]
    n_past = list(b.n_past)
    for f in range(3):
        codes = b.st.run(b.kv_d, n_past, b.d_trail.ptr, s_gpu, b.seeds, [f] * n, d_step_in=b.d_step.ptr if f == 0 else None)
        _, lg, cpl = b.st.taps(n)
        for i in range(n):
            tseed, cseed = rng.frame_seeds(b.seeds[i], f)
            cb0 = osamp.sample_talker(lg[i], seen[i], s_ora, tseed, f, 2050, 2048)
            cps = [osamp.sample_cp(cpl[i][p - 1], s_ora, cseed, p) for p in range(1, 16)]
            log(f"step {f} stream {i}: gpu {list(codes[i])} oracle {[cb0] + cps}")
            assert [cb0] + cps == list(codes[i])
            if cb0 != 2050:
                seen[i][cb0] = True
            n_past[i] += 1


def test_streams_are_independent(batch):
    """A stream's codes do not depend on which other streams share the batch (sampled)."""
    b = batch
    s = b.abi.Sampling.make(min_frames=2)
    n = len(b.n_past)
    np_ = list(b.n_past)
    b.st.reset()
    all_codes = b.st.run(b.kv_d, np_, b.d_trail.ptr, s, b.seeds, [0] * n, d_step_in=b.d_step.ptr)
    b.st.reset()
    one = b.st.run(b.kv_d[2:3], np_[2:3], b.d_trail.ptr + 2 * 4096, s, b.seeds[2:3], [0], d_step_in=b.d_step.ptr + 2 * 4096)
    log(f"stream 2 in the batch {list(all_codes[2])} alone {list(one[0])}")
    # 1 and 5 rows use the same row tiles and K splits, so the sums run in the same order
    assert list(one[0]) == list(all_codes[2])


def test_errors(batch):
    b = batch
    s = b.abi.Sampling.greedy()
    with pytest.raises(b.abi.NaviError) as e:
        b.st.run(b.kv_d[:1], [MAX_POS], b.d_trail.ptr, s, [0], [0], d_step_in=b.d_step.ptr)
    assert e.value.status == b.abi.NAVI_ERR_KV_FULL and "KV cache full" in str(e.value)
    with pytest.raises(b.abi.NaviError) as e:
        b.st.run(b.kv_d * 2, [1] * 10, b.d_trail.ptr, s, [0] * 10, [0] * 10, d_step_in=b.d_step.ptr)
    assert e.value.status == b.abi.NAVI_ERR_INVALID


def test_graph_replays_match_eager(batch):
    """Runs replayed from the captured graph (the default) give the codes and next step inputs of
    runs whose kernels the host launches one by one: four sampled steps from the same start, each
    replay preceded by the run's own uploads and followed by its copies and synchronisation."""
    b = batch
    n = len(b.n_past)
    s = b.abi.Sampling.make(min_frames=2)

    def steps(graphs):
        b.st.set_graphs(graphs)
        b.st.reset()
        out = []
        for f in range(4):
            codes = b.st.run(b.kv_d, [p + f for p in b.n_past], b.d_trail.ptr, s, b.seeds, [f] * n,
                             d_step_in=b.d_step.ptr if f == 0 else None)
            out.append((codes.copy(), b.st.step_out(n).copy()))
        return out

    b.st.set_taps(False)
    eager = steps(False)
    graph = steps(True)
    for f, ((ce, se), (cg, sg)) in enumerate(zip(eager, graph)):
        log(f"step {f}: eager {ce[:, :4].tolist()} graph {cg[:, :4].tolist()}")
        np.testing.assert_array_equal(cg, ce)
        np.testing.assert_array_equal(sg, se)
