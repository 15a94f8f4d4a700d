"""navi_synth (Graph::synth, graph.cpp:52-111) on the GPU.

The streamed request (first batch 2 frames, then batches of 4) must give exactly the PCM of
the same request run by hand through the three modules (prompt -> prefill -> frames, then the
vocoder on all codes at once), the batches must have the requested sizes, and the stats must
be consistent (time to first audio after the prefill, the frame count, EOS vs cap).
"""
import numpy as np
import pytest

from gpu_util import log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full_small(scratch_dir):
    from navi_amd import blob
    path = scratch_dir / "small_all.navi"
    if not path.exists():
        blob.write_random_blob(path, 0, parts=("talker", "cp", "codec"), talker_layers=2, cp_layers=2)
    return path


def _ids(kv, n_text, seed):
    rng = np.random.default_rng(seed)
    return [kv["text.im_start_id"], kv["text.assistant_id"], 198] + rng.integers(0, 151643, n_text).tolist() + \
           [kv["text.im_end_id"], 198, kv["text.im_start_id"], kv["text.assistant_id"], 198]


def test_synth_streams_the_same_pcm_as_the_modules(full_small):
    from navi_amd import abi
    abi.device_open()
    W = abi.DeviceWeights(full_small, select=lambda t: t.dtype != 4)
    talker = abi.Talker(W, max_prompt_tokens=128, max_positions=256)
    frame = abi.Frame(W)
    voc = abi.Vocoder(W, max_chunk_frames=16)
    ids = _ids(W.kv, 12, 7)
    spk = np.random.default_rng(8).standard_normal(1024).astype(np.float32)
    n = 10
    s = abi.Sampling.make(min_frames=n)
    log("synth: 10 frames, first batch 2, then 4")
    st, pcm, sizes = abi.synth(talker, frame, voc, ids=ids, speaker=spk, seed=5, max_frames=n, sampling=s,
                               vocoder_batch=4, first_batch=2)
    log(f"  stats {st.as_dict()}")
    assert st.n_frames == n and st.hit_cap == 1 and st.eos == 0 and st.n_tokens == 12
    assert sizes == [2 * 1920, 4 * 1920, 4 * 1920]
    assert st.prefill_ms < st.ttfa_ms <= st.total_ms and st.rtf > 0

    # the same request by hand, vocoder in one call
    pr = talker.build_prompt(ids, "english", spk)
    talker.prefill(pr.prefill, pr.n_prefill)
    frame.reset()
    codes = []
    for i in range(n):
        trail = pr.trailing + 4 * 1024 * i if i < pr.n_trailing else pr.tts_pad
        r = frame.run_first(talker.d_hidden, talker.d_logits, trail, s, 5, 0) if i == 0 else \
            frame.run(talker.kv, pr.n_prefill + i - 1, trail, s, 5, i)
        assert r.ok, r.error
        codes.append(list(r.codes))
    voc.reset()
    want = voc.decode(np.array(codes))
    assert pcm.shape == want.shape and np.array_equal(pcm, want)


def test_synth_reports_frame_errors(full_small):
    """A KV cache too small for the request fails the request with the frame's error."""
    from navi_amd import abi
    W = abi.DeviceWeights(full_small, select=lambda t: t.dtype != 4)
    talker = abi.Talker(W, max_prompt_tokens=32, max_positions=32)
    frame = abi.Frame(W)
    voc = abi.Vocoder(W, max_chunk_frames=4)
    ids = _ids(W.kv, 12, 9)
    spk = np.zeros(1024, np.float32)
    with pytest.raises(abi.NaviError) as e:
        abi.synth(talker, frame, voc, ids=ids, speaker=spk, max_frames=40, sampling=abi.Sampling.make(min_frames=40))
    assert "KV cache full" in str(e.value)


def test_synth_matches_oracle_greedy(full_small):
    """A whole request against the oracle (Graph::synth, graph.cpp:52-111, restated on the CPU):
    prompt rows -> prefill -> greedy frames -> the codec decoder, streamed by navi_synth in batches
    of 2 then 4 frames. The oracle runs the same request frame by frame and decodes its codes in
    one shot; the PCM must reach the vocoder bar (SNR >= 40 dB), which also requires every code to
    be the oracle's (one different code changes its frame's audio completely)."""
    import torch
    from navi_amd import abi
    from oracle import sampler as osamp
    from oracle.model import Oracle
    from oracle.vocoder import Vocoder as OVoc
    abi.device_open()
    W = abi.DeviceWeights(full_small, select=lambda t: t.dtype != 4)
    talker = abi.Talker(W, max_prompt_tokens=128, max_positions=256)
    frame = abi.Frame(W)
    voc = abi.Vocoder(W, max_chunk_frames=16)
    ids = _ids(W.kv, 14, 21)
    spk = np.random.default_rng(22).standard_normal(1024).astype(np.float32)
    n = 12
    st, pcm, sizes = abi.synth(talker, frame, voc, ids=ids, speaker=spk, seed=3, max_frames=n,
                               sampling=abi.Sampling.greedy(min_frames=n), vocoder_batch=4, first_batch=2)
    assert st.n_frames == n and sizes == [2 * 1920] + [4 * 1920] * 2 + [2 * 1920]
    ora = Oracle(full_small)
    pre, trail, pad = ora.build_prompt(ids, "english", spk)
    kvo = ora.new_kv(64)
    hid, lg = ora.prefill(pre, kvo)
    so = osamp.Sampling(temperature=0.0, cp_temperature=0.0, repetition_penalty=1.05, min_frames=n)
    ora.reset()
    codes, step = [], None
    with torch.no_grad():
        for i in range(n):
            th = trail[i] if i < trail.shape[0] else pad
            if i == 0:
                c, step = ora.frame(so, 3, 0, th, hidden=hid, logits=lg)
            else:
                c, step = ora.frame(so, 3, i, th, kv=kvo, n_past=pre.shape[0] + i - 1, step_in=step)
            codes.append(c)
    want = OVoc(full_small).decode(np.array(codes))
    err = pcm.astype(np.float64) - want
    snr = 10 * np.log10(np.sum(want.astype(np.float64) ** 2) / max(np.sum(err ** 2), 1e-300))
    log(f"synth vs oracle request: {n} frames, first codes {codes[0][:4]}, PCM SNR {snr:.1f} dB")
    assert pcm.shape == want.shape and snr >= 40.0
