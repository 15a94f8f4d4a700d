"""BASELINE configs[2] at its own shape, end to end on the device against the oracle.

128 synthetic text ids and a speaker N(0, 1) (seed 2): the device builds the prompt rows
(navi_talker_build_prompt), prefills 130 of them (the reference layout's 10 rows plus the
first 120 trailing text rows, as bench.py's streaming utterance does), then runs 240 frames as
one on-device loop (navi_frame_run_many) while the context grows from 130 to 369; the codes are
decoded by the streaming vocoder in the server's batches (4, then 16). On the 2-layer model with
full widths (the oracle runs 240 frames in seconds), greedy instead of top-k sampling so the
codes can be compared (the sampler itself is checked on the device's own logits elsewhere).

Checked against the oracle doing the same request: the prompt rows; the prefill's post-norm hidden
and logits (2e-2 max abs, cosine > 0.9995); every one of the 240 x 16 decisions, the oracle
teacher-forced with the device's codes: a device code differs from the oracle's only where the
oracle's own scores put it within the near-tie bound of their maximum (gpu_util.NEAR_TIE), at
most 3 such flips; the PCM of the device's codes against the oracle's decode (SNR >= 40 dB).
"""
import numpy as np
import pytest

from gpu_util import NEAR_TIE, compare, log

pytestmark = pytest.mark.gpu

N_TEXT, N_PRE_TEXT, N_FRAMES, SEED = 128, 120, 240, 2


@pytest.fixture(scope="module")
def blob_all(scratch_dir):
    from navi_amd import blob
    path = scratch_dir / "small_all.navi"
    if not path.exists():
        blob.write_random_blob(path, 0, parts=("talker", "cp", "codec"), talker_layers=2, cp_layers=2)
    return path


def test_config2_shape_end_to_end_against_oracle(blob_all):
    import torch
    from navi_amd import abi
    from oracle import sampler as osamp
    from oracle.model import Oracle
    from oracle.vocoder import Vocoder as OVoc
    abi.device_open()
    W = abi.DeviceWeights(blob_all, select=lambda t: t.dtype != 4)
    kvd = W.kv
    rng = np.random.default_rng(SEED)
    ids = [kvd["text.im_start_id"], kvd["text.assistant_id"], 198] + rng.integers(0, 151643, N_TEXT).tolist() + \
          [kvd["text.im_end_id"], 198, kvd["text.im_start_id"], kvd["text.assistant_id"], 198]
    spk = rng.standard_normal(1024).astype(np.float32)

    ora = Oracle(blob_all)
    pre, trail, pad = ora.build_prompt(ids, "english", spk)
    rows_o = np.concatenate([pre, trail[:N_PRE_TEXT]])
    trail_o = trail[N_PRE_TEXT:]
    n_pre = rows_o.shape[0]
    assert n_pre == 130 and trail_o.shape[0] == N_TEXT - N_PRE_TEXT

    talker = abi.Talker(W, max_prompt_tokens=256, max_positions=512)
    frame = abi.Frame(W)
    pr = talker.build_prompt(ids, "english", spk)
    rows = abi.DeviceBuffer(4 * 1024 * n_pre)
    abi.lib().navi_mem_d2d(rows.ptr, pr.prefill, 4 * 1024 * pr.n_prefill)
    abi.lib().navi_mem_d2d(rows.ptr + 4 * 1024 * pr.n_prefill, pr.trailing, 4 * 1024 * N_PRE_TEXT)
    n_tr = pr.n_trailing - N_PRE_TEXT
    d_trail = abi.DeviceBuffer(4 * 1024 * (n_tr + 1))
    abi.lib().navi_mem_d2d(d_trail.ptr, pr.trailing + 4 * 1024 * N_PRE_TEXT, 4 * 1024 * n_tr)
    abi.lib().navi_mem_d2d(d_trail.ptr + 4 * 1024 * n_tr, pr.tts_pad, 4 * 1024)
    got_rows = abi.download(rows.ptr, np.float32, n_pre * 1024).reshape(n_pre, 1024)
    d_rows = float(np.abs(got_rows - rows_o).max())
    log(f"configs[2] shape: {n_pre}-row prompt, device vs oracle rows max {d_rows:.2e}")
    assert d_rows < 1e-4

    talker.prefill(rows.ptr, n_pre)
    kv_o = ora.new_kv(512)
    with torch.no_grad():
        hid_o, lg_o = ora.prefill(rows_o, kv_o)
    hid_d = abi.download(talker.d_hidden, np.float32, 1024)
    lg_d = abi.download(talker.d_logits, np.float32, lg_o.size)
    for name, g, w in (("hidden", hid_d, hid_o), ("logits", lg_d, lg_o)):
        err, cos = compare(g, w)
        log(f"  prefill {name}: max abs {err:.2e}, cosine {cos:.7f}")
        assert err < 2e-2 and cos > 0.9995

    s = abi.Sampling.greedy(min_frames=N_FRAMES)
    frame.reset()
    codes, eos, us = frame.run_many(talker.kv, n_pre - 1, d_trail.ptr, n_tr, d_trail.ptr + 4 * 1024 * n_tr, s, SEED, 0,
                                    N_FRAMES, skip_first=True, d_hidden=talker.d_hidden, d_logits=talker.d_logits)
    log(f"  {len(codes)} frames on the device loop, {us / 1e3 / max(len(codes), 1):.3f} ms/frame")
    assert not eos and codes.shape == (N_FRAMES, 16)

    so = osamp.Sampling(temperature=0.0, cp_temperature=0.0, repetition_penalty=1.05, min_frames=N_FRAMES)
    ora.reset()
    flips, decisions, step = [], 0, None
    with torch.no_grad():
        for i in range(N_FRAMES):
            th = trail_o[i] if i < trail_o.shape[0] else pad
            dbg = {}
            if i == 0:
                c, step = ora.frame(so, SEED, 0, th, hidden=hid_o, logits=lg_o, debug=dbg, force=codes[i])
            else:
                c, step = ora.frame(so, SEED, i, th, kv=kv_o, n_past=n_pre + i - 1, step_in=step, debug=dbg,
                                    force=codes[i])
            scores = [np.asarray(dbg["cb0_scores"], np.float64)] + [np.asarray(x, np.float64) for x in dbg["cp_logits"]]
            choices = [dbg["cb0_choice"]] + list(dbg["cp_choice"])
            for p in range(16):
                decisions += 1
                dc, oc = int(codes[i][p]), int(choices[p])
                if dc != oc:
                    gap = float(scores[p].max() - scores[p][dc])
                    flips.append((i, p, dc, oc, gap))
                    assert gap <= NEAR_TIE, f"frame {i} position {p}: device {dc} vs oracle {oc}, oracle gap {gap:.3e}"
    log(f"  {decisions - len(flips)} of {decisions} greedy decisions identical; flips {flips}")
    assert len(flips) <= 3

    voc = abi.Vocoder(W, max_chunk_frames=16)
    parts = [voc.decode(codes[:4])] + [voc.decode(codes[f:f + 16]) for f in range(4, N_FRAMES, 16)]
    pcm = np.concatenate(parts)
    want = OVoc(blob_all).decode(codes)
    err = pcm.astype(np.float64) - want
    snr = 10 * np.log10(np.sum(want.astype(np.float64) ** 2) / max(np.sum(err ** 2), 1e-300))
    log(f"  streamed PCM of the 240 frames vs the oracle's decode: SNR {snr:.1f} dB")
    assert pcm.shape == want.shape == (N_FRAMES * 1920,) and snr >= 40.0
