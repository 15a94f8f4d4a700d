"""BASELINE configs[0] end to end on the full model (28 talker + 5 code-predictor layers).

Random-init weights N(0, 0.02) seed 0; 32 text ids uniform in [0, 151643) from a torch
Generator seeded 0 inside the 3-id role header and the 5-id trailer; speaker N(0, 1) seed 0;
language "english"; 24 greedy frames with repetition penalty 1.05 and EOS suppressed for all
24 frames. Everything runs on the device through the C ABI (prompt rows, prefill, frames)
and is compared with the oracle doing the same on the CPU: the prefill's hidden and logits
within 2e-2 max abs and cosine > 0.9995; every frame's logits within 2e-2; every one of the
24 x 16 greedy decisions gated by gpu_util.check_greedy_frame: the device's code is the argmax of
its own logits (bit-exact given identical logits) and the oracle's code, unless the oracle's scores
put the device's code within the fixed near-tie bound 2e-3 of their maximum, at most 2 such flips
in the 384 decisions. The oracle is teacher-forced with the device's codes, so such a flip does
not end the comparison. The decision
record (count, flips, row errors, margins) is written when NAVI_DECISION_LOG names a directory.
"""
import numpy as np
import pytest
import torch

from gpu_util import check_greedy_frame, compare, log, summarize_decisions

pytestmark = pytest.mark.gpu

N_FRAMES = 24


def config0_inputs(kv):
    g = torch.Generator().manual_seed(0)
    text = torch.randint(0, 151643, (32,), generator=g).tolist()
    head = [kv["text.im_start_id"], kv["text.assistant_id"], 198]
    tail = [kv["text.im_end_id"], 198, kv["text.im_start_id"], kv["text.assistant_id"], 198]
    spk = torch.randn(1024, generator=torch.Generator().manual_seed(0)).numpy().astype(np.float32)
    return head + text + tail, spk


def test_config0_greedy_end_to_end(full_blob):
    from navi_amd import abi
    from oracle import sampler as osamp
    from oracle.model import Oracle
    abi.device_open()
    ora = Oracle(full_blob)
    ids, spk = config0_inputs(ora.kv)
    W = abi.DeviceWeights(full_blob, select=lambda t: t.name.startswith("talker."))
    talker = abi.Talker(W, max_prompt_tokens=128, max_positions=256)
    frame = abi.Frame(W)
    pr = talker.build_prompt(ids, "english", spk)
    assert (pr.n_prefill, pr.n_trailing) == (10, 32)
    talker.prefill(pr.prefill, pr.n_prefill)
    log(f"config0: device prefill of {pr.n_prefill} rows {talker.last_ms():.3f} ms")
    opre, otrail, opad = ora.build_prompt(ids, "english", spk)
    kvo = ora.new_kv(256)
    ohid, olg = ora.prefill(opre, kvo)
    hid, lg = talker.hidden_logits()
    for name, got, want in (("hidden", hid, ohid), ("logits", lg, olg)):
        mx, cos = compare(got, want)
        log(f"  prefill {name}: max abs {mx:.3e} cosine {cos:.7f}")
        assert mx < 2e-2 and cos > 0.9995
    s = abi.Sampling.greedy(min_frames=N_FRAMES)
    so = osamp.Sampling(temperature=0.0, cp_temperature=0.0, repetition_penalty=1.05, min_frames=N_FRAMES)
    frame.reset()
    ora.reset()
    frame.set_taps(True)
    step = None
    record, us = [], []
    for i in range(N_FRAMES):
        trail_d = pr.trailing + 4 * 1024 * i if i < pr.n_trailing else pr.tts_pad
        trail_h = otrail[i] if i < otrail.shape[0] else opad
        dbg = {}
        if i == 0:
            r = frame.run_first(talker.d_hidden, talker.d_logits, trail_d, s, 0, 0)
        else:
            r = frame.run(talker.kv, pr.n_prefill + i - 1, trail_d, s, 0, i)
        assert r.ok, r.error
        codes = list(r.codes)
        if i == 0:
            c, step = ora.frame(so, 0, 0, trail_h, hidden=ohid, logits=olg, debug=dbg, force=codes)
        else:
            c, step = ora.frame(so, 0, i, trail_h, kv=kvo, n_past=pr.n_prefill + i - 1, step_in=step, debug=dbg,
                                force=codes)
        us.append(r.us)
        thid, tlg, tcp = frame.taps()
        lg_err = max(compare(tlg, dbg["logits"])[0], compare(tcp, np.stack(dbg["cp_logits"]))[0])
        exact = [dbg["cb0_choice"]] + list(dbg["cp_choice"]) == codes
        log(f"  frame {i:2d}: {'exact' if exact else 'flip'} cb0 {codes[0]}, logits max abs err {lg_err:.2e}, "
            f"{r.us:.0f} us")
        assert lg_err < 2e-2
        check_greedy_frame(i, codes, dbg, record, tlg, tcp)
    summarize_decisions("config0_greedy_24_frames", record, max_flips=2)
    log(f"config0: mean device {np.mean(us[1:]):.0f} us/frame (talker frames)")
