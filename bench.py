#!/usr/bin/env python3
"""Benchmark: one batch-1 frame of navi-tts's token loop on one MI355X.

A step is one frame (talker decode step + codebook-0 sampling + the 15-step
code-predictor pass with sampling + next-step assembly), the workload
BASELINE.json's metric is quoted on, at configs[1]'s context: the full
Qwen3-TTS-0.6B random-init weights N(0, 0.02) seed 1, 256 cached positions
with f16 K/V from N(0, 1), hidden input from N(0, 1). Sampling uses the model
defaults (top-k 50, temperature 0.9, repetition penalty 1.05).

`value` is the mean device time per frame (hipEvent around each launch on the
library stream: the reference's frame_ms definition, runtime/bench/bench.cpp:148),
`ms_per_step` the wall time per frame including the host tail. `roofline.achieved`
is the frame's algorithmic bytes (weights streamed once per pass, KV of 257 positions)
over that device time. `cpu_baseline` times the CPU oracle (PyTorch restatement)
on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "navi-tts_amd"))

HBM_PEAK_GBS = 8000.0
N_PAST = 256
SEED = 1


def algorithmic_bytes(kv: dict, n_past: int) -> dict:
    """Bytes one frame must read at least once: every weight of the talker, the K/V rows of the
    context, and the code predictor's layers and heads once per position."""
    def layer_bytes(ns):
        H, F = kv[f"{ns}.hidden_size"], kv[f"{ns}.intermediate_size"]
        Q = kv[f"{ns}.num_attention_heads"] * kv[f"{ns}.head_dim"]
        K = kv[f"{ns}.num_key_value_heads"] * kv[f"{ns}.head_dim"]
        D = kv[f"{ns}.head_dim"]
        return 2 * (Q * H + 2 * K * H + H * Q + 3 * F * H) + 4 * (2 * H + 2 * D)
    H = kv["talker.hidden_size"]
    talker = kv["talker.num_hidden_layers"] * layer_bytes("talker") + 2 * kv["talker.vocab_size"] * H + 4 * H
    kvb = kv["talker.num_hidden_layers"] * 2 * kv["talker.num_key_value_heads"] * kv["talker.head_dim"] * 2 * (n_past + 1)
    passes = kv["talker.num_code_groups"] - 1
    cp = passes * (kv["cp.num_hidden_layers"] * layer_bytes("cp") + 4 * H)
    heads = passes * 2 * kv["cp.vocab_size"] * H
    return {"talker": talker, "kv": kvb, "cp": cp, "cp_heads": heads, "total": talker + kvb + cp + heads}


TRAFFIC_FILE = ROOT / "profiles" / "k_frame_n256_traffic.json"


def copy_calibration(gib: float, reps: int):
    """A plain copy kernel of known size (torch's elementwise `neg` over f32: reads and writes
    exactly `gib` GiB once each) for scaling the FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch
    n = int(gib * (1 << 30)) // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(reps):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"bytes_read": 4 * n, "bytes_written": 4 * n, "dispatches": reps}}), flush=True)


FRAME_SOURCES = ("frame.hip", "sampler.h", "dev_common.h", "host_util.h")


def frame_source_digest() -> str:
    """sha1 over the sources k_frame is compiled from: the counter run behind the traffic figure is
    valid only for the kernel those sources build."""
    import hashlib
    h = hashlib.sha1()
    for name in FRAME_SOURCES:
        h.update((ROOT / "navi-tts_amd" / "csrc" / "hip" / name).read_bytes())
    return h.hexdigest()


def measured_traffic():
    """HBM bytes per k_frame launch from the committed counter runs: None when the file is absent or
    was measured on other kernel sources than the ones built now (its `frame_sources_sha1`)."""
    if not TRAFFIC_FILE.exists():
        return None
    t = json.loads(TRAFFIC_FILE.read_text())
    if t.get("frame_sources_sha1") != frame_source_digest():
        print("[bench] profiles/k_frame_n256_traffic.json was measured on other k_frame sources: traffic null",
              file=sys.stderr)
        return None
    return int(t["frame_bytes_per_launch"])


def make_blob(path: Path):
    from navi_amd import blob
    if not path.exists():
        blob.write_random_blob(path, SEED, parts=("talker", "cp", "codec", "speaker"))


def vocoder_flops_per_frame(kv: dict) -> float:
    """Multiply-adds x 2 of one frame through the codec decoder (the convolutions and linears;
    attention, norms and activations excluded): the work the matrix cores must do once."""
    ns = "codec.decoder"
    VH, FF = kv[f"{ns}.hidden_size"], kv[f"{ns}.intermediate_size"]
    HDT = kv[f"{ns}.num_attention_heads"] * kv[f"{ns}.head_dim"]
    L, CD, DD = kv[f"{ns}.latent_dim"], kv[f"{ns}.codebook_dim"], kv[f"{ns}.decoder_dim"]
    mac = CD * CD + 3 * CD * L + L * VH + kv[f"{ns}.num_hidden_layers"] * (3 * HDT * VH + HDT * VH + 3 * FF * VH) + VH * L
    rows = 1
    for r in kv[f"{ns}.upsampling_ratios"]:
        mac += rows * r * L * L                       # transposed conv, k = s
        rows *= r
        mac += rows * 8 * L * L                       # pwconv1 + pwconv2 (4L hidden)
    mac += rows * 7 * L * DD
    w = DD
    for r in kv[f"{ns}.upsample_rates"]:
        mac += rows * r * 2 * w * (w // 2)            # transposed conv: 2 taps per output phase
        rows *= r
        w //= 2
        mac += rows * 3 * (7 * w * w + w * w)         # three residual units
    mac += rows * 7 * w
    return 2.0 * mac


def multistream(W, kv: dict, abi, steps: int = 12, warmup: int = 3, n_streams: int = 32, ctx: int = 1024) -> dict:
    """32 independent streams, each with its own f16 N(0,1) KV cache at
    context 1024, advanced one frame per navi_streams_run (talker + code predictor as MFMA GEMMs
    over the streams), top-k 50 with per-stream seeds 0..31. Every step reads the weights once and
    every stream's KV once: bytes = weights + 32 x KV(1025 positions)."""
    from navi_amd import blob
    n_layer = kv["talker.num_hidden_layers"]
    kvs = []
    host = np.empty((ctx, 1024), np.uint16)
    ri = blob._randinit()
    for i in range(n_streams):
        c = abi.KvCache(n_layer, ctx + 8, 1024)
        for l in range(n_layer):
            for which, dst in (("k", c.k[l]), ("v", c.v[l])):
                ri.navi_fill_normal_f16(SEED, f"bench.kv.{i}.{l}.{which}".encode(), 1.0, host.ctypes.data, host.size)
                abi.upload(dst, host)
        kvs.append(c)
    st = abi.Streams(W, max_streams=n_streams, max_positions=ctx + 8)
    rng = np.random.default_rng(SEED)
    step_in = abi.DeviceBuffer(4 * 1024 * n_streams)
    step_in.upload(rng.standard_normal((n_streams, 1024)).astype(np.float32))
    trail = abi.DeviceBuffer(4 * 1024 * n_streams)
    trail.upload(np.zeros((n_streams, 1024), np.float32))
    s = abi.Sampling.make(min_frames=10 ** 6)
    seeds = list(range(n_streams))
    n_past = [ctx] * n_streams
    for i in range(warmup):
        st.run(kvs, n_past, trail.ptr, s, seeds, [i] * n_streams, d_step_in=step_in.ptr if i == 0 else None)
    dev, t0 = [], time.perf_counter()
    for i in range(steps):
        st.run(kvs, n_past, trail.ptr, s, seeds, [warmup + i] * n_streams)
        dev.append(st.last_ms())
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ms = float(np.mean(dev))
    b = algorithmic_bytes(kv, ctx)
    total = b["total"] - b["kv"] + n_streams * b["kv"]
    gbs = total / (ms * 1e-3) / 1e9
    return {"multistream": {"config": f"configs[4]: {n_streams} streams, KV f16 N(0,1) at context {ctx} each, "
                                      "top-k 50, T 0.9, seeds 0..31",
                            "streams": n_streams, "ms_per_step": round(ms, 3), "wall_ms_per_step": round(wall, 3),
                            "frames_per_s": round(n_streams / (ms * 1e-3), 1), "bytes_per_step": int(total),
                            "achieved_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}}


def streaming_and_vocoder(W, kv: dict, abi, parts=("prefill", "streaming", "vocoder")) -> dict:
    """BASELINE configs[2] (streaming utterance) through navi_synth and configs[3] (vocoder),
    plus the prefill times. The 128 text ids are prefilled with the prompt (130 rows: the
    reference layout's 10 rows + the first 120 trailing text rows; the last 8 text rows and
    tts_eos stream as trailing rows), so the context grows to ~370 as the config states.
    `parts` selects what runs (a profiler run of one part)."""
    prefill_roofline = prefill_roofline_for(kv)
    rng = np.random.default_rng(SEED)
    talker = abi.Talker(W, max_prompt_tokens=256, max_positions=512)
    frame = abi.Frame(W)
    head = [kv["text.im_start_id"], kv["text.assistant_id"], 198]
    tail = [kv["text.im_end_id"], 198, kv["text.im_start_id"], kv["text.assistant_id"], 198]
    ids = head + rng.integers(0, 151643, 128).tolist() + tail
    spk = rng.standard_normal(1024).astype(np.float32)
    builds = []
    for _ in range(3):                  # the first call also loads the kernels: report a warm one
        t0 = time.perf_counter()
        pr = talker.build_prompt(ids, "english", spk)
        builds.append((time.perf_counter() - t0) * 1e3)
    build_ms = builds[-1]
    n_pre = pr.n_prefill + 120
    rows = abi.DeviceBuffer(4 * 1024 * n_pre)
    abi.lib().navi_mem_d2d(rows.ptr, pr.prefill, 4 * 1024 * pr.n_prefill)
    abi.lib().navi_mem_d2d(rows.ptr + 4 * 1024 * pr.n_prefill, pr.trailing, 4 * 1024 * 120)
    trail = abi.DeviceBuffer(4 * 1024 * (pr.n_trailing - 120))
    abi.lib().navi_mem_d2d(trail.ptr, pr.trailing + 4 * 1024 * 120, 4 * 1024 * (pr.n_trailing - 120))
    pad = abi.DeviceBuffer(4 * 1024)
    abi.lib().navi_mem_d2d(pad.ptr, pr.tts_pad, 4 * 1024)
    out = {}
    pre_ms = {}
    for n in ((pr.n_prefill, n_pre) if "prefill" in parts else ()):
        t = []
        for _ in range(5):
            talker.prefill(rows.ptr, n)
            t.append(talker.last_ms())
        pre_ms[n] = float(np.median(t))
    if "prefill" in parts:
        out["prefill_ms"] = {"rows_10": round(pre_ms[pr.n_prefill], 3), "rows_130": round(pre_ms[n_pre], 3)}
        out["prefill_roofline"] = {"bound": "hbm (weights once per prefill); MFMA work x2 for the hi/lo split",
                                   "rows_10": prefill_roofline(pr.n_prefill, pre_ms[pr.n_prefill]),
                                   "rows_130": prefill_roofline(n_pre, pre_ms[n_pre])}
    if "streaming" in parts:
        out["streaming"] = streaming(W, abi, talker, frame, rows, n_pre, trail, pr, pad, build_ms)
    if "vocoder" in parts:
        out["vocoder"] = vocoder_block(W, kv, abi, rng)
    return out


def prefill_roofline_for(kv: dict):
    def prefill_roofline(T, ms):
        """The prefill reads the talker weights once (the algorithmic bytes: layers + norms + head)
        and does 2 x T x (layer MACs) + the head's row on the matrix cores (x2 for the hi/lo split
        of the activations, which the matrix cores also execute)."""
        H, Fd = kv["talker.hidden_size"], kv["talker.intermediate_size"]
        Q = kv["talker.num_attention_heads"] * kv["talker.head_dim"]
        KV = kv["talker.num_key_value_heads"] * kv["talker.head_dim"]
        L = kv["talker.num_hidden_layers"]
        macs = T * L * (H * (Q + 2 * KV) + Q * H + 3 * H * Fd) + H * kv["talker.vocab_size"]
        b = algorithmic_bytes(kv, 0)
        wbytes = b["talker"] + T * b["kv"]           # weights once + the T rows of K/V written
        gbs = wbytes / (ms * 1e-3) / 1e9
        tfl = 2 * 2 * macs / (ms * 1e-3) / 1e12
        return {"rows": T, "ms": round(ms, 3), "bytes": int(wbytes), "achieved_gbs": round(gbs, 1),
                "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "mfma_tflops": round(tfl, 2),
                "mfma_frac": round(tfl / 2500.0, 5)}
    return prefill_roofline


def streaming(W, abi, talker, frame, rows, n_pre, trail, pr, pad, build_ms) -> dict:
    """the 240-frame streaming utterance through navi_synth."""
    voc = abi.Vocoder(W, max_chunk_frames=32)
    s = abi.Sampling.make(min_frames=240)
    prompt = (rows.ptr, n_pre, trail.ptr, pr.n_trailing - 120, pad.ptr)
    # warm-up: the first batch and full batches of both chunk sizes
    abi.synth(talker, frame, voc, prompt=prompt, seed=2, max_frames=52, sampling=s, vocoder_batch=16, first_batch=4)
    abi.synth(talker, frame, voc, prompt=prompt, seed=2, max_frames=52, sampling=s, vocoder_batch=16, first_batch=4)
    # three identical utterances; the figures are those of the run with the median TTFA
    runs = [abi.synth(talker, frame, voc, prompt=prompt, seed=2, max_frames=240, sampling=s, vocoder_batch=16,
                      first_batch=4)[0] for _ in range(3)]
    st = sorted(runs, key=lambda r: r.ttfa_ms)[1]
    return {"config": "configs[2]: 128 text ids prefilled (130 rows), speaker N(0,1), 240 frames, "
                      "top-k 50, T 0.9, seed 2, first vocoder batch 4 then 16",
            "runs": 3, "ttfa_ms_each": [round(r.ttfa_ms, 2) for r in runs],
            "ttfa_ms": round(st.ttfa_ms, 2), "prompt_build_ms": round(build_ms, 3),
            # the reference's TTFA starts at the request, before the prompt rows exist
            "ttfa_with_prompt_build_ms": round(st.ttfa_ms + build_ms, 2),
            "rtf": round(st.rtf, 4), "total_ms": round(st.total_ms, 1),
            "frames_ms_per_frame": round(st.frames_ms / max(st.n_frames, 1), 4),
            "vocoder_ms": round(st.vocoder_ms, 2), "n_frames": st.n_frames, "audio_s": round(st.audio_s, 2)}


def vocoder_block(W, kv: dict, abi, rng) -> dict:
    """240 frames of codes U[0, 2048) in 16-frame chunks and as one block."""
    codes = rng.integers(0, 2048, (240, 16))
    v16 = abi.Vocoder(W, max_chunk_frames=16)
    v240 = abi.Vocoder(W, max_chunk_frames=240)
    # warm-up: both chunk sizes
    v16.decode(codes[:32])
    v240.decode(codes)
    v240.decode(codes)
    t16, t240 = [], []
    for _ in range(3):
        v16.reset()
        v16.decode(codes)
        t16.append(v16.last_ms() / 240)
        v240.reset()
        v240.decode(codes)
        t240.append(v240.last_ms() / 240)
    ms16, ms240 = float(np.median(t16)), float(np.median(t240))
    fl = vocoder_flops_per_frame(kv)
    return {"config": "configs[3]: codes U[0,2048), 240 frames", "ms_per_frame_chunk16": round(ms16, 4),
            "ms_per_frame_block240": round(ms240, 4), "gflop_per_frame": round(fl / 1e9, 3),
            "tflops_block240": round(fl / (ms240 * 1e-3) / 1e12, 2),
            "mfma_frac_block240": round(fl / (ms240 * 1e-3) / 2.5e15, 5)}


def speaker_flops_per_frame(kv: dict) -> float:
    """Dense multiply-adds per mel frame of the ECAPA-TDNN (speaker.hip:175-217), x 2 flops:
    block 0 (k5, 128 -> 512), per SE-Res2Net block two 512 x 512 k1 convs and seven 64 x 64 k3
    convs, MFA 1536 x 1536, attentive pooling 1536 -> 128 -> 1536 (its mean/std columns are a
    per-utterance bias, not per frame); the SE and fc GEMVs are per utterance and left out."""
    M = kv["speaker.mel.num_mels"]
    per = 512 * M * 5 + 3 * (2 * 512 * 512 + 7 * 64 * 64 * 3) + 1536 * 1536 + 2 * 1536 * 128
    return 2.0 * per


def speaker_encoder(W, kv: dict, abi, seconds=(3.0, 10.0)) -> dict:
    """navi_speaker_embed on synthetic audio (the per-clone step before the prompt, bench.cpp:144):
    host log-mel + device ECAPA-TDNN; device time of the network from its own events."""
    rng = np.random.default_rng(SEED)
    spk = abi.Speaker(W, max_seconds=max(seconds))
    out = {"config": "voice clone: N(0, 0.1) audio at 24 kHz, random-init ECAPA-TDNN (seed 1)"}
    fl = speaker_flops_per_frame(kv)
    for sec in seconds:
        wav = (rng.standard_normal(int(sec * kv["speaker.sample_rate"])) * 0.1).astype(np.float32)
        mel = spk.mel(wav)
        spk.embed_mel(mel)
        dev = []
        for _ in range(5):
            spk.embed_mel(mel)
            dev.append(spk.last_ms())
        t0 = time.perf_counter()
        spk.embed(wav)
        wall = (time.perf_counter() - t0) * 1e3
        ms = float(np.median(dev))
        out[f"{sec:g}s"] = {"frames": int(mel.shape[1]), "device_ms": round(ms, 3), "embed_wall_ms": round(wall, 2),
                            "tflops": round(fl * mel.shape[1] / (ms * 1e-3) / 1e12, 2)}
    out["gflop_per_second_of_audio"] = round(fl * kv["speaker.sample_rate"] / kv["speaker.mel.hop_size"] / 1e9, 3)
    spk.close()
    return {"speaker": out}


def host_cpu() -> str:
    """The host CPU's model name and the cores this process may use."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{name}, {len(os.sched_getaffinity(0))} cores available"


def cpu_baseline(path: Path, frames: int) -> dict:
    """The oracle (PyTorch f32 on the host cores) on the same workload, `frames` frames."""
    import torch
    from oracle import sampler as osamp
    from oracle.model import Oracle
    threads = int(os.environ.get("NAVI_CPU_THREADS", "0")) or min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    ora = Oracle(path)
    rng = np.random.default_rng(SEED)
    kvo = ora.new_kv(N_PAST + frames + 1)
    for l in range(ora.tp.n_layer):
        kvo[l][0][:N_PAST] = torch.from_numpy(rng.standard_normal((N_PAST, 1024)).astype(np.float16).astype(np.float32))
        kvo[l][1][:N_PAST] = torch.from_numpy(rng.standard_normal((N_PAST, 1024)).astype(np.float16).astype(np.float32))
    step = rng.standard_normal(1024).astype(np.float32)
    trail = np.zeros(1024, np.float32)
    s = osamp.Sampling(min_frames=10 ** 6)
    ora.reset()
    ora.frame(s, 2, 1, trail, kv=kvo, n_past=N_PAST, step_in=step)   # warm-up
    t0 = time.perf_counter()
    for i in range(frames):
        _, step = ora.frame(s, 2, i + 1, trail, kv=kvo, n_past=N_PAST, step_in=step)
    ms = (time.perf_counter() - t0) * 1e3 / frames
    # the same restatement's prefill (10 prompt rows, N(0,1)) and codec decoder (8 frames of codes
    # U[0, 2048) in one call), each timed once after one warm-up call
    rows = rng.standard_normal((10, 1024)).astype(np.float32)
    kvp = ora.new_kv(16)
    ora.prefill(rows, kvp)
    t0 = time.perf_counter()
    ora.prefill(rows, kvp)
    pre_ms = (time.perf_counter() - t0) * 1e3
    from oracle.vocoder import Vocoder as OVoc
    voc = OVoc(path)
    codes = rng.integers(0, 2048, (8, 16))
    voc.decode(codes[:2])
    t0 = time.perf_counter()
    voc.decode(codes)
    voc_ms = (time.perf_counter() - t0) * 1e3 / len(codes)
    return {"value": round(ms, 2), "unit": "ms/frame", "cores": threads, "kind": "port", "cpu": host_cpu(),
            "prefill_ms_rows_10": round(pre_ms, 1), "vocoder_ms_per_frame": round(voc_ms, 1),
            "sample": f"{frames} frames at n_past={N_PAST} after 1 warm-up frame, full 0.6B random-init model, "
                      f"PyTorch f32 restatement (oracle/) with torch.set_num_threads({threads}); "
                      "a 10-row prefill and an 8-frame codec decode, each once after a warm-up call"}


def frame_phase_table(P: np.ndarray, n_tl: int, n_cl: int, n_cb: int = 16) -> dict:
    """Reduces one profiled frame's stamps (navi_frame_set_profile: per block, the 100 MHz real-time
    counter at the start and end of every wait, in the kernel's phase order) to a phase table in
    microseconds: medians over the blocks of when each phase ended, relative to the moment the
    layer's input vector arrived, averaged over the talker layers 1.. and over the code predictor's
    one-row layers that are not the first of their pass; then the time per code-predictor pass with
    its logits hop and sampling. Blocks 0..15 run the attention combines (talker) and the cp
    attention, so their stamp sequences carry those marks too."""
    NB = P.shape[0]
    t0 = P[:, 0][P[:, 0] > 0].min()
    per_block = []
    for b in range(NB):
        row = P[b]
        n = int((row > 0).sum())
        t = (row[:n].astype(np.int64) - int(t0)) / 100.0
        i, L, C = 0, [], []
        att = b < 16
        for _ in range(n_tl):
            d = dict(zip(("att_start", "qkv_arrived", "kv_staged", "values", "partial_put"), t[i:i + 5])); i += 5
            if att:
                d.update(zip(("partials_wait", "partials_got", "head_put"), t[i:i + 3])); i += 3
            d.update(zip(("att_gs", "att_ge", "x2_gs", "x2_ge", "h_gs", "h_ge", "x_gs", "x_ge"), t[i:i + 8])); i += 8
            L.append(d)
        head = dict(zip(("lg_gs", "lg_ge", "s0", "s1"), t[i:i + 4])); i += 4
        for p in range(n_cb - 1):
            for _ in range(n_cl):
                d = {}
                if att:
                    d.update(zip(("cpa_start", "cpa_qkv", "cpa_put"), t[i:i + 3])); i += 3
                # every gather takes both rows of a two-row pass in one wait: two stamps each
                v = t[i:i + 8]; i += 8
                d.update({"att_gs": v[0], "att_ge": v[1], "x2_gs": v[2], "x2_ge": v[3],
                          "h_gs": v[4], "h_ge": v[5], "x_gs": v[6], "x_ge": v[7]})
                C.append(d)
            C[-1].update(zip(("lg_gs", "lg_ge", "s0", "s1"), t[i:i + 4])); i += 4
        per_block.append((L, head, C, t[i] if i < n else np.nan))

    def med(kind, idx, key, blocks):
        return float(np.median([per_block[b][kind][idx][key] for b in blocks]))

    def layer_table(kind, idxs, steps):
        out = {}
        for name, key, blocks in steps:
            out[name] = round(float(np.mean([med(kind, li, key, blocks) - med(kind, li - 1, "x_ge", range(NB))
                                              for li in idxs])), 2)
        return out
    allb, att = range(NB), range(16)
    talker = layer_table(0, range(1, n_tl), [
        ("qkv published, K/V staging issued", "att_start", allb), ("q/k/v arrived", "qkv_arrived", allb),
        ("range partial published", "partial_put", allb), ("partials combined, head published", "head_put", att),
        ("attention output gathered", "att_ge", allb), ("o published", "x2_gs", allb), ("x2 gathered", "x2_ge", allb),
        ("gate/up published", "h_gs", allb), ("h gathered", "h_ge", allb), ("down published", "x_gs", allb),
        ("x gathered (layer end)", "x_ge", allb)])
    cp_idx = [i for i in range(1, (n_cb - 1) * n_cl) if i % n_cl != 0 and i >= n_cl]
    cp = layer_table(2, cp_idx, [
        ("qkv published", "att_gs", range(16, NB)), ("q/k/v arrived at the attention blocks", "cpa_qkv", att),
        ("attention output published", "cpa_put", att), ("attention output gathered", "att_ge", allb),
        ("o published", "x2_gs", allb), ("x2 gathered", "x2_ge", allb), ("gate/up published", "h_gs", allb),
        ("h gathered", "h_ge", allb), ("down published", "x_gs", allb), ("x gathered (layer end)", "x_ge", allb)])
    prev = float(np.median([per_block[b][1]["s1"] for b in allb]))
    talker_end = prev
    passes = []
    for p in range(n_cb - 1):
        last = p * n_cl + n_cl - 1
        s1, lg, xe = (med(2, last, k, allb) for k in ("s1", "lg_ge", "x_ge"))
        passes.append({"pass": p, "us": round(s1 - prev, 1), "logits_hop_us": round(lg - xe, 2),
                       "sampling_us": round(s1 - lg, 2)})
        prev = s1
    end = float(np.nanmedian([pb[3] for pb in per_block]))
    return {"unit": "us", "talker_layer_cumulative": talker, "cp_layer_cumulative": cp,
            "talker_and_cb0_us": round(talker_end, 1), "cp_passes": passes, "frame_us": round(end, 1)}


def frame_profile(frame, kv, trail, s, warmup: int) -> dict:
    """One frame at n_past 256 with the kernel's own phase stamps on (no profiler attached)."""
    frame.set_profile(True)
    r = frame.run(kv, N_PAST, trail.ptr, s, 2, warmup + 1000)
    if not r.ok:
        raise SystemExit(f"profiled frame failed: {r.error.decode()}")
    P = frame.profile(frame.grid_blocks(), 4096)
    frame.set_profile(False)
    return {"frame_phases": {"profiled_frame_device_us": round(r.us, 1), **frame_phase_table(P, 28, 5)}}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--greedy", action="store_true", help="greedy sampling instead of the model defaults")
    ap.add_argument("--cpu-frames", type=int, default=36, help="frames timed for the CPU baseline (0: skip)")
    ap.add_argument("--blob", default="", help="path for the random-init blob (default /dev/shm)")
    ap.add_argument("--keep-blob", action="store_true")
    ap.add_argument("--no-streaming", action="store_true", help="skip the prefill / streaming / vocoder extras")
    ap.add_argument("--only", choices=("prefill", "streaming", "vocoder", "multistream", "speaker"), default="",
                    help="run only this part (for a profiler run) and print its JSON instead of the bench line")
    ap.add_argument("--frame-profile", action="store_true",
                    help="after the warm-up, run one frame with the kernel's phase stamps on, print the phase table "
                         "(JSON) and exit")
    ap.add_argument("--copy-calibration", type=float, default=0.0, metavar="GIB",
                    help="only run the counter-calibration copy kernel over GIB GiB and exit")
    args = ap.parse_args()
    if args.copy_calibration > 0:
        copy_calibration(args.copy_calibration, 4)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the batch-1 frame is a chain of dependent phases; the path shards by stream, one process per GPU)", file=sys.stderr)
        sys.exit(2)

    from navi_amd import abi
    shm = "/dev/shm" if os.access("/dev/shm", os.W_OK) else "/tmp"
    path = Path(args.blob or f"{shm}/navi_bench_seed{SEED}_{os.getpid()}.navi")
    try:
        print("[bench] writing random-init blob", flush=True, file=sys.stderr)
        make_blob(path)
        info = abi.device_open()
        W = abi.DeviceWeights(path, select=lambda t: t.dtype != 4)
        if args.only:
            kvd = W.kv
            print(f"[bench] only {args.only}", flush=True, file=sys.stderr)
            if args.only == "multistream":
                part = multistream(W, kvd, abi)
            elif args.only == "speaker":
                part = speaker_encoder(W, kvd, abi)
            else:
                part = streaming_and_vocoder(W, kvd, abi, parts=(args.only,))
            abi.lib().navi_device_synchronize()
            print(json.dumps(part), flush=True)
            return
        frame = abi.Frame(W)
        kvd = W.kv
        n_layer = kvd["talker.num_hidden_layers"]
        kv = abi.KvCache(n_layer, 2048, 1024)
        rng = np.random.default_rng(SEED)
        for l in range(n_layer):
            kv.fill(l, rng.standard_normal((N_PAST, 1024)).astype(np.float16), rng.standard_normal((N_PAST, 1024)).astype(np.float16))
        abi.upload(frame.d_step_out, rng.standard_normal(1024).astype(np.float32))
        trail = abi.DeviceBuffer(4 * 1024)
        trail.upload(np.zeros(1024, np.float32))
        s = abi.Sampling.greedy(min_frames=10 ** 6) if args.greedy else abi.Sampling.make(min_frames=10 ** 6)
        frame.reset()
        print(f"[bench] device {info.name.decode()} {info.arch.decode()} CUs {info.multiprocessors}; grid {frame.grid_blocks()}", flush=True, file=sys.stderr)
        for i in range(args.warmup):
            r = frame.run(kv, N_PAST, trail.ptr, s, 2, i)
            if not r.ok:
                raise SystemExit(f"warm-up frame {i} failed: {r.error.decode()}")
        abi.lib().navi_device_synchronize()
        if args.frame_profile:
            print(json.dumps(frame_profile(frame, kv, trail, s, args.warmup)), flush=True)
            return
        dev_us = []
        t0 = time.perf_counter()
        for i in range(args.steps):
            r = frame.run(kv, N_PAST, trail.ptr, s, 2, args.warmup + i)
            if not r.ok:
                raise SystemExit(f"frame {i} failed: {r.error.decode()}")
            dev_us.append(r.us)
        abi.lib().navi_device_synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
        dev = np.asarray(dev_us)
        dev_ms = float(dev.mean()) / 1e3
        b = algorithmic_bytes(kvd, N_PAST)
        gbs = b["total"] / (dev_ms * 1e-3) / 1e9
        print(f"[bench] device ms/frame mean {dev_ms:.4f} median {np.median(dev)/1e3:.4f} min {dev.min()/1e3:.4f}; "
              f"wall {wall_ms:.4f} ms/frame; {gbs:.0f} GB/s over {b['total']/1e9:.4f} GB", flush=True, file=sys.stderr)
        # the same frames as one on-device loop (navi_frame_run_many): no host round trip per frame
        pad = trail.ptr
        t0 = time.perf_counter()
        codes, _, loop_us = frame.run_many(kv, N_PAST, trail.ptr, 0, pad, s, 2, args.warmup, args.steps)
        abi.lib().navi_device_synchronize()
        loop_wall = (time.perf_counter() - t0) * 1e3 / args.steps
        loop = {"frames": int(len(codes)), "n_past": f"{N_PAST}..{N_PAST + args.steps - 1}",
                "device_ms_per_frame": round(loop_us / 1e3 / args.steps, 4), "wall_ms_per_frame": round(loop_wall, 4)}
        print(f"[bench] frame loop: {json.dumps(loop)}", flush=True, file=sys.stderr)
        extra = None
        if not args.no_streaming:
            print("[bench] prefill, streaming utterance and vocoder", flush=True, file=sys.stderr)
            extra = streaming_and_vocoder(W, kvd, abi)
            print(f"[bench] {json.dumps(extra)}", flush=True, file=sys.stderr)
            print("[bench] multi-stream decode", flush=True, file=sys.stderr)
            ms_ = multistream(W, kvd, abi)
            print(f"[bench] {json.dumps(ms_)}", flush=True, file=sys.stderr)
            extra.update(ms_)
            print("[bench] speaker encoder", flush=True, file=sys.stderr)
            sp = speaker_encoder(W, kvd, abi)
            print(f"[bench] {json.dumps(sp)}", flush=True, file=sys.stderr)
            extra.update(sp)
        del frame, W, kv
        cpu = None
        if args.cpu_frames > 0:
            print("[bench] CPU baseline", flush=True, file=sys.stderr)
            sys.path.insert(0, str(ROOT))
            cpu = cpu_baseline(path, args.cpu_frames)
        line = {
            "metric": "ms/frame at batch 1 (talker + code predictor + sampling), device time",
            "value": round(dev_ms, 4), "unit": "ms/frame", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(wall_ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "f16 weights, f32 accumulate", "data": "synthetic (random-init weights N(0,0.02) seed 1, KV/hidden N(0,1))",
            "config": {"workload": "frame @ n_past=256 (configs[1] context): talker step + 15 cp steps + top-k 50 sampling",
                       "model": "Qwen3-TTS-12Hz-0.6B shapes", "global_batch": 1, "n_past": N_PAST,
                       "sampling": "greedy" if args.greedy else "top-k 50, T 0.9, rep 1.05", "parallelism": "none"},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                         "bytes_per_frame": b["total"], "kernel": "k_frame"},
            "cpu_baseline": cpu,
            "frame_loop": loop,
        }
        if extra:
            line.update(extra)
        print(json.dumps(line), flush=True)
    finally:
        if not args.keep_blob and not args.blob and path.exists():
            path.unlink()


if __name__ == "__main__":
    main()
