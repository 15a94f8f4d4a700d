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
    """Bytes one frame must read at least once (BASELINE.md / SURVEY 8d accounting)."""
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


def measured_traffic():
    """HBM bytes per k_frame launch from the committed counter runs (None when absent)."""
    if not TRAFFIC_FILE.exists():
        return None
    t = json.loads(TRAFFIC_FILE.read_text())
    return int(t["frame_bytes_per_launch"])


def make_blob(path: Path):
    from navi_amd import blob
    if not path.exists():
        blob.write_random_blob(path, SEED, parts=("talker", "cp"))


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
    return {"value": round(ms, 2), "unit": "ms/frame", "cores": threads, "kind": "port",
            "sample": f"{frames} frames at n_past={N_PAST} after 1 warm-up frame, full 0.6B random-init model, "
                      f"PyTorch f32 restatement (oracle/) with torch.set_num_threads({threads})"}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--greedy", action="store_true", help="greedy sampling instead of the model defaults")
    ap.add_argument("--cpu-frames", type=int, default=36, help="frames timed for the CPU baseline (0: skip)")
    ap.add_argument("--blob", default="", help="path for the random-init blob (default /dev/shm)")
    ap.add_argument("--keep-blob", action="store_true")
    ap.add_argument("--copy-calibration", type=float, default=0.0, metavar="GIB",
                    help="only run the counter-calibration copy kernel over GIB GiB and exit")
    args = ap.parse_args()
    if args.copy_calibration > 0:
        copy_calibration(args.copy_calibration, 4)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the batch-1 frame is a chain of dependent phases; see DESIGN.md, 'More than one GPU')", file=sys.stderr)
        sys.exit(2)

    from navi_amd import abi
    shm = "/dev/shm" if os.access("/dev/shm", os.W_OK) else "/tmp"
    path = Path(args.blob or f"{shm}/navi_bench_seed{SEED}_{os.getpid()}.navi")
    try:
        print("[bench] writing random-init blob", flush=True, file=sys.stderr)
        make_blob(path)
        info = abi.device_open()
        W = abi.DeviceWeights(path, select=lambda t: t.name.startswith("talker."))
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
        }
        print(json.dumps(line), flush=True)
    finally:
        if not args.keep_blob and not args.blob and path.exists():
            path.unlink()


if __name__ == "__main__":
    main()
