"""Shared helpers for the GPU parity tests (compare, cosine, oracle prefill on device)."""
from __future__ import annotations

import sys

import numpy as np


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def compare(got, want):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    d = np.abs(got - want)
    cos = float(np.dot(got, want) / (np.linalg.norm(got) * np.linalg.norm(want) + 1e-300))
    return float(d.max()), cos


def top2_margin(v):
    s = np.sort(np.asarray(v, np.float64))[::-1]
    return float(s[0] - s[1])


def device_from_oracle_prefill(ora, kv_oracle, n_prefill, kv_dev):
    """Copies the oracle's prefill K/V rows (f16 values) into the device KV cache."""
    for l in range(ora.tp.n_layer):
        k = kv_oracle[l][0][:n_prefill].numpy()
        v = kv_oracle[l][1][:n_prefill].numpy()
        kv_dev.fill(l, k, v, 0)
    kv_dev.n_used = n_prefill


# A greedy decision the device may take differently from the oracle only when the oracle's own
# scores put the device's pick within NEAR_TIE of its maximum: accumulation order (f32 sums in a
# different order, the K/V cache in f16) moves logits by ~1e-4..1e-3 at the full model's depth,
# so a tie closer than that is not decidable across implementations.
NEAR_TIE = 5e-3


def greedy_decisions(codes, dbg):
    """[(position, device code, oracle code, oracle score gap)] for the 16 decisions of a frame run
    with teacher forcing; gap = oracle max score - oracle score of the device's code."""
    out = []
    scores = [np.asarray(dbg["cb0_scores"], np.float64)] + [np.asarray(x, np.float64) for x in dbg["cp_logits"]]
    choices = [dbg["cb0_choice"]] + list(dbg["cp_choice"])
    for p, (sc, oc) in enumerate(zip(scores, choices)):
        dc = int(codes[p])
        out.append((p, dc, int(oc), float(sc.max() - sc[dc])))
    return out


def check_greedy_frame(i, codes, dbg, flips):
    """Asserts every decision of frame i is the oracle's, or a near tie (recorded in flips)."""
    for p, dc, oc, gap in greedy_decisions(codes, dbg):
        if dc == oc:
            continue
        log(f"  frame {i} position {p}: device {dc} oracle {oc}, oracle score gap {gap:.2e}")
        assert gap <= NEAR_TIE, f"frame {i} position {p}: device {dc} vs oracle {oc}, gap {gap:.3e} is not a near tie"
        flips.append((i, p, dc, oc, gap))
