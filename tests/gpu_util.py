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
