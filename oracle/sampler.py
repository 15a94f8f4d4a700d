"""The reference sampler, restated on the CPU (test infrastructure).

Follows model/qwen3tts/frame.hip:
* `talker_modified_logits` - tl_modified_logit, frame.hip:413-419;
* `greedy`                 - block_argmax, frame.hip:178-203 (lowest index wins ties);
* `kth_largest`            - block_kth_largest's result, frame.hip:221-256 (exact k-th largest,
                              duplicates counted); restated as a sort;
* `draw`                   - block_draw, frame.hip:258-296 (fused f32 running sum over nonzero
                              entries in index order, first cum >= u, else V-1);
* `sample_talker` / `sample_cp` - tl_sample / cp_sample, frame.hip:421-500.

Arithmetic is f32 where the kernel's is (division by the temperature, the
running sum); expf and the softmax denominator are computed in f64 and
rounded, i.e. the correctly rounded values the device approximates.
"""
from __future__ import annotations

from dataclasses import dataclass
from fractions import Fraction

import numpy as np

from . import rng

F32 = np.float32


@dataclass
class Sampling:
    """model/qwen3tts/frame.h:24-31 defaults."""
    temperature: float = 0.9
    top_k: int = 50
    repetition_penalty: float = 1.05
    cp_temperature: float = 0.9
    cp_top_k: int = 50
    min_frames: int = 2


def talker_modified_logits(logits, seen, eos_id: int, suppress_from: int, frame_index: int, min_frames: int,
                           repetition_penalty: float) -> np.ndarray:
    v = np.asarray(logits, dtype=F32).copy()
    idx = np.arange(v.size)
    kill = (idx >= suppress_from) & (idx != eos_id)
    if frame_index < min_frames:
        kill |= idx == eos_id
    if repetition_penalty > 0:
        p = F32(repetition_penalty)
        pen = np.asarray(seen, dtype=bool) & ~kill
        v = np.where(pen, np.where(v > 0, v / p, v * p), v).astype(F32)
    v[kill] = -np.inf
    return v


def greedy(v) -> int:
    return int(np.argmax(np.asarray(v, dtype=F32)))   # first maximum = lowest index on ties


def kth_largest(xs, k: int) -> float:
    xs = np.asarray(xs, dtype=F32)
    return float(np.sort(xs)[::-1][k - 1])


def softmax_weights(xs, top_k: int):
    """(e, inv_sum, threshold): e_i = exp(x_i - max) for x_i >= threshold, else 0."""
    xs = np.asarray(xs, dtype=F32)
    V = xs.size
    mx = F32(np.max(xs))
    thr = F32(kth_largest(xs, top_k)) if 0 < top_k < V else F32(-np.inf)
    d = (xs - mx).astype(F32)
    e = np.where(xs >= thr, np.exp(d.astype(np.float64)), 0.0).astype(F32)
    ssum = F32(np.sum(e.astype(np.float64)))
    return e, F32(F32(1.0) / ssum), thr


def fma_f32(a, b, c) -> np.float32:
    """f32(a*b + c) rounded once (round to nearest, ties to even), from the exact rational value."""
    a, b, c = F32(a), F32(b), F32(c)
    if not (np.isfinite(a) and np.isfinite(b) and np.isfinite(c)):
        return F32(float(a) * float(b) + float(c))
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    r = F32(float(exact))                     # within one f32 ulp of the exact value
    best = None
    for cand in (np.nextafter(r, F32(-np.inf)), r, np.nextafter(r, F32(np.inf))):
        if not np.isfinite(cand):
            continue
        d = abs(Fraction(float(cand)) - exact)
        if best is None or d < best[0] or (d == best[0] and (int(cand.view(np.uint32)) & 1) == 0):
            best = (d, cand)
    return F32(best[1])


def draw(e, inv_sum, seed: int) -> tuple[int, float]:
    """(index, margin): margin = |cum - u| at the decision (a near-tie indicator). The running sum
    is fused (cum = fma(p, inv_sum, cum)): the reference's `cum += p[i] * inv_sum` (frame.hip:290-292)
    is contracted by hipcc's default -ffp-contract=fast-honor-pragmas."""
    u = F32(rng.draw_uniform(seed))
    cum = F32(0.0)
    inv_sum = F32(inv_sum)
    last_gap = np.inf
    for i in np.flatnonzero(np.asarray(e) != 0):
        cum = fma_f32(e[i], inv_sum, cum)
        last_gap = min(last_gap, abs(float(cum) - float(u)))
        if cum >= u:
            return int(i), last_gap
    return int(np.asarray(e).size - 1), last_gap


def sample_talker(logits, seen, s: Sampling, talker_seed: int, frame_index: int, eos_id: int, suppress_from: int):
    v = talker_modified_logits(logits, seen, eos_id, suppress_from, frame_index, s.min_frames, s.repetition_penalty)
    if s.temperature <= 0:
        return greedy(v)
    xs = (v / F32(s.temperature)).astype(F32)
    e, inv, _ = softmax_weights(xs, s.top_k)
    return draw(e, inv, talker_seed)[0]


def sample_cp(logits, s: Sampling, cp_seed: int, pos: int):
    lg = np.asarray(logits, dtype=F32)
    if s.cp_temperature <= 0:
        return greedy(lg)
    xs = (lg / F32(s.cp_temperature)).astype(F32)
    e, inv, _ = softmax_weights(xs, s.cp_top_k)
    return draw(e, inv, rng.cp_pos_seed(cp_seed, pos))[0]
