"""bench.py's frame phase table (the k_frame evidence that needs no profiler) on synthetic stamps laid
out as the kernel writes them: per block, 100 MHz stamps in phase order, blocks 0..15 with the
attention marks. Every phase of the synthetic frame takes a known time, so the table's figures
are known."""
import importlib.util
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent


def _bench():
    spec = importlib.util.spec_from_file_location("navi_bench", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _stamps(n_tl=28, n_cl=5, step=10):
    """Each stamp 0.1 us (10 ticks) after the previous one."""
    P = np.zeros((256, 4096), np.uint64)
    for b in range(256):
        att = b < 16
        n = n_tl * (5 + (3 if att else 0) + 8) + 4
        for p in range(15):
            n += n_cl * ((3 if att else 0) + 8) + 4
        n += 1
        P[b, :n] = 1000 + step * np.arange(n, dtype=np.uint64)
    return P


def test_frame_phase_table_on_synthetic_stamps():
    b = _bench()
    t = b.frame_phase_table(_stamps(), 28, 5)
    assert len(t["cp_passes"]) == 15
    # a one-row cp layer of a non-attention block is 8 stamps: its gathered x sits 8 stamps (0.8 us)
    # after the previous layer's
    assert abs(t["cp_layer_cumulative"]["x gathered (layer end)"] - 0.8) < 1e-6
    vals = list(t["talker_layer_cumulative"].values())
    assert all(v > 0 for v in vals)
    assert all(p["us"] > 0 and p["logits_hop_us"] > 0 and p["sampling_us"] > 0 for p in t["cp_passes"])
    assert t["frame_us"] > t["talker_and_cb0_us"] > 0
