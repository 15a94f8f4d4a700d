"""bench.py's roofline.traffic comes from the committed counter runs (profiles/k_frame_n256_traffic.json).
The file records the sha1 of the k_frame sources it was measured on; bench.py reports the figure only
while the sources still hash the same, and this test fails when a change to the frame kernel's sources
leaves the committed counter figure stale."""
import importlib.util
import json
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _bench():
    spec = importlib.util.spec_from_file_location("navi_bench", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_traffic_file_matches_the_frame_sources():
    b = _bench()
    t = json.loads(b.TRAFFIC_FILE.read_text())
    assert t["frame_sources_sha1"] == b.frame_source_digest(), "k_frame changed: rerun the FETCH_SIZE / WRITE_SIZE passes"
    assert b.measured_traffic() == t["frame_bytes_per_launch"]


def test_traffic_is_null_for_other_sources(tmp_path, monkeypatch):
    b = _bench()
    t = json.loads(b.TRAFFIC_FILE.read_text())
    t["frame_sources_sha1"] = "0" * 40
    f = tmp_path / "traffic.json"
    f.write_text(json.dumps(t))
    monkeypatch.setattr(b, "TRAFFIC_FILE", f)
    assert b.measured_traffic() is None
