import os
import sys
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "navi-tts_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def scratch_dir():
    base = os.environ.get("NAVI_TEST_SCRATCH")
    if not base:
        base = "/dev/shm" if os.access("/dev/shm", os.W_OK) else tempfile.gettempdir()
    d = Path(tempfile.mkdtemp(prefix="navi_tests_", dir=base))
    yield d
    for p in d.glob("*"):
        try:
            p.unlink()
        except OSError:
            pass
    try:
        d.rmdir()
    except OSError:
        pass


def _blob(scratch_dir, name, seed, **kw):
    from navi_amd import blob
    path = scratch_dir / name
    if not path.exists():
        blob.write_random_blob(path, seed, **kw)
    return path


@pytest.fixture(scope="session")
def small_blob(scratch_dir):
    """Full widths, 2 talker layers, 2 cp layers: a fast oracle."""
    return _blob(scratch_dir, "small.navi", 0, parts=("talker", "cp"), talker_layers=2, cp_layers=2)


@pytest.fixture(scope="session")
def full_blob(scratch_dir):
    """the full 0.6B talker + 5-layer code predictor, seed 0."""
    return _blob(scratch_dir, "full_seed0.navi", 0, parts=("talker", "cp"))


@pytest.fixture(scope="session")
def speaker_blob(scratch_dir):
    """The speaker encoder's tensors only (random init, seed 3)."""
    return _blob(scratch_dir, "speaker.navi", 3, parts=("speaker",))


@pytest.fixture(scope="session")
def speaker_fixture():
    """The reference's own speaker fixture, first 2 s (tests/golden/make_speaker_fixture.py):
    (wav f32 as runtime/audio/wav.cpp reads it, log-mel frames 0..185 [128][186])."""
    import numpy as np
    z = np.load(ROOT / "tests" / "golden" / "speaker_mel_prefix.npz", allow_pickle=False)
    return z["wav_s16"].astype(np.float32) / np.float32(32768.0), z["mel"]
