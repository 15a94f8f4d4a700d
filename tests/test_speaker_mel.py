"""The library's host mel front end (navi_speaker_mel, SpeakerEncoder::mel speaker.hip:269-303).

Host code only (no device call), so it runs in the CPU suite: against the reference's own
fixture (the first 2 s of tests/reference/voice_1.wav -> speaker_mels.npy frames 0..185, see
tests/golden/make_speaker_fixture.py) and against oracle.speaker.log_mel on ragged lengths,
including the shortest input the reflect padding allows; too-short input and a too-small output
buffer are errors, as in the reference.
"""
import ctypes as C

import numpy as np
import pytest

KV = {"speaker.sample_rate": 24000, "speaker.enc_dim": 1024, "speaker.mel.n_fft": 1024, "speaker.mel.num_mels": 128,
      "speaker.mel.hop_size": 256, "speaker.mel.win_size": 1024, "speaker.mel.fmin": 0.0, "speaker.mel.fmax": 12000.0}


@pytest.fixture(scope="module")
def abi():
    from navi_amd import abi
    return abi


def rel_rms(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.sqrt(np.mean((got - want) ** 2) / np.mean(want ** 2)))


def test_mel_matches_reference_fixture(abi, speaker_fixture):
    wav, mel_ref = speaker_fixture
    got = abi.speaker_mel(KV, wav)
    # 2 s of audio: the library's last frames see the reflect padding at the cut, the fixture's
    # (from the whole file) do not, so compare the frames whose windows lie inside the 2 s.
    T = got.shape[1]
    assert got.shape == (128, (len(wav) + 768 - 1024) // 256 + 1)
    inner = T - 3
    r = rel_rms(got[:, :inner], mel_ref[:, :inner])
    print(f"frames {T}, rel rms vs fixture {r:.2e}, max abs {np.abs(got[:, :inner] - mel_ref[:, :inner]).max():.2e}")
    assert r < 1e-4


@pytest.mark.parametrize("n", [385, 1300, 4801, 24000 + 37])
def test_mel_matches_oracle_on_ragged_lengths(abi, n):
    from oracle.speaker import log_mel
    wav = (np.random.default_rng(n).standard_normal(n) * 0.3).astype(np.float32)
    got = abi.speaker_mel(KV, wav)
    want = log_mel(wav)
    assert got.shape == want.shape
    assert np.abs(got - want).max() < 1e-4


def test_mel_errors(abi):
    with pytest.raises(abi.NaviError, match="too short"):
        abi.speaker_mel(KV, np.zeros(384, np.float32))
    p = abi.speaker_params(KV)
    wav = np.zeros(4800, np.float32)
    n = C.c_int32()
    err = C.create_string_buffer(256)
    out = np.empty(16, np.float32)
    st = abi.lib().navi_speaker_mel(C.byref(p), wav.ctypes.data, wav.size, out.ctypes.data, out.size, C.byref(n), err, 256)
    assert st == abi.NAVI_ERR_INVALID and b"mel buffer" in err.value
    bad = dict(KV, **{"speaker.mel.win_size": 800})
    with pytest.raises(abi.NaviError, match="unsupported front end"):
        abi.speaker_mel(bad, wav)
