"""The speaker encoder on the GPU vs the CPU oracle (through the C ABI).

Same f16 weights (random init, seed 3) on both sides; the device stages activations as f16
hi + lo pairs through the matrix cores and accumulates in f32, the oracle is PyTorch f32, so the
bar is on the embedding as a whole: relative RMS error <= 1e-3 and cosine >= 0.99999.
Inputs: the reference's own fixture mel (speaker_mels.npy frames 0..185) and audio (voice_1.wav,
first 2 s), ragged noise lengths from the 5-frame minimum to 30 s (the default bound), two calls
in a row on one handle
(long then short), the max_seconds bound, and the reference's error cases (too short, too long).
"""
import numpy as np
import pytest

from gpu_util import compare, log

pytestmark = pytest.mark.gpu

REL, COS = 1e-3, 0.99999


@pytest.fixture(scope="module")
def spk(speaker_blob):
    from navi_amd import abi
    from oracle.speaker import SpeakerOracle
    abi.device_open()
    W = abi.DeviceWeights(speaker_blob, select=lambda t: t.name.startswith("speaker_encoder."))
    return abi, W, SpeakerOracle(speaker_blob)


def check(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    rel = float(np.sqrt(np.mean((got - want) ** 2) / np.mean(want ** 2)))
    d, cos = compare(got, want)
    log(f"  {what}: rel rms {rel:.2e}, max abs {d:.2e}, cosine {cos:.8f}")
    assert got.shape == want.shape
    assert np.isfinite(got).all()
    assert rel <= REL and cos >= COS


def test_embed_mel_fixture_matches_oracle(spk, speaker_fixture):
    abi, W, ora = spk
    _, mel = speaker_fixture
    s = abi.Speaker(W, max_seconds=30.0)
    log(f"speaker embed_mel, fixture mel {mel.shape}")
    got = s.embed_mel(mel)
    log(f"  device {s.last_ms():.3f} ms")
    check(got, ora.embed_mel(mel), "fixture mel")
    again = s.embed_mel(mel)
    assert np.array_equal(got, again), "two runs on the same input differ"


def test_embed_audio_matches_oracle(spk, speaker_fixture):
    abi, W, ora = spk
    wav, _ = speaker_fixture
    s = abi.Speaker(W)
    log(f"speaker embed, fixture audio {wav.size} samples")
    check(s.embed(wav), ora.embed(wav), "fixture audio")


def test_device_mel_matches_host_mel_and_fixture(spk, speaker_fixture):
    """navi_speaker_embed's front end (k_logmel, double-precision FFT in LDS) against the host's
    navi_speaker_mel (double, another FFT algorithm): equal up to float rounding of the output
    (1e-5 absolute on values down to log(1e-5) = -11.5), including a pure tone whose high bins
    sit at sidelobe level. Against the reference's f32 fixture: within its own f32 error (the
    host's double result sits 3.3e-4 from it)."""
    abi, W, _ = spk
    wav, mel_ref = speaker_fixture
    s = abi.Speaker(W)
    for name, x in (("fixture audio", wav),
                    ("noise 1300", (np.random.default_rng(5).standard_normal(1300) * 0.2).astype(np.float32)),
                    ("tone + silence", np.concatenate([np.sin(np.arange(24000) * 0.05).astype(np.float32) * 0.5,
                                                       np.zeros(7000, np.float32)]))):
        log(f"speaker device mel, {name}")
        s.embed(x)
        dev = s.tap_mel()
        host = s.mel(x)
        assert dev.shape == host.shape
        d = np.abs(dev.astype(np.float64) - host)
        rel = float(np.sqrt(np.mean(d ** 2) / np.mean(host.astype(np.float64) ** 2)))
        log(f"  {dev.shape[1]} frames: max abs {d.max():.2e}, rel rms {rel:.2e}, device {s.last_ms():.3f} ms")
        assert d.max() <= 1e-5 and rel <= 1e-7
        if name == "fixture audio":
            inner = dev.shape[1] - 3
            assert np.abs(dev[:, :inner] - mel_ref[:, :inner]).max() <= 1e-3


@pytest.mark.parametrize("n", [1300, 9001, 3 * 24000 + 517])
def test_ragged_lengths(spk, n):
    abi, W, ora = spk
    wav = (np.random.default_rng(n).standard_normal(n) * 0.2).astype(np.float32)
    s = abi.Speaker(W, max_seconds=5.0)
    log(f"speaker embed, noise {n} samples ({abi.speaker_mel(W.kv, wav).shape[1]} frames)")
    check(s.embed(wav), ora.embed(wav), f"{n} samples")


def test_thirty_seconds_the_default_maximum(spk):
    """The longest clip a default handle takes (max_seconds 30: 2,814 mel frames of audio)."""
    abi, W, ora = spk
    s = abi.Speaker(W)                            # max_seconds = 30
    n = 30 * 24000 - 256                          # 2,811 frames: inside the 2,814-frame bound
    wav = (np.random.default_rng(30).standard_normal(n) * 0.1).astype(np.float32)
    log(f"speaker embed, 30 s of noise ({abi.speaker_mel(W.kv, wav).shape[1]} frames)")
    got = s.embed(wav)
    log(f"  device {s.last_ms():.3f} ms")
    check(got, ora.embed(wav), "30 s")


def test_long_then_short_on_one_handle(spk):
    abi, W, ora = spk
    rng = np.random.default_rng(7)
    long_mel = rng.standard_normal((128, 300)).astype(np.float32) - 4.0
    short_mel = rng.standard_normal((128, 23)).astype(np.float32) - 4.0
    s = abi.Speaker(W, max_seconds=4.0)
    log("speaker long (300 frames) then short (23 frames) on one handle")
    a = s.embed_mel(long_mel)
    b = s.embed_mel(short_mel)
    check(a, ora.embed_mel(long_mel), "300 frames")
    check(b, ora.embed_mel(short_mel), "23 frames after 300")
    fresh = abi.Speaker(W, max_seconds=4.0).embed_mel(short_mel)
    assert np.array_equal(b, fresh), "a previous longer call changed the result"


def test_max_seconds_bound_and_errors(spk):
    abi, W, ora = spk
    s = abi.Speaker(W, max_seconds=1.0)           # max frames = int(1.0 * 24000 / 256) + 2 = 95
    rng = np.random.default_rng(11)
    mel = rng.standard_normal((128, 95)).astype(np.float32) - 4.0
    log("speaker max_seconds bound: 95 frames ok, 96 refused")
    check(s.embed_mel(mel), ora.embed_mel(mel), "95 frames (the bound)")
    with pytest.raises(abi.NaviError, match="max_seconds"):
        s.embed_mel(rng.standard_normal((128, 96)).astype(np.float32))
    with pytest.raises(abi.NaviError, match="max_seconds"):
        s.embed(np.zeros(24000 * 2, np.float32))
    with pytest.raises(abi.NaviError, match="too short"):
        s.embed(np.zeros(300, np.float32))
    with pytest.raises(abi.NaviError, match="5..95"):
        s.embed_mel(mel[:, :4])
    with pytest.raises(ValueError):
        s.embed_mel(mel[:64])
    # the handle still works after the refusals
    check(s.embed_mel(mel[:, :40]), ora.embed_mel(mel[:, :40]), "40 frames after errors")
