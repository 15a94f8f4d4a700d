"""Pins the speaker-encoder oracle (oracle/speaker.py) on the CPU.

* the log-mel front end against the reference's own fixture (voice_1.wav -> speaker_mels.npy, first
  2 s; the reference's gate is rel-rms < 1e-4, tests/test_speaker.cpp:61);
* the reflect-padded "same" conv against torch.nn.Conv1d(padding="same", padding_mode="reflect");
* the weighted statistics against numpy.average;
* the whole ECAPA-TDNN on a time-constant mel against a closed form: every conv of a constant
  signal is its summed taps times the value, the pooled std is sqrt(1e-12) and the attention is
  uniform, so the network reduces to a chain of matrix products. A planted mistake (the SE-Res2Net
  residual dropped) must break the agreement;
* the whole ECAPA-TDNN on real speech frames against transformers' ECAPA_TimeDelayNet (an independent
  implementation, same weights by tensor name), with a planted mistake (Res2Net slices reversed).
"""
import numpy as np
import pytest
import torch

from oracle import speaker as osp


def rel_rms(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2) / np.mean(b ** 2)))


def test_log_mel_matches_reference_fixture(speaker_fixture):
    wav, want = speaker_fixture
    got = osp.log_mel(wav)[:, :want.shape[1]]
    e = rel_rms(got, want)
    print(f"log-mel vs reference fixture: rel-rms {e:.2e}, max |d| {np.abs(got - want).max():.2e}")
    assert e < 1e-4


def test_log_mel_frame_count_and_floor():
    wav = np.zeros(24000, np.float32)
    m = osp.log_mel(wav)
    assert m.shape == (128, (24000 + 2 * 384 - 1024) // 256 + 1)
    # silence: every mel band is the filterbank row sum times sqrt(1e-9), under the 1e-5 floor or not
    fb = osp.mel_filterbank(24000, 1024, 128, 0.0, 12000.0).astype(np.float64)
    np.testing.assert_allclose(m[:, 0], np.log(np.maximum(fb.sum(1) * np.sqrt(1e-9), 1e-5)), rtol=1e-5)


@pytest.mark.parametrize("K,dil", [(5, 1), (3, 2), (3, 3), (3, 4), (1, 1)])
def test_same_conv_matches_torch_reflect_conv(K, dil):
    g = torch.Generator().manual_seed(K * 10 + dil)
    x = torch.randn(16, 37, generator=g)
    conv = torch.nn.Conv1d(16, 24, K, dilation=dil, padding="same", padding_mode="reflect")
    with torch.no_grad():
        conv.weight.copy_(torch.randn(24, 16, K, generator=g))
        conv.bias.copy_(torch.randn(24, generator=g))
        want = conv(x[None])[0]
        got = osp.same_conv(x, conv.weight, conv.bias, dil)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_weighted_stats_matches_numpy_average():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((8, 50))
    w = rng.random((8, 50))
    w /= w.sum(1, keepdims=True)
    m, s = osp.weighted_stats(torch.from_numpy(x), torch.from_numpy(w))
    mw = np.average(x, axis=1, weights=w)
    sw = np.sqrt(np.average((x - mw[:, None]) ** 2, axis=1, weights=w))
    np.testing.assert_allclose(m.numpy(), mw, rtol=1e-12)
    np.testing.assert_allclose(s.numpy(), sw, rtol=1e-12)
    m, s = osp.weighted_stats(torch.from_numpy(x))
    np.testing.assert_allclose(m.numpy(), x.mean(1), rtol=1e-12)
    np.testing.assert_allclose(s.numpy(), x.std(1), rtol=1e-12)


def closed_form(p, v, drop_residual=False):
    """ECAPA-TDNN of a mel constant over time (value v[128]) in f64 matrix form."""
    relu = lambda z: np.maximum(z, 0.0)
    sig = lambda z: 1.0 / (1.0 + np.exp(-z))

    def lin(name, z):
        return p[name + ".weight"].numpy().astype(np.float64).sum(-1) @ z + p[name + ".bias"].numpy()

    h = relu(lin("blocks.0.conv", v))
    outs = []
    for bi in range(3):
        bp = f"blocks.{bi + 1}."
        b = relu(lin(bp + "tdnn1.conv", h))
        parts = np.split(b, 8)
        c = [parts[0]]
        for i in range(1, 8):
            c.append(relu(lin(bp + f"res2net_block.blocks.{i - 1}.conv", parts[i] if i == 1 else parts[i] + c[i - 1])))
        b2 = relu(lin(bp + "tdnn2.conv", np.concatenate(c)))
        gse = sig(lin(bp + "se_block.conv2", relu(lin(bp + "se_block.conv1", b2))))
        h = b2 * gse + (0.0 if drop_residual else h)
        outs.append(h)
    att = relu(lin("mfa.conv", np.concatenate(outs)))
    return lin("fc", np.concatenate([att, np.full_like(att, 1e-6)]))


def test_embed_mel_time_constant_closed_form(speaker_blob):
    ora = osp.SpeakerOracle(speaker_blob)
    v = np.random.default_rng(1).uniform(-8.0, 1.0, 128)
    got = ora.embed_mel(np.repeat(v[:, None], 24, axis=1).astype(np.float32))
    want = closed_form(ora.p, v)
    e = rel_rms(got, want)
    print(f"constant-mel embedding vs closed form: rel-rms {e:.2e}")
    assert e < 1e-4
    assert rel_rms(got, closed_form(ora.p, v, drop_residual=True)) > 1e-2     # the check can fail


def _library_ecapa(ora):
    """transformers' ECAPA_TimeDelayNet (qwen2_5_omni/modeling_qwen2_5_omni.py:2630), an independent
    implementation of the same network, configured with Qwen3-TTS's shapes and loaded with the
    blob's weights by tensor name (the reference's names, params.cpp:165-195, are the HF ones)."""
    from transformers.models.qwen2_5_omni.configuration_qwen2_5_omni import Qwen2_5OmniDiTConfig
    from transformers.models.qwen2_5_omni.modeling_qwen2_5_omni import ECAPA_TimeDelayNet
    cfg = Qwen2_5OmniDiTConfig()
    cfg.mel_dim, cfg.enc_dim = 128, ora.p["fc.weight"].shape[0]
    cfg.enc_channels = [512, 512, 512, 512, 1536]
    cfg.enc_kernel_sizes = [5, 3, 3, 3, 1]
    cfg.enc_dilations = [1, 2, 3, 4, 1]
    cfg.enc_attention_channels, cfg.enc_res2net_scale, cfg.enc_se_channels = 128, 8, 128
    net = ECAPA_TimeDelayNet(cfg).eval()
    net.load_state_dict({k: v.clone() for k, v in ora.p.items()}, strict=True)
    return net


@pytest.mark.parametrize("T", [5, 37, 186])
def test_embed_mel_matches_transformers_ecapa(speaker_blob, speaker_fixture, T):
    """The whole network (block wiring, Res2Net slice order, SE, MFA concatenation order, attentive
    pooling) against the library model on real speech frames (the reference's mel fixture) and on
    the 5-frame minimum. A planted mistake (Res2Net slices fed in reverse order) must fail."""
    ora = osp.SpeakerOracle(speaker_blob)
    net = _library_ecapa(ora)
    mel = np.ascontiguousarray(speaker_fixture[1][:, :T], dtype=np.float32)
    with torch.no_grad():
        want = net(torch.from_numpy(mel.T)[None])[0].numpy()
    got = ora.embed_mel(mel)
    e = rel_rms(got, want)
    print(f"T={T}: oracle vs transformers ECAPA rel-rms {e:.2e}")
    assert e < 1e-5
    # planted: the Res2Net chain visits its slices in reverse order
    orig = torch.split
    try:
        torch.split = lambda t, n, dim=0: tuple(reversed(orig(t, n, dim=dim))) if n == ora.R else orig(t, n, dim=dim)
        bad = ora.embed_mel(mel)
    finally:
        torch.split = orig
    assert rel_rms(bad, want) > 1e-2
