"""The speaker encoder on the CPU: 24 kHz audio -> log-mel [n_mels][T] -> ECAPA-TDNN -> f32[enc_dim].

Test infrastructure (see oracle/__init__.py). A restatement of model/qwen3tts/speaker.hip (and
docs/model.md "Speaker encoder") in numpy f64 (front end) and PyTorch f32 (network; f16 weights
as stored, upcast):

* `mel_filterbank` - librosa.filters.mel with the slaney mel scale and slaney norm (speaker.hip:45-71);
* `log_mel`        - SpeakerEncoder::mel (speaker.hip:262-300): reflect padding (n_fft - hop) / 2 at both
                     ends, periodic Hann window, |FFT| as sqrt(re^2 + im^2 + 1e-9), the filterbank,
                     log(max(., 1e-5)); frames = (len + 2 pad - n_fft) // hop + 1;
* `same_conv`      - k_conv with reflect = 1 and pad_left = (K - 1) dil / 2 (speaker.hip:155-173,
                     kernels.h:72-242): PyTorch Conv1d, "same" output length, reflect padding;
* `weighted_stats` - k_weighted_stats (speaker.hip:92-107): per channel, mean and std over time with
                     weights w[t][c] (uniform 1/T when none), std = sqrt(max(var, 1e-12));
* `SpeakerOracle.embed_mel` - SpeakerEncoder::Impl::run (speaker.hip:175-220): block 0 (k5 conv +
                     ReLU) -> 3 SE-Res2Net blocks (dilations 2, 3, 4: tdnn1, Res2Net scale 8 where
                     slice 0 passes, slice 1 is conv(slice 1) and slice i is conv(slice i + out i-1),
                     tdnn2, squeeze-excitation on the time mean, + the block input) -> MFA conv over
                     the three block outputs concatenated -> attentive statistics pooling
                     ([x | mean | std] -> tdnn + ReLU + tanh -> conv -> softmax over time ->
                     weighted mean and std) -> fc.

Pinning (tests/test_oracle_speaker.py): `log_mel` and `mel_filterbank` against the reference's own
fixture (tests/reference/voice_1.wav -> speaker_mels.npy, first 2 s; tests/golden/); `same_conv`
against torch.nn.Conv1d(padding="same", padding_mode="reflect"); `weighted_stats` against
numpy.average; `embed_mel` on a time-constant mel against a closed form (every conv reduces to a
matrix of summed taps, the pooled std to 1e-6, the attention to 1/T). The block wiring (slice
order, residuals, concatenation orders) follows speaker.hip:175-220 and is pinned by that closed
form and by transformers' ECAPA_TimeDelayNet (qwen2_5_omni/modeling_qwen2_5_omni.py:2630), an
independent implementation of the same network loaded with the same weights (equal on real speech).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from .navi_read import NaviBlob

SPK = "speaker_encoder."


def mel_filterbank(sr: int, n_fft: int, n_mels: int, fmin: float, fmax: float) -> np.ndarray:
    """[n_mels][n_fft / 2 + 1] float32 (slaney scale: linear below 1 kHz, log above; slaney norm)."""
    f_sp, min_log_hz = 200.0 / 3.0, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0

    def hz_to_mel(f):
        return min_log_mel + np.log(f / min_log_hz) / logstep if f >= min_log_hz else f / f_sp

    def mel_to_hz(m):
        return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), f_sp * m)

    n_bins = n_fft // 2 + 1
    fftfreqs = np.arange(n_bins, dtype=np.float64) * (sr / 2.0) / (n_bins - 1)
    mels = hz_to_mel(fmin) + (hz_to_mel(fmax) - hz_to_mel(fmin)) * np.arange(n_mels + 2) / (n_mels + 1)
    mel_f = mel_to_hz(mels)
    lower = (fftfreqs[None, :] - mel_f[:n_mels, None]) / (mel_f[1:n_mels + 1] - mel_f[:n_mels])[:, None]
    upper = (mel_f[2:, None] - fftfreqs[None, :]) / (mel_f[2:] - mel_f[1:n_mels + 1])[:, None]
    w = np.maximum(0.0, np.minimum(lower, upper)) * (2.0 / (mel_f[2:] - mel_f[:n_mels]))[:, None]
    return w.astype(np.float32)


def log_mel(wav: np.ndarray, sr: int = 24000, n_fft: int = 1024, hop: int = 256, n_mels: int = 128,
            fmin: float = 0.0, fmax: float = 12000.0) -> np.ndarray:
    """[n_mels][T] float32 log-mel of a mono waveform in [-1, 1]."""
    x = np.asarray(wav, dtype=np.float64)
    pad = (n_fft - hop) // 2
    y = np.pad(x, (pad, pad), mode="reflect")
    T = (len(y) - n_fft) // hop + 1
    hann = 0.5 - 0.5 * np.cos(2.0 * np.pi * np.arange(n_fft) / n_fft)      # periodic
    idx = np.arange(T)[:, None] * hop + np.arange(n_fft)[None, :]
    spec = np.fft.rfft(y[idx] * hann[None, :], axis=1)                     # [T][n_bins]
    mag = np.sqrt(spec.real ** 2 + spec.imag ** 2 + 1e-9)
    fb = mel_filterbank(sr, n_fft, n_mels, fmin, fmax).astype(np.float64)
    return np.log(np.maximum(fb @ mag.T, 1e-5)).astype(np.float32)


def same_conv(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, dil: int = 1) -> torch.Tensor:
    """x [Cin][T], w [Cout][Cin][K] -> [Cout][T]: output t reads x[t - (K-1) dil / 2 + j dil],
    rows outside [0, T) mirrored (PyTorch padding_mode="reflect")."""
    K = w.shape[-1]
    H = (K - 1) * dil
    xp = F.pad(x[None], (H // 2, H - H // 2), mode="reflect") if H else x[None]
    return F.conv1d(xp, w, b, dilation=dil)[0]


def weighted_stats(x: torch.Tensor, w: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """x [C][T] -> (mean [C], std [C]) over time with weights w [C][T] (uniform 1/T if None)."""
    if w is None:
        w = torch.full_like(x, 1.0 / x.shape[1])
    m = (w * x).sum(1)
    v = (w * (x - m[:, None]) ** 2).sum(1)
    return m, torch.sqrt(torch.clamp(v, min=1e-12))


class SpeakerOracle:
    """The ECAPA-TDNN of one `.navi` file (f16 weights upcast to f32)."""

    C, R, SCALE, DILS = 512, 64, 8, (2, 3, 4)

    def __init__(self, path):
        self.blob = NaviBlob(path)

        def t(name):
            return torch.from_numpy(np.asarray(self.blob.f32(name), dtype=np.float32))

        self.p = {name[len(SPK):]: t(name) for name in self.blob.tensors if name.startswith(SPK)}

    def conv(self, name: str, x: torch.Tensor, dil: int = 1) -> torch.Tensor:
        return same_conv(x, self.p[name + ".weight"], self.p[name + ".bias"], dil)

    def dense(self, name: str, v: torch.Tensor) -> torch.Tensor:
        """A k=1 conv over one time step (the SE block and the fc)."""
        return self.conv(name, v[:, None])[:, 0]

    @torch.no_grad()
    def embed_mel(self, mel: np.ndarray) -> np.ndarray:
        """mel [n_mels][T] -> embedding f32[enc_dim]."""
        x = torch.from_numpy(np.ascontiguousarray(mel, dtype=np.float32))
        h = torch.relu(self.conv("blocks.0.conv", x))
        outs = []
        for bi, dil in enumerate(self.DILS):
            bp = f"blocks.{bi + 1}."
            b = torch.relu(self.conv(bp + "tdnn1.conv", h))
            parts = list(torch.split(b, self.R, dim=0))
            c = [parts[0]]
            for i in range(1, self.SCALE):
                xi = parts[i] if i == 1 else parts[i] + c[i - 1]
                c.append(torch.relu(self.conv(bp + f"res2net_block.blocks.{i - 1}.conv", xi, dil)))
            b2 = torch.relu(self.conv(bp + "tdnn2.conv", torch.cat(c, 0)))
            mean = b2.mean(1)
            g = torch.relu(self.dense(bp + "se_block.conv1", mean))
            gse = torch.sigmoid(self.dense(bp + "se_block.conv2", g))
            h = b2 * gse[:, None] + h
            outs.append(h)
        att = torch.relu(self.conv("mfa.conv", torch.cat(outs, 0)))
        m, s = weighted_stats(att)
        T = att.shape[1]
        catx = torch.cat([att, m[:, None].expand(-1, T), s[:, None].expand(-1, T)], 0)
        a = torch.tanh(torch.relu(self.conv("asp.tdnn.conv", catx)))
        a = torch.softmax(self.conv("asp.conv", a), dim=1)
        pm, ps = weighted_stats(att, a)
        return self.dense("fc", torch.cat([pm, ps], 0)).numpy().astype(np.float32)

    def embed(self, wav: np.ndarray, **mel_kw) -> np.ndarray:
        return self.embed_mel(log_mel(wav, **mel_kw))
