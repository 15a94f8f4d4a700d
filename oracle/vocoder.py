"""The codec decoder (vocoder) on the CPU: codes [T][16] -> 24 kHz PCM [T * 1920].

Test infrastructure (see oracle/__init__.py). A one-shot restatement in PyTorch f32 (f16 weights
as stored, upcast) of the reference's streaming decoder, model/qwen3tts/vocoder.hip:261-343 with
the conv semantics of kernels.h:72-242:

* `rvq_embed`     - k_rvq (vocoder.hip:125-143): [cb_first[c0] | sum_{q=1..15} cb_rest[q-1][c_q]],
                    then the two output projections as one k=1 conv over the concatenation;
* `causal_conv`   - k_conv: y[t] = bias + sum_{ci,j} W[co][ci][j] x[t - (K-1-j) dil][ci], zero history;
* `trans_conv`    - ConvTranspose1d with stride s, kernel k, output trimmed on the right by k - s
                    (transposed_phases, vocoder.hip:369-385);
* `snake`         - PRO_SNAKE (kernels.h:120-126): x + sin^2(x e^alpha) / (e^beta + 1e-9);
* `convnext`      - k_dwconv_ln + pwconv1 (GELU, erf form) + pwconv2 * gamma + residual
                    (vocoder.hip:20-54, 320-327);
* `transformer_layer` - RMSNorm (eps 1e-5) -> q/k/v -> RoPE (theta 1e4, rotate-half) -> causal
                    attention over the last `window` positions (k_attention, vocoder.hip:87-122) ->
                    o * attn_scale + x -> RMSNorm -> SwiGLU -> down * mlp_scale + x (vocoder.hip:290-302);
* `Vocoder.decode` - the whole chain (decode_chunk, vocoder.hip:280-342), clamp to [-1, 1].
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from .model import inv_freq, rmsnorm, rope
from .navi_read import NaviBlob

F32 = np.float32
DEC = "codec.decoder."


def snake(x: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
    """x [C][T]; alpha/beta [C] as stored (log scale)."""
    a = torch.exp(alpha)[:, None]
    b = 1.0 / (torch.exp(beta)[:, None] + 1e-9)
    return x + b * torch.sin(x * a) ** 2


def causal_conv(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, dil: int = 1) -> torch.Tensor:
    """x [Cin][T], w [Cout][Cin][K] -> [Cout][T], left zero padding (K-1)*dil."""
    K = w.shape[-1]
    xp = F.pad(x[None], ((K - 1) * dil, 0))
    return F.conv1d(xp, w, b, dilation=dil)[0]


def trans_conv(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, s: int) -> torch.Tensor:
    """x [Cin][T], w [Cin][Cout][k] -> [Cout][T * s] (right trim k - s)."""
    T = x.shape[-1]
    return F.conv_transpose1d(x[None], w, b, stride=s)[0][:, :T * s]


def convnext(x: torch.Tensor, p: dict) -> torch.Tensor:
    """x [C][T]."""
    C = x.shape[0]
    h = F.conv1d(F.pad(x[None], (6, 0)), p["dw"], p["dw_b"], groups=C)[0]            # causal depthwise k7
    h = F.layer_norm(h.T, (C,), p["ln_w"], p["ln_b"], eps=1e-6)                        # [T][C]
    h = F.gelu(F.linear(h, p["pw1"], p["pw1_b"]))                                       # erf form
    h = F.linear(h, p["pw2"], p["pw2_b"]) * p["gamma"]
    return x + h.T


def transformer_layer(x: torch.Tensor, w: dict, n_head: int, head_dim: int, eps: float, invf: torch.Tensor,
                      window: int, pos0: int = 0) -> torch.Tensor:
    """x [T][H] at positions pos0..; one-shot (no cache): keys are the rows of x itself."""
    T = x.shape[0]
    xn = rmsnorm(x, w["ln1"], eps)
    q = F.linear(xn, w["wq"]).view(T, n_head, head_dim)
    k = F.linear(xn, w["wk"]).view(T, n_head, head_dim)
    v = F.linear(xn, w["wv"]).view(T, n_head, head_dim)
    pos = torch.arange(pos0, pos0 + T)
    q, k = rope(q, pos, invf), rope(k, pos, invf)
    s = torch.einsum("thd,jhd->htj", q.double(), k.double()) / np.sqrt(head_dim)
    i = torch.arange(T)
    allowed = (i[None, :] <= i[:, None]) & (i[:, None] - i[None, :] < window)
    s = s.masked_fill(~allowed[None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    att = torch.einsum("htj,jhd->thd", p, v.double()).float().reshape(T, n_head * head_dim)
    x = (x.double() + F.linear(att, w["wo"]).double() * w["attn_scale"].double()).float()
    xn = rmsnorm(x, w["ln2"], eps)
    g = F.linear(xn, w["wg"]).double()
    u = F.linear(xn, w["wu"]).double()
    h = (g / (1.0 + torch.exp(-g)) * u).float()
    return (x.double() + F.linear(h, w["wd"]).double() * w["mlp_scale"].double()).float()


class Vocoder:
    def __init__(self, path_or_blob):
        self.blob = b = path_or_blob if isinstance(path_or_blob, NaviBlob) else NaviBlob(path_or_blob)
        kv = b.kv
        t = lambda n: torch.from_numpy(b.f32(DEC + n))
        self.n_q = kv["codec.decoder.num_quantizers"]
        self.n_sem = kv["codec.decoder.num_semantic_quantizers"]
        self.window = kv["codec.decoder.sliding_window"]
        self.hidden = kv["codec.decoder.hidden_size"]
        self.n_head = kv["codec.decoder.num_attention_heads"]
        self.head_dim = kv["codec.decoder.head_dim"]
        self.eps = float(kv["codec.decoder.rms_norm_eps"])
        self.invf = inv_freq(float(kv["codec.decoder.rope_theta"]), self.head_dim)
        self.ratios = list(kv["codec.decoder.upsampling_ratios"])
        self.rates = list(kv["codec.decoder.upsample_rates"])
        self.samples_per_frame = kv["codec.decode_upsample_rate"]
        q = "quantizer."
        self.cb_first = t(q + "rvq_first.vq.layers.0._codebook.codebook")
        self.cb_rest = [t(q + f"rvq_rest.vq.layers.{i}._codebook.codebook") for i in range(self.n_q - self.n_sem)]
        self.proj_first = t(q + "rvq_first.output_proj.weight")[:, :, 0]
        self.proj_rest = t(q + "rvq_rest.output_proj.weight")[:, :, 0]
        self.pre_conv = (t("pre_conv.conv.weight"), t("pre_conv.conv.bias"))
        pt = "pre_transformer."
        self.in_proj = (t(pt + "input_proj.weight"), t(pt + "input_proj.bias"))
        self.out_proj = (t(pt + "output_proj.weight"), t(pt + "output_proj.bias"))
        self.final_norm = t(pt + "norm.weight")
        self.layers = []
        for l in range(kv["codec.decoder.num_hidden_layers"]):
            lp = pt + f"layers.{l}."
            self.layers.append({
                "ln1": t(lp + "input_layernorm.weight"), "ln2": t(lp + "post_attention_layernorm.weight"),
                "wq": t(lp + "self_attn.q_proj.weight"), "wk": t(lp + "self_attn.k_proj.weight"),
                "wv": t(lp + "self_attn.v_proj.weight"), "wo": t(lp + "self_attn.o_proj.weight"),
                "wg": t(lp + "mlp.gate_proj.weight"), "wu": t(lp + "mlp.up_proj.weight"),
                "wd": t(lp + "mlp.down_proj.weight"),
                "attn_scale": t(lp + "self_attn_layer_scale.scale"), "mlp_scale": t(lp + "mlp_layer_scale.scale")})
        self.ups = []
        for j in range(len(self.ratios)):
            up = f"upsample.{j}."
            self.ups.append(((t(up + "0.conv.weight"), t(up + "0.conv.bias")), {
                "dw": t(up + "1.dwconv.conv.weight"), "dw_b": t(up + "1.dwconv.conv.bias"),
                "ln_w": t(up + "1.norm.weight"), "ln_b": t(up + "1.norm.bias"),
                "pw1": t(up + "1.pwconv1.weight"), "pw1_b": t(up + "1.pwconv1.bias"),
                "pw2": t(up + "1.pwconv2.weight"), "pw2_b": t(up + "1.pwconv2.bias"), "gamma": t(up + "1.gamma")}))
        self.dec0 = (t("decoder.0.conv.weight"), t("decoder.0.conv.bias"))
        self.blocks = []
        for i in range(len(self.rates)):
            bp = f"decoder.{i + 1}.block."
            units = []
            for r in range(3):
                rp = bp + f"{2 + r}."
                units.append({"a1": (t(rp + "act1.alpha"), t(rp + "act1.beta")),
                              "c1": (t(rp + "conv1.conv.weight"), t(rp + "conv1.conv.bias")),
                              "a2": (t(rp + "act2.alpha"), t(rp + "act2.beta")),
                              "c2": (t(rp + "conv2.conv.weight"), t(rp + "conv2.conv.bias"))})
            self.blocks.append({"snake": (t(bp + "0.alpha"), t(bp + "0.beta")),
                                "up": (t(bp + "1.conv.weight"), t(bp + "1.conv.bias")), "units": units})
        n = len(self.rates)
        self.tail_snake = (t(f"decoder.{n + 1}.alpha"), t(f"decoder.{n + 1}.beta"))
        self.final_conv = (t(f"decoder.{n + 2}.conv.weight"), t(f"decoder.{n + 2}.conv.bias"))

    def rvq_embed(self, codes: np.ndarray) -> torch.Tensor:
        """codes [T][16] -> [T][512]."""
        c = torch.from_numpy(np.asarray(codes, np.int64))
        first = self.cb_first[c[:, 0]]
        rest = torch.zeros_like(first)
        for q in range(1, self.n_q):
            rest = rest + self.cb_rest[q - 1][c[:, q]]
        return F.linear(first, self.proj_first) + F.linear(rest, self.proj_rest)

    def stages(self, codes: np.ndarray) -> dict:
        """Every intermediate of decode, time-major [T'][C] (for stage-by-stage comparison)."""
        out = {}
        h = self.rvq_embed(codes)                                       # [T][512]
        out["rvq"] = h
        a = causal_conv(h.T, *self.pre_conv).T                          # [T][1024]
        out["pre_conv"] = a
        x = F.linear(a, *self.in_proj)
        for l, w in enumerate(self.layers):
            x = transformer_layer(x, w, self.n_head, self.head_dim, self.eps, self.invf, self.window)
            out[f"layer{l}"] = x
        x = F.linear(rmsnorm(x, self.final_norm, self.eps), *self.out_proj)
        out["pre_transformer"] = x
        y = x.T                                                         # [C][T]
        for j, (upw, cx) in enumerate(self.ups):
            y = trans_conv(y, upw[0], upw[1], self.ratios[j])
            y = convnext(y, cx)
            out[f"up{j}"] = y.T
        y = causal_conv(y, *self.dec0)
        out["dec0"] = y.T
        for i, bk in enumerate(self.blocks):
            y = trans_conv(snake(y, *bk["snake"]), bk["up"][0], bk["up"][1], self.rates[i])
            for r, u in enumerate(bk["units"]):
                z = causal_conv(snake(y, *u["a1"]), *u["c1"], dil=(1, 3, 9)[r])
                y = y + causal_conv(snake(z, *u["a2"]), *u["c2"])
            out[f"block{i + 1}"] = y.T
        pcm = causal_conv(snake(y, *self.tail_snake), *self.final_conv).clamp(-1.0, 1.0)
        out["pcm"] = pcm[0]
        return out

    def decode(self, codes: np.ndarray) -> np.ndarray:
        with torch.no_grad():
            return self.stages(codes)["pcm"].numpy().astype(F32)
