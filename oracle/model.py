"""Talker decode step, code-predictor pass, prompt assembly and prefill on the CPU.

Test infrastructure (see oracle/__init__.py). Restates, in PyTorch f32 on the CPU:
* `rmsnorm`           - block_rmsnorm / k_rmsnorm: x * rsqrt(mean(x^2) + eps) * w
                        (model/qwen3tts/frame.hip:107-114, kernels.h:342-350);
* `inv_freq`, `rope`  - rotate-half RoPE, pair (i, i + hd/2), angle = f32(pos) * f32(theta^(-2i/hd))
                        (frame.hip:327-334, talker.hip:64-73);
* `decoder_layer`     - RMSNorm -> q/k/v -> per-head q/k RMSNorm -> RoPE -> f16 K/V store ->
                        causal GQA attention -> o + residual -> RMSNorm -> SiLU(g)*u -> down + residual
                        (frame.hip:300-402 and 539-549 for one row; talker.hip:362-389 for T rows);
* `Oracle.talker_step` - frame.hip:537-550 (talker phases of k_frame);
* `Oracle.code_predictor` - frame.hip:554-575 (16 positions, lm_head[pos-1], cp KV per frame);
* `Oracle.assemble_step` - frame.hip:503-513 (f32 adds in the kernel's order);
* `text_projection`   - talker.hip:333-335 (fc1 -> SiLU -> fc2, both with bias);
* `Oracle.build_prompt` - talker.hip:283-352 (10-row prefill layout, trailing rows, tts_pad);
* `Oracle.prefill`    - talker.hip:354-399;
* `Oracle.frame`      - one frame: run_first / run of frame.hip:787-810 with Impl::launch's seeds (653-659).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import rng, sampler
from .navi_read import NaviBlob

F32 = np.float32


@dataclass
class Xf:
    hidden: int
    n_layer: int
    n_head: int
    n_kv_head: int
    head_dim: int
    ff: int
    vocab: int
    eps: float
    theta: float

    @staticmethod
    def from_kv(kv: dict, ns: str) -> "Xf":
        return Xf(kv[f"{ns}.hidden_size"], kv[f"{ns}.num_hidden_layers"], kv[f"{ns}.num_attention_heads"],
                  kv[f"{ns}.num_key_value_heads"], kv[f"{ns}.head_dim"], kv[f"{ns}.intermediate_size"],
                  kv.get(f"{ns}.vocab_size", 0), float(kv[f"{ns}.rms_norm_eps"]), float(kv[f"{ns}.rope_theta"]))


def f16_round(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float16).to(torch.float32)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    x64 = x.double()
    scale = torch.rsqrt(torch.mean(x64 * x64, dim=-1, keepdim=True) + eps)
    return (x64 * scale * w.double()).float()


def inv_freq(theta: float, hd: int) -> torch.Tensor:
    """f32(1 / theta^(2i/hd)) computed in double (talker.hip:67)."""
    i = np.arange(hd // 2, dtype=np.float64)
    return torch.from_numpy((1.0 / np.power(theta, 2.0 * i / hd)).astype(F32))


def rope(x: torch.Tensor, pos: torch.Tensor, invf: torch.Tensor) -> torch.Tensor:
    """x: [T, heads, hd]; pos: [T] int. Angle in f32, sin/cos in f64, rotate-half."""
    half = x.shape[-1] // 2
    ang = (pos.to(torch.float32)[:, None] * invf[None, :]).double()      # f32 product, exact in f64
    c, s = torch.cos(ang).float()[:, None, :], torch.sin(ang).float()[:, None, :]
    x0, x1 = x[..., :half].double(), x[..., half:].double()
    c, s = c.double(), s.double()
    return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1).float()


@dataclass
class LayerW:
    ln1: torch.Tensor
    ln2: torch.Tensor
    qn: torch.Tensor
    kn: torch.Tensor
    wq: torch.Tensor
    wk: torch.Tensor
    wv: torch.Tensor
    wo: torch.Tensor
    wg: torch.Tensor
    wu: torch.Tensor
    wd: torch.Tensor


def load_layers(blob: NaviBlob, prefix: str, n: int) -> list[LayerW]:
    t = lambda name: torch.from_numpy(blob.f32(name))
    out = []
    for l in range(n):
        p = f"{prefix}.layers.{l}."
        out.append(LayerW(t(p + "input_layernorm.weight"), t(p + "post_attention_layernorm.weight"),
                          t(p + "self_attn.q_norm.weight"), t(p + "self_attn.k_norm.weight"),
                          t(p + "self_attn.q_proj.weight"), t(p + "self_attn.k_proj.weight"),
                          t(p + "self_attn.v_proj.weight"), t(p + "self_attn.o_proj.weight"),
                          t(p + "mlp.gate_proj.weight"), t(p + "mlp.up_proj.weight"), t(p + "mlp.down_proj.weight")))
    return out


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.linear(x, w)


def silu(a: torch.Tensor) -> torch.Tensor:
    return a / (1.0 + torch.exp(-a))


def text_projection(rows: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor,
                    b2: torch.Tensor) -> torch.Tensor:
    """talker.hip:333-335: fc2(SiLU(fc1(rows) + b1)) + b2 (the gemm's EPI_SILU epilogue on fc1,
    kernels.h:262-350); f32 products, bias and activation in f64, rounded to f32 per stage."""
    a = silu(linear(rows, w1).double() + b1.double()).float()
    return (linear(a, w2).double() + b2.double()).float()


def decoder_layer(P: Xf, w: LayerW, x: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int,
                  invf: torch.Tensor) -> torch.Tensor:
    """x: [T, hidden] rows at positions pos0..pos0+T-1; kc/vc: [max_pos, n_kv*hd] f32 holding
    f16-rounded values, written in place at those positions. Returns the new x."""
    T = x.shape[0]
    hd, nh, nkv = P.head_dim, P.n_head, P.n_kv_head
    xn = rmsnorm(x, w.ln1, P.eps)
    q = linear(xn, w.wq).view(T, nh, hd)
    k = linear(xn, w.wk).view(T, nkv, hd)
    v = linear(xn, w.wv).view(T, nkv, hd)
    q = rmsnorm(q, w.qn, P.eps)
    k = rmsnorm(k, w.kn, P.eps)
    pos = torch.arange(pos0, pos0 + T)
    q = rope(q, pos, invf)
    k = rope(k, pos, invf)
    kc[pos0:pos0 + T] = f16_round(k.reshape(T, nkv * hd))
    vc[pos0:pos0 + T] = f16_round(v.reshape(T, nkv * hd))
    n = pos0 + T
    K = kc[:n].view(n, nkv, hd).double()
    V = vc[:n].view(n, nkv, hd).double()
    grp = nh // nkv
    scale = 1.0 / np.sqrt(hd)
    att = torch.empty(T, nh, hd, dtype=torch.float64)
    for t in range(T):
        m = pos0 + t + 1
        for h in range(nh):
            g = h // grp
            s = (K[:m, g, :] @ q[t, h].double()) * scale
            s = s.float().double()
            e = torch.exp(s - s.max())
            p = e / e.sum()
            att[t, h] = p @ V[:m, g, :]
    att = att.float().view(T, nh * hd)
    x = (x.double() + linear(att, w.wo).double()).float()
    xn = rmsnorm(x, w.ln2, P.eps)
    g = linear(xn, w.wg).double()
    u = linear(xn, w.wu).double()
    hmid = (g / (1.0 + torch.exp(-g)) * u).float()
    return (x.double() + linear(hmid, w.wd).double()).float()


class Oracle:
    """CPU model over a random-init (or converted) `.navi` blob."""

    def __init__(self, path_or_blob, threads: int | None = None):
        if threads:
            torch.set_num_threads(threads)
        self.blob = b = path_or_blob if isinstance(path_or_blob, NaviBlob) else NaviBlob(path_or_blob)
        kv = b.kv
        self.kv = kv
        self.tp = Xf.from_kv(kv, "talker")
        self.cpp = Xf.from_kv(kv, "cp")
        self.n_groups = kv["talker.num_code_groups"]
        self.eos_id = kv["talker.codec_eos_token_id"]
        t = lambda name: torch.from_numpy(b.f32(name))
        self.talker = load_layers(b, "talker.model", self.tp.n_layer)
        self.talker_norm = t("talker.model.norm.weight")
        self.codec_head = t("talker.codec_head.weight")
        self.codec_emb = t("talker.model.codec_embedding.weight")
        self.cp = load_layers(b, "talker.code_predictor.model", self.cpp.n_layer)
        self.cp_norm = t("talker.code_predictor.model.norm.weight")
        self.cp_emb = [t(f"talker.code_predictor.model.codec_embedding.{i}.weight") for i in range(self.n_groups - 1)]
        self.lm_head = [t(f"talker.code_predictor.lm_head.{i}.weight") for i in range(self.n_groups - 1)]
        self.invf_t = inv_freq(self.tp.theta, self.tp.head_dim)
        self.invf_c = inv_freq(self.cpp.theta, self.cpp.head_dim)
        self.seen = np.zeros(self.tp.vocab, dtype=bool)

    # -- KV cache ----------------------------------------------------------
    def new_kv(self, max_pos: int = 2048):
        kvd = self.tp.n_kv_head * self.tp.head_dim
        return [(torch.zeros(max_pos, kvd), torch.zeros(max_pos, kvd)) for _ in range(self.tp.n_layer)]

    # -- talker --------------------------------------------------------------
    def talker_forward(self, x: torch.Tensor, kv, pos0: int):
        """x: [T, hidden]. Returns (post-norm hidden rows, logits rows)."""
        for l, w in enumerate(self.talker):
            x = decoder_layer(self.tp, w, x, kv[l][0], kv[l][1], pos0, self.invf_t)
        h = rmsnorm(x, self.talker_norm, self.tp.eps)
        return h, linear(h, self.codec_head)

    def talker_step(self, step_in: np.ndarray, kv, n_past: int):
        h, lg = self.talker_forward(torch.from_numpy(np.asarray(step_in, F32)).view(1, -1), kv, n_past)
        return h[0].numpy(), lg[0].numpy()

    # -- code predictor ------------------------------------------------------
    def cp_layers(self, x: torch.Tensor, ckv, pos0: int) -> torch.Tensor:
        for l, w in enumerate(self.cp):
            x = decoder_layer(self.cpp, w, x, ckv[l][0], ckv[l][1], pos0, self.invf_c)
        return x

    def code_predictor(self, hidden: np.ndarray, cb0: int, s: sampler.Sampling, cp_seed: int, debug=None, force=None):
        """codes[1..15] from the talker's post-norm hidden and cb0 (positions 0 and 1 run as one
        2-row pass; causal, so identical to two single-row passes). With `force` (16 codes), the
        oracle records its own choice at each position in debug["cp_choice"] and continues with
        the forced code (teacher forcing, so a comparison survives a near-tie flip)."""
        G = self.n_groups
        kvd = self.cpp.n_kv_head * self.cpp.head_dim
        ckv = [(torch.zeros(G, kvd), torch.zeros(G, kvd)) for _ in range(self.cpp.n_layer)]
        codes = [cb0]
        x = torch.stack([torch.from_numpy(np.asarray(hidden, F32)), self.codec_emb[cb0]])
        x = self.cp_layers(x, ckv, 0)[1:2]
        for pos in range(1, G):
            if pos >= 2:
                x = self.cp_layers(self.cp_emb[pos - 2][codes[pos - 1]].view(1, -1), ckv, pos)
            h = rmsnorm(x, self.cp_norm, self.cpp.eps)
            lg = linear(h, self.lm_head[pos - 1])[0].numpy()
            if debug is not None:
                debug.setdefault("cp_logits", []).append(lg)
            c = sampler.sample_cp(lg, s, cp_seed, pos)
            if debug is not None:
                debug.setdefault("cp_choice", []).append(c)
            codes.append(int(force[pos]) if force is not None else c)
        return codes

    def assemble_step(self, codes, trailing: np.ndarray) -> np.ndarray:
        v = self.codec_emb[codes[0]].numpy().astype(F32).copy()
        for cb in range(self.n_groups - 1):
            v = (v + self.cp_emb[cb][codes[cb + 1]].numpy()).astype(F32)
        return (v + np.asarray(trailing, F32)).astype(F32)

    # -- one frame -----------------------------------------------------------
    def reset(self):
        self.seen[:] = False

    def frame(self, s: sampler.Sampling, seed: int, frame_index: int, trailing: np.ndarray, *,
              kv=None, n_past: int | None = None, step_in=None, hidden=None, logits=None, debug=None, force=None):
        """run_first (hidden/logits given) or run (kv, n_past, step_in). Returns (codes, step_out).
        With `force` (16 codes): teacher forcing; the oracle's own choices go to debug["cb0_choice"]
        and debug["cp_choice"], the forced codes drive the repetition set, the code predictor and
        the next step. debug["cb0_scores"] holds the modified logits cb0 is chosen from, debug["modify"]
        applies the same modification (this frame's repetition set and gates) to other logits."""
        if hidden is None:
            hidden, logits = self.talker_step(step_in, kv, n_past)
        if debug is not None:
            debug["hidden"], debug["logits"] = np.asarray(hidden, F32), np.asarray(logits, F32)
            debug["cb0_scores"] = sampler.talker_modified_logits(logits, self.seen, self.eos_id, self.tp.vocab - 1024,
                                                                 frame_index, s.min_frames, s.repetition_penalty)
            seen0 = self.seen.copy()
            debug["modify"] = lambda lg: sampler.talker_modified_logits(lg, seen0, self.eos_id, self.tp.vocab - 1024,
                                                                        frame_index, s.min_frames, s.repetition_penalty)
        tseed, cseed = rng.frame_seeds(seed, frame_index)
        cb0 = sampler.sample_talker(logits, self.seen, s, tseed, frame_index, self.eos_id, self.tp.vocab - 1024)
        if debug is not None:
            debug["cb0_choice"] = cb0
        if force is not None:
            cb0 = int(force[0])
        if cb0 != self.eos_id:
            self.seen[cb0] = True
        codes = self.code_predictor(hidden, cb0, s, cseed, debug, force)
        return codes, self.assemble_step(codes, trailing)

    # -- prompt + prefill ----------------------------------------------------
    def build_prompt(self, ids, language: str, speaker: np.ndarray):
        """talker.hip:283-352. Returns (prefill rows, trailing rows, tts_pad row) as f32 arrays."""
        kv, b = self.kv, self.blob
        ids = [int(i) for i in ids]
        n_text = len(ids) - 8
        if n_text < 1:
            raise ValueError("empty text")
        tids = ids[:3] + ids[3:3 + n_text]
        i_bos, i_eos, i_pad = len(tids), len(tids) + 1, len(tids) + 2
        tids += [kv["text.tts_bos_id"], kv["text.tts_eos_id"], kv["text.tts_pad_id"]]
        table = b.array("talker.model.text_embedding.weight")
        rows = torch.from_numpy(table[np.asarray(tids)].astype(F32))
        t = lambda name: torch.from_numpy(b.f32(name))
        tp = "talker.text_projection."
        proj = text_projection(rows, t(tp + "linear_fc1.weight"), t(tp + "linear_fc1.bias"),
                               t(tp + "linear_fc2.weight"), t(tp + "linear_fc2.bias")).numpy()
        if language in ("", "auto"):
            cids = [kv["talker.codec_nothink_id"], kv["talker.codec_think_bos_id"], kv["talker.codec_think_eos_id"]]
        else:
            cids = [kv["talker.codec_think_id"], kv["talker.codec_think_bos_id"], kv[f"talker.language.{language}"],
                    kv["talker.codec_think_eos_id"]]
        n_think = len(cids)
        cids += [kv["talker.codec_pad_id"], kv["talker.codec_bos_id"]]
        crow = self.codec_emb.numpy()[np.asarray(cids)]
        spk = np.asarray(speaker, F32)
        pre = [proj[r] for r in range(3)]
        pre += [(proj[i_pad] + crow[r]).astype(F32) for r in range(n_think)]
        pre.append((proj[i_pad] + spk).astype(F32))
        pre.append((proj[i_bos] + crow[n_think]).astype(F32))
        pre.append((proj[3] + crow[n_think + 1]).astype(F32))
        trail = [proj[3 + r] for r in range(1, n_text)] + [proj[i_eos]]
        return np.stack(pre).astype(F32), np.stack(trail).astype(F32), proj[i_pad].astype(F32)

    def prefill(self, prefill_rows: np.ndarray, kv):
        """talker.hip:354-399: rows at positions 0..T-1; returns (hidden, logits) of the last row."""
        h, lg = self.talker_forward(torch.from_numpy(np.asarray(prefill_rows, F32)), kv, 0)
        return h[-1].numpy(), lg[-1].numpy()
