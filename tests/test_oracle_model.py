"""Pins the oracle's transformer layer and frame assembly (oracle/model.py).

* decoder_layer against an independent implementation: transformers' Qwen3DecoderLayer (same
  QK-norm structure), built from a local Qwen3Config with random weights and non-unit norms;
* decode-vs-prefill invariant: T rows as one prefill == T sequential one-row steps (rows and
  the f16 K/V cache rows);
* RoPE: identity at position 0, norm preserving, scores depend only on the position difference;
* RMSNorm closed form on a constant vector;
* assemble_step: the f32 sum order codec_emb[cb0] + cp_emb[0][c1] + ... + trailing.
"""
import numpy as np
import pytest
import torch

from oracle import model as M

F32 = np.float32


def _qwen3_pair(seed=0, T=7):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer, Qwen3RotaryEmbedding
    H, nh, nkv, hd, ff = 256, 4, 2, 64, 512
    cfg = Qwen3Config(hidden_size=H, intermediate_size=ff, num_attention_heads=nh, num_key_value_heads=nkv,
                      head_dim=hd, rms_norm_eps=1e-6, rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                      num_hidden_layers=1, attention_bias=False)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    layer = Qwen3DecoderLayer(cfg, 0).eval()
    with torch.no_grad():
        for p in layer.parameters():
            if p.dim() == 2:
                p.copy_(torch.randn_like(p) * 0.05)
            else:
                p.copy_(1.0 + 0.3 * torch.randn_like(p))
    P = M.Xf(H, 1, nh, nkv, hd, ff, 0, 1e-6, 1e6)
    a = layer.self_attn
    w = M.LayerW(layer.input_layernorm.weight.detach(), layer.post_attention_layernorm.weight.detach(),
                 a.q_norm.weight.detach(), a.k_norm.weight.detach(), a.q_proj.weight.detach(), a.k_proj.weight.detach(),
                 a.v_proj.weight.detach(), a.o_proj.weight.detach(), layer.mlp.gate_proj.weight.detach(),
                 layer.mlp.up_proj.weight.detach(), layer.mlp.down_proj.weight.detach())
    return cfg, layer, Qwen3RotaryEmbedding(cfg), P, w


def test_decoder_layer_matches_transformers_qwen3(monkeypatch):
    monkeypatch.setattr(M, "f16_round", lambda t: t)      # the library layer keeps K/V in f32
    T = 7
    cfg, layer, rot, P, w = _qwen3_pair(T=T)
    x = torch.randn(T, cfg.hidden_size)
    pos = torch.arange(T)[None]
    mask = torch.full((T, T), float("-inf")).triu(1)[None, None]
    with torch.no_grad():
        cos, sin = rot(x[None], pos)
        want = layer(x[None], attention_mask=mask, position_ids=pos, position_embeddings=(cos, sin))
        want = want[0] if isinstance(want, tuple) else want
    kvd = P.n_kv_head * P.head_dim
    kc, vc = torch.zeros(16, kvd), torch.zeros(16, kvd)
    got = M.decoder_layer(P, w, x, kc, vc, 0, M.inv_freq(P.theta, P.head_dim))
    err = (got - want[0]).abs().max().item()
    assert err < 2e-4 * max(1.0, want.abs().max().item()), err


def test_decoder_layer_detects_a_dropped_qk_norm(monkeypatch):
    """The comparison above is sensitive: a layer whose q_norm weight is ignored fails it."""
    monkeypatch.setattr(M, "f16_round", lambda t: t)
    T = 5
    cfg, layer, rot, P, w = _qwen3_pair(seed=1, T=T)
    x = torch.randn(T, cfg.hidden_size)
    pos = torch.arange(T)[None]
    mask = torch.full((T, T), float("-inf")).triu(1)[None, None]
    with torch.no_grad():
        cos, sin = rot(x[None], pos)
        want = layer(x[None], attention_mask=mask, position_ids=pos, position_embeddings=(cos, sin))
        want = want[0] if isinstance(want, tuple) else want
    w.qn = torch.ones_like(w.qn)
    kvd = P.n_kv_head * P.head_dim
    got = M.decoder_layer(P, w, x, torch.zeros(8, kvd), torch.zeros(8, kvd), 0, M.inv_freq(P.theta, P.head_dim))
    assert (got - want[0]).abs().max().item() > 1e-2


def test_prefill_equals_sequential_decode():
    cfg, layer, rot, P, w = _qwen3_pair(seed=2)
    invf = M.inv_freq(P.theta, P.head_dim)
    T = 9
    x = torch.randn(T, P.hidden)
    kvd = P.n_kv_head * P.head_dim
    kp, vp = torch.zeros(T, kvd), torch.zeros(T, kvd)
    yp = M.decoder_layer(P, w, x, kp, vp, 0, invf)
    ks, vs = torch.zeros(T, kvd), torch.zeros(T, kvd)
    ys = torch.cat([M.decoder_layer(P, w, x[t:t + 1], ks, vs, t, invf) for t in range(T)])
    assert torch.allclose(yp, ys, atol=1e-5, rtol=1e-5)
    # the same f16 cache rows, up to one f16 ulp where GEMM and GEMV accumulation orders round apart
    for a, b in ((kp, ks), (vp, vs)):
        assert torch.allclose(a, b, rtol=2 ** -10, atol=2 ** -24)
        assert (a != b).float().mean().item() < 0.01


def test_rope_invariants():
    invf = M.inv_freq(1e6, 128)
    r = torch.Generator().manual_seed(0)
    q = torch.randn(1, 16, 128, generator=r)
    k = torch.randn(1, 8, 128, generator=r)
    assert torch.allclose(M.rope(q, torch.tensor([0]), invf), q)
    for p in (1, 17, 300):
        rq = M.rope(q, torch.tensor([p]), invf)
        assert torch.allclose(rq.norm(dim=-1), q.norm(dim=-1), rtol=1e-5)
    # <R(m) q, R(n) k> depends on m - n only
    a = (M.rope(q[:, :1], torch.tensor([40]), invf) * M.rope(k[:, :1], torch.tensor([33]), invf)).sum()
    b = (M.rope(q[:, :1], torch.tensor([107]), invf) * M.rope(k[:, :1], torch.tensor([100]), invf)).sum()
    assert abs(a.item() - b.item()) < 1e-4
    # rotate-half pairing: dims (i, i + 64) rotate together by pos * invf[i]
    e = torch.zeros(1, 1, 128)
    e[0, 0, 3] = 1.0
    out = M.rope(e, torch.tensor([5]), invf)[0, 0]
    ang = 5.0 * float(invf[3])
    assert abs(out[3].item() - np.cos(ang)) < 1e-6 and abs(out[67].item() - np.sin(ang)) < 1e-6
    assert out.abs().sum().item() == pytest.approx(abs(np.cos(ang)) + abs(np.sin(ang)), rel=1e-6)


def test_inv_freq_closed_form():
    invf = M.inv_freq(1e6, 128).numpy()
    assert invf[0] == 1.0
    assert invf[32] == F32(1e6 ** -0.5)
    assert np.all(np.diff(invf) < 0)


def test_rmsnorm_closed_form():
    x = torch.full((1, 1024), 3.0)
    w = torch.linspace(0.5, 1.5, 1024)
    y = M.rmsnorm(x, w, 1e-6)
    want = 3.0 / np.sqrt(9.0 + 1e-6) * w.double()
    assert torch.allclose(y.double(), want[None], atol=1e-7)


def test_assemble_step_sum_order():
    class O:                      # a stand-in holding tables chosen so the order matters in f32
        n_groups = 16
    o = O()
    big, tiny = F32(2 ** 24), F32(1.0)
    o.codec_emb = torch.tensor([[big]])
    o.cp_emb = [torch.tensor([[tiny]]) for _ in range(15)]
    out = M.Oracle.assemble_step(o, [0] * 16, np.array([-big], F32))
    # left to right: 2^24 + 1 rounds back to 2^24 fifteen times, then - 2^24 = 0
    assert out[0] == 0.0
