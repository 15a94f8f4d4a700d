"""Pins the oracle's code-predictor wiring (oracle/model.py `Oracle.code_predictor`) against an
independent implementation: transformers' Qwen3-Omni talker code predictor
(`Qwen3OmniMoeTalkerCodePredictorModelForConditionalGeneration`,
transformers/models/qwen3_omni_moe/modeling_qwen3_omni_moe.py:2534-2612), the same architecture
as Qwen3-TTS's: a 2-row prefill of [talker post-norm hidden, talker codec_embedding(cb0)], then one
row per generation step whose input is codec_embedding[step - 1](previous code), scored by
lm_head[step] (reference: model/qwen3tts/frame.hip:458-500).

Built from a local config with random weights (no checkpoint). Greedy (argmax) codes and every
position's logits must agree; planted mistakes in the oracle's wiring (lm_head[pos] instead of
lm_head[pos - 1], the embedding table one off, a step written at the previous position, the cp's
own table for position 1 instead of the talker's) must each break the agreement. (A uniform shift
of every position is invisible by construction: RoPE scores depend on position differences only.)
"""
import numpy as np
import pytest
import torch

from oracle import model as M
from oracle import sampler as osamp

H, FF, NL, NH, NKV, HD, V, VT, G = 64, 128, 2, 4, 2, 16, 40, 56, 8


def _pair(seed=0):
    from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import \
        Qwen3OmniMoeTalkerCodePredictorConfig
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import \
        Qwen3OmniMoeTalkerCodePredictorModelForConditionalGeneration as CP
    cfg = Qwen3OmniMoeTalkerCodePredictorConfig(
        vocab_size=V, hidden_size=H, intermediate_size=FF, num_hidden_layers=NL, num_attention_heads=NH,
        num_key_value_heads=NKV, head_dim=HD, rms_norm_eps=1e-6,
        rope_parameters={"rope_type": "default", "rope_theta": 1e6}, num_code_groups=G)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    model = CP(cfg).eval()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() == 2:
                p.copy_(torch.randn_like(p) * (0.5 if "embedding" in name else 0.15))
            else:
                p.copy_(1.0 + 0.3 * torch.randn_like(p))
    o = M.Oracle.__new__(M.Oracle)
    o.n_groups = G
    o.cpp = M.Xf(H, NL, NH, NKV, HD, FF, V, 1e-6, 1e6)
    o.invf_c = M.inv_freq(1e6, HD)
    d = lambda t: t.detach().clone()
    o.cp = []
    for L in model.model.layers:
        a = L.self_attn
        o.cp.append(M.LayerW(d(L.input_layernorm.weight), d(L.post_attention_layernorm.weight), d(a.q_norm.weight),
                             d(a.k_norm.weight), d(a.q_proj.weight), d(a.k_proj.weight), d(a.v_proj.weight),
                             d(a.o_proj.weight), d(L.mlp.gate_proj.weight), d(L.mlp.up_proj.weight),
                             d(L.mlp.down_proj.weight)))
    o.cp_norm = d(model.model.norm.weight)
    o.cp_emb = [d(e.weight) for e in model.model.codec_embedding]
    o.lm_head = [d(h.weight) for h in model.lm_head]
    g = torch.Generator().manual_seed(seed + 100)
    o.codec_emb = torch.randn(VT, H, generator=g) * 0.5          # the talker's own codec table
    hidden = torch.randn(H, generator=g)
    return model, cfg, o, hidden


@torch.no_grad()
def _library_greedy(model, cfg, talker_emb_row, hidden, cb0):
    """Greedy generation with the library model, step by step with its KV cache."""
    from transformers import DynamicCache
    cache = DynamicCache(config=cfg)
    out = model(inputs_embeds=torch.stack([hidden, talker_emb_row])[None], past_key_values=cache, use_cache=True)
    logits = [out.logits[0, -1].numpy()]
    codes = [cb0, int(np.argmax(logits[-1]))]
    for step in range(1, G - 1):
        out = model(input_ids=torch.tensor([[codes[-1]]]), past_key_values=cache, use_cache=True,
                    generation_steps=step)
        logits.append(out.logits[0, -1].numpy())
        codes.append(int(np.argmax(logits[-1])))
    return codes, logits


def _oracle_greedy(o, hidden, cb0):
    dbg = {}
    s = osamp.Sampling(temperature=0.0, cp_temperature=0.0)
    codes = o.code_predictor(hidden.numpy(), cb0, s, 0, debug=dbg)
    return codes, dbg["cp_logits"]


def _max_logit_diff(a, b):
    return max(float(np.abs(np.asarray(x, np.float64) - np.asarray(y, np.float64)).max()) for x, y in zip(a, b))


@pytest.fixture
def no_f16_cache(monkeypatch):
    monkeypatch.setattr(M, "f16_round", lambda t: t)     # the library keeps its cache in f32


@pytest.mark.parametrize("seed,cb0", [(0, 3), (1, 17), (2, 51)])
def test_code_predictor_matches_transformers(no_f16_cache, seed, cb0):
    model, cfg, o, hidden = _pair(seed)
    want_codes, want_lg = _library_greedy(model, cfg, o.codec_emb[cb0], hidden, cb0)
    got_codes, got_lg = _oracle_greedy(o, hidden, cb0)
    err = _max_logit_diff(got_lg, want_lg)
    scale = max(float(np.abs(x).max()) for x in want_lg)
    print(f"seed {seed}: codes {got_codes} (library {want_codes}), max |dlogit| {err:.2e} of {scale:.2f}")
    assert got_codes == want_codes
    assert err < 2e-5 * max(1.0, scale)
    assert len(set(got_codes[1:])) > 2          # the comparison is not degenerate


def _planted(o, kind):
    if kind == "lm_head[pos]":
        o.lm_head = o.lm_head[1:] + o.lm_head[:1]
    elif kind == "cp_emb[pos-1]":
        o.cp_emb = o.cp_emb[1:] + o.cp_emb[:1]
    elif kind == "step position one back":
        inner = M.Oracle.cp_layers
        o.cp_layers = lambda x, ckv, pos0: inner(o, x, ckv, pos0 - 1 if pos0 >= 2 else pos0)
    elif kind == "cp table at position 1":
        o.codec_emb = torch.cat([o.cp_emb[0], o.codec_emb[V:]])
    return o


@pytest.mark.parametrize("kind", ["lm_head[pos]", "cp_emb[pos-1]", "step position one back",
                                  "cp table at position 1"])
def test_code_predictor_pin_detects_wiring_mistakes(no_f16_cache, kind):
    model, cfg, o, hidden = _pair(0)
    cb0 = 3
    _, want_lg = _library_greedy(model, cfg, o.codec_emb[cb0], hidden, cb0)
    _, got_lg = _oracle_greedy(_planted(o, kind), hidden, cb0)
    err = _max_logit_diff(got_lg, want_lg)
    print(f"planted {kind}: max |dlogit| {err:.2e}")
    assert err > 1e-2
