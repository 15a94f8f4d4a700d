"""Pins the oracle's two front ends against independent implementations in transformers:

* the codec decoder's RVQ front end (`oracle.vocoder.Vocoder.rvq_embed`; reference
  model/qwen3tts/vocoder.hip:119-137 with the concatenated output projections at :554-556)
  against `MimiSplitResidualVectorQuantizer.decode` (transformers/models/mimi/modeling_mimi.py):
  one semantic codebook through its own 1x1 `output_proj`, plus the N-1 acoustic codebooks
  summed and sent through theirs. The codebooks are held as Mimi holds them (`embed_sum` over a
  non-unit `cluster_usage`); the blob stores the quotient (tools/convert.py:303-308), and that
  quotient is what the oracle is given.
* the talker's text projection (`oracle.model.text_projection`; reference
  model/qwen3tts/talker.hip:333-335, fc1 with the SiLU epilogue, then fc2) against
  `Qwen3OmniMoeTalkerResizeMLP` with `hidden_act="silu"`.

Random weights from a local config (no checkpoint). Each pin has planted-mistake controls: the
same comparison must fail for a mistaken oracle (acoustic codebook index one off, the two
projections swapped, the last acoustic codebook dropped; GELU for SiLU, fc1's or fc2's bias
dropped).
"""
import numpy as np
import pytest
import torch

from oracle import model as M
from oracle import vocoder as V

N_Q, N_SEM, CB, VQ, CD, T = 16, 1, 64, 32, 48, 7


def _mimi(seed=0):
    from transformers import MimiConfig
    from transformers.models.mimi.modeling_mimi import MimiSplitResidualVectorQuantizer
    cfg = MimiConfig(hidden_size=CD, codebook_dim=VQ, vector_quantization_hidden_dimension=VQ,
                     num_quantizers=N_Q, num_semantic_quantizers=N_SEM, codebook_size=CB)
    torch.manual_seed(seed)
    q = MimiSplitResidualVectorQuantizer(cfg).eval()
    with torch.no_grad():
        for rvq in (q.semantic_residual_vector_quantizer, q.acoustic_residual_vector_quantizer):
            for layer in rvq.layers:
                cb = layer.codebook
                cb.cluster_usage.copy_(0.5 + torch.rand(CB) * 3.0)
                cb.embed_sum.copy_(torch.randn(CB, VQ) * cb.cluster_usage[:, None])
                cb._embed = None
            rvq.output_proj.weight.copy_(torch.randn_like(rvq.output_proj.weight) * 0.2)
    return q


def _oracle_rvq(q) -> V.Vocoder:
    """A Vocoder holding only the front end's tensors, laid out as the blob stores them."""
    o = V.Vocoder.__new__(V.Vocoder)
    sem, ac = q.semantic_residual_vector_quantizer, q.acoustic_residual_vector_quantizer
    baked = lambda layer: (layer.codebook.embed_sum / layer.codebook.cluster_usage[:, None]).detach().clone()
    o.n_q, o.n_sem = N_Q, N_SEM
    o.cb_first = baked(sem.layers[0])
    o.cb_rest = [baked(l) for l in ac.layers]
    o.proj_first = sem.output_proj.weight[:, :, 0].detach().clone()
    o.proj_rest = ac.output_proj.weight[:, :, 0].detach().clone()
    return o


def _codes(seed=1):
    return np.random.default_rng(seed).integers(0, CB, (T, N_Q))


@torch.no_grad()
def _mimi_decode(q, codes):
    return q.decode(torch.from_numpy(codes.T.copy())[None].long())[0].T        # [B, K, T] -> [T][CD]


def _planted_rvq(o, kind):
    if kind == "acoustic index q instead of q-1":
        o.cb_rest = o.cb_rest[1:] + o.cb_rest[:1]
    elif kind == "projections swapped":
        o.proj_first, o.proj_rest = o.proj_rest, o.proj_first
    elif kind == "last acoustic codebook dropped":
        o.n_q = N_Q - 1
    return o


def test_rvq_embed_matches_mimi():
    q = _mimi()
    codes = _codes()
    want = _mimi_decode(q, codes)
    with torch.no_grad():
        got = _oracle_rvq(q).rvq_embed(codes)
    err = float((got - want).abs().max())
    print(f"rvq: max |d| {err:.2e} of {float(want.abs().max()):.2f}")
    assert got.shape == (T, CD)
    assert err < 1e-4


@pytest.mark.parametrize("kind", ["acoustic index q instead of q-1", "projections swapped",
                                  "last acoustic codebook dropped"])
def test_rvq_pin_detects_mistakes(kind):
    q = _mimi()
    codes = _codes()
    want = _mimi_decode(q, codes)
    with torch.no_grad():
        got = _planted_rvq(_oracle_rvq(q), kind).rvq_embed(codes)
    err = float((got - want).abs().max())
    print(f"planted {kind}: max |d| {err:.2e}")
    assert err > 1e-1


D_IN, D_MID, D_OUT, R = 40, 56, 24, 9


def _resize_mlp(seed=0):
    from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import Qwen3OmniMoeTalkerConfig
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import Qwen3OmniMoeTalkerResizeMLP
    cfg = Qwen3OmniMoeTalkerConfig(thinker_hidden_size=D_IN,
                                   text_config={"hidden_size": D_OUT, "intermediate_size": D_MID,
                                                "hidden_act": "silu"})
    torch.manual_seed(seed)
    m = Qwen3OmniMoeTalkerResizeMLP(cfg).eval()
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn_like(p) * (0.3 if p.dim() == 2 else 1.0))
    return m


def _proj_args(m):
    d = lambda t: t.detach().clone()
    return [d(m.linear_fc1.weight), d(m.linear_fc1.bias), d(m.linear_fc2.weight), d(m.linear_fc2.bias)]


def test_text_projection_matches_resize_mlp():
    m = _resize_mlp()
    rows = torch.randn(R, D_IN)
    with torch.no_grad():
        want = m(rows)
        got = M.text_projection(rows, *_proj_args(m))
    err = float((got - want).abs().max())
    print(f"text projection: max |d| {err:.2e} of {float(want.abs().max()):.2f}")
    assert err < 1e-5 * max(1.0, float(want.abs().max()))


@pytest.mark.parametrize("kind", ["GELU for SiLU", "fc1 bias dropped", "fc2 bias dropped"])
def test_text_projection_pin_detects_mistakes(monkeypatch, kind):
    m = _resize_mlp()
    rows = torch.randn(R, D_IN)
    args = _proj_args(m)
    if kind == "GELU for SiLU":
        monkeypatch.setattr(M, "silu", torch.nn.functional.gelu)
    elif kind == "fc1 bias dropped":
        args[1] = torch.zeros_like(args[1])
    elif kind == "fc2 bias dropped":
        args[3] = torch.zeros_like(args[3])
    with torch.no_grad():
        want = m(rows)
        got = M.text_projection(rows, *args)
    err = float((got - want).abs().max())
    print(f"planted {kind}: max |d| {err:.2e}")
    assert err > 1e-2


def test_build_prompt_uses_the_pinned_projection(small_blob):
    """Every prompt row is a text_projection row (plus a codec or speaker row): the 3 role rows
    equal the pinned function applied to the first three embedding-table rows."""
    o = M.Oracle(small_blob)
    b = o.blob
    ids = [o.kv["text.im_start_id"], o.kv["text.assistant_id"], 198, 1000, 2000,
           o.kv["text.im_end_id"], 198, o.kv["text.im_start_id"], o.kv["text.assistant_id"], 198]
    pre, _, _ = o.build_prompt(ids, "english", np.zeros(1024, np.float32))
    rows = torch.from_numpy(b.array("talker.model.text_embedding.weight")[np.asarray(ids[:3])].astype(np.float32))
    t = lambda n: torch.from_numpy(b.f32("talker.text_projection." + n))
    want = M.text_projection(rows, t("linear_fc1.weight"), t("linear_fc1.bias"), t("linear_fc2.weight"),
                             t("linear_fc2.bias")).numpy()
    assert np.array_equal(pre[:3], want)
