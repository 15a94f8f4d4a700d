"""Pins the oracle's codec decoder (oracle/vocoder.py).

* building blocks against an independent implementation with the same structure:
  transformers' Qwen3-Omni code2wav modules (SnakeBeta, the decoder residual unit with causal
  k7 convs at dilations 1/3/9, the ConvNeXt block, the layer-scaled sliding-window transformer
  layer), loaded with the same random weights. (Omni's transposed conv trims both sides and
  its front end differs; those two parts follow the reference instead and are pinned below.)
* the right-trimmed transposed conv and the causal conv against brute-force loops;
* (the RVQ front end is pinned against transformers' Mimi quantizer in test_oracle_front_ends.py);
* causality of the whole decoder: decoding the first n frames gives exactly the first n * 1920
  samples of decoding all frames (what makes chunked streaming equal one-shot decoding).
"""
import numpy as np
import pytest
import torch

from oracle import vocoder as V

torch.manual_seed(0)


def _omni():
    from transformers.models.qwen3_omni_moe import modeling_qwen3_omni_moe as m
    return m


def test_snake_matches_transformers():
    m = _omni()
    ref = m.Qwen3OmniMoeSnakeBeta(24)
    with torch.no_grad():
        ref.alpha.copy_(torch.randn(24) * 0.3)
        ref.beta.copy_(torch.randn(24) * 0.3)
    x = torch.randn(24, 50) * 2
    with torch.no_grad():
        want = ref(x[None])[0]
    assert torch.allclose(V.snake(x, ref.alpha.detach(), ref.beta.detach()), want, atol=1e-6)


@pytest.mark.parametrize("dil", [1, 3, 9])
def test_residual_unit_matches_transformers(dil):
    m = _omni()
    ref = m.Qwen3OmniMoeCode2WavDecoderResidualUnit(16, dil)
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(torch.randn_like(p) * 0.2)
    x = torch.randn(16, 40)
    with torch.no_grad():
        want = ref(x[None])[0]
        z = V.causal_conv(V.snake(x, ref.act1.alpha, ref.act1.beta), ref.conv1.conv.weight, ref.conv1.conv.bias, dil)
        got = x + V.causal_conv(V.snake(z, ref.act2.alpha, ref.act2.beta), ref.conv2.conv.weight, ref.conv2.conv.bias)
    assert torch.allclose(got, want, atol=1e-5)


def test_convnext_matches_transformers():
    m = _omni()
    C = 32
    ref = m.Qwen3OmniMoeConvNeXtBlock(C)
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(torch.randn_like(p) * 0.2)
    x = torch.randn(C, 30)
    p = {"dw": ref.dwconv.conv.weight, "dw_b": ref.dwconv.conv.bias, "ln_w": ref.norm.weight, "ln_b": ref.norm.bias,
         "pw1": ref.pwconv1.weight, "pw1_b": ref.pwconv1.bias, "pw2": ref.pwconv2.weight, "pw2_b": ref.pwconv2.bias,
         "gamma": ref.gamma}
    with torch.no_grad():
        want = ref(x[None])[0]
        got = V.convnext(x, p)
    assert torch.allclose(got, want, atol=1e-5)


def test_transformer_layer_matches_transformers():
    m = _omni()
    from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import Qwen3OmniMoeCode2WavConfig
    H, nh, hd, W, T = 64, 4, 16, 8, 21
    cfg = Qwen3OmniMoeCode2WavConfig(hidden_size=H, num_attention_heads=nh, num_key_value_heads=nh, head_dim=hd,
                                     intermediate_size=128, rms_norm_eps=1e-5, sliding_window=W,
                                     layer_scale_initial_scale=0.1, hidden_act="silu", attention_bias=False)
    cfg._attn_implementation = "eager"
    ref = m.Qwen3OmniMoeCode2WavTransformerLayer(cfg, 0).eval()
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(torch.randn_like(p) * 0.1 + (1.0 if p.dim() == 1 else 0.0))
    x = torch.randn(T, H)
    invf = V.inv_freq(10000.0, hd)
    ang = torch.arange(T, dtype=torch.float32)[:, None] * invf[None]
    cos = torch.cat([ang.cos(), ang.cos()], -1)[None]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[None]
    i = torch.arange(T)
    ok = (i[None, :] <= i[:, None]) & (i[:, None] - i[None, :] < W)
    mask = torch.zeros(T, T).masked_fill(~ok, float("-inf"))[None, None]
    with torch.no_grad():
        want = ref(x[None], attention_mask=mask, position_embeddings=(cos, sin))
        want = (want[0] if isinstance(want, tuple) else want)[0]
        a, mlp = ref.self_attn, ref.mlp
        w = {"ln1": ref.input_layernorm.weight, "ln2": ref.post_attention_layernorm.weight, "wq": a.q_proj.weight,
             "wk": a.k_proj.weight, "wv": a.v_proj.weight, "wo": a.o_proj.weight, "wg": mlp.gate_proj.weight,
             "wu": mlp.up_proj.weight, "wd": mlp.down_proj.weight, "attn_scale": ref.self_attn_layer_scale.scale,
             "mlp_scale": ref.mlp_layer_scale.scale}
        got = V.transformer_layer(x, w, nh, hd, 1e-5, invf, W)
    assert torch.allclose(got, want, atol=2e-5), (got - want).abs().max()


def test_causal_conv_brute_force():
    r = np.random.default_rng(0)
    x = r.standard_normal((3, 9))
    w = r.standard_normal((2, 3, 4))
    b = r.standard_normal(2)
    dil = 2
    want = np.zeros((2, 9))
    for co in range(2):
        for t in range(9):
            acc = b[co]
            for ci in range(3):
                for j in range(4):
                    tt = t - (4 - 1 - j) * dil
                    if tt >= 0:
                        acc += w[co, ci, j] * x[ci, tt]
            want[co, t] = acc
    got = V.causal_conv(torch.tensor(x), torch.tensor(w), torch.tensor(b), dil).numpy()
    assert np.allclose(got, want)


@pytest.mark.parametrize("s,k", [(2, 2), (3, 6), (5, 10)])
def test_trans_conv_brute_force(s, k):
    r = np.random.default_rng(s)
    Cin, Cout, T = 3, 2, 5
    x = r.standard_normal((Cin, T))
    w = r.standard_normal((Cin, Cout, k))
    b = r.standard_normal(Cout)
    want = np.zeros((Cout, T * s))
    for co in range(Cout):
        for i in range(T):
            for p in range(s):
                acc = b[co]
                for m in range(k // s):                  # out[i*s+p] = sum_m W[ci][co][p+m*s] x[i-m]
                    if i - m >= 0:
                        acc += sum(w[ci, co, p + m * s] * x[ci, i - m] for ci in range(Cin))
                want[co, i * s + p] = acc
    got = V.trans_conv(torch.tensor(x), torch.tensor(w), torch.tensor(b), s).numpy()
    assert np.allclose(got, want)


@pytest.fixture(scope="module")
def voc(scratch_dir):
    from navi_amd import blob
    path = scratch_dir / "codec_only.navi"
    if not path.exists():
        blob.write_random_blob(path, 0, parts=("codec",))
    return V.Vocoder(path)


def test_decoder_is_causal(voc):
    codes = np.random.default_rng(2).integers(0, 2048, (6, 16))
    full = voc.decode(codes)
    part = voc.decode(codes[:4])
    assert full.shape == (6 * 1920,) and part.shape == (4 * 1920,)
    assert np.abs(full[:4 * 1920] - part).max() < 1e-5
    assert np.abs(full).max() < 1.0 and full.std() > 0.02      # a non-degenerate, unclipped signal
