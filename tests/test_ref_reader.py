"""The random-init `.navi` writer (navi_amd/blob.py) read by the reference's own reader.

tests/native/ref_navi_check.cpp is compiled together with the reference's
runtime/weights/navi_file.cpp and model/qwen3tts/params.cpp, where they lie under
/root/reference (outputs into a temporary directory), and run on a blob holding every part the
reference's table lists (talker, code predictor, speaker encoder, codec decoder, tokenizer
files), with 2 talker and 2 code-predictor layers. It must:

* open the file (NaviFile::open, navi_file.cpp:79-148: magic, version, size, page-aligned
  in-bounds tensors, byte length == numel * dtype size, unique names);
* read every parameter (read_params, params.cpp:59-130) as the writer meant it;
* validate (params.cpp:286-303) with no missing, shape-mismatched or unused tensor;
* see each tensor with the writer's dtype (f16 for >= 2-D, f32 for 1-D, u8 for the tokenizer
  files), dims and byte length, and bytes whose two checksums equal those of the data the
  writer generated for it.

So every tensor name the kernels bind, and the format itself, is pinned by the reference's
reader on the CPU. Skipped where /root/reference is absent (the GPU box).
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference")
SRC = ["runtime/weights/navi_file.cpp", "model/qwen3tts/params.cpp"]
PARTS = ("talker", "cp", "speaker", "codec", "tokenizer")

pytestmark = pytest.mark.skipif(not all((REF / s).exists() for s in SRC), reason="reference sources absent")

DTYPE_NAME = {0: "f32", 1: "f16", 2: "bf16", 3: "i32", 4: "u8"}


def _checksums(raw: bytes):
    pad = (-len(raw)) % 8
    w = np.frombuffer(raw + b"\0" * pad, dtype="<u8")
    i = np.arange(w.size, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return int(w.sum(dtype=np.uint64)), int((w * (2 * i + 1)).sum(dtype=np.uint64))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    d = tmp_path_factory.mktemp("ref_reader")
    exe = d / "ref_navi_check"
    r = subprocess.run(["g++", "-std=c++20", "-O2", "-Wall", f"-I{REF}", "-o", str(exe),
                        str(ROOT / "tests" / "native" / "ref_navi_check.cpp"), *[str(REF / s) for s in SRC]],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def _run(exe, path):
    out = subprocess.run([str(exe), str(path)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr
    lines = out.stdout.splitlines()
    assert lines[-1] == "OK", lines[-1]
    return lines[:-1]


@pytest.fixture(scope="module")
def checked(checker, scratch_dir):
    from navi_amd import blob
    path = scratch_dir / "all_parts.navi"
    kw = dict(talker_layers=2, cp_layers=2)
    blob.write_random_blob(path, 11, parts=PARTS, **kw)
    lines = _run(checker, path)
    params = {}
    tensors = []
    flags = []
    for ln in lines:
        tag, rest = ln.split(" ", 1)
        if tag == "P":
            k, _, v = rest.partition(" ")
            params[k] = v
        elif tag == "T":
            f = rest.split(" ")
            nd = int(f[2])
            tensors.append(dict(name=f[0], dtype=f[1], dims=tuple(int(x) for x in f[3:3 + nd]),
                                offset=int(f[3 + nd]), nbytes=int(f[4 + nd]), sum=int(f[5 + nd]), wsum=int(f[6 + nd])))
        else:
            flags.append(ln)
    kv = blob.qwen3tts_0p6b_kv(**kw)
    specs = blob.tensor_table(kv, PARTS)
    yield dict(params=params, tensors=tensors, flags=flags, kv=kv, specs=specs, seed=11)
    path.unlink()


def test_reference_validate_reports_nothing(checked):
    """No MISSING, MISMATCH or UNUSED line: the blob holds exactly the reference's table."""
    assert checked["flags"] == []


def test_reference_validate_flags_a_wrong_blob(checker, scratch_dir):
    """Control: a blob without the tokenizer files, one codec tensor transposed and one extra
    tensor draws exactly those MISSING, MISMATCH and UNUSED lines from the same checker."""
    from navi_amd import blob
    kv = blob.qwen3tts_0p6b_kv(talker_layers=1, cp_layers=1, text_vocab=64)
    specs = blob.tensor_table(kv, ("talker", "cp", "speaker", "codec"))
    name = "codec.decoder.pre_transformer.input_proj.weight"
    i = [s.name for s in specs].index(name)
    specs[i] = blob.TensorSpec(name, tuple(reversed(specs[i].shape)), specs[i].init)
    specs.append(blob.TensorSpec("codec.encoder.extra.weight", (4, 4), ("normal", 0.02)))
    path = scratch_dir / "wrong.navi"
    blob.write_navi(path, kv, specs, 0)
    flags = [ln for ln in _run(checker, path) if not ln.startswith(("P ", "T "))]
    path.unlink()
    assert sorted(f.split(" ")[0] + " " + f.split(" ")[1].rstrip(":") for f in flags) == sorted(
        ["MISSING tokenizer.vocab.json", "MISSING tokenizer.merges.txt", "MISSING tokenizer.config.json",
         f"MISMATCH {name}", "UNUSED codec.encoder.extra.weight"])


def test_reference_reads_the_parameters_written(checked):
    p, kv = checked["params"], checked["kv"]
    ints = {"im_start_id": "text.im_start_id", "im_end_id": "text.im_end_id", "assistant_id": "text.assistant_id",
            "tts_bos_id": "text.tts_bos_id", "tts_eos_id": "text.tts_eos_id", "tts_pad_id": "text.tts_pad_id",
            "text_vocab": "talker.text_vocab_size", "text_hidden": "talker.text_hidden_size",
            "n_code_groups": "talker.num_code_groups", "position_id_per_second": "talker.position_id_per_seconds",
            "mrope_interleaved": "talker.mrope_interleaved", "codec_bos_id": "talker.codec_bos_id",
            "codec_eos_id": "talker.codec_eos_token_id", "codec_pad_id": "talker.codec_pad_id",
            "codec_think_id": "talker.codec_think_id", "codec_nothink_id": "talker.codec_nothink_id",
            "codec_think_bos_id": "talker.codec_think_bos_id", "codec_think_eos_id": "talker.codec_think_eos_id",
            "spk_dim": "speaker.enc_dim", "spk_sample_rate": "speaker.sample_rate", "mel_n_fft": "speaker.mel.n_fft",
            "mel_num_mels": "speaker.mel.num_mels", "mel_hop": "speaker.mel.hop_size", "mel_win": "speaker.mel.win_size",
            "codec_sample_rate": "codec.output_sample_rate", "codec_upsample": "codec.decode_upsample_rate",
            "vq_latent": "codec.decoder.latent_dim", "vq_codebook_dim": "codec.decoder.codebook_dim",
            "vq_codebook_size": "codec.decoder.codebook_size", "vq_n_q": "codec.decoder.num_quantizers",
            "vq_n_semantic": "codec.decoder.num_semantic_quantizers", "vocoder_decoder_dim": "codec.decoder.decoder_dim",
            "vocoder_sliding_window": "codec.decoder.sliding_window", "top_k": "gen.top_k",
            "cp_top_k": "gen.subtalker_top_k"}
    for field, key in ints.items():
        assert int(p[field]) == int(kv[key]), (field, p[field], kv[key])
    floats = {"mel_fmin": "speaker.mel.fmin", "mel_fmax": "speaker.mel.fmax", "temperature": "gen.temperature",
              "top_p": "gen.top_p", "repetition_penalty": "gen.repetition_penalty",
              "cp_temperature": "gen.subtalker_temperature", "cp_top_p": "gen.subtalker_top_p"}
    for field, key in floats.items():
        assert np.float32(p[field]) == np.float32(kv[key]), (field, p[field], kv[key])
    for ns, key in (("talker", "talker"), ("cp", "cp"), ("vocoder", "codec.decoder")):
        for field, k in (("hidden", "hidden_size"), ("n_layer", "num_hidden_layers"),
                         ("n_head", "num_attention_heads"), ("n_kv_head", "num_key_value_heads"),
                         ("head_dim", "head_dim"), ("ff", "intermediate_size")):
            assert int(p[f"{ns}.{field}"]) == int(kv[f"{key}.{k}"]), (ns, field)
        assert int(p[f"{ns}.vocab"]) == int(kv.get(f"{key}.vocab_size", 0))
        assert int(p[f"{ns}.max_pos"]) == int(kv.get(f"{key}.max_position_embeddings", 0))
        assert np.float32(p[f"{ns}.rms_eps"]) == np.float32(kv[f"{key}.rms_norm_eps"])
        assert float(p[f"{ns}.rope_theta"]) == float(kv[f"{key}.rope_theta"])
    assert [int(x) for x in p["mrope_section"].split()] == list(kv["talker.mrope_section"])
    assert [int(x) for x in p["vocoder_upsample_rates"].split()] == list(kv["codec.decoder.upsample_rates"])
    assert [int(x) for x in p["vocoder_upsampling_ratios"].split()] == list(kv["codec.decoder.upsampling_ratios"])
    langs = {k[len("talker.language."):]: v for k, v in kv.items() if k.startswith("talker.language.")}
    assert {k[len("language."):]: int(v) for k, v in p.items() if k.startswith("language.")} == langs
    assert p["dtype"] == kv["general.dtype"] and p["name"] == kv["general.name"]
    assert int(p["has_codec_encoder"]) == 0


def test_reference_sees_the_tensors_written(checked):
    from navi_amd import blob
    got, specs = checked["tensors"], checked["specs"]
    assert [t["name"] for t in got] == [s.name for s in specs]
    for t, s in zip(got, specs):
        want_dtype = "u8" if s.name.startswith("tokenizer.") else ("f16" if len(s.shape) >= 2 else "f32")
        assert t["dtype"] == DTYPE_NAME[s.dtype] == want_dtype, s.name
        assert t["dims"] == tuple(s.shape) and t["nbytes"] == s.nbytes, s.name
        data = np.ascontiguousarray(blob.materialize(s, checked["seed"]))
        assert (t["sum"], t["wsum"]) == _checksums(data.tobytes()), s.name
