"""The `.navi` writer and readers, and the random-init fill.

* The writer's bytes are parsed here with `struct` straight from the documented layout
  (reference docs/navi-format.md: header, KV table, tensor table, page-aligned data), not with
  the readers, so writer and readers cannot share a mistake;
* both readers (navi_amd.navi_file and the oracle's navi_read) return the written arrays and
  reject corrupted files;
* the f16 conversion is round-to-nearest-even (numpy's float16 cast is the independent check),
  including subnormals, overflow and NaN;
* the random fill is deterministic per (seed, name) and has the requested scale; the tensor
  table follows the converter's dtype rule (>= 2-D f16, 1-D f32).
"""
import struct

import numpy as np
import pytest

from navi_amd import blob
from navi_amd.navi_file import NaviFile, NaviFormatError


def _parse(path):
    b = open(path, "rb").read()
    assert b[:4] == b"NAVI"
    version, data_offset, n_kv, n_t, size = struct.unpack_from("<IQIIQ", b, 4)
    assert version == 1 and data_offset % 4096 == 0 and size == len(b)
    p = 32

    def string():
        nonlocal p
        (n,) = struct.unpack_from("<I", b, p)
        s = b[p + 4:p + 4 + n].decode()
        p += 4 + n
        return s

    kv = {}
    for _ in range(n_kv):
        k = string()
        t = b[p]
        p += 1
        if t == 0:
            (kv[k],) = struct.unpack_from("<q", b, p)
            p += 8
        elif t == 1:
            (kv[k],) = struct.unpack_from("<d", b, p)
            p += 8
        elif t == 2:
            kv[k] = string()
        elif t == 3:
            (n,) = struct.unpack_from("<I", b, p)
            kv[k] = list(struct.unpack_from(f"<{n}q", b, p + 4))
            p += 4 + 8 * n
        else:
            raise AssertionError(f"kv type {t}")
    tensors = {}
    for _ in range(n_t):
        name = string()
        dt, nd = b[p], b[p + 1]
        p += 2
        dims = struct.unpack_from(f"<{nd}Q", b, p)
        p += 8 * nd
        off, nbytes = struct.unpack_from("<QQ", b, p)
        p += 16
        assert off % 4096 == 0 and data_offset + off + nbytes <= size
        tensors[name] = (dt, dims, b[data_offset + off:data_offset + off + nbytes])
    assert p <= data_offset
    return kv, tensors


@pytest.fixture
def tiny(tmp_path):
    kv = {"general.arch": "qwen3-tts", "a.int": -5, "a.float": 0.25, "a.list": [1, -2, 3], "a.bool": True}
    specs = [blob.TensorSpec("w.matrix", (3, 5), ("normal", 0.5)), blob.TensorSpec("w.vector", (7,), ("const", 1.5)),
             blob.TensorSpec("w.big", (1100, 2), ("normal", 1.0))]
    path = tmp_path / "tiny.navi"
    blob.write_navi(path, kv, specs, seed=3)
    return path, kv, specs


def test_writer_bytes_follow_the_documented_layout(tiny):
    path, kv, specs = tiny
    got_kv, tensors = _parse(path)
    assert got_kv == {**kv, "a.bool": 1}
    assert set(tensors) == {s.name for s in specs}
    dt, dims, raw = tensors["w.matrix"]
    assert dt == 1 and dims == (3, 5) and len(raw) == 30
    dt, dims, raw = tensors["w.vector"]
    assert dt == 0 and dims == (7,) and np.all(np.frombuffer(raw, np.float32) == 1.5)
    assert np.array_equal(np.frombuffer(tensors["w.big"][2], np.uint16).reshape(1100, 2),
                          blob.materialize(specs[2], 3))


def test_readers_return_written_arrays(tiny):
    from oracle.navi_read import NaviBlob
    path, kv, specs = tiny
    f = NaviFile(path)
    o = NaviBlob(path)
    for s in specs:
        want = blob.materialize(s, 3)
        assert np.array_equal(f.array(s.name), want)
        oa = o.array(s.name)
        assert np.array_equal(oa.view(want.dtype) if oa.dtype.itemsize == want.dtype.itemsize else oa, want)
    assert f.kv["a.list"] == [1, -2, 3] and o.kv["a.float"] == 0.25
    f.close()


@pytest.mark.parametrize("corrupt", ["magic", "version", "truncate", "size"])
def test_reader_rejects_corrupt_files(tiny, tmp_path, corrupt):
    path, _, _ = tiny
    b = bytearray(open(path, "rb").read())
    if corrupt == "magic":
        b[0:4] = b"NAVX"
    elif corrupt == "version":
        b[4:8] = struct.pack("<I", 2)
    elif corrupt == "truncate":
        b = b[:-4096]
    else:
        b[24:32] = struct.pack("<Q", len(b) + 4096)
    bad = tmp_path / f"bad_{corrupt}.navi"
    bad.write_bytes(bytes(b))
    with pytest.raises(NaviFormatError):
        NaviFile(bad)


def test_f16_conversion_is_round_to_nearest_even():
    r = np.random.default_rng(0)
    x = np.concatenate([r.standard_normal(100000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 65504, 65520, 65519.99, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8, -1e-5, 1e6,
                                  np.inf, -np.inf, 1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32)])
    got = blob.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    nan = blob.f32_to_f16_bits(np.array([np.nan], np.float32)).view(np.float16)
    assert np.isnan(nan[0])


def test_random_fill_is_deterministic_and_scaled():
    s = blob.TensorSpec("talker.model.layers.0.mlp.up_proj.weight", (512, 1024), ("normal", 0.02))
    a, b = blob.materialize(s, 1), blob.materialize(s, 1)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, blob.materialize(s, 2))
    other = blob.TensorSpec("talker.model.layers.1.mlp.up_proj.weight", (512, 1024), ("normal", 0.02))
    assert not np.array_equal(a, blob.materialize(other, 1))
    v = a.view(np.float16).astype(np.float64)
    assert abs(v.mean()) < 1e-3 and abs(v.std() - 0.02) < 5e-4
    # Gaussian shape: about 68.3% within one sigma, 95.4% within two
    assert abs(np.mean(np.abs(v) < 0.02) - 0.6827) < 0.01 and abs(np.mean(np.abs(v) < 0.04) - 0.9545) < 0.01


def test_tensor_table_dtype_rule_and_names():
    kv = blob.qwen3tts_0p6b_kv(talker_layers=2, cp_layers=1)
    table = blob.tensor_table(kv, ("talker", "cp", "codec"))
    names = {t.name for t in table}
    assert len(names) == len(table)
    for t in table:
        assert t.dtype == (1 if len(t.shape) >= 2 else 0), t.name
    for want in ("talker.model.layers.1.self_attn.q_proj.weight", "talker.codec_head.weight",
                 "talker.model.text_embedding.weight", "talker.code_predictor.lm_head.14.weight",
                 "talker.code_predictor.model.codec_embedding.14.weight", "talker.text_projection.linear_fc1.weight"):
        assert want in names
    shapes = {t.name: t.shape for t in table}
    assert shapes["talker.model.layers.0.self_attn.q_proj.weight"] == (2048, 1024)
    assert shapes["talker.model.layers.0.self_attn.k_proj.weight"] == (1024, 1024)
    assert shapes["talker.model.layers.0.mlp.down_proj.weight"] == (1024, 3072)
    assert shapes["talker.codec_head.weight"] == (3072, 1024)
    assert shapes["talker.code_predictor.lm_head.0.weight"] == (2048, 1024)
    assert shapes["talker.model.text_embedding.weight"] == (151936, 2048)
