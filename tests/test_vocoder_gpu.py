"""The codec decoder on the GPU vs the CPU oracle (through the C ABI).

Bar (north star): PCM SNR >= 40 dB against the f32 reference on the same f16 weights.
Streaming (the reference's vocoder gate, tests/test_vocoder.cpp:101-107): decoding in chunks
(first batch 4 then 16, or any chunk size) equals decoding in one call; reset starts a new
utterance; codes outside the codebook are an error.
"""
import numpy as np
import pytest

from gpu_util import log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def codec(scratch_dir):
    from navi_amd import abi, blob
    from oracle.vocoder import Vocoder as OVoc
    path = scratch_dir / "codec_gpu.navi"
    if not path.exists():
        blob.write_random_blob(path, 0, parts=("codec",))
    abi.device_open()
    W = abi.DeviceWeights(path, select=lambda t: t.name.startswith("codec.decoder."))
    return abi, W, OVoc(path)


def snr_db(got, want):
    err = np.asarray(got, np.float64) - np.asarray(want, np.float64)
    return 10 * np.log10(np.sum(np.asarray(want, np.float64) ** 2) / max(np.sum(err ** 2), 1e-300))


def test_vocoder_matches_oracle(codec):
    abi, W, ora = codec
    codes = np.random.default_rng(0).integers(0, 2048, (12, 16))
    v = abi.Vocoder(W, max_chunk_frames=16)
    log("vocoder 12 frames, one chunk")
    pcm = v.decode(codes)
    want = ora.decode(codes)
    snr = snr_db(pcm, want)
    log(f"  SNR {snr:.1f} dB, max abs err {np.abs(pcm - want).max():.2e}, device {v.last_ms():.3f} ms")
    assert pcm.shape == want.shape == (12 * 1920,)
    assert snr >= 40.0


def test_chunked_equals_one_shot(codec):
    abi, W, _ = codec
    codes = np.random.default_rng(1).integers(0, 2048, (20, 16))
    one = abi.Vocoder(W, max_chunk_frames=32)
    ref = one.decode(codes)
    small = abi.Vocoder(W, max_chunk_frames=4)
    log("vocoder chunked 4 x 5 vs one shot")
    got = small.decode(codes)
    d1 = np.abs(got - ref).max()
    streamed = abi.Vocoder(W, max_chunk_frames=16)
    log("vocoder streamed 4 then 16 vs one shot")
    got2 = np.concatenate([streamed.decode(codes[:4]), streamed.decode(codes[4:])])
    d2 = np.abs(got2 - ref).max()
    log(f"  chunk-4 max diff {d1:.2e}, 4+16 max diff {d2:.2e}")
    assert d1 <= 1e-5 and d2 <= 1e-5


def test_tile_shapes_do_not_change_the_pcm(codec):
    """The decoder blocks' convs pick their tiles by the chunk's row count (k_conv_wide: 128- or
    64-row tiles; the 768- and 384-channel convs, whose input channels are split in ranges fixed at
    create, run the ranges as separate blocks with partials for short chunks and in one block for
    long ones) and the transformer's row kernels more row tiles per block for more rows: a column's
    sums keep their order in every case, so 64 frames decoded as one block and as 16-frame chunks
    give the same PCM bit for bit. (Both handles hold at least 16 frames, so their split counts,
    fixed at create from a 16-frame chunk, agree.)"""
    abi, W, _ = codec
    codes = np.random.default_rng(5).integers(0, 2048, (64, 16))
    one = abi.Vocoder(W, max_chunk_frames=64)
    block = one.decode(codes)
    small = abi.Vocoder(W, max_chunk_frames=16)
    chunks = small.decode(codes)
    log(f"64-frame block vs 16-frame chunks: max diff {np.abs(block - chunks).max():.2e}")
    assert np.array_equal(block, chunks)


def test_reset_restarts_the_utterance(codec):
    abi, W, _ = codec
    codes = np.random.default_rng(2).integers(0, 2048, (6, 16))
    v = abi.Vocoder(W, max_chunk_frames=8)
    a = v.decode(codes)
    v.decode(codes)
    v.reset()
    b = v.decode(codes)
    assert np.array_equal(a, b)


def test_bad_code_is_an_error(codec):
    abi, W, _ = codec
    v = abi.Vocoder(W, max_chunk_frames=4)
    codes = np.zeros((2, 16), np.int32)
    codes[1, 3] = 2048
    with pytest.raises(abi.NaviError) as e:
        v.decode(codes)
    assert e.value.status == abi.NAVI_ERR_INVALID


def test_activation_outside_f16_is_an_error(codec, scratch_dir):
    """A conv input at or above 65504 (outside f16, where the staging's hi/lo split breaks) is an
    error, not an infinity in the PCM, also when only the third chunk of a call holds it; the next
    call starts clean. Row 7 of the first two rest codebooks is set to 40000 in every channel, so a
    frame whose codes 1 and 2 are both 7 sums to 80000 in the RVQ front end's rows."""
    abi, _, _ = codec
    W2 = abi.DeviceWeights(scratch_dir / "codec_gpu.navi", select=lambda t: t.name.startswith("codec.decoder."))
    for q in (0, 1):
        name = f"codec.decoder.quantizer.rvq_rest.vq.layers.{q}._codebook.codebook"
        vq = W2.tensors[name][2][1]
        abi.upload(W2.ptr(name) + 7 * vq * 2, np.full(vq, 40000, np.float16).view(np.uint16))
    v = abi.Vocoder(W2, max_chunk_frames=4)
    codes = np.random.default_rng(3).integers(0, 2048, (12, 16)).astype(np.int32)
    codes[:, 1:3][codes[:, 1:3] == 7] = 8
    log("vocoder f16-range flag: 8 clean frames, then 12 with the overflow in frame 9 (chunk 3 of 3)")
    clean = v.decode(codes[:8])
    assert np.isfinite(clean).all()
    bad = codes.copy()
    bad[9, 1] = bad[9, 2] = 7
    v.reset()
    with pytest.raises(abi.NaviError) as e:
        v.decode(bad)
    assert e.value.status == abi.NAVI_ERR_INVALID and "f16 range" in str(e.value)
    v.reset()
    assert np.array_equal(v.decode(codes[:8]), clean)


def test_stage_hook_stages_match_oracle(codec):
    """Vocoder::set_stage_hook (vocoder.h:46-48): every stage of a chunk reaches the hook under the
    reference's stage names, in the model's order; the stages compare one by one with the oracle's
    intermediates (rel-RMS, the SNR bar's equivalent), and "pcm" is exactly what decode returns."""
    abi, W, ora = codec
    codes = np.random.default_rng(3).integers(0, 2048, (8, 16))
    v = abi.Vocoder(W, max_chunk_frames=8)
    got = {}
    names = []

    def hook(name, arr):
        names.append(name)
        got[name] = arr.copy()
    v.set_stage_hook(hook)
    pcm = v.decode(codes)
    v.set_stage_hook(None)
    L = len([n for n in names if n.startswith("layer")])
    want_order = (["rvq", "pre_conv", "in_proj"]
                  + sum([[f"norm1_{l}", f"qkv_{l}", f"attnraw{l}", f"xattn_{l}", f"layer{l}"] for l in range(L)], [])
                  + ["pre_transformer"] + sum([[f"up{j}_t", f"up{j}_ln", f"up{j}_cnx"] for j in range(2)], [])
                  + ["dec0"] + sum([[f"dec{b}_b{k}" for k in range(1, 5)] for b in range(1, 5)], []) + ["pcm"])
    log(f"stage hook: {len(names)} stages, {L} transformer layers")
    assert names == want_order
    np.testing.assert_array_equal(got["pcm"][:, 0], pcm)
    ostages = ora.stages(codes)
    pairs = [("rvq", "rvq"), ("pre_conv", "pre_conv"), (f"layer{L - 1}", f"layer{L - 1}"),
             ("pre_transformer", "pre_transformer"), ("up0_cnx", "up0"), ("up1_cnx", "up1"), ("dec0", "dec0")]
    pairs += [(f"dec{b}_b4", f"block{b}") for b in range(1, 5)]
    for dn, on in pairs:
        a = np.asarray(got[dn], np.float64)
        b = ostages[on].numpy().astype(np.float64)
        assert a.shape == b.shape, (dn, a.shape, b.shape)
        rel = np.sqrt(np.sum((a - b) ** 2) / max(np.sum(b ** 2), 1e-300))
        log(f"  {dn:16s} vs oracle {on:16s}: rel-rms {rel:.2e}")
        assert rel < 1e-3
    # no hook: the same PCM, no callbacks
    v.reset()
    names.clear()
    assert np.array_equal(v.decode(codes), pcm) and not names


def test_graph_replays_match_eager(codec):
    """Chunks replayed from captured HIP graphs (navi_vocoder_set_graphs) give the PCM of chunks whose kernels
    the host launches one by one: a stream of 4 then 16-frame chunks (both history parities, a
    partial last chunk), replayed several times with resets and eager decodes in between; every
    replay is compared with the eager result."""
    abi, W, _ = codec
    codes = np.random.default_rng(4).integers(0, 2048, (45, 16))
    v = abi.Vocoder(W, max_chunk_frames=16)

    def stream():
        v.reset()
        return np.concatenate([v.decode(codes[:4]), v.decode(codes[4:20]), v.decode(codes[20:36]), v.decode(codes[36:])])
    v.set_graphs(False)
    eager = stream()
    v.set_graphs(True)
    for rep in range(3):
        got = stream()
        assert np.array_equal(got, eager), f"replay {rep} differs: max {np.abs(got - eager).max():.3e}"
        v.set_graphs(False)                     # eager work between the replays
        assert np.array_equal(stream(), eager)
        v.set_graphs(True)
    v.set_graphs(False)
    log(f"vocoder graph replays == eager over 45 frames (4 + 16 + 16 + 9), 3 rounds")


def test_config3_240_frames_block_and_stream(codec):
    """BASELINE configs[3] at its own size: 240 frames of uniform codes decoded as one 240-frame
    block and as a stream of 4 then 16-frame chunks, both against the oracle's one-shot decode
    (SNR >= 40 dB), and block == stream within 1e-5. Past frame 72 the pre-transformer's attention
    drops keys older than its 72-position window (reference k_attention, vocoder.hip:86-117), and
    with 16-frame chunks its K/V ring of next_pow2(72 + 16) = 128 slots (vocoder.hip:473-474)
    wraps from frame 128 on, so both paths run here under the oracle's windowed mask."""
    abi, W, ora = codec
    codes = np.random.default_rng(7).integers(0, 2048, (240, 16))
    want = ora.decode(codes)
    block = abi.Vocoder(W, max_chunk_frames=240)
    log("vocoder configs[3]: 240-frame block")
    got_block = block.decode(codes)
    stream = abi.Vocoder(W, max_chunk_frames=16)
    log("vocoder configs[3]: 240 frames as 4 + 16 x 14 + 12")
    parts = [stream.decode(codes[:4])]
    for f in range(4, 240, 16):
        parts.append(stream.decode(codes[f:f + 16]))
    got_stream = np.concatenate(parts)
    assert got_block.shape == got_stream.shape == want.shape == (240 * 1920,)
    s_block, s_stream = snr_db(got_block, want), snr_db(got_stream, want)
    # the windowed and wrapped region on its own: frames 128..239 (ring wrapped, keys truncated)
    tail = slice(128 * 1920, 240 * 1920)
    s_tail = snr_db(got_stream[tail], want[tail])
    d = float(np.abs(got_block - got_stream).max())
    log(f"  SNR block {s_block:.1f} dB, stream {s_stream:.1f} dB, stream frames 128-239 {s_tail:.1f} dB; "
        f"block vs stream max diff {d:.2e}")
    assert s_block >= 40.0 and s_stream >= 40.0 and s_tail >= 40.0
    assert d <= 1e-5
