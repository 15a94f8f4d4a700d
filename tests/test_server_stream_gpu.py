"""The server's streaming path on this backend (runtime/server/server.cpp:401-495, 770-788).

tests/native/server_stream.cpp drives navi::qwen3tts::Graph (navi-tts_amd/csrc/host/
navi_graph.hpp, the reference's graph.h signatures over the C ABI) the way the server does: a
worker thread runs synth and pushes each vocoder batch as s16 into a bounded queue, the
consumer drains it or aborts it. Checked: the streamed audio equals the one-shot request's
sample for sample, batches arrive as 4 then 16 frames while the request is still running, a
client that goes away stops the request at its next batch with the consumer's exception, the
Graph serves the next request identically, errors arrive as navi::Error. The Python binding's
on_pcm follows the same rule (an exception stops the request and propagates).
"""
import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

from gpu_util import log

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
HARNESS = ROOT / "tests" / "native" / "lib" / "libserver_stream.so"


@pytest.fixture(scope="module")
def graph(scratch_dir):
    from navi_amd import abi, blob
    path = scratch_dir / "small_all_spk.navi"
    if not path.exists():
        blob.write_random_blob(path, 0, parts=("talker", "cp", "codec", "speaker"), talker_layers=2, cp_layers=2)
    abi.device_open()
    W = abi.DeviceWeights(path, select=lambda t: t.dtype != 4)
    talker = abi.Talker(W, max_prompt_tokens=128, max_positions=256)
    frame = abi.Frame(W)
    voc = abi.Vocoder(W, max_chunk_frames=16)
    spk = abi.Speaker(W, max_seconds=4.0)
    return abi, W, talker, frame, voc, spk


def _ids(kv, n_text, seed):
    rng = np.random.default_rng(seed)
    return [kv["text.im_start_id"], kv["text.assistant_id"], 198] + rng.integers(0, 151643, n_text).tolist() + \
           [kv["text.im_end_id"], 198, kv["text.im_start_id"], kv["text.assistant_id"], 198]


def test_server_streaming_path_through_graph(graph):
    abi, W, talker, frame, voc, spk = graph
    if not HARNESS.exists():
        pytest.fail(f"{HARNESS} is not built (run __graft_entry__.build())")
    lib = C.CDLL(str(HARNESS))
    fn = lib.navi_test_server_stream
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_uint64,
                   C.c_int32, C.c_char_p, C.c_size_t]
    ids = np.asarray(_ids(W.kv, 20, 3), np.int32)
    out = C.create_string_buffer(8192)
    log("server streaming path: warm-up, stream, one-shot, abort, next request, bad request (40 frames)")
    rc = fn(talker.h, frame.h, voc.h, spk.h, int(W.kv["talker.language.english"]), ids.ctypes.data, ids.size, 11, 40,
            out, 8192)
    rep = json.loads(out.value.decode())
    log(f"  {rep}")
    assert rc == 0 and "fatal" not in rep, rep
    assert np.isfinite(rep["warmup_speaker_norm"]) and rep["warmup_speaker_norm"] > 0
    assert 1 <= rep["warmup_frames"] <= 16
    assert rep["stream_error"] == "" and rep["stream_frames"] == 40
    assert rep["stream_sizes"] == [4 * 1920, 16 * 1920, 16 * 1920, 4 * 1920]
    assert rep["stream_first_before_done"], "the first batch only arrived after the request ended"
    assert rep["stream_ttfa_ms"] < rep["stream_total_ms"]
    assert rep["oneshot_frames"] == 40 and rep["stream_equals_oneshot"]
    assert rep["abort_error"] == "client stopped reading" and rep["abort_pushed"] == 1
    assert rep["after_abort_equals_oneshot"]
    assert "unknown language" in rep["bad_language_error"]


def test_python_on_pcm_exception_stops_the_request(graph):
    abi, W, talker, frame, voc, _ = graph
    ids = _ids(W.kv, 12, 5)
    spk = np.random.default_rng(2).standard_normal(1024).astype(np.float32)
    s = abi.Sampling.make(min_frames=40)
    seen = []

    class Gone(Exception):
        pass

    def on_pcm(chunk):
        seen.append(chunk.size)
        if len(seen) == 2:
            raise Gone("client stopped reading")

    log("python on_pcm raising at the second batch of a 40-frame request")
    with pytest.raises(Gone):
        abi.synth(talker, frame, voc, ids=ids, speaker=spk, seed=4, max_frames=40, sampling=s, vocoder_batch=16,
                  first_batch=4, on_pcm=on_pcm)
    assert seen == [4 * 1920, 16 * 1920]
    # the modules serve the next request normally, with the same audio as a fresh one
    st, pcm, sizes = abi.synth(talker, frame, voc, ids=ids, speaker=spk, seed=4, max_frames=8, sampling=s,
                               vocoder_batch=4, first_batch=4)
    st2, pcm2, _ = abi.synth(talker, frame, voc, ids=ids, speaker=spk, seed=4, max_frames=8, sampling=s,
                             vocoder_batch=8, first_batch=8)
    assert st.n_frames == 8 and sizes == [4 * 1920, 4 * 1920]
    assert np.array_equal(pcm, pcm2)


def _to_s16(pcm):
    """runtime/audio/wav.cpp:13-22: clamp to [-1, 1], scale by 32767, round to nearest (even)."""
    return np.rint(np.clip(np.asarray(pcm, np.float32), -1.0, 1.0) * np.float32(32767.0)).astype(np.int16)


def test_server_stream_matches_oracle_greedy(graph, scratch_dir):
    """The server's streaming path (server.cpp:398-495: the worker's synth into the bounded s16
    queue, drained by the consumer) against the oracle's request: greedy prompt -> prefill -> 40
    frames -> the codec decoder in one shot, then the server's s16 conversion. The streamed s16
    must reach SNR >= 40 dB against the oracle's s16, and the device vocoder fed the ORACLE's codes
    in the server's batches (4, then 16) must give the streamed s16 sample for sample: the stream
    carries exactly the oracle's codes."""
    import torch
    from oracle import sampler as osamp
    from oracle.model import Oracle
    from oracle.vocoder import Vocoder as OVoc
    abi, W, talker, frame, voc, _ = graph
    if not HARNESS.exists():
        pytest.fail(f"{HARNESS} is not built (run __graft_entry__.build())")
    lib = C.CDLL(str(HARNESS))
    fn = lib.navi_test_server_stream_request
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p, C.c_uint64,
                   C.c_int32, C.c_float, C.c_float, C.c_void_p, C.c_int64, C.POINTER(C.c_int64), C.c_void_p,
                   C.c_int32, C.POINTER(C.c_int32), C.c_char_p, C.c_size_t]
    n = 40
    ids = np.asarray(_ids(W.kv, 16, 31), np.int32)
    spk = np.random.default_rng(32).standard_normal(1024).astype(np.float32)
    pcm = np.zeros(n * 1920, np.int16)
    sizes = np.zeros(16, np.int32)
    n_pcm, n_sizes = C.c_int64(0), C.c_int32(0)
    err = C.create_string_buffer(512)
    log("server streaming path, greedy 40 frames, against the oracle's request")
    rc = fn(talker.h, frame.h, voc.h, int(W.kv["talker.language.english"]), ids.ctypes.data, ids.size,
            spk.ctypes.data, 6, n, 0.0, 0.0, pcm.ctypes.data, pcm.size, C.byref(n_pcm), sizes.ctypes.data,
            sizes.size, C.byref(n_sizes), err, 512)
    assert rc == 0, err.value.decode()
    sizes = sizes[:n_sizes.value].tolist()
    assert n_pcm.value == n * 1920 and sizes == [4 * 1920, 16 * 1920, 16 * 1920, 4 * 1920]

    path = scratch_dir / "small_all_spk.navi"
    ora = Oracle(path)
    pre, trail, pad = ora.build_prompt(ids.tolist(), "english", spk)
    kvo = ora.new_kv(128)
    hid, lg = ora.prefill(pre, kvo)
    so = osamp.Sampling(temperature=0.0, cp_temperature=0.0, repetition_penalty=1.05, min_frames=n)
    ora.reset()
    codes, step = [], None
    with torch.no_grad():
        for i in range(n):
            th = trail[i] if i < trail.shape[0] else pad
            if i == 0:
                c, step = ora.frame(so, 6, 0, th, hidden=hid, logits=lg)
            else:
                c, step = ora.frame(so, 6, i, th, kv=kvo, n_past=pre.shape[0] + i - 1, step_in=step)
            codes.append(c)
    want = _to_s16(OVoc(path).decode(np.array(codes))).astype(np.float64)
    got = pcm.astype(np.float64)
    snr = 10 * np.log10(np.sum(want ** 2) / max(np.sum((got - want) ** 2), 1e-300))
    voc.reset()
    b = np.asarray(codes)
    dev = np.concatenate([voc.decode(b[:4]), voc.decode(b[4:20]), voc.decode(b[20:36]), voc.decode(b[36:])])
    same = np.array_equal(_to_s16(dev), pcm)
    log(f"  server stream vs oracle: SNR {snr:.1f} dB (s16); device vocoder on the oracle's codes == stream: {same}")
    assert snr >= 40.0
    assert same
