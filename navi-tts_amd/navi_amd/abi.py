"""ctypes binding of include/navi_amd.h and the Python mirror of the host objects.

This is plumbing: it loads the in-tree libnavi_amd.so (and fails loudly when it
is missing), declares the C structs, and wraps the handles the way the
reference's C++ classes wrap their Impl: `DeviceWeights` (one device arena per
`.navi`, device_weights.cpp:18-76), `KvCache` (talker.h:20-24) and `Frame`
(frame.h:46-71). Nothing here computes; every operation is a C ABI call.
"""
from __future__ import annotations

import atexit
import ctypes as C
import weakref
from pathlib import Path

import numpy as np

from .navi_file import NaviFile

LIB_PATH = Path(__file__).resolve().parent.parent / "lib" / "libnavi_amd.so"

(NAVI_OK, NAVI_ERR_TIMEOUT, NAVI_ERR_LAUNCH, NAVI_ERR_KV_FULL, NAVI_ERR_INVALID, NAVI_ERR_HIP, NAVI_ERR_UNSUPPORTED,
 NAVI_ERR_CANCELLED) = range(8)

# The exported entry points include/navi_amd.h declares (checked by the CPU tests).
EXPORTS = [
    "navi_device_open", "navi_device_stream", "navi_device_synchronize", "navi_device_close", "navi_build_arch",
    "navi_mem_alloc", "navi_mem_free", "navi_mem_h2d", "navi_mem_d2h", "navi_mem_d2d", "navi_mem_zero",
    "navi_frame_create", "navi_frame_destroy", "navi_frame_reset", "navi_frame_run", "navi_frame_run_many", "navi_frame_step_out",
    "navi_frame_grid_blocks", "navi_frame_occupancy_per_mp", "navi_frame_set_taps", "navi_frame_tap_hidden",
    "navi_frame_tap_logits", "navi_frame_tap_cp_logits", "navi_frame_set_profile", "navi_frame_profile",
    "navi_frame_set_epoch", "navi_frame_epoch", "navi_frame_set_spin_cap",
    "navi_talker_create", "navi_talker_destroy", "navi_talker_build_prompt", "navi_talker_prefill", "navi_talker_kv",
    "navi_talker_hidden", "navi_talker_logits", "navi_talker_last_ms", "navi_talker_set_graphs", "navi_linear", "navi_linear_noalloc",
    "navi_vocoder_create", "navi_vocoder_destroy", "navi_vocoder_reset", "navi_vocoder_decode",
    "navi_vocoder_samples_per_frame", "navi_vocoder_max_chunk_frames", "navi_vocoder_last_ms", "navi_synth",
    "navi_vocoder_set_stage_hook", "navi_vocoder_owns_tensor", "navi_vocoder_set_graphs",
    "navi_streams_create", "navi_streams_destroy", "navi_streams_reset", "navi_streams_run", "navi_streams_step_out",
    "navi_streams_max_streams", "navi_streams_last_ms", "navi_streams_set_taps", "navi_streams_set_graphs",
    "navi_speaker_mel", "navi_speaker_create", "navi_speaker_destroy", "navi_speaker_embed_mel", "navi_speaker_embed",
    "navi_speaker_last_ms", "navi_speaker_tap_mel", "navi_speaker_dim",
    "navi_streams_tap_hidden",
    "navi_streams_tap_logits", "navi_streams_tap_cp_logits",
]


class NaviError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"[{status}] {msg}")
        self.status = status


class DeviceInfo(C.Structure):
    _fields_ = [("index", C.c_int32), ("name", C.c_char * 64), ("arch", C.c_char * 32),
                ("multiprocessors", C.c_int32), ("warp_size", C.c_int32), ("cooperative_launch", C.c_int32),
                ("max_threads_per_block", C.c_int32), ("lds_per_block", C.c_uint64),
                ("clock_khz", C.c_int32), ("mem_clock_khz", C.c_int32), ("mem_bus_width", C.c_int32),
                ("vram_total", C.c_uint64), ("vram_free", C.c_uint64), ("l2_bytes", C.c_uint64),
                ("hip_runtime_version", C.c_int32)]


class XformerParams(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("n_layer", C.c_int32), ("n_head", C.c_int32), ("n_kv_head", C.c_int32),
                ("head_dim", C.c_int32), ("ff", C.c_int32), ("vocab", C.c_int32), ("rms_eps", C.c_float),
                ("rope_theta", C.c_double)]


class ModelParams(C.Structure):
    _fields_ = [("talker", XformerParams), ("cp", XformerParams), ("n_code_groups", C.c_int32),
                ("codec_eos_id", C.c_int32), ("text_hidden", C.c_int32), ("text_vocab", C.c_int32),
                ("tts_bos_id", C.c_int32), ("tts_eos_id", C.c_int32), ("tts_pad_id", C.c_int32),
                ("codec_bos_id", C.c_int32), ("codec_pad_id", C.c_int32), ("codec_think_id", C.c_int32),
                ("codec_nothink_id", C.c_int32), ("codec_think_bos_id", C.c_int32), ("codec_think_eos_id", C.c_int32)]


class TensorRef(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ptr", C.c_void_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
                ("dims", C.c_uint64 * 4)]


class KvView(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("max_pos", C.c_int32), ("kv_dim", C.c_int32),
                ("k", C.POINTER(C.c_void_p)), ("v", C.POINTER(C.c_void_p))]


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("repetition_penalty", C.c_float),
                ("cp_temperature", C.c_float), ("cp_top_k", C.c_int32), ("min_frames", C.c_int32)]

    @staticmethod
    def make(temperature=0.9, top_k=50, repetition_penalty=1.05, cp_temperature=0.9, cp_top_k=50, min_frames=2):
        return Sampling(temperature, top_k, repetition_penalty, cp_temperature, cp_top_k, min_frames)

    @staticmethod
    def greedy(min_frames=2, repetition_penalty=1.05):
        return Sampling(0.0, 50, repetition_penalty, 0.0, 50, min_frames)


class FrameOptions(C.Structure):
    _fields_ = [("blocks_per_mp", C.c_int32), ("spin_cap", C.c_uint64)]


class FrameResult(C.Structure):
    _fields_ = [("ok", C.c_int32), ("eos", C.c_int32), ("codes", C.c_int32 * 16), ("us", C.c_double),
                ("status", C.c_int32), ("error", C.c_char * 160)]


class VocoderParams(C.Structure):
    _fields_ = [("xf", XformerParams), ("latent_dim", C.c_int32), ("codebook_dim", C.c_int32),
                ("codebook_size", C.c_int32), ("n_q", C.c_int32), ("n_semantic", C.c_int32),
                ("decoder_dim", C.c_int32), ("sliding_window", C.c_int32), ("upsampling_ratios", C.c_int32 * 2),
                ("upsample_rates", C.c_int32 * 4), ("samples_per_frame", C.c_int32)]


class SpeakerParams(C.Structure):
    _fields_ = [("sample_rate", C.c_int32), ("enc_dim", C.c_int32), ("n_fft", C.c_int32), ("num_mels", C.c_int32),
                ("hop", C.c_int32), ("win", C.c_int32), ("fmin", C.c_float), ("fmax", C.c_float)]


class SynthRequest(C.Structure):
    _fields_ = [("ids", C.c_void_p), ("n_ids", C.c_int32), ("language_id", C.c_int32), ("speaker", C.c_void_p),
                ("d_prefill", C.c_void_p), ("d_trailing", C.c_void_p), ("d_tts_pad", C.c_void_p),
                ("n_prefill", C.c_int32), ("n_trailing", C.c_int32), ("seed", C.c_uint64), ("max_frames", C.c_int32),
                ("sampling", Sampling), ("vocoder_batch", C.c_int32), ("first_batch", C.c_int32)]


class SynthStats(C.Structure):
    _fields_ = [("n_tokens", C.c_int32), ("n_frames", C.c_int32), ("hit_cap", C.c_int32), ("eos", C.c_int32),
                ("prefill_ms", C.c_double), ("frames_ms", C.c_double), ("vocoder_ms", C.c_double),
                ("total_ms", C.c_double), ("ttfa_ms", C.c_double), ("audio_s", C.c_double), ("rtf", C.c_double)]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


PCM_CALLBACK = C.CFUNCTYPE(C.c_int32, C.POINTER(C.c_float), C.c_int32, C.c_void_p)
STAGE_CALLBACK = C.CFUNCTYPE(None, C.c_void_p, C.c_char_p, C.c_void_p, C.c_int32, C.c_int32)


class Prompt(C.Structure):
    _fields_ = [("prefill", C.c_void_p), ("trailing", C.c_void_p), ("tts_pad", C.c_void_p),
                ("n_prefill", C.c_int32), ("n_trailing", C.c_int32)]


_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built (there is no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build(); there is no CPU fallback")
    L = C.CDLL(str(LIB_PATH))
    E = C.c_char_p
    L.navi_device_open.argtypes = [C.POINTER(DeviceInfo), E, C.c_size_t]
    L.navi_device_stream.restype = C.c_void_p
    L.navi_build_arch.restype = C.c_char_p
    L.navi_mem_alloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    L.navi_mem_free.argtypes = [C.c_void_p]
    for f in ("navi_mem_h2d", "navi_mem_d2h", "navi_mem_d2d"):
        getattr(L, f).argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    L.navi_mem_zero.argtypes = [C.c_void_p, C.c_size_t]
    L.navi_frame_create.argtypes = [C.POINTER(ModelParams), C.POINTER(TensorRef), C.c_int32, C.POINTER(FrameOptions),
                                    C.POINTER(C.c_void_p), E, C.c_size_t]
    L.navi_frame_destroy.argtypes = [C.c_void_p]
    L.navi_frame_destroy.restype = None
    L.navi_frame_reset.argtypes = [C.c_void_p]
    L.navi_frame_run.argtypes = [C.c_void_p, C.POINTER(KvView), C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.POINTER(Sampling), C.c_uint64, C.c_int32, C.POINTER(FrameResult)]
    L.navi_frame_run_many.argtypes = [C.c_void_p, C.POINTER(KvView), C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_int32, C.c_void_p, C.POINTER(Sampling), C.c_uint64, C.c_int32, C.c_int32, C.c_void_p,
                                      C.POINTER(C.c_int32), C.POINTER(C.c_int32), C.POINTER(C.c_double), E, C.c_size_t]
    L.navi_frame_step_out.argtypes = [C.c_void_p]
    L.navi_frame_step_out.restype = C.c_void_p
    for f in ("navi_frame_grid_blocks", "navi_frame_occupancy_per_mp"):
        getattr(L, f).argtypes = [C.c_void_p]
    L.navi_frame_set_taps.argtypes = [C.c_void_p, C.c_int32]
    L.navi_frame_set_profile.argtypes = [C.c_void_p, C.c_int32]
    L.navi_frame_profile.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32]
    L.navi_frame_set_epoch.argtypes = [C.c_void_p, C.c_uint32]
    L.navi_frame_epoch.argtypes = [C.c_void_p]
    L.navi_frame_epoch.restype = C.c_uint32
    L.navi_frame_set_spin_cap.argtypes = [C.c_void_p, C.c_uint64]
    for f in ("navi_frame_tap_hidden", "navi_frame_tap_logits", "navi_frame_tap_cp_logits"):
        getattr(L, f).argtypes = [C.c_void_p]
        getattr(L, f).restype = C.c_void_p
    L.navi_talker_set_graphs.argtypes = [C.c_void_p, C.c_int32]
    L.navi_talker_create.argtypes = [C.POINTER(ModelParams), C.POINTER(TensorRef), C.c_int32, C.c_int32, C.c_int32,
                                     C.POINTER(C.c_void_p), E, C.c_size_t]
    L.navi_talker_destroy.argtypes = [C.c_void_p]
    L.navi_talker_destroy.restype = None
    L.navi_talker_build_prompt.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.POINTER(Prompt),
                                           E, C.c_size_t]
    L.navi_talker_prefill.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, E, C.c_size_t]
    L.navi_talker_kv.argtypes = [C.c_void_p, C.POINTER(KvView), C.POINTER(C.c_int32)]
    for f in ("navi_talker_hidden", "navi_talker_logits"):
        getattr(L, f).argtypes = [C.c_void_p]
        getattr(L, f).restype = C.c_void_p
    L.navi_talker_last_ms.argtypes = [C.c_void_p]
    L.navi_talker_last_ms.restype = C.c_double
    L.navi_vocoder_create.argtypes = [C.POINTER(VocoderParams), C.POINTER(TensorRef), C.c_int32, C.c_int32,
                                      C.POINTER(C.c_void_p), E, C.c_size_t]
    L.navi_vocoder_destroy.argtypes = [C.c_void_p]
    L.navi_vocoder_destroy.restype = None
    L.navi_vocoder_reset.argtypes = [C.c_void_p]
    L.navi_vocoder_decode.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, E, C.c_size_t]
    for f in ("navi_vocoder_samples_per_frame", "navi_vocoder_max_chunk_frames"):
        getattr(L, f).argtypes = [C.c_void_p]
    L.navi_vocoder_last_ms.argtypes = [C.c_void_p]
    L.navi_vocoder_set_stage_hook.argtypes = [C.c_void_p, STAGE_CALLBACK, C.c_void_p]
    L.navi_vocoder_owns_tensor.argtypes = [C.c_char_p]
    L.navi_vocoder_set_graphs.argtypes = [C.c_void_p, C.c_int32]
    L.navi_vocoder_last_ms.restype = C.c_double
    L.navi_speaker_mel.argtypes = [C.POINTER(SpeakerParams), C.c_void_p, C.c_int64, C.c_void_p, C.c_int64,
                                   C.POINTER(C.c_int32), E, C.c_size_t]
    L.navi_speaker_create.argtypes = [C.POINTER(SpeakerParams), C.POINTER(TensorRef), C.c_int32, C.c_double,
                                      C.POINTER(C.c_void_p), E, C.c_size_t]
    L.navi_speaker_destroy.argtypes = [C.c_void_p]
    L.navi_speaker_destroy.restype = None
    L.navi_speaker_embed_mel.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, E, C.c_size_t]
    L.navi_speaker_embed.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, E, C.c_size_t]
    L.navi_speaker_last_ms.argtypes = [C.c_void_p]
    L.navi_speaker_last_ms.restype = C.c_double
    L.navi_speaker_dim.argtypes = [C.c_void_p]
    L.navi_speaker_dim.restype = C.c_int32
    L.navi_speaker_tap_mel.argtypes = [C.c_void_p, C.POINTER(C.c_int32)]
    L.navi_speaker_tap_mel.restype = C.c_void_p
    L.navi_synth.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(SynthRequest), PCM_CALLBACK, C.c_void_p,
                             C.POINTER(SynthStats), E, C.c_size_t]
    L.navi_linear.argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p,
                              C.c_int32, C.c_void_p, C.c_int32, E, C.c_size_t]
    L.navi_linear_noalloc.argtypes = L.navi_linear.argtypes
    L.navi_streams_create.argtypes = [C.POINTER(ModelParams), C.POINTER(TensorRef), C.c_int32, C.c_int32, C.c_int32,
                                      C.POINTER(C.c_void_p), E, C.c_size_t]
    L.navi_streams_destroy.argtypes = [C.c_void_p]
    L.navi_streams_destroy.restype = None
    L.navi_streams_reset.argtypes = [C.c_void_p, C.c_int32]
    L.navi_streams_run.argtypes = [C.c_void_p, C.c_int32, C.POINTER(KvView), C.c_void_p, C.c_void_p, C.c_void_p,
                                   C.POINTER(Sampling), C.c_void_p, C.c_void_p, C.c_void_p, E, C.c_size_t]
    L.navi_streams_set_taps.argtypes = [C.c_void_p, C.c_int32]
    L.navi_streams_set_graphs.argtypes = [C.c_void_p, C.c_int32]
    for f in ("navi_streams_step_out", "navi_streams_tap_hidden", "navi_streams_tap_logits", "navi_streams_tap_cp_logits"):
        getattr(L, f).argtypes = [C.c_void_p]
        getattr(L, f).restype = C.c_void_p
    L.navi_streams_max_streams.argtypes = [C.c_void_p]
    L.navi_streams_last_ms.argtypes = [C.c_void_p]
    L.navi_streams_last_ms.restype = C.c_double
    _lib = L
    return L


def _check(st: int, err: C.Array | None = None, what: str = ""):
    if st != NAVI_OK:
        msg = err.value.decode(errors="replace") if err is not None else what
        raise NaviError(st, msg or what)


# Every live handle and device buffer, released before the process exits (below).
_live = weakref.WeakSet()


def _track(obj):
    _live.add(obj)
    return obj


@atexit.register
def _release_all():
    """Destroys every live handle, frees every device buffer and closes the library's device
    (navi_device_close) while the interpreter shuts down: nothing of the library's is left for
    the C runtime's exit handlers, which run after any tool attached to HIP (a profiler) has
    finalised."""
    if _lib is None:
        return
    objs = list(_live)
    for o in objs:
        if not isinstance(o, DeviceBuffer):
            o.close()
    for o in objs:
        if isinstance(o, DeviceBuffer):
            o.free()
    _lib.navi_device_close()


def device_open() -> DeviceInfo:
    info = DeviceInfo()
    err = C.create_string_buffer(256)
    _check(lib().navi_device_open(C.byref(info), err, 256), err)
    return info


# ---- device memory -------------------------------------------------------------

class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(lib().navi_mem_alloc(C.byref(p), self.nbytes), what="navi_mem_alloc")
        self.ptr = p.value
        _track(self)

    def upload(self, arr: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes
        _check(lib().navi_mem_h2d(self.ptr + offset, a.ctypes.data, a.nbytes), what="navi_mem_h2d")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        _check(lib().navi_mem_d2h(out.ctypes.data, self.ptr + offset, out.nbytes), what="navi_mem_d2h")
        return out

    def free(self):
        if self.ptr:
            lib().navi_mem_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def download(ptr: int, dtype, count: int) -> np.ndarray:
    out = np.empty(count, dtype=dtype)
    _check(lib().navi_mem_d2h(out.ctypes.data, ptr, out.nbytes), what="navi_mem_d2h")
    return out


def upload(ptr: int, arr: np.ndarray):
    a = np.ascontiguousarray(arr)
    _check(lib().navi_mem_h2d(ptr, a.ctypes.data, a.nbytes), what="navi_mem_h2d")


# ---- weights ---------------------------------------------------------------------

ARENA_ALIGN = 256


class DeviceWeights:
    """One device arena holding every selected tensor of a `.navi`
    (DeviceWeights::upload, device_weights.cpp:18-76: 256-byte aligned, file order,
    `groups` placed adjacently)."""

    def __init__(self, path, select=None, groups=()):
        nf = NaviFile(path)
        self.kv = dict(nf.kv)
        chosen, seen_groups = [], set()
        group_of = {n: gi for gi, g in enumerate(groups) for n in g}
        take = (lambda t: select(t)) if select else (lambda t: t.dtype != 4)
        for t in nf.tensors:
            gi = group_of.get(t.name)
            if gi is None:
                if take(t):
                    chosen.append(t)
                continue
            if gi in seen_groups:
                continue
            seen_groups.add(gi)
            for n in groups[gi]:
                m = nf.find(n)
                if m is not None and take(m):
                    chosen.append(m)
        arena = sum((t.nbytes + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN for t in chosen)
        self.buf = DeviceBuffer(max(arena, 1))
        self.tensors = {}
        off = 0
        for t in chosen:
            _check(lib().navi_mem_h2d(self.buf.ptr + off, C.addressof(C.c_char.from_buffer_copy(b"\0")) if t.nbytes == 0 else
                                      np.frombuffer(nf.bytes_of(t), dtype=np.uint8).ctypes.data, t.nbytes), what=t.name)
            self.tensors[t.name] = (self.buf.ptr + off, t.dtype, t.dims)
            off += (t.nbytes + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN
        self.bytes = arena
        nf.close()

    def ptr(self, name: str) -> int:
        return self.tensors[name][0]

    def refs(self):
        """(TensorRef array, keepalive) for the ABI's create() calls."""
        names = list(self.tensors)
        arr = (TensorRef * len(names))()
        keep = []
        for i, n in enumerate(names):
            p, dt, dims = self.tensors[n]
            b = n.encode()
            keep.append(b)
            arr[i].name = b
            arr[i].ptr = p
            arr[i].dtype = dt
            arr[i].ndim = len(dims)
            for k, d in enumerate(dims[:4]):
                arr[i].dims[k] = d
        return arr, keep


def model_params(kv: dict) -> ModelParams:
    """read_params (params.cpp:59-130) for the fields the path uses."""
    def xf(ns):
        return XformerParams(kv[f"{ns}.hidden_size"], kv[f"{ns}.num_hidden_layers"], kv[f"{ns}.num_attention_heads"],
                             kv[f"{ns}.num_key_value_heads"], kv[f"{ns}.head_dim"], kv[f"{ns}.intermediate_size"],
                             kv.get(f"{ns}.vocab_size", 0), float(kv[f"{ns}.rms_norm_eps"]), float(kv[f"{ns}.rope_theta"]))
    if kv.get("general.arch") != "qwen3-tts":
        raise ValueError(f"architecture '{kv.get('general.arch')}' is not qwen3-tts")
    return ModelParams(xf("talker"), xf("cp"), kv["talker.num_code_groups"], kv["talker.codec_eos_token_id"],
                       kv["talker.text_hidden_size"], kv["talker.text_vocab_size"], kv["text.tts_bos_id"],
                       kv["text.tts_eos_id"], kv["text.tts_pad_id"], kv["talker.codec_bos_id"], kv["talker.codec_pad_id"],
                       kv["talker.codec_think_id"], kv["talker.codec_nothink_id"], kv["talker.codec_think_bos_id"],
                       kv["talker.codec_think_eos_id"])


# ---- KV cache ----------------------------------------------------------------------

class KvCache:
    """talker.h:20-24: per layer [max_pos][kv_dim] f16 K and V, device-resident."""

    def __init__(self, n_layer: int, max_pos: int, kv_dim: int):
        self.n_layer, self.max_pos, self.kv_dim = n_layer, max_pos, kv_dim
        per = max_pos * kv_dim * 2
        self.buf = DeviceBuffer(2 * n_layer * per)
        self.k = [self.buf.ptr + l * per for l in range(n_layer)]
        self.v = [self.buf.ptr + (n_layer + l) * per for l in range(n_layer)]
        self.n_used = 0
        self._kp = (C.c_void_p * n_layer)(*self.k)
        self._vp = (C.c_void_p * n_layer)(*self.v)
        self.view = KvView(n_layer, max_pos, kv_dim, C.cast(self._kp, C.POINTER(C.c_void_p)),
                           C.cast(self._vp, C.POINTER(C.c_void_p)))

    def fill(self, layer: int, k_rows: np.ndarray, v_rows: np.ndarray, pos0: int = 0):
        """Writes f16 rows (uint16 bit patterns or float arrays) at positions pos0..."""
        def bits(a):
            a = np.asarray(a)
            return a if a.dtype == np.uint16 else a.astype(np.float16).view(np.uint16)
        kb, vb = bits(k_rows), bits(v_rows)
        off = pos0 * self.kv_dim * 2
        upload(self.k[layer] + off, kb)
        upload(self.v[layer] + off, vb)

    def read(self, layer: int, n: int):
        k = download(self.k[layer], np.uint16, n * self.kv_dim).view(np.float16).astype(np.float32)
        v = download(self.v[layer], np.uint16, n * self.kv_dim).view(np.float16).astype(np.float32)
        return k.reshape(n, self.kv_dim), v.reshape(n, self.kv_dim)


# ---- frame -------------------------------------------------------------------------

class Frame:
    """frame.h:46-71 over navi_frame_*."""

    def __init__(self, weights: DeviceWeights, params: ModelParams | None = None, spin_cap: int = 0):
        self.params = params or model_params(weights.kv)
        refs, self._keep = weights.refs()
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        opt = FrameOptions(1, spin_cap)
        _check(lib().navi_frame_create(C.byref(self.params), refs, len(refs), C.byref(opt), C.byref(h), err, 256), err)
        self.h = h.value
        self.hidden = self.params.talker.hidden
        _track(self)

    def close(self):
        if self.h:
            lib().navi_frame_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        _check(lib().navi_frame_reset(self.h), what="navi_frame_reset")

    def set_taps(self, on: bool):
        _check(lib().navi_frame_set_taps(self.h, 1 if on else 0), what="navi_frame_set_taps")

    def set_epoch(self, epoch: int):
        """Test hook: the next launch uses epoch + 4096 (wrapping past 2^32 - 4096)."""
        _check(lib().navi_frame_set_epoch(self.h, epoch), what="navi_frame_set_epoch")

    @property
    def epoch(self) -> int:
        return int(lib().navi_frame_epoch(self.h))

    def set_spin_cap(self, spin_cap: int):
        _check(lib().navi_frame_set_spin_cap(self.h, C.c_uint64(spin_cap)), what="navi_frame_set_spin_cap")

    def _run(self, kv, n_past, skip, d_hidden, d_logits, d_trailing, s, seed, frame_index) -> FrameResult:
        r = FrameResult()
        lib().navi_frame_run(self.h, C.byref(kv.view) if kv is not None else None, n_past, skip, d_hidden, d_logits,
                             d_trailing, C.byref(s), C.c_uint64(seed & ((1 << 64) - 1)), frame_index, C.byref(r))
        return r

    def run_first(self, d_hidden: int, d_logits: int, d_trailing: int, s: Sampling, seed: int, frame_index: int):
        return self._run(None, 0, 1, d_hidden, d_logits, d_trailing, s, seed, frame_index)

    def run(self, kv: KvCache, n_past: int, d_trailing: int, s: Sampling, seed: int, frame_index: int):
        r = self._run(kv, n_past, 0, None, None, d_trailing, s, seed, frame_index)
        if r.ok:
            kv.n_used = n_past + 1
        return r

    def run_many(self, kv, n_past0: int, d_trailing: int, n_trailing: int, d_tts_pad: int, s: Sampling, seed: int,
                 frame_index0: int, n_frames: int, skip_first: bool = False, d_hidden: int | None = None,
                 d_logits: int | None = None):
        """navi_frame_run_many: (codes [n_done][16], eos, device us of the loop)."""
        codes = np.zeros((n_frames, 16), dtype=np.int32)
        done, eos, us = C.c_int32(), C.c_int32(), C.c_double()
        err = C.create_string_buffer(256)
        _check(lib().navi_frame_run_many(self.h, C.byref(kv.view) if kv is not None else None, n_past0, 1 if skip_first else 0,
                                         d_hidden, d_logits, d_trailing, n_trailing, d_tts_pad, C.byref(s),
                                         C.c_uint64(seed & ((1 << 64) - 1)), frame_index0, n_frames, codes.ctypes.data,
                                         C.byref(done), C.byref(eos), C.byref(us), err, 256), err)
        last = n_past0 + done.value - 1
        if kv is not None and done.value > (1 if skip_first else 0):
            kv.n_used = last + 1
        return codes[:done.value], bool(eos.value), us.value

    @property
    def d_step_out(self) -> int:
        return lib().navi_frame_step_out(self.h)

    def grid_blocks(self) -> int:
        return lib().navi_frame_grid_blocks(self.h)

    def taps(self):
        L = lib()
        hid = download(L.navi_frame_tap_hidden(self.h), np.float32, self.hidden)
        lg = download(L.navi_frame_tap_logits(self.h), np.float32, self.params.talker.vocab)
        cp = download(L.navi_frame_tap_cp_logits(self.h), np.float32, 15 * self.params.cp.vocab).reshape(15, -1)
        return hid, lg, cp

    def set_profile(self, on: bool):
        _check(lib().navi_frame_set_profile(self.h, 1 if on else 0), what="navi_frame_set_profile")

    def profile(self, n_blocks: int = 256, n_slots: int = 4096) -> np.ndarray:
        """[n_blocks][n_slots] 100 MHz stamps of the last run with profiling on."""
        out = np.zeros((n_blocks, n_slots), dtype=np.uint64)
        _check(lib().navi_frame_profile(self.h, out.ctypes.data, n_blocks, n_slots), what="navi_frame_profile")
        return out

    def step_out(self) -> np.ndarray:
        return download(self.d_step_out, np.float32, self.hidden)


# ---- multi-stream decode ---------------------------------------------------------------

class Streams:
    """navi_streams_*: one frame for each of n independent streams per call."""

    def __init__(self, weights: DeviceWeights, max_streams: int, max_positions: int, params: ModelParams | None = None):
        self.params = params or model_params(weights.kv)
        refs, self._keep = weights.refs()
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        _check(lib().navi_streams_create(C.byref(self.params), refs, len(refs), max_streams, max_positions, C.byref(h),
                                         err, 256), err)
        self.h = h.value
        self.max_streams = max_streams
        self.hidden = self.params.talker.hidden
        _track(self)

    def close(self):
        if self.h:
            lib().navi_streams_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self, stream: int = -1):
        _check(lib().navi_streams_reset(self.h, stream), what="navi_streams_reset")

    def set_taps(self, on: bool):
        _check(lib().navi_streams_set_taps(self.h, 1 if on else 0), what="navi_streams_set_taps")

    def set_graphs(self, on: bool):
        _check(lib().navi_streams_set_graphs(self.h, 1 if on else 0), what="navi_streams_set_graphs")

    def run(self, kvs, n_past, d_trailing: int, s: Sampling, seeds, frame_index, d_step_in: int | None = None):
        """codes [n][16] (int32) for streams 0..n-1; kvs: one KvCache (or TalkerKv) per stream."""
        n = len(kvs)
        views = (KvView * n)(*[k.view for k in kvs])
        npast = np.ascontiguousarray(n_past, dtype=np.int32)
        sd = np.ascontiguousarray([x & ((1 << 64) - 1) for x in seeds], dtype=np.uint64)
        fi = np.ascontiguousarray(frame_index, dtype=np.int32)
        codes = np.zeros((n, 16), dtype=np.int32)
        err = C.create_string_buffer(256)
        _check(lib().navi_streams_run(self.h, n, views, npast.ctypes.data, d_step_in, d_trailing, C.byref(s),
                                      sd.ctypes.data, fi.ctypes.data, codes.ctypes.data, err, 256), err)
        for i, k in enumerate(kvs):
            k.n_used = int(npast[i]) + 1
        return codes

    @property
    def d_step_out(self) -> int:
        return lib().navi_streams_step_out(self.h)

    def step_out(self, n: int) -> np.ndarray:
        return download(self.d_step_out, np.float32, n * self.hidden).reshape(n, self.hidden)

    def taps(self, n: int):
        """(post-norm hidden [n][H], raw logits [n][VT], cp logits [n][15][VC]) of the last run."""
        L, p = lib(), self.params
        ms, H, VT, VC = self.max_streams, self.hidden, p.talker.vocab, p.cp.vocab
        hid = download(L.navi_streams_tap_hidden(self.h), np.float32, ms * H).reshape(ms, H)[:n]
        lg = download(L.navi_streams_tap_logits(self.h), np.float32, ms * VT).reshape(ms, VT)[:n]
        cp = download(L.navi_streams_tap_cp_logits(self.h), np.float32, ms * 15 * VC).reshape(ms, 15, VC)[:n]
        return hid, lg, cp

    def last_ms(self) -> float:
        return lib().navi_streams_last_ms(self.h)


# ---- talker: prompt rows + prefill ----------------------------------------------------

class TalkerKv:
    """The talker-owned KV cache seen as the KvCache the frame takes (talker.h:20-24, 48)."""

    def __init__(self, view: KvView, n_used: int):
        self.view = view
        self.n_layer, self.max_pos, self.kv_dim = view.n_layer, view.max_pos, view.kv_dim
        self.k = [view.k[l] for l in range(view.n_layer)]
        self.v = [view.v[l] for l in range(view.n_layer)]
        self.n_used = n_used

    def read(self, layer: int, n: int):
        k = download(self.k[layer], np.uint16, n * self.kv_dim).view(np.float16).astype(np.float32)
        v = download(self.v[layer], np.uint16, n * self.kv_dim).view(np.float16).astype(np.float32)
        return k.reshape(n, self.kv_dim), v.reshape(n, self.kv_dim)

    def fill(self, layer: int, k_rows: np.ndarray, v_rows: np.ndarray, pos0: int = 0):
        KvCache.fill(self, layer, k_rows, v_rows, pos0)


class Talker:
    """talker.h:34-67 over navi_talker_*: prompt rows, the causal prefill, the KV cache."""

    def __init__(self, weights: DeviceWeights, max_prompt_tokens: int = 1024, max_positions: int = 2048,
                 params: ModelParams | None = None):
        self.params = params or model_params(weights.kv)
        self.kv_meta = weights.kv
        refs, self._keep = weights.refs()
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        _check(lib().navi_talker_create(C.byref(self.params), refs, len(refs), max_prompt_tokens, max_positions,
                                        C.byref(h), err, 256), err)
        self.h = h.value
        self.hidden = self.params.talker.hidden
        v, n = KvView(), C.c_int32()
        _check(lib().navi_talker_kv(self.h, C.byref(v), C.byref(n)), what="navi_talker_kv")
        self.kv = TalkerKv(v, n.value)
        _track(self)

    def close(self):
        if self.h:
            lib().navi_talker_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_graphs(self, on: bool):
        _check(lib().navi_talker_set_graphs(self.h, 1 if on else 0), what="navi_talker_set_graphs")

    def language_id(self, language: str) -> int:
        if language in ("", "auto"):
            return -1
        key = f"talker.language.{language}"
        if key not in self.kv_meta:
            raise NaviError(NAVI_ERR_INVALID, f"talker: unknown language '{language}'")
        return int(self.kv_meta[key])

    def build_prompt(self, ids, language: str, speaker: np.ndarray) -> Prompt:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        spk = np.ascontiguousarray(speaker, dtype=np.float32)
        pr = Prompt()
        err = C.create_string_buffer(256)
        _check(lib().navi_talker_build_prompt(self.h, a.ctypes.data, a.size, self.language_id(language), spk.ctypes.data,
                                              C.byref(pr), err, 256), err)
        return pr

    def prompt_arrays(self, pr: Prompt):
        """(prefill rows, trailing rows, tts_pad row) downloaded as f32 arrays."""
        H = self.hidden
        return (download(pr.prefill, np.float32, pr.n_prefill * H).reshape(pr.n_prefill, H),
                download(pr.trailing, np.float32, pr.n_trailing * H).reshape(pr.n_trailing, H),
                download(pr.tts_pad, np.float32, H))

    def prefill(self, d_rows: int, n_rows: int):
        err = C.create_string_buffer(256)
        _check(lib().navi_talker_prefill(self.h, d_rows, n_rows, err, 256), err)
        self.kv.n_used = n_rows

    @property
    def d_hidden(self) -> int:
        return lib().navi_talker_hidden(self.h)

    @property
    def d_logits(self) -> int:
        return lib().navi_talker_logits(self.h)

    def hidden_logits(self):
        return (download(self.d_hidden, np.float32, self.hidden),
                download(self.d_logits, np.float32, self.params.talker.vocab))

    def last_ms(self) -> float:
        return lib().navi_talker_last_ms(self.h)


def linear(d_x: int, ldx: int, M: int, w: int, K: int, N: int, d_y: int, ldy: int, bias: int | None = None,
           residual: int | None = None, act: int = 0, noalloc: bool = False):
    """navi_linear (navi_linear_noalloc with noalloc): d_y = act(d_x . w^T + bias) + residual on the device."""
    err = C.create_string_buffer(256)
    fn = lib().navi_linear_noalloc if noalloc else lib().navi_linear
    _check(fn(d_x, ldx, M, w, K, N, bias, residual, act, d_y, ldy, err, 256), err)


# ---- vocoder ---------------------------------------------------------------------------

def vocoder_params(kv: dict) -> VocoderParams:
    """The codec decoder fields of read_params (params.cpp:106-117)."""
    ns = "codec.decoder"
    xf = XformerParams(kv[f"{ns}.hidden_size"], kv[f"{ns}.num_hidden_layers"], kv[f"{ns}.num_attention_heads"],
                       kv[f"{ns}.num_key_value_heads"], kv[f"{ns}.head_dim"], kv[f"{ns}.intermediate_size"], 0,
                       float(kv[f"{ns}.rms_norm_eps"]), float(kv[f"{ns}.rope_theta"]))
    p = VocoderParams()
    p.xf = xf
    p.latent_dim, p.codebook_dim = kv[f"{ns}.latent_dim"], kv[f"{ns}.codebook_dim"]
    p.codebook_size, p.n_q = kv[f"{ns}.codebook_size"], kv[f"{ns}.num_quantizers"]
    p.n_semantic, p.decoder_dim = kv[f"{ns}.num_semantic_quantizers"], kv[f"{ns}.decoder_dim"]
    p.sliding_window = kv.get(f"{ns}.sliding_window", 0)
    for i, r in enumerate(kv[f"{ns}.upsampling_ratios"]):
        p.upsampling_ratios[i] = r
    for i, r in enumerate(kv[f"{ns}.upsample_rates"]):
        p.upsample_rates[i] = r
    p.samples_per_frame = kv["codec.decode_upsample_rate"]
    return p


class Vocoder:
    """vocoder.h:27-55 over navi_vocoder_*."""

    def __init__(self, weights: DeviceWeights, max_chunk_frames: int = 32):
        self.params = vocoder_params(weights.kv)
        refs, self._keep = weights.refs()
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        _check(lib().navi_vocoder_create(C.byref(self.params), refs, len(refs), max_chunk_frames, C.byref(h), err, 256), err)
        self.h = h.value
        self.samples_per_frame = lib().navi_vocoder_samples_per_frame(self.h)
        self.n_q = self.params.n_q
        _track(self)

    def close(self):
        if self.h:
            lib().navi_vocoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        _check(lib().navi_vocoder_reset(self.h), what="navi_vocoder_reset")

    def decode(self, codes) -> np.ndarray:
        c = np.ascontiguousarray(codes, dtype=np.int32).reshape(-1, self.n_q)
        out = np.empty(c.shape[0] * self.samples_per_frame, np.float32)
        err = C.create_string_buffer(256)
        _check(lib().navi_vocoder_decode(self.h, c.ctypes.data, c.shape[0], out.ctypes.data, err, 256), err)
        return out

    def last_ms(self) -> float:
        return lib().navi_vocoder_last_ms(self.h)

    def set_graphs(self, on: bool):
        _check(lib().navi_vocoder_set_graphs(self.h, 1 if on else 0), what="navi_vocoder_set_graphs")

    def set_stage_hook(self, fn):
        """Vocoder::set_stage_hook: fn(name, host f32 [rows][cols]) after every stage (None = off)."""
        if fn is None:
            self._hook = None
            _check(lib().navi_vocoder_set_stage_hook(self.h, STAGE_CALLBACK(), None), what="navi_vocoder_set_stage_hook")
            return

        def tramp(_user, name, d_buf, rows, cols):
            fn(name.decode(), download(d_buf, np.float32, rows * cols).reshape(rows, cols))
        self._hook = STAGE_CALLBACK(tramp)
        _check(lib().navi_vocoder_set_stage_hook(self.h, self._hook, None), what="navi_vocoder_set_stage_hook")


# ---- speaker encoder -------------------------------------------------------------------

def speaker_params(kv: dict) -> SpeakerParams:
    """The speaker fields of read_params (params.cpp:97-104)."""
    return SpeakerParams(kv["speaker.sample_rate"], kv["speaker.enc_dim"], kv["speaker.mel.n_fft"],
                         kv["speaker.mel.num_mels"], kv["speaker.mel.hop_size"], kv["speaker.mel.win_size"],
                         float(kv["speaker.mel.fmin"]), float(kv["speaker.mel.fmax"]))


def speaker_mel(kv_or_params, wav) -> np.ndarray:
    """navi_speaker_mel (SpeakerEncoder::mel, speaker.hip:269-303): log-mel [num_mels][T] of a mono
    waveform in [-1, 1], computed on the host by the library."""
    p = kv_or_params if isinstance(kv_or_params, SpeakerParams) else speaker_params(kv_or_params)
    x = np.ascontiguousarray(wav, dtype=np.float32).reshape(-1)
    n = C.c_int32()
    err = C.create_string_buffer(256)
    _check(lib().navi_speaker_mel(C.byref(p), x.ctypes.data, x.size, None, 0, C.byref(n), err, 256), err)
    out = np.empty((p.num_mels, n.value), np.float32)
    _check(lib().navi_speaker_mel(C.byref(p), x.ctypes.data, x.size, out.ctypes.data, out.size, C.byref(n), err, 256), err)
    return out


class Speaker:
    """speaker.h:17-38 (SpeakerEncoder) over navi_speaker_*."""

    def __init__(self, weights: DeviceWeights, max_seconds: float = 30.0):
        self.params = speaker_params(weights.kv)
        refs, self._keep = weights.refs()
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        _check(lib().navi_speaker_create(C.byref(self.params), refs, len(refs), max_seconds, C.byref(h), err, 256), err)
        self.h = h.value
        _track(self)

    def close(self):
        if self.h:
            lib().navi_speaker_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def mel(self, wav) -> np.ndarray:
        return speaker_mel(self.params, wav)

    def embed(self, wav) -> np.ndarray:
        """[enc_dim] embedding of a mono 24 kHz waveform in [-1, 1]."""
        x = np.ascontiguousarray(wav, dtype=np.float32).reshape(-1)
        out = np.empty(self.params.enc_dim, np.float32)
        err = C.create_string_buffer(256)
        _check(lib().navi_speaker_embed(self.h, x.ctypes.data, x.size, out.ctypes.data, err, 256), err)
        return out

    def embed_mel(self, mel) -> np.ndarray:
        """... from a precomputed mel [num_mels][T]."""
        m = np.ascontiguousarray(mel, dtype=np.float32)
        if m.ndim != 2 or m.shape[0] != self.params.num_mels:
            raise ValueError(f"speaker: mel must be [{self.params.num_mels}][T], got {m.shape}")
        out = np.empty(self.params.enc_dim, np.float32)
        err = C.create_string_buffer(256)
        _check(lib().navi_speaker_embed_mel(self.h, m.ctypes.data, m.shape[1], out.ctypes.data, err, 256), err)
        return out

    def last_ms(self) -> float:
        return lib().navi_speaker_last_ms(self.h)

    def tap_mel(self) -> np.ndarray:
        """The device log-mel of the last embed as [num_mels][T] (navi_speaker_tap_mel)."""
        n = C.c_int32()
        ptr = lib().navi_speaker_tap_mel(self.h, C.byref(n))
        out = np.empty((n.value, self.params.num_mels), np.float32)
        _check(lib().navi_mem_d2h(out.ctypes.data, ptr, out.nbytes), what="navi_mem_d2h")
        return out.T.copy()


# ---- one request end to end ------------------------------------------------------------

def synth(talker: "Talker", frame: Frame, vocoder: "Vocoder", *, ids=None, language: str = "english", speaker=None,
          prompt=None, seed: int = 0, max_frames: int = 600, sampling: Sampling | None = None, vocoder_batch: int = 0,
          first_batch: int = 0, on_pcm=None):
    """navi_synth (Graph::synth, graph.cpp:52-111). ids + speaker build the prompt; or `prompt` =
    (d_prefill, n_prefill, d_trailing, n_trailing, d_tts_pad) gives the rows directly.
    on_pcm(chunk f32 array), if given, sees each vocoder batch as it is produced; an exception it
    raises stops the request (no further frame runs) and propagates out of synth, as an exception
    from Graph::synth's on_pcm does.
    Returns (SynthStats, pcm f32 array, [samples per vocoder batch])."""
    req = SynthRequest()
    keep = []
    if prompt is None:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        spk = np.ascontiguousarray(speaker, dtype=np.float32)
        keep += [a, spk]
        req.ids, req.n_ids, req.speaker = a.ctypes.data, a.size, spk.ctypes.data
        req.language_id = talker.language_id(language)
    else:
        req.d_prefill, req.n_prefill, req.d_trailing, req.n_trailing, req.d_tts_pad = prompt
    req.seed = seed & ((1 << 64) - 1)
    req.max_frames = max_frames
    req.sampling = sampling or Sampling.make()
    req.vocoder_batch, req.first_batch = vocoder_batch, first_batch
    chunks, raised = [], []

    def trampoline(ptr, n, _user):
        chunk = np.ctypeslib.as_array(ptr, shape=(n,)).copy()
        chunks.append(chunk)
        if on_pcm is not None:
            try:
                on_pcm(chunk)
            except BaseException as e:        # handed back to the caller after navi_synth returns
                raised.append(e)
                return 1
        return 0

    cb = PCM_CALLBACK(trampoline)
    st = SynthStats()
    err = C.create_string_buffer(256)
    status = lib().navi_synth(talker.h, frame.h, vocoder.h, C.byref(req), cb, None, C.byref(st), err, 256)
    if raised and status == NAVI_ERR_CANCELLED:
        raise raised[0]
    _check(status, err)
    pcm = np.concatenate(chunks) if chunks else np.zeros(0, np.float32)
    return st, pcm, [c.size for c in chunks]
