"""ctypes view of the C restatement in oracle/csrc/sampler.c (test infrastructure).

Built by `make -C oracle/csrc` (run by __graft_entry__.build()) into oracle/lib/.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "lib" / "liboracle_sampler.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C oracle/csrc`")
        L = C.CDLL(str(LIB_PATH))
        L.ora_splitmix64.argtypes = [C.c_uint64]
        L.ora_splitmix64.restype = C.c_uint64
        L.ora_pcg32_next_inc.argtypes = [C.POINTER(C.c_uint64), C.c_uint64]
        L.ora_pcg32_next_inc.restype = C.c_uint32
        L.ora_pcg32_next.argtypes = [C.POINTER(C.c_uint64)]
        L.ora_pcg32_next.restype = C.c_uint32
        L.ora_draw_uniform.argtypes = [C.c_uint64]
        L.ora_draw_uniform.restype = C.c_float
        L.ora_frame_seeds.argtypes = [C.c_uint64, C.c_int32, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
        L.ora_frame_seeds.restype = None
        L.ora_cp_pos_seed.argtypes = [C.c_uint64, C.c_int32]
        L.ora_cp_pos_seed.restype = C.c_uint64
        fp = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        L.ora_kth_largest.argtypes = [fp, C.c_int32, C.c_int32]
        L.ora_kth_largest.restype = C.c_float
        L.ora_draw.argtypes = [fp, C.c_int32, C.c_float, C.c_uint64]
        L.ora_draw.restype = C.c_int32
        L.ora_argmax.argtypes = [fp, C.c_int32]
        L.ora_argmax.restype = C.c_int32
        _lib = L
    return _lib


def splitmix64(x: int) -> int:
    return lib().ora_splitmix64(x)


def pcg32_stream(state: int, n: int, inc: int | None = None) -> list[int]:
    st = C.c_uint64(state)
    if inc is None:
        return [lib().ora_pcg32_next(C.byref(st)) for _ in range(n)]
    return [lib().ora_pcg32_next_inc(C.byref(st), inc) for _ in range(n)]


def draw_uniform(seed: int) -> float:
    return lib().ora_draw_uniform(seed)


def frame_seeds(seed: int, frame_index: int) -> tuple[int, int]:
    t, c = C.c_uint64(), C.c_uint64()
    lib().ora_frame_seeds(seed, frame_index, C.byref(t), C.byref(c))
    return t.value, c.value


def cp_pos_seed(cp_seed: int, pos: int) -> int:
    return lib().ora_cp_pos_seed(cp_seed, pos)


def kth_largest(xs, k: int) -> float:
    a = np.ascontiguousarray(xs, dtype=np.float32)
    return float(lib().ora_kth_largest(a, a.size, k))


def draw(p, inv_sum: float, seed: int) -> int:
    a = np.ascontiguousarray(p, dtype=np.float32)
    return int(lib().ora_draw(a, a.size, np.float32(inv_sum), seed))


def argmax(v) -> int:
    a = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().ora_argmax(a, a.size))
