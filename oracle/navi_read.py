"""Minimal `.navi` reader for the oracle (docs/navi-format.md:1-47).

Test infrastructure: memory-maps the file and hands out numpy views. Mirrors
runtime/weights/navi_file.cpp:79-148 (header, KV table, tensor table checks).
"""
from __future__ import annotations

import struct

import numpy as np

_DT = {0: np.float32, 1: np.float16, 2: np.uint16, 3: np.int32, 4: np.uint8}


class NaviBlob:
    def __init__(self, path):
        self.path = str(path)
        self.mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        b = self.mm
        if bytes(b[:4]) != b"NAVI":
            raise ValueError(f"{path}: bad magic")
        version, data_offset, n_kv, n_t, size = struct.unpack_from("<IQIIQ", b, 4)
        if version != 1 or size != b.size or data_offset % 4096:
            raise ValueError(f"{path}: bad header")
        self.data_offset = data_offset
        p = 32

        def string():
            nonlocal p
            (n,) = struct.unpack_from("<I", b, p)
            s = bytes(b[p + 4:p + 4 + n]).decode()
            p += 4 + n
            return s

        self.kv = {}
        for _ in range(n_kv):
            key = string()
            t = int(b[p])
            p += 1
            if t == 0:
                (v,) = struct.unpack_from("<q", b, p); p += 8
            elif t == 1:
                (v,) = struct.unpack_from("<d", b, p); p += 8
            elif t == 2:
                v = string()
            elif t == 3:
                (n,) = struct.unpack_from("<I", b, p); p += 4
                v = list(struct.unpack_from(f"<{n}q", b, p)); p += 8 * n
            else:
                raise ValueError(f"{path}: kv {key} has unknown type {t}")
            self.kv[key] = v
        self.tensors = {}
        for _ in range(n_t):
            name = string()
            dt, nd = int(b[p]), int(b[p + 1])
            p += 2
            dims = struct.unpack_from(f"<{nd}Q", b, p); p += 8 * nd
            off, nbytes = struct.unpack_from("<QQ", b, p); p += 16
            self.tensors[name] = (int(dt), tuple(int(d) for d in dims), int(off), int(nbytes))

    def array(self, name) -> np.ndarray:
        dt, dims, off, nbytes = self.tensors[name]
        start = self.data_offset + off
        return np.frombuffer(self.mm, dtype=_DT[dt], count=int(np.prod(dims, dtype=np.int64)), offset=start).reshape(dims)

    def f32(self, name) -> np.ndarray:
        """The tensor as f32 (exact for f16 storage)."""
        return self.array(name).astype(np.float32)
