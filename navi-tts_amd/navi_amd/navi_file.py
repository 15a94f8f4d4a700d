"""`.navi` reader (runtime/weights/navi_file.cpp:79-148 semantics) for the Python plumbing.

Memory-maps the file, parses the KV and tensor tables with the same checks the
C++ reader makes (magic, version, file size, page-aligned in-bounds tensors,
byte length == numel * dtype size, unique names) and hands out numpy views.
"""
from __future__ import annotations

import mmap
import struct

import numpy as np

PAGE = 4096
DTYPE_SIZE = {0: 4, 1: 2, 2: 2, 3: 4, 4: 1}
DTYPE_NP = {0: np.float32, 1: np.uint16, 2: np.uint16, 3: np.int32, 4: np.uint8}


class NaviFormatError(ValueError):
    pass


class TensorInfo:
    __slots__ = ("name", "dtype", "dims", "offset", "nbytes")

    def __init__(self, name, dtype, dims, offset, nbytes):
        self.name, self.dtype, self.dims, self.offset, self.nbytes = name, dtype, dims, offset, nbytes

    @property
    def numel(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n


class NaviFile:
    def __init__(self, path):
        self.path = str(path)
        self._f = open(self.path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        b = self._mm
        if len(b) < 32:
            raise NaviFormatError(f"{path}: not a .navi file (too small)")
        if b[:4] != b"NAVI":
            raise NaviFormatError(f"{path}: bad magic; not a .navi file")
        version, self.data_offset, n_kv, n_t, size = struct.unpack_from("<IQIIQ", b, 4)
        if version != 1:
            raise NaviFormatError(f"{path}: .navi format version {version} (this build reads 1)")
        if size != len(b):
            raise NaviFormatError(f"{path}: header says {size} bytes, file is {len(b)} (truncated or corrupt)")
        if self.data_offset % PAGE or self.data_offset > len(b):
            raise NaviFormatError(f"{path}: bad data_offset")
        p, end = 32, self.data_offset

        def need(n):
            if p + n > end:
                raise NaviFormatError(f"{path}: truncated header")

        def string():
            nonlocal p
            need(4)
            (n,) = struct.unpack_from("<I", b, p)
            need(4 + n)
            s = bytes(b[p + 4:p + 4 + n]).decode("utf-8")
            p += 4 + n
            return s

        def take(fmt):
            nonlocal p
            sz = struct.calcsize(fmt)
            need(sz)
            v = struct.unpack_from(fmt, b, p)
            p += sz
            return v

        self.kv: dict = {}
        for _ in range(n_kv):
            key = string()
            (t,) = take("<B")
            if t == 0:
                (v,) = take("<q")
            elif t == 1:
                (v,) = take("<d")
            elif t == 2:
                v = string()
            elif t == 3:
                (n,) = take("<I")
                v = list(take(f"<{n}q"))
            else:
                raise NaviFormatError(f"{path}: kv '{key}' has unknown type")
            self.kv[key] = v
        self.tensors: list[TensorInfo] = []
        self._index: dict[str, int] = {}
        for _ in range(n_t):
            name = string()
            dt, nd = take("<BB")
            if dt not in DTYPE_SIZE:
                raise NaviFormatError(f"{path}: tensor '{name}' has unknown dtype")
            dims = tuple(take(f"<{nd}Q"))
            off, nbytes = take("<QQ")
            t = TensorInfo(name, dt, dims, off, nbytes)
            if off % PAGE or self.data_offset + off + nbytes > len(b):
                raise NaviFormatError(f"{path}: tensor '{name}' lies outside the file")
            if t.numel * DTYPE_SIZE[dt] != nbytes:
                raise NaviFormatError(f"{path}: tensor '{name}' shape does not match its byte length")
            if name in self._index:
                raise NaviFormatError(f"{path}: duplicate tensor '{name}'")
            self._index[name] = len(self.tensors)
            self.tensors.append(t)

    def find(self, name: str):
        i = self._index.get(name)
        return None if i is None else self.tensors[i]

    def get(self, name: str) -> TensorInfo:
        t = self.find(name)
        if t is None:
            raise KeyError(f"{self.path}: missing tensor '{name}'")
        return t

    def bytes_of(self, t: TensorInfo) -> memoryview:
        start = self.data_offset + t.offset
        return memoryview(self._mm)[start:start + t.nbytes]

    def array(self, name: str) -> np.ndarray:
        t = self.get(name)
        return np.frombuffer(self.bytes_of(t), dtype=DTYPE_NP[t.dtype]).reshape(t.dims)

    def close(self):
        if self._mm is not None:
            self._mm.close()
            self._f.close()
            self._mm = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
