"""GgufFile: the checkpoint reader of the Q8_0 path over libmi_sdvk.so.

Mirrors ofc::GgufFile (src/Modules/Model/Gguf.hpp:90-140, Gguf.cpp:290-583):
the same method names, argument meaning and error behaviour -- `open` returns
False and fills `err`, `readFloat` returns an empty list and `readQ8` False
when the tensor is missing or has the wrong type. The parsing and decoding run
in the library (mi_gguf_* in include/mi_sdvk.h); this module only moves
results into numpy arrays. Upload helpers write caller-owned device buffers in
the layouts the GEMM entries read (sdvkgen.cpp:549-611).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from ._lib import MiGgufMetaInfo, MiGgufTensorInfo, call, ptr

# ggml tensor type ids (Gguf.hpp:15-31)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, BF16 = 0, 1, 2, 3, 6, 7, 8, 9, 30
# GGUF metadata value types (Gguf.hpp:71-85)
(GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, GGUF_BOOL, GGUF_STRING,
 GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64) = range(13)


@dataclass(frozen=True)
class GgufTensor:
    """Gguf.hpp:36-47 (+ the logical rows / cols of ggdims, sdvkgen.cpp:151-176)."""
    index: int
    name: str
    dims: tuple
    type: int
    offset: int
    nbytes: int
    rows: int
    cols: int

    def nElems(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def shape(self) -> tuple:
        """(rows, cols) = (dims[1], dims[0]); 1-D -> (1, n); N-D folds dims[1:]."""
        if len(self.dims) == 1:
            return (1, self.dims[0])
        r = 1
        for d in self.dims[1:]:
            r *= d
        return (r, self.dims[0])


@dataclass(frozen=True)
class GgufMeta:
    """Gguf.hpp:50-68: one metadata value (scalars in u / f / b / s, arrays as lists)."""
    type: int
    u: int = 0
    f: float = 0.0
    b: bool = False
    s: str = ""
    arrType: int = 0
    items: tuple = ()

    def isArray(self) -> bool:
        return self.type == GGUF_ARRAY

    def isStr(self) -> bool:
        return self.type == GGUF_STRING

    def isNum(self) -> bool:
        return self.type not in (GGUF_STRING, GGUF_ARRAY)


class GgufFile:
    def __init__(self):
        self._h = ctypes.c_void_p()
        self._tensors: list[GgufTensor] = []
        self._version = 0
        self._data_offset = 0
        self._file_size = 0

    # -- lifetime --------------------------------------------------------------
    def open(self, path: str, err: Optional[list] = None, prefix: str = "") -> bool:
        """Gguf.cpp:290-416. On failure returns False and appends the reason to err."""
        self.close()
        lib = _lib.load()
        h = ctypes.c_void_p()
        st = lib.mi_gguf_open(str(path).encode(), prefix.encode() if prefix else None, ctypes.byref(h))
        if st != _lib.MI_OK:
            if err is not None:
                err.append(lib.mi_last_error().decode())
            return False
        self._h = h
        ver, n, off, size = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        call("mi_gguf_info", h, ctypes.byref(ver), ctypes.byref(n), ctypes.byref(off), ctypes.byref(size))
        self._version, self._data_offset, self._file_size = ver.value, off.value, size.value
        self._tensors = [self._tensor(i) for i in range(n.value)]
        return True

    def close(self) -> None:
        if self._h:
            _lib.load().mi_gguf_close(self._h)
            self._h = ctypes.c_void_p()
        self._tensors = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- table -----------------------------------------------------------------
    def _tensor(self, i: int) -> GgufTensor:
        info = MiGgufTensorInfo()
        call("mi_gguf_tensor", self._h, i, ctypes.byref(info))
        return GgufTensor(i, info.name.decode(), tuple(info.dims[: info.n_dims]), info.type, info.offset, info.nbytes,
                          info.rows, info.cols)

    def version(self) -> int:
        return self._version

    def tensorCount(self) -> int:
        return len(self._tensors)

    def tensors(self) -> list:
        return list(self._tensors)

    def find(self, name: str) -> Optional[GgufTensor]:
        idx = ctypes.c_uint64()
        st = _lib.load().mi_gguf_find(self._h, name.encode(), ctypes.byref(idx))
        return self._tensors[idx.value] if st == _lib.MI_OK else None

    def dataOffset(self) -> int:
        return self._data_offset

    def fileSize(self) -> int:
        return self._file_size

    # -- metadata ----------------------------------------------------------------
    def meta(self, key: str) -> Optional[GgufMeta]:
        lib = _lib.load()
        info = MiGgufMetaInfo()
        if lib.mi_gguf_meta(self._h, key.encode(), ctypes.byref(info)) != _lib.MI_OK:
            return None
        s = ctypes.string_at(info.str, info.str_len).decode("utf-8", "replace") if info.str else ""
        items: tuple = ()
        if info.type == GGUF_ARRAY and info.arr_len:
            n = info.arr_len
            if info.arr_type == GGUF_STRING:
                strs = (ctypes.c_char_p * n)()
                call("mi_gguf_meta_array", self._h, key.encode(), 0, n, None, None, strs)
                items = tuple(x.decode("utf-8", "replace") for x in strs)
            elif info.arr_type in (GGUF_FLOAT32, GGUF_FLOAT64):
                f = np.zeros(n, dtype=np.float64)
                call("mi_gguf_meta_array", self._h, key.encode(), 0, n, None, f.ctypes.data, None)
                items = tuple(float(x) for x in f)
            else:
                u = np.zeros(n, dtype=np.uint64)
                call("mi_gguf_meta_array", self._h, key.encode(), 0, n, u.ctypes.data, None, None)
                items = tuple(bool(x) for x in u) if info.arr_type == GGUF_BOOL else tuple(int(x) for x in u)
        return GgufMeta(info.type, int(info.u), float(info.f), bool(info.b), s, info.arr_type, items)

    def has(self, key: str) -> bool:
        return self.meta(key) is not None

    def getU64(self, key: str, default: int = 0) -> int:
        m = self.meta(key)
        return m.u if m is not None and m.isNum() else default

    def getI64(self, key: str, default: int = 0) -> int:
        m = self.meta(key)
        if m is None or not m.isNum():
            return default
        return m.u - (1 << 64) if m.u >= (1 << 63) else m.u

    def getF64(self, key: str, default: float = 0.0) -> float:
        m = self.meta(key)
        if m is None or not m.isNum():
            return default
        return m.f if m.type in (GGUF_FLOAT32, GGUF_FLOAT64) else float(m.u)

    def getF32(self, key: str, default: float = 0.0) -> float:
        return float(np.float32(self.getF64(key, default)))

    def getStr(self, key: str, default: str = "") -> str:
        m = self.meta(key)
        return m.s if m is not None and m.isStr() else default

    def archU64(self, arch: str, key: str, default: int = 0) -> int:
        return self.getU64(arch + "." + key, default)

    def archF32(self, arch: str, key: str, default: float = 0.0) -> float:
        return self.getF32(arch + "." + key, default)

    # -- data --------------------------------------------------------------------
    def readRaw(self, t: GgufTensor) -> Optional[np.ndarray]:
        out = np.empty(t.nbytes, dtype=np.uint8)
        st = _lib.load().mi_gguf_read_raw(self._h, t.index, out.ctypes.data, t.nbytes)
        return out if st == _lib.MI_OK else None

    def readFloat(self, name: str, err: Optional[list] = None) -> np.ndarray:
        """Gguf.cpp:489-527: fp32 decode of F32 / F16 / BF16 / Q4_0 / Q8_0 (empty on error)."""
        t = self.find(name)
        if t is None:
            if err is not None:
                err.append("tensor not found: " + name)
            return np.empty(0, dtype=np.float32)
        out = np.empty(t.nElems(), dtype=np.float32)
        lib = _lib.load()
        if lib.mi_gguf_read_f32(self._h, t.index, out.ctypes.data, out.size) != _lib.MI_OK:
            if err is not None:
                err.append(lib.mi_last_error().decode())
            return np.empty(0, dtype=np.float32)
        return out

    def readQ8(self, name: str, err: Optional[list] = None):
        """Gguf.cpp:530-583 (readQ8 / readQ8Into): (ok, int8 payload, fp32 scales)."""
        t = self.find(name)
        if t is None:
            if err is not None:
                err.append("tensor not found: " + name)
            return False, None, None
        q = np.empty(t.nElems(), dtype=np.int8)
        s = np.empty(t.nElems() // 32, dtype=np.float32)
        lib = _lib.load()
        if lib.mi_gguf_read_q8_split(self._h, t.index, q.ctypes.data, s.ctypes.data) != _lib.MI_OK:
            if err is not None:
                err.append(lib.mi_last_error().decode())
            return False, None, None
        return True, q, s

    # -- device uploads (stream-ordered, caller-owned buffers) ----------------------
    def upload_raw(self, t: GgufTensor, dst, stream=None) -> None:
        """Stored bytes -> device (a Q8_0 weight as the 34-byte blocks of mi_gemm_nt_q8_0)."""
        call("mi_gguf_upload_raw", self._h, t.index, ptr(dst), t.nbytes, _stream(stream))

    def upload_f32(self, t: GgufTensor, dst, stream=None) -> None:
        """readFloat decode -> device fp32 (biases, norms, non-Q8 weights)."""
        call("mi_gguf_upload_f32", self._h, t.index, ptr(dst), t.nElems(), _stream(stream))

    def upload_q8_split(self, t: GgufTensor, payload, scales, stream=None) -> None:
        """Q8_0 -> the reference's device layout (int8 payload, fp32 scale per block)."""
        call("mi_gguf_upload_q8_split", self._h, t.index, ptr(payload), ptr(scales), _stream(stream))


def _stream(stream) -> Optional[int]:
    if stream is None:
        return None
    return stream.handle.value if hasattr(stream, "handle") else int(stream)
