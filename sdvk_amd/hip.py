"""Minimal HIP runtime plumbing over ctypes: device buffers, streams, events.

The kernels live in libmi_sdvk.so; this module only moves bytes and times
launches. It binds the same libamdhip64 that libmi_sdvk.so links against
(ROCm's, via the library's rpath), so both share one HIP runtime instance.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

_hip = None


class HipError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        cands = [ROCM / "lib" / "libamdhip64.so.7", ROCM / "lib" / "libamdhip64.so"]
        path = next((p for p in cands if p.exists()), None)
        if path is None:
            raise HipError(f"libamdhip64 not found under {ROCM / 'lib'}")
        h = ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        h.hipFree.argtypes = [vp]
        h.hipMemcpy.argtypes = [vp, vp, sz, ctypes.c_int]
        h.hipMemcpyAsync.argtypes = [vp, vp, sz, ctypes.c_int, vp]
        h.hipMemsetAsync.argtypes = [vp, ctypes.c_int, sz, vp]
        h.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
        h.hipStreamDestroy.argtypes = [vp]
        h.hipStreamSynchronize.argtypes = [vp]
        h.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(vp), ctypes.c_uint]
        h.hipEventDestroy.argtypes = [vp]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventSynchronize.argtypes = [vp]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        h.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        h.hipDeviceGetAttribute.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        h.hipDeviceGetName.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int]
        h.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        h.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, sz]
        h.hipGraphLaunch.argtypes = [vp, vp]
        h.hipGraphExecDestroy.argtypes = [vp]
        h.hipGraphDestroy.argtypes = [vp]
        _hip = h
    return _hip


def check(err: int, what: str = "") -> None:
    if err != 0:
        msg = lib().hipGetErrorString(err).decode()
        raise HipError(f"{what}: HIP error {err}: {msg}")


H2D, D2H, D2D = 1, 2, 3


def device_count() -> int:
    n = ctypes.c_int(0)
    err = lib().hipGetDeviceCount(ctypes.byref(n))
    return n.value if err == 0 else 0


def device_name(dev: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    check(lib().hipDeviceGetName(buf, 256, dev), "hipDeviceGetName")
    return buf.value.decode()


def synchronize() -> None:
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceBuffer:
    """An owning device allocation of `nbytes` bytes."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        check(lib().hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 1)), f"hipMalloc({nbytes})")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    @property
    def value(self) -> int:
        return self.ptr.value or 0

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes, "upload past the end of the buffer"
        check(lib().hipMemcpy(ctypes.c_void_p(self.value + offset), a.ctypes.data_as(ctypes.c_void_p),
                              a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes, "download past the end of the buffer"
        check(lib().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.value + offset),
                              out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def copy_from(self, src: "DeviceBuffer", nbytes: int, stream: "Stream | None" = None) -> None:
        """Device-to-device copy of the first `nbytes` of `src` (asynchronous on `stream`)."""
        assert nbytes <= self.nbytes and nbytes <= src.nbytes, "copy past the end of a buffer"
        s = stream.handle if stream else None
        check(lib().hipMemcpyAsync(ctypes.c_void_p(self.value), ctypes.c_void_p(src.value), nbytes, D2D, s),
              "hipMemcpyAsync D2D")

    def fill_zero(self, stream: "Stream | None" = None) -> None:
        s = stream.handle if stream else None
        check(lib().hipMemsetAsync(ctypes.c_void_p(self.value), 0, self.nbytes, s), "hipMemsetAsync")

    def free(self) -> None:
        if self.ptr.value:
            lib().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(lib().hipStreamCreate(ctypes.byref(self.handle)), "hipStreamCreate")

    def synchronize(self) -> None:
        check(lib().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.handle.value:
                lib().hipStreamDestroy(self.handle)
        except Exception:
            pass


# hipEventReleaseToDevice: the event's completion releases at device scope
# only (no system-scope fence, which writes the L2 back to memory), the flag
# HIP documents for timing the commands between events.
EVENT_RELEASE_TO_DEVICE = 0x40000000


class Event:
    def __init__(self, flags: int = 0):
        self.handle = ctypes.c_void_p()
        if flags:
            check(lib().hipEventCreateWithFlags(ctypes.byref(self.handle), flags), "hipEventCreateWithFlags")
        else:
            check(lib().hipEventCreate(ctypes.byref(self.handle)), "hipEventCreate")

    def record(self, stream: Stream | None = None) -> None:
        check(lib().hipEventRecord(self.handle, stream.handle if stream else None), "hipEventRecord")

    def synchronize(self) -> None:
        check(lib().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle.value:
                lib().hipEventDestroy(self.handle)
        except Exception:
            pass


class Graph:
    """A stream capture turned into an executable graph (hipStreamBeginCapture /
    hipStreamEndCapture / hipGraphInstantiate): the launches issued on `stream`
    between begin() and end() are recorded, not run, and launch() replays them.
    Only kernel launches belong in a graph here (no hipMemsetAsync nodes)."""

    CAPTURE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal

    def __init__(self, stream: Stream):
        self.stream = stream
        self.graph = ctypes.c_void_p()
        self.exec = ctypes.c_void_p()

    def begin(self) -> None:
        check(lib().hipStreamBeginCapture(self.stream.handle, self.CAPTURE_THREAD_LOCAL), "hipStreamBeginCapture")

    def end(self) -> None:
        check(lib().hipStreamEndCapture(self.stream.handle, ctypes.byref(self.graph)), "hipStreamEndCapture")
        check(lib().hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0), "hipGraphInstantiate")

    def launch(self) -> None:
        check(lib().hipGraphLaunch(self.exec, self.stream.handle), "hipGraphLaunch")

    def __del__(self):
        try:
            if self.exec.value:
                lib().hipGraphExecDestroy(self.exec)
            if self.graph.value:
                lib().hipGraphDestroy(self.graph)
        except Exception:
            pass
