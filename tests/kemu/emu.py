"""Python side of the kernel emulator: loads the emulation build of the
library (tests/kemu/kemu_build.py) and hands out guarded host buffers that stand
in for device memory. Test infrastructure only."""
from __future__ import annotations

import ctypes
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for _p in (ROOT, HERE):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import kemu_build as _build  # noqa: E402
from sdvk_amd._lib import SIGNATURES  # noqa: E402  (the C-ABI signatures)


class Buf:
    """A guarded allocation: the byte after its 16-byte-rounded end (or the
    byte before its start, `front=True`) is on a PROT_NONE page."""

    def __init__(self, emu: "Emu", nbytes: int, front: bool = False):
        self.emu, self.nbytes = emu, int(nbytes)
        self.ptr = emu.lib.kemu_alloc(max(self.nbytes, 1), 1 if front else 0)
        if not self.ptr:
            raise MemoryError("kemu_alloc failed")

    def view(self, dtype, count: int | None = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else int(count)
        raw = (ctypes.c_uint8 * (n * dt.itemsize)).from_address(self.ptr)
        return np.frombuffer(raw, dtype=dt, count=n)

    def get(self, dtype, count: int | None = None) -> np.ndarray:
        return self.view(dtype, count).copy()

    def fill(self, byte: int) -> "Buf":
        ctypes.memset(self.ptr, byte, self.nbytes)
        return self


class Emu:
    def __init__(self):
        self.lib = ctypes.CDLL(str(_build.build()))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(self.lib, name, None)
            if f is not None:
                f.restype, f.argtypes = res, args
        self.lib.kemu_alloc.restype, self.lib.kemu_alloc.argtypes = ctypes.c_void_p, [ctypes.c_size_t, ctypes.c_int]
        self.lib.kemu_set_order.argtypes = [ctypes.c_int, ctypes.c_int]
        self.lib.kemu_launches.restype = ctypes.c_uint64
        self.lib.kemu_blocks_run.restype = ctypes.c_uint64
        self.lib.kemu_set_sample.argtypes = [ctypes.c_char_p]
        self.lib.kemu_last_grid.argtypes = [ctypes.POINTER(ctypes.c_uint32)]
        self.lib.kemu_last_kernel.restype = ctypes.c_char_p
        self.lib.kemu_sync.restype = None

    def buf(self, arr=None, *, nbytes: int | None = None, front: bool = False) -> Buf:
        if arr is not None:
            a = np.ascontiguousarray(arr)
            b = Buf(self, a.nbytes, front)
            ctypes.memmove(b.ptr, a.ctypes.data, a.nbytes)
            return b
        return Buf(self, nbytes, front)

    def call(self, name: str, *args) -> None:
        st = getattr(self.lib, name)(*args)
        if st != 0:
            raise RuntimeError(f"{name}: status {st}: {self.lib.mi_last_error().decode()}")

    def status(self, name: str, *args) -> int:
        return getattr(self.lib, name)(*args)

    def sample(self, spec: str = "") -> None:
        """Emulate only some workgroups: rules "kernel|x|y|z" joined by ';', each
        dimension '*' (all), '-' (none) or indices (negative: from the end);
        kernels that no rule names run in full. "" runs everything."""
        self.lib.kemu_set_sample(spec.encode())

    def last_launch(self) -> tuple[str, tuple[int, int, int]]:
        """(kernel text, grid) of the most recent launch."""
        g = (ctypes.c_uint32 * 4)()
        self.lib.kemu_last_grid(g)
        return self.lib.kemu_last_kernel().decode(), (g[0], g[1], g[2])

    def last_block_threads(self) -> int:
        g = (ctypes.c_uint32 * 4)()
        self.lib.kemu_last_grid(g)
        return g[3]

    def order(self, order: int, reverse_blocks: bool = False) -> None:
        """order bits: 1 lanes reversed, 2 waves reversed, 4 wave-major."""
        self.lib.kemu_set_order(int(order), int(reverse_blocks))
