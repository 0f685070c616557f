"""mi_gemm_nt_q8_0_noalloc (the GEMM entry that allocates nothing: its K-split
partials live in the library's per-GPU scratch array) against the workspace
entry mi_gemm_nt_q8_0_ws through the C-ABI: bit-identical on two calls in a
row, the second smaller (the scratch keeps the first call's contents), for
K-split plans, an unsplit plan, mode 1 and mode 2. A plan needing more scratch
than the maximum is rejected before any launch. In a fresh process, the first
call captured into a HIP graph after mi_gemm_noalloc_init replays to the
workspace entry's bits, and without the init it is refused."""
import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_parity, q8_weights
from sdvk_amd import _lib
from sdvk_amd.hip import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu

SCRATCH_MAX = 32 << 20


def _call(lib, name, *args):
    st = getattr(lib, name)(*args)
    assert st == _lib.MI_OK, f"{name}: status {st}: {lib.mi_last_error().decode()}"


def _run(lib, oracle, M, N, K, mode, seed):
    """One shape through both entries; returns (noalloc C, workspace C, oracle C or None)."""
    print(f"[case] noalloc M={M} N={N} K={K} mode={mode} seed={seed}", flush=True)
    A = oracle.normal(seed, M * K)
    blocks = q8_weights(oracle, seed + 1, N, K)
    bias = oracle.normal(seed + 2, N, 0.0, 0.02)
    C0 = oracle.normal(seed + 3, M * N)
    dA, dW, dB = DeviceBuffer.from_array(A), DeviceBuffer.from_array(blocks), DeviceBuffer.from_array(bias)
    nws = lib.mi_gemm_nt_q8_workspace_bytes(M, N, K, 1)
    assert nws <= SCRATCH_MAX
    ws = DeviceBuffer(max(nws, 16))
    outs = []
    for entry in ("noalloc", "ws"):
        dC = DeviceBuffer.from_array(C0)
        if entry == "noalloc":
            _call(lib, "mi_gemm_nt_q8_0_noalloc", dA.value, dW.value, dB.value, dC.value, M, N, K, mode, 0, 0, 1, 0,
                  0, None)
        else:
            _call(lib, "mi_gemm_nt_q8_0_ws", dA.value, dW.value, dB.value, dC.value, M, N, K, mode, 0, 0, 1, 0, 0,
                  ws.value, nws, None)
        synchronize()
        outs.append(dC.download(np.float32, M * N))
    ref = oracle.gemm_nt_q8_0(A, blocks, M, N, K, bias=None if mode == 1 else bias)
    if mode:
        ref = ref + C0
    return outs[0], outs[1], ref, nws


@pytest.mark.parametrize("first,second", [
    ((154, 1280, 2048, 0), (100, 640, 1024, 0)),    # 64x64 tiles, 4 then 8 K splits
    ((2048, 1280, 5120, 2), (1000, 700, 4096, 1)),  # 256x128 tiles with 3 K splits, then 64x64 splits
    ((520, 384, 640, 0), (33, 96, 64, 2)),           # splits, then a single-step K
])
def test_noalloc_matches_workspace_entry(gpu, oracle, first, second):
    lib = _lib.load()
    sizes = []
    for i, (M, N, K, mode) in enumerate((first, second)):
        got, want, ref, nws = _run(lib, oracle, M, N, K, mode, 10 * i + 1)
        sizes.append(nws)
        if (M, N, K) == (2048, 1280, 5120):  # the planner's 3-way split of 80 tiles of 256 x 128
            assert nws == 3 * M * N * 4, f"2048x1280x5120 plans {nws} bytes of partials, not 3 planes"
        assert np.array_equal(got, want), f"call {i + 1}: noalloc differs from the workspace entry"
        assert_parity(got, ref, what=f"noalloc call {i + 1} vs oracle")
    assert sizes[0] > 0, "the first call was meant to use the scratch"


def test_noalloc_unsplit_shape_equals_plain_entry(gpu, oracle):
    lib = _lib.load()
    M, N, K = 8192, 640, 640
    got, want, ref, nws = _run(lib, oracle, M, N, K, 0, 7)
    assert nws == 0
    assert np.array_equal(got, want)
    assert_parity(got, ref, what="noalloc unsplit")


def test_noalloc_rejects_plans_beyond_the_scratch(gpu, oracle, tune):
    """A forced 8-way split of a large shape needs 8 M N floats (> 32 MiB):
    rejected with MI_ERR_UNSUPPORTED before anything is launched."""
    lib = _lib.load()
    M, N, K = 4096, 1280, 2048
    tune("gemm_cfg", "3:8")
    dA = DeviceBuffer(M * K * 4)
    dW = DeviceBuffer(N * (K // 32) * 34 + 16)
    dC = DeviceBuffer(M * N * 4)
    st = lib.mi_gemm_nt_q8_0_noalloc(dA.value, dW.value, None, dC.value, M, N, K, 0, 0, 0, 1, 0, 0, None)
    assert st == _lib.MI_ERR_UNSUPPORTED
    assert b"scratch" in lib.mi_last_error()


_CAPTURE_CHILD = r"""
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np
from oracle import binding as ob
from sdvk_amd import _lib, hip
from sdvk_amd.hip import DeviceBuffer, Graph, Stream
init = sys.argv[2] == "init"
lib = _lib.load()
M, N, K = 154, 1280, 2048  # 64 x 64 tiles with K splits: the call uses the scratch
A = ob.normal(1, M * K)
W = ob.q8_0_quantize(ob.normal(2, N * K, 0.0, 0.02))
dA, dW, dC, dR = DeviceBuffer.from_array(A), DeviceBuffer.from_array(W), DeviceBuffer(M * N * 4), DeviceBuffer(M * N * 4)
nws = lib.mi_gemm_nt_q8_workspace_bytes(M, N, K, 1)
assert nws > 0
ws = DeviceBuffer(nws)
st = lib.mi_gemm_nt_q8_0_ws(dA.value, dW.value, None, dR.value, M, N, K, 0, 0, 0, 1, 0, 0, ws.value, nws, None)
assert st == 0, lib.mi_last_error()
hip.synchronize()
if init:
    assert lib.mi_gemm_noalloc_init() == 0, lib.mi_last_error()
s = Stream()
g = Graph(s)
g.begin()
st = lib.mi_gemm_nt_q8_0_noalloc(dA.value, dW.value, None, dC.value, M, N, K, 0, 0, 0, 1, 0, 0, s.handle)
print(f"[child] first noalloc call inside the capture (init={init}): status {st}", flush=True)
if not init:
    assert st == _lib.MI_ERR_UNSUPPORTED, st
    assert b"mi_gemm_noalloc_init" in lib.mi_last_error()
    graph = __import__("ctypes").c_void_p()
    hip.check(hip.lib().hipStreamEndCapture(s.handle, __import__("ctypes").byref(graph)), "end capture")
    print("OK refused", flush=True)
    sys.exit(0)
assert st == 0, lib.mi_last_error()
g.end()
for rep in range(3):
    g.launch()
    s.synchronize()
    got, want = dC.download(np.float32, M * N), dR.download(np.float32, M * N)
    assert np.array_equal(got, want), f"replay {rep}: captured noalloc differs from the workspace entry"
print("OK replays", flush=True)
"""


@pytest.mark.parametrize("init", ["init", "noinit"])
def test_noalloc_first_call_inside_a_capture(gpu, init):
    """A fresh process whose first mi_gemm_nt_q8_0_noalloc call is made inside a
    stream capture: after mi_gemm_noalloc_init the graph replays (three times)
    to the workspace entry's bits; without it the call is refused with
    MI_ERR_UNSUPPORTED, and the capture ends cleanly."""
    root = str(Path(__file__).resolve().parents[1])
    print(f"[case] noalloc capture in a child process ({init})", flush=True)
    r = subprocess.run([sys.executable, "-u", "-c", _CAPTURE_CHILD, root, init], capture_output=True, text=True,
                       timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, f"child exited {r.returncode}"
    assert ("OK replays" if init == "init" else "OK refused") in r.stdout
