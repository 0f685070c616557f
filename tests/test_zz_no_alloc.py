"""mi_gemm_nt_q8_0_noalloc (the GEMM entry that allocates nothing: its K-split
partials live in the library's per-GPU scratch array) against the workspace
entry mi_gemm_nt_q8_0_ws through the C-ABI: bit-identical on two calls in a
row, the second smaller (the scratch keeps the first call's contents), for
K-split plans, an unsplit plan, mode 1 and mode 2. A plan needing more scratch
than the maximum is rejected before any launch."""
import ctypes

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
    ((2048, 1280, 5120, 2), (1000, 700, 4096, 1)),  # 128x128 tiles with 2 K splits, then 64x64 splits
    ((520, 384, 640, 0), (33, 96, 64, 2)),           # splits, then a single-step K
])
def test_noalloc_matches_workspace_entry(gpu, oracle, first, second):
    lib = _lib.load()
    sizes = []
    for i, (M, N, K, mode) in enumerate((first, second)):
        got, want, ref, nws = _run(lib, oracle, M, N, K, mode, 10 * i + 1)
        sizes.append(nws)
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


def test_noalloc_rejects_plans_beyond_the_scratch(gpu, oracle, monkeypatch):
    """A forced 8-way split of a large shape needs 8 M N floats (> 32 MiB):
    rejected with MI_ERR_UNSUPPORTED before anything is launched."""
    lib = _lib.load()
    M, N, K = 4096, 1280, 2048
    monkeypatch.setenv("MI_GEMM_CFG", "3:8")
    dA = DeviceBuffer(M * K * 4)
    dW = DeviceBuffer(N * (K // 32) * 34 + 16)
    dC = DeviceBuffer(M * N * 4)
    st = lib.mi_gemm_nt_q8_0_noalloc(dA.value, dW.value, None, dC.value, M, N, K, 0, 0, 0, 1, 0, 0, None)
    assert st == _lib.MI_ERR_UNSUPPORTED
    assert b"scratch" in lib.mi_last_error()
