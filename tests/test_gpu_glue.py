"""GPU parity of the block glue kernels (LayerNorm, GEGLU, residual add)
against the CPU oracle (layernorm_fwd.comp:15-38, unary_fwd.comp:28-36,
sdvkgen.cpp:1709-1720 / add2).

Bars: LayerNorm and GEGLU are fp32 on both sides, differing only in
summation order and in the expf implementation: max |err| <= 4e-6 (LayerNorm,
outputs O(1..5)) and <= 2e-6 x (1 + |y|) (GEGLU). The add is exact.
"""
import numpy as np
import pytest

from sdvk_amd import ops
from sdvk_amd._lib import MiError
from sdvk_amd.hip import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,d,affine", [(2048, 1280, True), (7, 320, True), (5, 1001, True), (3, 4100, False),
                                           (1, 4, False), (9, 4096, True)])
def test_layernorm(gpu, oracle, rows, d, affine):
    x = oracle.normal(11, rows * d, 0.5, 3.0)
    g = oracle.normal(12, d, 1.0, 0.2) if affine else None
    b = oracle.normal(13, d, 0.0, 0.2) if affine else None
    want = oracle.layernorm(x, g, b, rows, d)
    dx = DeviceBuffer.from_array(x)
    dy = DeviceBuffer(x.nbytes)
    dg = DeviceBuffer.from_array(g) if affine else None
    db = DeviceBuffer.from_array(b) if affine else None
    ops.layernorm(dx, dg, db, dy, rows, d)
    synchronize()
    got = dy.download(np.float32, rows * d)
    assert np.max(np.abs(got - want)) <= 4e-6
    # in place
    ops.layernorm(dx, dg, db, dx, rows, d)
    synchronize()
    assert np.max(np.abs(dx.download(np.float32, rows * d) - want)) <= 4e-6


@pytest.mark.parametrize("rows,F", [(2048, 5120), (3, 37), (5, 8)])
def test_geglu(gpu, oracle, rows, F):
    h = oracle.normal(21, rows * 2 * F, 0.0, 2.0)
    want = oracle.geglu(h, rows, F)
    dh, dy = DeviceBuffer.from_array(h), DeviceBuffer(rows * F * 4)
    ops.geglu(dh, dy, rows, F)
    synchronize()
    got = dy.download(np.float32, rows * F)
    assert np.all(np.abs(got - want) <= 2e-6 * (1 + np.abs(want)))


@pytest.mark.parametrize("n", [2048 * 1280, 1001, 4])
def test_add(gpu, oracle, n):
    a, b = oracle.normal(31, n), oracle.normal(32, n)
    dx, da = DeviceBuffer.from_array(a), DeviceBuffer.from_array(b)
    ops.add2(dx, da, n)
    synchronize()
    assert np.array_equal(dx.download(np.float32, n), oracle.add(a, b))


def test_errors(gpu):
    x = DeviceBuffer(4096)
    with pytest.raises(MiError):
        ops.layernorm(x, x, None, x, 4, 64)          # gamma without beta
    with pytest.raises(MiError):
        ops.geglu(x, x.value + 16, 4, 16)             # y overlaps h
    with pytest.raises(MiError):
        ops.add2(x, x.value + 4, 100)                 # partial overlap
    with pytest.raises(MiError):
        ops.layernorm(None, None, None, x, 4, 64)
