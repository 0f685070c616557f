"""GPU parity for the Q8_0 decode entry points (bit-exact against the oracle and
against the fixture written by the reference's own GGUF reader)."""
from pathlib import Path

import numpy as np
import pytest

from sdvk_amd import MI_F16, MI_F32, ops
from sdvk_amd.hip import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"


def _bits_equal(got, want):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _dequant(blocks, n, dtype):
    db = DeviceBuffer.from_array(blocks)
    out = DeviceBuffer(n * (4 if dtype == MI_F32 else 2))
    ops.q8_0_dequant(db, out, n, out_dtype=dtype)
    synchronize()
    return out.download(np.float32 if dtype == MI_F32 else np.float16, n)


def test_dequant_reference_fixture_bit_exact(gpu):
    f = np.load(GOLDEN / "q8_0_reference.npz")
    n = int(f["rows"]) * int(f["cols"])
    _bits_equal(_dequant(f["blocks"], n, MI_F32), f["dequant"])


@pytest.mark.parametrize("n", [32, 32 * 7, 1280 * 640, 10240 * 1280])
def test_dequant_f32_bit_exact_and_f16_rne(gpu, oracle, n):
    print(f"[case] dequant n={n}", flush=True)
    blocks = oracle.q8_0_quantize(oracle.normal(n, n, 0.0, 0.02))
    want = oracle.q8_0_dequant(blocks, n)
    _bits_equal(_dequant(blocks, n, MI_F32), want)
    got16 = _dequant(blocks, n, MI_F16)
    assert np.array_equal(got16.view(np.uint16), want.astype(np.float16).view(np.uint16))


def test_split_dequant_and_repack_bit_exact(gpu, oracle):
    f = np.load(GOLDEN / "q8_0_reference.npz")
    blocks = f["blocks"]
    n = int(f["rows"]) * int(f["cols"])
    db = DeviceBuffer.from_array(blocks)
    payload = DeviceBuffer(n)
    scales = DeviceBuffer(n // 32 * 4)
    ops.q8_0_to_split(db, payload, scales, n)
    synchronize()
    assert np.array_equal(payload.download(np.int8, n), f["payload"])
    assert np.array_equal(scales.download(np.uint32, n // 32), f["scales"].view(np.uint32))
    out = DeviceBuffer(n * 4)
    ops.q8_split_dequant(payload, scales, out, n)
    synchronize()
    _bits_equal(out.download(np.float32, n), f["dequant"])


def test_split_dequant_arbitrary_fp32_scales(gpu, oracle):
    n = 4 * 1000
    payload = oracle.uniform_int(3, -128, 127, n).astype(np.int8)
    scales = oracle.normal(4, (n + 31) // 32, 0.01, 0.003)
    want = oracle.q8_split_dequant(payload, scales, n)
    out = DeviceBuffer(n * 4)
    ops.q8_split_dequant(DeviceBuffer.from_array(payload), DeviceBuffer.from_array(scales), out, n)
    synchronize()
    _bits_equal(out.download(np.float32, n), want)


def test_quantize_bit_exact(gpu, oracle):
    """mi_q8_0_quantize vs the oracle's restatement of sdvkgen.cpp:533-544:
    N(0, 0.02^2) weights plus edge blocks (all zero, exact halves, one
    non-zero, huge / tiny magnitudes)."""
    w = oracle.normal(41, 32 * 4096, 0.0, 0.02)
    edge = np.zeros(32 * 6, np.float32)
    edge[32:64] = np.arange(32, dtype=np.float32) - 15.5          # .5 steps relative to amax
    edge[64] = 1e-3                                                # one non-zero
    edge[96:128] = np.linspace(-6e4, 6e4, 32, dtype=np.float32)    # near the fp16 top
    edge[128:160] = np.linspace(-1e-6, 1e-6, 32, dtype=np.float32) # fp16 subnormal scale
    edge[160:192] = 127.0 * np.sign(np.arange(32) - 15.5).astype(np.float32)
    for x in (w, edge):
        n = x.size
        dw, db = DeviceBuffer.from_array(x), DeviceBuffer(n // 32 * 34)
        ops.q8_0_quantize(dw, db, n)
        synchronize()
        assert np.array_equal(db.download(np.uint8, n // 32 * 34), oracle.q8_0_quantize(x))
