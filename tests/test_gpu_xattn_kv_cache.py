"""Cross-attention K / V caching of the SDXL transformer block
(mi_block_ctx_kv once per job, mi_sdxl_block_forward_kv per call): the
context's to_k / to_v projections that crossAttention recomputes on every call
(sdvkgen.cpp:1283-1290) are made once and reused.
"""
import numpy as np
import pytest

from helpers import record, rms
from sdvk_amd import ops
from sdvk_amd.hip import DeviceBuffer, synchronize
from test_gpu_block import BLOCK_TOL, make_weights, run_block, to_device

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,T,C,H,Tc,Cc,F,masked", [(2, 100, 320, 5, 77, 2048, 1280, True),
                                                    (1, 33, 64, 1, 5, 96, 160, False)])
@pytest.mark.parametrize("flags", [0, ops.MI_BLOCK_FP16_ATTENTION | ops.MI_BLOCK_FP16_ACTIVATIONS |
                                   ops.MI_BLOCK_FUSED_EPILOGUES])
def test_block_cached_ctx_kv(gpu, oracle, B, T, C, H, Tc, Cc, F, masked, flags):
    """K / V of the context projected once (mi_block_ctx_kv) and reused by two
    block applications (mi_sdxl_block_forward_kv): within the block bar of the
    oracle's two blocks, and bit-identical to two uncached calls (both project
    with the same unsplit GEMMs and every sum has a fixed order)."""
    print(f"[case] block cached kv B={B} T={T} C={C} Tc={Tc} Cc={Cc} flags={flags}", flush=True)
    w = make_weights(oracle, C, Cc, F, seed=500)
    x = oracle.normal(3, B * T * C)
    ctx = oracle.normal(4, B * Tc * Cc).astype(np.float16).astype(np.float32)
    kl = oracle.uniform_int(8, 1, Tc, B) if masked else None
    dims = ops.BlockDims(B, T, C, H, Tc, Cc, F, flags)
    dev, bw = to_device(w)
    dx, dc = DeviceBuffer.from_array(x), DeviceBuffer.from_array(ctx)
    dl = DeviceBuffer.from_array(np.asarray(kl, np.int32)) if kl is not None else None
    kv = DeviceBuffer(ops.block_ctx_kv_bytes(dims))
    ws = DeviceBuffer(ops.block_workspace_bytes(dims))
    ops.block_ctx_kv(bw, dims, dc, kv)
    for _ in range(2):
        ops.sdxl_block_forward_kv(bw, dims, dx, kv, ws, ctx_len=dl)
    synchronize()
    got = dx.download(np.float32, x.size)
    once = oracle.sdxl_block(w, x, ctx, batch=B, tokens=T, channels=C, heads=H, ctx_tokens=Tc, ctx_channels=Cc,
                             ff_inner=F, ctx_len=kl, threads=oracle.max_threads())
    want = oracle.sdxl_block(w, once, ctx, batch=B, tokens=T, channels=C, heads=H, ctx_tokens=Tc, ctx_channels=Cc,
                             ff_inner=F, ctx_len=kl, threads=oracle.max_threads())
    e2 = np.max(np.abs(got - want)) / rms(want - x)
    print(f"  two blocks vs oracle err/rms = {e2:.3e}", flush=True)
    record(e2, 2 * BLOCK_TOL)
    assert np.all(np.isfinite(got)) and e2 <= 2 * BLOCK_TOL
    fresh = run_block(w, dims, x, ctx, kl, blocks=2)
    diff = float(np.max(np.abs(got - fresh)))
    print(f"  cached vs fresh: max |diff| = {diff:.3e}", flush=True)
    assert np.array_equal(got, fresh)


def test_kv_buffer_checks(gpu, oracle):
    C, Cc, F = 64, 96, 160
    w = make_weights(oracle, C, Cc, F)
    dims = ops.BlockDims(1, 8, C, 1, 5, Cc, F)
    dev, bw = to_device(w)
    x, ctx = DeviceBuffer(8 * C * 4), DeviceBuffer(5 * Cc * 4)
    ws = DeviceBuffer(ops.block_workspace_bytes(dims))
    with pytest.raises(ops.MiError):  # K / V buffer shorter than mi_block_ctx_kv_bytes
        ops.block_ctx_kv(bw, dims, ctx, DeviceBuffer(ops.block_ctx_kv_bytes(dims) - 256))
    with pytest.raises(ops.MiError):
        ops.sdxl_block_forward_kv(bw, dims, x, DeviceBuffer(ops.block_ctx_kv_bytes(dims) - 256), ws)
