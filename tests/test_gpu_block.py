"""GPU parity of one SDXL transformer block (config 4 semantics,
sdvkgen.cpp:1739-1763) against the oracle's composition of the same block.

The block chains three fp16-MFMA stages (projection GEMM -> attention ->
output GEMM, and FF up -> GEGLU -> FF down), each within 2e-3 x RMS of its
fp32 result. The check is on the block's update (x_out - x_in), whose RMS is
what those errors are relative to: max |err| <= 5e-3 x RMS(update).
"""
import numpy as np
import pytest

from helpers import record, rms
from sdvk_amd import ops
from sdvk_amd.hip import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu
BLOCK_TOL = 5e-3


def make_weights(oracle, C, Cc, F, seed=300, std=0.02):
    """Config 4: linear weights Q8_0 from N(0, std^2), biases N(0, std^2), LayerNorm gamma = 1, beta = 0."""
    w, s = {}, seed
    for nm in ("norm1", "norm2", "norm3"):
        w[nm + "_w"] = np.ones(C, np.float32)
        w[nm + "_b"] = np.zeros(C, np.float32)
    for nm, (n, k) in {"attn1_q": (C, C), "attn1_k": (C, C), "attn1_v": (C, C), "attn1_out": (C, C),
                       "attn2_q": (C, C), "attn2_k": (C, Cc), "attn2_v": (C, Cc), "attn2_out": (C, C),
                       "ff_up": (2 * F, C), "ff_down": (C, F)}.items():
        w[nm] = oracle.q8_0_quantize(oracle.normal(s, n * k, 0.0, std))
        s += 1
    for nm, n in {"attn1_out_b": C, "attn2_out_b": C, "ff_up_b": 2 * F, "ff_down_b": C}.items():
        w[nm] = oracle.normal(s, n, 0.0, std)
        s += 1
    return w


def to_device(w):
    dev = {k: DeviceBuffer.from_array(v) for k, v in w.items()}
    return dev, ops.BlockWeights(**dev)


def run_block(w, dims, x, ctx, ctx_len=None, blocks=1):
    dev, bw = to_device(w)
    dx, dc = DeviceBuffer.from_array(x), DeviceBuffer.from_array(ctx)
    dl = DeviceBuffer.from_array(np.asarray(ctx_len, np.int32)) if ctx_len is not None else None
    ws = DeviceBuffer(ops.block_workspace_bytes(dims))
    for _ in range(blocks):
        ops.sdxl_block_forward(bw, dims, dx, dc, ws, ctx_len=dl)
    synchronize()
    return dx.download(np.float32, x.size)


@pytest.mark.parametrize("B,T,C,H,Tc,Cc,F,masked", [(2, 64, 128, 2, 77, 256, 256, False),
                                                    (2, 100, 320, 5, 77, 2048, 1280, True),
                                                    (1, 33, 64, 1, 5, 96, 160, False)])
def test_block_small(gpu, oracle, B, T, C, H, Tc, Cc, F, masked):
    print(f"[case] block B={B} T={T} C={C} H={H} Tc={Tc} Cc={Cc} F={F} masked={masked}", flush=True)
    w = make_weights(oracle, C, Cc, F)
    x = oracle.normal(1, B * T * C)
    ctx = oracle.normal(2, B * Tc * Cc).astype(np.float16).astype(np.float32)
    kl = oracle.uniform_int(7, 1, Tc, B) if masked else None
    dims = ops.BlockDims(B, T, C, H, Tc, Cc, F)
    got = run_block(w, dims, x, ctx, kl)
    want = oracle.sdxl_block(w, x, ctx, batch=B, tokens=T, channels=C, heads=H, ctx_tokens=Tc, ctx_channels=Cc,
                             ff_inner=F, ctx_len=kl, threads=oracle.max_threads())
    upd = want - x
    e = np.max(np.abs(got - want)) / rms(upd)
    print(f"  update err/rms = {e:.3e}", flush=True)
    record(e, BLOCK_TOL)
    assert np.all(np.isfinite(got)) and e <= BLOCK_TOL


def test_block_config4_full(gpu, oracle):
    """BASELINE config 4 at full size (level 2: 1280 channels, 2 x 1024 tokens,
    20 heads, context 2 x 77 x 2048, FF 1280 -> 10240 -> 5120 -> 1280), one block."""
    B, T, C, H, Tc, Cc, F = 2, 1024, 1280, 20, 77, 2048, 5120
    print("[case] block config 4 full size", flush=True)
    w = make_weights(oracle, C, Cc, F, seed=400)
    x = oracle.normal(1, B * T * C)
    ctx = oracle.normal(6, B * Tc * Cc).astype(np.float16).astype(np.float32)
    dims = ops.BlockDims(B, T, C, H, Tc, Cc, F)
    got = run_block(w, dims, x, ctx)
    want = oracle.sdxl_block(w, x, ctx, batch=B, tokens=T, channels=C, heads=H, ctx_tokens=Tc, ctx_channels=Cc,
                             ff_inner=F, threads=oracle.max_threads())
    e = np.max(np.abs(got - want)) / rms(want - x)
    print(f"  update err/rms = {e:.3e}", flush=True)
    record(e, BLOCK_TOL)
    assert np.all(np.isfinite(got)) and e <= BLOCK_TOL


def test_workspace_checks(gpu, oracle):
    C, Cc, F = 64, 96, 160
    w = make_weights(oracle, C, Cc, F)
    dims = ops.BlockDims(1, 8, C, 1, 5, Cc, F)
    dev, bw = to_device(w)
    x, ctx = DeviceBuffer(8 * C * 4), DeviceBuffer(5 * Cc * 4)
    small = DeviceBuffer(1024)
    with pytest.raises(ops.MiError):
        ops.sdxl_block_forward(bw, dims, x, ctx, small)
    with pytest.raises(ops.MiError):
        ops.sdxl_block_forward(bw, ops.BlockDims(1, 8, 100, 3, 5, Cc, F), x, ctx,
                               DeviceBuffer(ops.block_workspace_bytes(dims)))

