"""The config-4 block stack exactly as the bench times it (bench.BlockStack:
ten blocks, each with its own weights, every block flag, context K / V cached
per block): each block against the oracle's block applied to that block's own
input (the per-block bar, derived in test_block_bar.py), and the stack's final
output against the chained oracle (ten oracle blocks from the same input)."""
from __future__ import annotations

import numpy as np
import pytest

import bench
from helpers import record, rms
from sdvk_amd import hip, ops
from test_gpu_block import BLOCK_TOL

pytestmark = pytest.mark.gpu


def _host_weights(st, i):
    """Block i's weights as the oracle takes them (Q8_0 bytes, fp32 vectors), read back from the device."""
    d = st.keep[1 + i]
    B, T, C, H, Tc, Cc, F = st.DIMS
    shapes = {"attn1_q": (C, C), "attn1_k": (C, C), "attn1_v": (C, C), "attn1_out": (C, C), "attn2_q": (C, C),
              "attn2_k": (C, Cc), "attn2_v": (C, Cc), "attn2_out": (C, C), "ff_up": (2 * F, C), "ff_down": (C, F)}
    w = {}
    joint = d["_qkv"].download(np.uint8, d["_qkv"].nbytes) if "_qkv" in d else None
    for nm, (n, k) in shapes.items():
        nb = n * k // 32 * 34
        v = d[nm]
        if isinstance(v, int):  # the joint Q / K / V matrix: an address inside d["_qkv"]
            off = v - d["_qkv"].value
            w[nm] = joint[off:off + nb].copy()
        else:
            w[nm] = v.download(np.uint8, nb)
    for nm, n in {"attn1_out_b": C, "attn2_out_b": C, "ff_up_b": 2 * F, "ff_down_b": C}.items():
        w[nm] = d[nm].download(np.float32, n)
    for nm in ("norm1", "norm2", "norm3"):
        w[nm + "_w"] = d[nm + "_w"].download(np.float32, C)
        w[nm + "_b"] = d[nm + "_b"].download(np.float32, C)
    return w


@pytest.mark.parametrize("hattn", [True, False], ids=["fp16_attention", "fp32_attention_inputs"])
def test_block_stack_against_chained_oracle(gpu, oracle, hattn):
    print(f"[case] config-4 stack, 10 blocks, all flags, fp16_attention={hattn}", flush=True)
    st = bench.BlockStack(np.random.default_rng(1), hip, ops, nblocks=10, joint_qkv=True, fused=True, half=True,
                          hattn=hattn)
    B, T, C, H, Tc, Cc, F = st.DIMS
    stream = hip.Stream()
    kv = []
    for w in st.weights:
        buf = hip.DeviceBuffer(ops.block_ctx_kv_bytes(st.dims))
        ops.block_ctx_kv(w, st.dims, st.ctx, buf, stream=stream)
        kv.append(buf)
    stream.synchronize()
    xs = [st.x.download(np.float32, B * T * C)]
    ctx = st.ctx.download(np.float32, B * Tc * Cc)
    for w, buf in zip(st.weights, kv):
        ops.sdxl_block_forward_kv(w, st.dims, st.x, buf, st.ws, stream=stream)
        stream.synchronize()
        xs.append(st.x.download(np.float32, B * T * C))
    kw = dict(batch=B, tokens=T, channels=C, heads=H, ctx_tokens=Tc, ctx_channels=Cc, ff_inner=F,
              threads=oracle.max_threads())
    worst, chained = 0.0, xs[0]
    for i in range(st.nblocks):
        wh = _host_weights(st, i)
        want = oracle.sdxl_block(wh, xs[i], ctx, **kw)
        e = float(np.max(np.abs(xs[i + 1] - want)) / rms(want - xs[i]))
        record(e, BLOCK_TOL)
        worst = max(worst, e)
        chained = oracle.sdxl_block(wh, chained, ctx, **kw)
        print(f"  block {i}: err/rms(update) = {e:.3e}", flush=True)
    e_total = float(np.max(np.abs(xs[-1] - chained)) / rms(chained - xs[0]))
    print(f"  stack vs chained oracle: err/rms(stack update) = {e_total:.3e}", flush=True)
    assert np.all(np.isfinite(xs[-1]))
    assert worst <= BLOCK_TOL, f"worst block {worst:.3e}"
    record(e_total, BLOCK_TOL)
    assert e_total <= BLOCK_TOL
