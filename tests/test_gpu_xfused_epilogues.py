"""GPU checks of the fused block epilogues: GEMM mode 2 (C += A.W^T + bias,
the residual add of sdvkgen.cpp:1746,1751,1762 folded into the GEMM) and the
GEGLU GEMM (linear(ff_up) + geglu, sdvkgen.cpp:1709-1720, in one kernel); and
the block's joint Q/K/V projection (to_q / to_k / to_v stored back to back).

Bars: mode 2 to the GEMM bar on the update (C - C0); GEGLU against the
oracle within the GEMM bar propagated through v * gelu(g), and bit for bit
against the separate path (GEMM into [M, 2F] + mi_geglu: the same MFMA sums
and the same fp32 epilogue operations); the block with
MI_BLOCK_FUSED_EPILOGUES and / or MI_BLOCK_JOINT_QKV against the oracle's
block to the block bar and bit for bit against the plain block (every flag
combination computes the same sums in the same order).
"""
from __future__ import annotations

from math import erf

import numpy as np
import pytest

from helpers import assert_parity, q8_weights, record, rms
from sdvk_amd import ops
from sdvk_amd.hip import DeviceBuffer, synchronize
from test_gpu_block import BLOCK_TOL, make_weights, to_device

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K,cfg", [(77, 96, 64, None), (130, 257, 320, None), (2048, 1280, 1280, None),
                                       (300, 200, 256, "0:2"), (154, 1280, 5120, None)])
def test_residual_mode(gpu, oracle, tune, M, N, K, cfg):
    print(f"[case] gemm mode 2 M={M} N={N} K={K} cfg={cfg}", flush=True)
    if cfg:
        tune("gemm_cfg", cfg)
    A = oracle.normal(1, M * K)
    blocks = q8_weights(oracle, 2, N, K)
    bias = oracle.normal(3, N, 0.0, 0.02)
    C0 = oracle.normal(4, M * N)
    dC = DeviceBuffer.from_array(C0)
    nws = ops.gemm_workspace_bytes(M, N, K)
    ops.gemm_nt_q8_0(DeviceBuffer.from_array(A), DeviceBuffer.from_array(blocks), dC, M, N, K,
                     bias=DeviceBuffer.from_array(bias), mode=2, workspace=DeviceBuffer(nws) if nws else None)
    synchronize()
    got = dC.download(np.float32, M * N) - C0
    want = oracle.gemm_nt_q8_0(A, blocks, M, N, K, bias=bias, threads=oracle.max_threads())
    e = assert_parity(got, want, what="mode 2")
    print(f"  err/rms = {e:.3e}", flush=True)


@pytest.mark.parametrize("M,F,K,cfg", [(77, 48, 64, None), (300, 200, 256, "4"), (130, 100, 96, None),
                                       (2048, 5120, 1280, None), (300, 130, 256, "0"), (300, 130, 256, "5"),
                                       (300, 130, 256, "6")])
def test_geglu_gemm(gpu, oracle, tune, M, F, K, cfg):
    print(f"[case] gemm geglu M={M} F={F} K={K} cfg={cfg}", flush=True)
    if cfg:
        tune("gemm_cfg", cfg)
    A = oracle.normal(1, M * K)
    blocks = q8_weights(oracle, 2, 2 * F, K)
    bias = oracle.normal(3, 2 * F, 0.0, 0.5)
    dA, dW, dB = DeviceBuffer.from_array(A), DeviceBuffer.from_array(blocks), DeviceBuffer.from_array(bias)
    dG, dH, dY = DeviceBuffer(M * F * 4), DeviceBuffer(M * 2 * F * 4), DeviceBuffer(M * F * 4)
    ops.gemm_nt_q8_0_geglu(dA, dW, dG, M, F, K, bias=dB)
    ops.gemm_nt_q8_0(dA, dW, dH, M, 2 * F, K, bias=dB)
    ops.geglu(dH, dY, M, F)
    synchronize()
    got = dG.download(np.float32, M * F).reshape(M, F)
    sep = dY.download(np.float32, M * F).reshape(M, F)
    d_sep = float(np.max(np.abs(got - sep)) / rms(sep))
    print(f"  fused vs separate = {d_sep:.3e} x RMS", flush=True)
    if cfg:
        tune("gemm_cfg", None)
    h = oracle.gemm_nt_q8_0(A, blocks, M, 2 * F, K, bias=bias, threads=oracle.max_threads()).reshape(M, 2 * F)
    want = oracle.geglu(h, M, F).reshape(M, F)
    v, g = h[:, :F].astype(np.float64), h[:, F:].astype(np.float64)
    cdf = 0.5 * (1.0 + np.vectorize(erf)(g / np.sqrt(2.0)))
    dgelu = cdf + g * np.exp(-0.5 * g * g) / np.sqrt(2.0 * np.pi)
    bound = 2e-3 * rms(h) * (np.abs(g * cdf) + np.abs(v * dgelu)) + 1e-6 * np.abs(want)
    assert np.all(np.isfinite(got))
    worst = float(np.max(np.abs(got - want) / bound))
    print(f"  vs oracle: {worst:.2f} x the propagated GEMM bound", flush=True)
    assert worst <= 1.0
    assert np.array_equal(got, sep), "fused GEGLU differs from GEMM + mi_geglu"


@pytest.mark.parametrize("B,T,C,H,Tc,Cc,F,masked", [(2, 64, 128, 2, 77, 256, 256, True),
                                                    (2, 100, 320, 5, 77, 2048, 1280, True),
                                                    (2, 1024, 1280, 20, 77, 2048, 5120, False)])
@pytest.mark.parametrize("flags", [ops.MI_BLOCK_FUSED_EPILOGUES, ops.MI_BLOCK_JOINT_QKV,
                                   ops.MI_BLOCK_FUSED_EPILOGUES | ops.MI_BLOCK_JOINT_QKV,
                                   ops.MI_BLOCK_FP16_ACTIVATIONS,
                                   ops.MI_BLOCK_FP16_ACTIVATIONS | ops.MI_BLOCK_FUSED_EPILOGUES,
                                   ops.MI_BLOCK_FP16_ACTIVATIONS | ops.MI_BLOCK_FUSED_EPILOGUES |
                                   ops.MI_BLOCK_JOINT_QKV,
                                   ops.MI_BLOCK_FP16_ATTENTION | ops.MI_BLOCK_FP16_ACTIVATIONS |
                                   ops.MI_BLOCK_FUSED_EPILOGUES | ops.MI_BLOCK_JOINT_QKV,
                                   ops.MI_BLOCK_FP16_ATTENTION | ops.MI_BLOCK_JOINT_QKV])
def test_block_flags(gpu, oracle, B, T, C, H, Tc, Cc, F, masked, flags):
    """The block with fused epilogues, the joint Q/K/V projection and / or fp16
    activations: within the block bar of the oracle and bit-identical to the
    plain block (weights stored apart, separate epilogues, fp32 activations).
    With MI_BLOCK_FP16_ATTENTION (fp16 Q / K / V, a precision choice) the plain
    block of the comparison carries that flag alone."""
    print(f"[case] block flags={flags} B={B} T={T} C={C} F={F}", flush=True)
    base = flags & ops.MI_BLOCK_FP16_ATTENTION
    w = make_weights(oracle, C, Cc, F, seed=500)
    x = oracle.normal(3, B * T * C)
    ctx = oracle.normal(4, B * Tc * Cc).astype(np.float16).astype(np.float32)
    kl = oracle.uniform_int(8, 1, Tc, B) if masked else None
    dev, bw = to_device(w)
    if flags & ops.MI_BLOCK_JOINT_QKV:
        joint = DeviceBuffer.from_array(np.concatenate([w["attn1_q"], w["attn1_k"], w["attn1_v"]]))
        nb = w["attn1_q"].nbytes
        bw_f = ops.BlockWeights(**dict(dev, attn1_q=joint.value, attn1_k=joint.value + nb,
                                       attn1_v=joint.value + 2 * nb))
    else:
        bw_f = bw
    dc = DeviceBuffer.from_array(ctx)
    dl = DeviceBuffer.from_array(np.asarray(kl, np.int32)) if kl is not None else None
    outs = []
    for weights, dims in ((bw_f, ops.BlockDims(B, T, C, H, Tc, Cc, F, flags)),
                          (bw, ops.BlockDims(B, T, C, H, Tc, Cc, F, base))):
        ws = DeviceBuffer(ops.block_workspace_bytes(dims))
        dx = DeviceBuffer.from_array(x)
        ops.sdxl_block_forward(weights, dims, dx, dc, ws, ctx_len=dl)
        synchronize()
        outs.append(dx.download(np.float32, x.size))
    want = oracle.sdxl_block(w, x, ctx, batch=B, tokens=T, channels=C, heads=H, ctx_tokens=Tc, ctx_channels=Cc,
                             ff_inner=F, ctx_len=kl, threads=oracle.max_threads())
    e = float(np.max(np.abs(outs[0] - want)) / rms(want - x))
    print(f"  flags {flags} vs oracle err/rms(update) = {e:.3e}", flush=True)
    record(e, BLOCK_TOL)
    assert np.all(np.isfinite(outs[0])) and e <= BLOCK_TOL
    diff = float(np.max(np.abs(outs[0] - outs[1])))
    print(f"  flags {flags} vs plain: max |diff| = {diff:.3e}", flush=True)
    assert np.array_equal(outs[0], outs[1])


def test_joint_qkv_needs_adjacent_weights(gpu, oracle):
    """MI_BLOCK_JOINT_QKV with to_q / to_k / to_v not laid out as one [3C, C]
    matrix is an error, not a silent fallback."""
    C, Cc, F = 64, 96, 160
    w = make_weights(oracle, C, Cc, F)
    dev, bw = to_device(w)
    dims = ops.BlockDims(1, 8, C, 1, 5, Cc, F, ops.MI_BLOCK_JOINT_QKV)
    x, ctx = DeviceBuffer(8 * C * 4), DeviceBuffer(5 * Cc * 4)
    with pytest.raises(ops.MiError):
        ops.sdxl_block_forward(bw, dims, x, ctx, DeviceBuffer(ops.block_workspace_bytes(dims)))
