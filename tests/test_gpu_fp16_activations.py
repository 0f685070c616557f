"""GPU checks of the fp16-activation path (the config-4 block's
MI_BLOCK_FP16_ACTIVATIONS): every producer that stores fp16 gives exactly the
fp16 rounding (RNE) of its fp32 result, and the fp16-A GEMM gives exactly the
fp32 GEMM's result on the same fp16 values -- together the reason the block
computes the same bits either way.

  * mi_gemm_nt_q8_0_f16a vs mi_gemm_nt_q8_0_ws on A = fp16 values (every tile
    build, K splits, modes 0 / 1 / 2, batch / strides): bit for bit;
  * mi_gemm_nt_q8_0_geglu_f16 vs fp16(mi_gemm_nt_q8_0_geglu) on the same A;
  * mi_layernorm_f16 / mi_geglu_f16 vs fp16(mi_layernorm / mi_geglu);
  * fp16-output attention vs fp16(fp32-output attention), same precision mode.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_parity, q8_weights
from sdvk_amd import MI_ATTN_PREC_FP16, MI_F16, MI_F32, ops
from sdvk_amd.hip import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu


def _half_a(oracle, seed, n):
    """N(0, 1) activations that are fp16 numbers: the fp16 bits and the same values as fp32."""
    a16 = oracle.normal(seed, n).astype(np.float16)
    return a16, a16.astype(np.float32)


@pytest.mark.parametrize("M,N,K,mode,cfg", [(77, 96, 64, 0, None), (300, 260, 320, 1, None),
                                            (2048, 1280, 1280, 2, None), (154, 1280, 2048, 0, None),
                                            (2048, 1280, 5120, 2, None), (300, 200, 256, 0, "0"),
                                            (300, 200, 256, 0, "2"), (300, 300, 256, 1, "4"),
                                            (400, 300, 256, 0, "5"), (200, 300, 512, 2, "5:2"),
                                            (130, 100, 96, 0, None), (300, 200, 256, 1, "6")])
def test_f16a_gemm_equals_fp32_gemm(gpu, oracle, tune, M, N, K, mode, cfg):
    print(f"[case] f16a gemm M={M} N={N} K={K} mode={mode} cfg={cfg}", flush=True)
    if cfg:
        tune("gemm_cfg", cfg)
    a16, a32 = _half_a(oracle, 1, M * K)
    blocks = q8_weights(oracle, 2, N, K)
    bias = oracle.normal(3, N, 0.0, 0.02)
    C0 = oracle.normal(4, M * N)
    dW, dB = DeviceBuffer.from_array(blocks), DeviceBuffer.from_array(bias)
    nws = ops.gemm_workspace_bytes(M, N, K)
    outs = []
    for A, entry in ((a16, ops.gemm_nt_q8_0_f16a), (a32, ops.gemm_nt_q8_0)):
        dC = DeviceBuffer.from_array(C0)
        entry(DeviceBuffer.from_array(A), dW, dC, M, N, K, bias=dB, mode=mode,
              workspace=DeviceBuffer(nws) if nws else None)
        synchronize()
        outs.append(dC.download(np.float32, M * N))
    assert np.array_equal(outs[0], outs[1]), "fp16-A GEMM differs from the fp32 GEMM on the same values"
    want = oracle.gemm_nt_q8_0(a32, blocks, M, N, K, bias=None if mode == 1 else bias, threads=oracle.max_threads())
    got = outs[0] - (C0 if mode else 0)
    assert_parity(got, want, what="f16a gemm")


def test_f16a_gemm_batch_and_strides(gpu, oracle):
    """Batch items with strides (lda, sA multiples of 8 halves; ldc, sC padded)."""
    B, M, N, K = 2, 70, 36, 128
    lda, ldc, sA, sC = 136, 40, 70 * 136 + 8, 3000
    a16, a32 = _half_a(oracle, 5, (B - 1) * sA + (M - 1) * lda + K)
    blocks = q8_weights(oracle, 6, N, K)
    outs = []
    for A, entry in ((a16, ops.gemm_nt_q8_0_f16a), (a32, ops.gemm_nt_q8_0)):
        dC = DeviceBuffer.from_array(np.zeros((B - 1) * sC + (M - 1) * ldc + N, np.float32))
        entry(DeviceBuffer.from_array(A), DeviceBuffer.from_array(blocks), dC, M, N, K, lda=lda, ldc=ldc, batch=B,
              sA=sA, sC=sC)
        synchronize()
        outs.append(dC.download(np.float32))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("M,F,K", [(77, 48, 64), (300, 200, 256), (2048, 5120, 1280)])
def test_geglu_f16_equals_rounded_fp32(gpu, oracle, M, F, K):
    print(f"[case] geglu f16 M={M} F={F} K={K}", flush=True)
    a16, a32 = _half_a(oracle, 7, M * K)
    blocks = q8_weights(oracle, 8, 2 * F, K)
    bias = oracle.normal(9, 2 * F, 0.0, 0.5)
    dW, dB = DeviceBuffer.from_array(blocks), DeviceBuffer.from_array(bias)
    d16, d32 = DeviceBuffer(M * F * 2), DeviceBuffer(M * F * 4)
    ops.gemm_nt_q8_0_geglu_f16(DeviceBuffer.from_array(a16), dW, d16, M, F, K, bias=dB)
    ops.gemm_nt_q8_0_geglu(DeviceBuffer.from_array(a32), dW, d32, M, F, K, bias=dB)
    synchronize()
    got = d16.download(np.float16, M * F)
    want = d32.download(np.float32, M * F).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("rows,d", [(9, 1280), (2048, 1280), (5, 4096)])
def test_layernorm_f16_equals_rounded_fp32(gpu, oracle, rows, d):
    x = oracle.normal(11, rows * d, 0.5, 2.0)
    g, b = oracle.normal(12, d, 1.0, 0.1), oracle.normal(13, d, 0.0, 0.1)
    dx, dg, db = DeviceBuffer.from_array(x), DeviceBuffer.from_array(g), DeviceBuffer.from_array(b)
    d16, d32 = DeviceBuffer(rows * d * 2), DeviceBuffer(rows * d * 4)
    ops.layernorm_f16(dx, dg, db, d16, rows, d)
    ops.layernorm(dx, dg, db, d32, rows, d)
    synchronize()
    got, want = d16.download(np.float16, rows * d), d32.download(np.float32, rows * d).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_geglu_kernel_f16_equals_rounded_fp32(gpu, oracle):
    rows, F = 2048, 5120
    h = oracle.normal(14, rows * 2 * F)
    dh, d16, d32 = DeviceBuffer.from_array(h), DeviceBuffer(rows * F * 2), DeviceBuffer(rows * F * 4)
    ops.geglu_f16(dh, d16, rows, F)
    ops.geglu(dh, d32, rows, F)
    synchronize()
    got, want = d16.download(np.float16, rows * F), d32.download(np.float32, rows * F).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("B,H,Tq,Tk,ws,kv", [(2, 20, 1024, 1024, False, False), (2, 20, 1024, 77, False, True),
                                            (2, 10, 4096, 4096, True, False), (1, 3, 100, 130, False, False)])
def test_attention_f16_out_equals_rounded_fp32(gpu, oracle, B, H, Tq, Tk, ws, kv):
    """Both kernels (fp32 and fp16 inputs), the staged and the key-split
    stores: the fp16 output is the fp16 rounding of the fp32 output."""
    print(f"[case] attention f16 out B={B} H={H} Tq={Tq} Tk={Tk} ws={ws}", flush=True)
    C = 64 * H
    for in_dt, np_in in ((MI_F16, np.float16), (MI_F32, np.float32)):
        if ws and in_dt == MI_F32:
            continue
        q = oracle.normal(21, B * Tq * C).astype(np_in)
        k = oracle.normal(22, B * Tk * C).astype(np_in)
        v = oracle.normal(23, B * Tk * C).astype(np_in)
        kl = DeviceBuffer.from_array(oracle.uniform_int(24, 1, Tk, B).astype(np.int32)) if kv else None
        dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
        kw = dict(batch=B, Tq=Tq, Tk=Tk, C=C, heads=H, in_dtype=in_dt, kv_len=kl, precision=MI_ATTN_PREC_FP16)
        outs = []
        for odt, esz in ((MI_F16, 2), (MI_F32, 4)):
            do = DeviceBuffer(B * Tq * C * esz)
            n = ops.fused_attention_ws_bytes(out_dtype=odt, **kw) if ws else 0
            ops.fused_attention_ws(dq, dk, dv, do, DeviceBuffer(n) if n else None, out_dtype=odt, **kw)
            synchronize()
            outs.append(do.download(np.float16 if odt == MI_F16 else np.float32, B * Tq * C))
        assert np.array_equal(outs[0].view(np.uint16), outs[1].astype(np.float16).view(np.uint16)), \
            f"in {in_dt}: fp16 output is not the rounded fp32 output"


@pytest.mark.parametrize("M,N,K,ldc", [(77, 96, 64, 0), (2048, 3840, 1280, 0), (154, 1280, 2048, 0),
                                       (300, 260, 256, 264), (2048, 1280, 1280, 0)])
def test_f16o_gemm_is_the_rounded_fp32_gemm(gpu, oracle, M, N, K, ldc):
    """mi_gemm_nt_q8_0_f16o (the block's fp16 Q / K / V projections) stores the
    RNE rounding of mi_gemm_nt_q8_0's fp32 result, for fp32 and fp16 A; padding
    columns of a strided C stay untouched."""
    print(f"[case] f16o gemm M={M} N={N} K={K} ldc={ldc}", flush=True)
    a16, a32 = _half_a(oracle, 31, M * K)
    blocks = q8_weights(oracle, 32, N, K)
    bias = oracle.normal(33, N, 0.0, 0.02)
    dW, dB = DeviceBuffer.from_array(blocks), DeviceBuffer.from_array(bias)
    d32 = DeviceBuffer(M * N * 4)
    ops.gemm_nt_q8_0(DeviceBuffer.from_array(a32), dW, d32, M, N, K, bias=dB)
    synchronize()
    want = d32.download(np.float32, M * N).astype(np.float16)
    ld = ldc or N
    for a_dtype, A in ((MI_F32, a32), (MI_F16, a16)):
        dH = DeviceBuffer.from_array(np.full((M - 1) * ld + N, np.float16(7.0), np.float16))
        ops.gemm_nt_q8_0_f16o(DeviceBuffer.from_array(A), dW, dH, M, N, K, a_dtype=a_dtype, bias=dB, ldc=ldc)
        synchronize()
        got = dH.download(np.float16, (M - 1) * ld + N)
        rows = np.concatenate([got[m * ld:m * ld + N] for m in range(M)])
        assert np.array_equal(rows.view(np.uint16), want.view(np.uint16)), f"a_dtype {a_dtype}"
        if ld > N:
            assert all(np.all(got[m * ld + N:(m + 1) * ld] == np.float16(7.0)) for m in range(M - 1))
