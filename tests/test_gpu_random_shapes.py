"""GPU parity on seeded random shapes, beyond the hand-picked cases: the Q8_0
NT GEMM (workspace entry, so every plan the rules pick runs, K splits
included), the Q8 NN GEMM (tiled and untiled kernels, with and without K
splits) and the fused attention (fp16 kernel with masks, causal, partial query
blocks and key splits; fp32 reference-layout kernel), each against the CPU
oracle. Shapes and data come from fixed seeds, so a failure names a
reproducible case.

Bar: max |out - oracle| <= 2e-3 x RMS(oracle) (fp32 outputs), as in the other
parity tests; fp16 outputs add half an fp16 ulp of |out| per element.
"""
import numpy as np
import pytest

from helpers import REL_RMS_TOL, assert_parity, err_vs_rms, fp16_half_ulp, q8_weights, rms
from sdvk_amd import MI_ATTN_PREC_AUTO, MI_ATTN_PREC_FP16, MI_F16, MI_F32, ops
from sdvk_amd.hip import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu


def _gemm_shapes(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.integers(1, 2600))
        N = int(rng.integers(1, 2600))
        K = 32 * int(rng.integers(1, 160))
        out.append((M, N, K, int(rng.integers(0, 2)), bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("M,N,K,mode,bias", _gemm_shapes(12, 2024))
def test_random_gemm_nt_q8_0(gpu, oracle, M, N, K, mode, bias):
    print(f"[case] random gemm M={M} N={N} K={K} mode={mode} bias={bias}", flush=True)
    A = oracle.normal(M + 1, M * K)
    blocks = q8_weights(oracle, N + 2, N, K)
    b = oracle.normal(K + 3, N, 0.0, 0.02) if bias and mode == 0 else None  # mode 1 adds no bias
    C0 = oracle.normal(M + N, M * N) if mode == 1 else None
    nws = ops.gemm_workspace_bytes(M, N, K)
    dA, dW = DeviceBuffer.from_array(A), DeviceBuffer.from_array(blocks)
    dB = DeviceBuffer.from_array(b) if b is not None else None
    dC = DeviceBuffer.from_array(C0) if C0 is not None else DeviceBuffer(M * N * 4)
    ops.gemm_nt_q8_0(dA, dW, dC, M, N, K, bias=dB, mode=mode, workspace=DeviceBuffer(nws) if nws else None)
    synchronize()
    got = dC.download(np.float32, M * N).reshape(M, N)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).integers(0, M, min(M, 48))]))
    want = oracle.gemm_rows(A, blocks, M, N, K, rows.astype(np.uint32), bias=b, threads=oracle.max_threads())
    if mode == 1:
        want = want + C0.reshape(M, N)[rows]
        # accumulate mode: the bar is on the product, the stored C0 adds exactly
        e = float(np.max(np.abs(got[rows] - want))) / rms(want - C0.reshape(M, N)[rows])
    else:
        e = err_vs_rms(got[rows], want)
    print(f"  err/rms = {e:.3e} (split workspace {nws} B)", flush=True)
    assert e <= REL_RMS_TOL


def _nn_shapes(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.integers(1, 1400))
        N = 4 * int(rng.integers(1, 525))  # the NN entry takes N and K in multiples of 4 (gemm_nn_q8.comp)
        K = 64 * int(rng.integers(1, 90)) if i % 3 else 32 * int(rng.integers(1, 90)) + 32 * (i % 2)
        out.append((M, N, K, bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("M,N,K,ws", _nn_shapes(8, 77))
def test_random_gemm_nn_q8(gpu, oracle, M, N, K, ws):
    print(f"[case] random nn M={M} N={N} K={K} ws={ws}", flush=True)
    payload, scales = oracle.q8_0_to_split(q8_weights(oracle, M + 5, M, K), M * K)
    B = oracle.normal(N + 6, K * N)
    want = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K, threads=oracle.max_threads()).reshape(M, N)
    dq, ds, dB = DeviceBuffer.from_array(payload), DeviceBuffer.from_array(scales), DeviceBuffer.from_array(B)
    dC = DeviceBuffer(M * N * 4)
    kw = {}
    if ws:
        n = ops.gemm_nn_workspace_bytes(M, N, K)
        kw["workspace"] = DeviceBuffer(n) if n else None
    ops.gemm_nn_q8(dq, ds, dB, dC, M, N, K, **kw)
    synchronize()
    got = dC.download(np.float32, M * N).reshape(M, N)
    e = assert_parity(got, want, what="random nn")
    print(f"  err/rms = {e:.3e}", flush=True)


def _attn_shapes(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        B = int(rng.integers(1, 3))
        H = int(rng.integers(1, 9))
        Tq = int(rng.integers(1, 700))
        Tk = int(rng.integers(1, 900))
        hd = int(rng.choice([64, 64, 40, 32]))
        causal = bool(rng.integers(0, 4) == 0)
        masked = bool(rng.integers(0, 3) == 0) and not causal
        split = str(rng.choice(["", "", "1:2", "2:3"]))
        out.append((B, H, Tq, Tk, hd, causal, masked, split))
    return out


@pytest.mark.parametrize("B,H,Tq,Tk,hd,causal,masked,split",
                         [x for x in _attn_shapes(24, 977) if not x[5]][:10])
def test_random_burst_attention(gpu, oracle, tune, B, H, Tq, Tk, hd, causal, masked, split):
    """The burst build (attn_simd_waves "3", 4-wave workgroups, one fp16 P
    product) on random non-causal shapes: within the bar of the oracle and bit
    for bit the interleaved build's output (attn_simd_waves "2")."""
    print(f"[case] random burst attention B={B} H={H} Tq={Tq} Tk={Tk} hd={hd} masked={masked} "
          f"split={split or '-'}", flush=True)
    C = H * hd
    tune("attn_nw", "4")
    if split:
        tune("attn_split", split)
    q = oracle.normal(Tq + 11, B * Tq * C).astype(np.float16)
    k = oracle.normal(Tk + 12, B * Tk * C).astype(np.float16)
    v = oracle.normal(Tk + 13, B * Tk * C).astype(np.float16)
    kv_len = None
    if masked:
        kv_len = np.random.default_rng(Tk + 1).integers(0, Tk + 1, B).astype(np.int32)
        kv_len[0] = max(int(kv_len[0]), 1)
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=H, in_dtype=1, kv_len=kv_len,
                                     threads=oracle.max_threads()).astype(np.float64)
    dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
    dl = DeviceBuffer.from_array(kv_len) if kv_len is not None else None
    kw = dict(batch=B, Tq=Tq, Tk=Tk, C=C, heads=H, in_dtype=MI_F16, out_dtype=MI_F32, kv_len=dl,
              precision=MI_ATTN_PREC_FP16)
    outs = []
    for waves in ("2", "3"):
        tune("attn_simd_waves", waves)
        nws = ops.fused_attention_ws_bytes(**kw)
        do = DeviceBuffer(B * Tq * C * 4)
        ops.fused_attention_ws(dq, dk, dv, do, DeviceBuffer(nws) if nws else None, **kw)
        synchronize()
        outs.append(do.download(np.float32, B * Tq * C))
    assert np.array_equal(outs[0], outs[1]), "burst build differs from the interleaved build"
    assert_parity(outs[1].reshape(want.shape).astype(np.float64), want, what="random burst attention",
                  label="[precision=fp16]")


@pytest.mark.parametrize("B,H,Tq,Tk,hd,causal,masked,split", _attn_shapes(14, 4242))
def test_random_attention(gpu, oracle, tune, B, H, Tq, Tk, hd, causal, masked, split):
    """fp16 in / fp16 and fp32 out through the workspace entry (a forced key
    split where `split` is set: it applies to unmasked, non-causal, 4-wave
    launches), and the fp32 reference-layout entry for batch 1."""
    print(f"[case] random attention B={B} H={H} Tq={Tq} Tk={Tk} hd={hd} causal={causal} masked={masked} "
          f"split={split or '-'}", flush=True)
    C = H * hd
    if split:
        tune("attn_split", split)
    q = oracle.normal(Tq + 1, B * Tq * C).astype(np.float16)
    k = oracle.normal(Tk + 2, B * Tk * C).astype(np.float16)
    v = oracle.normal(Tk + 3, B * Tk * C).astype(np.float16)
    kv_len = None
    if masked:  # lengths 0..Tk, at least one batch item with a key (an all-zero output has no RMS)
        kv_len = np.random.default_rng(Tk).integers(0, Tk + 1, B).astype(np.int32)
        kv_len[0] = max(int(kv_len[0]), 1)
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=H, causal=causal, in_dtype=1,
                                     kv_len=kv_len, threads=oracle.max_threads()).astype(np.float64)
    dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
    dl = DeviceBuffer.from_array(kv_len) if kv_len is not None else None
    kw = dict(batch=B, Tq=Tq, Tk=Tk, C=C, heads=H, causal=causal, in_dtype=MI_F16, kv_len=dl)
    # fp32 out: the default (two-part P) to a tenth of the bar, and one fp16 P
    # product (MI_ATTN_PREC_FP16) to the bar; fp16 out: its default (one product)
    for odt, prec in ((MI_F32, MI_ATTN_PREC_AUTO), (MI_F32, MI_ATTN_PREC_FP16), (MI_F16, MI_ATTN_PREC_AUTO)):
        nws = ops.fused_attention_ws_bytes(out_dtype=odt, precision=prec, **kw)
        do = DeviceBuffer(B * Tq * C * (4 if odt == MI_F32 else 2))
        ops.fused_attention_ws(dq, dk, dv, do, DeviceBuffer(nws) if nws else None, out_dtype=odt, precision=prec,
                               **kw)
        synchronize()
        if odt == MI_F32:
            got = do.download(np.float32, B * Tq * C).reshape(want.shape).astype(np.float64)
            tol = REL_RMS_TOL / 10 if prec == MI_ATTN_PREC_AUTO else REL_RMS_TOL
            assert_parity(got, want, tol=tol, what=f"random attention fp32 out, precision {prec}",
                          label="" if prec == MI_ATTN_PREC_AUTO else "[precision=fp16]")
        else:
            got = do.download(np.float16, B * Tq * C).reshape(want.shape).astype(np.float64)
            bound = REL_RMS_TOL * rms(want) + fp16_half_ulp(want)
            assert np.all(np.abs(got - want) <= bound), "fp16 output beyond parity + storage rounding"
    if B == 1:
        # the reference call shape: fp32 [T, C] through mi_fused_attention
        dq32, dk32, dv32 = (DeviceBuffer.from_array(x.astype(np.float32)) for x in (q, k, v))
        do32 = DeviceBuffer(Tq * C * 4)
        ops.fused_attention(ops.FusedAttnArgs(dq32, dk32, dv32, do32, Tq, Tk, C, H, causal))
        synchronize()
        got = do32.download(np.float32, Tq * C).reshape(want.shape).astype(np.float64)
        if not masked:
            assert_parity(got, want, tol=REL_RMS_TOL / 10, what="random attention, reference layout")
