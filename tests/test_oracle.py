"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement (a wrong
sign or index, a dropped term, a transposed operand) fails it: the reference's
own GGUF reader compiled from /root/reference (oracle/_ref, when present),
golden fixtures written from that reader, independent library routes
(numpy float64 matmul / softmax, math.erf), closed forms and invariants.
"""
import math

import numpy as np
import pytest

from helpers import rms

pytestmark = []


# ------------------------------------------------------------------ fp16 --

def test_fp16_decode_exhaustive_vs_numpy(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([oracle.lib().or_fp16_to_fp32(int(b)) for b in bits], dtype=np.float32).view(np.uint32)
    nan = np.isnan(bits.view(np.float16))
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan(got.view(np.float32)[nan]))


def test_fp16_decode_exhaustive_vs_reference(oracle):
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("reference tree absent: oracle/_ref not built (pinned by the numpy check and fixtures)")
    for b in range(65536):
        a = oracle.lib().or_fp16_to_fp32(b)
        r = R.ref_fp16_to_fp32(b)
        if math.isnan(r):
            assert math.isnan(a), b
        else:
            assert np.float32(a).view(np.uint32) == np.float32(r).view(np.uint32), hex(b)


def test_fp16_encode_rne_vs_numpy(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 1e9, np.inf, -np.inf, 2 ** -24, 2 ** -25,
                  2 ** -25 * 1.0000001, 3 * 2 ** -26, 2 ** -14, 2 ** -14 - 2 ** -25, 6.1e-5, 1.0009765625,
                  1.00048828125, 1.00146484375], dtype=np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.lib().or_fp32_to_fp16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ Q8_0 --

def _kat_blocks() -> np.ndarray:
    """Known-answer blocks: q over {-128,-127,-1,0,1,127} and scales at the fp16 edges."""
    ds = [0x0000, 0x8000, 0x0001, 0x03ff, 0x0400, 0x3c00, 0xbc00, 0x7bff, 0x2e66, 0x7c00, 0xfc00, 0x7e00, 0x1234]
    qs = np.array([-128, -127, -1, 0, 1, 127] * 5 + [42, -42], dtype=np.int8)
    out = []
    for i, d in enumerate(ds):
        blk = np.zeros(34, dtype=np.uint8)
        blk[0], blk[1] = d & 0xff, d >> 8
        blk[2:] = np.roll(qs, i).view(np.uint8)
        out.append(blk)
    return np.concatenate(out)


def test_q8_0_dequant_kat_closed_form(oracle):
    blocks = _kat_blocks()
    n = blocks.size // 34 * 32
    got = oracle.q8_0_dequant(blocks, n)
    b = blocks.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    with np.errstate(invalid="ignore"):
        want = (d * q).reshape(-1)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_q8_0_decode_vs_reference_reader(oracle):
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("reference tree absent: oracle/_ref not built (pinned by tests/golden fixtures)")
    rows, cols = 24, 96
    w = oracle.normal(11, rows * cols, 0.0, 0.02)
    # 12 known-answer blocks append 4 more rows of 96 (3 blocks per row)
    blocks = np.concatenate([oracle.q8_0_quantize(w), _kat_blocks()[: 34 * 12]])
    rows += 4
    n = rows * cols
    ref_f, ref_q, ref_s, ref_q2, ref_s2 = oracle.ref_q8_0_decode(blocks, rows, cols)
    got = oracle.q8_0_dequant(blocks, n)
    nan = np.isnan(ref_f)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref_f[~nan].view(np.uint32))
    q, s = oracle.q8_0_to_split(blocks, n)
    assert np.array_equal(q, ref_q) and np.array_equal(q, ref_q2)
    assert np.array_equal(s.view(np.uint32), ref_s.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), ref_s2.view(np.uint32))


def test_q8_0_golden_fixture(oracle):
    """tests/golden/q8_0_reference.npz was written by the reference's own reader."""
    from pathlib import Path

    f = np.load(Path(__file__).parent / "golden" / "q8_0_reference.npz")
    blocks, rows, cols = f["blocks"], int(f["rows"]), int(f["cols"])
    got = oracle.q8_0_dequant(blocks, rows * cols)
    want = f["dequant"]
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    q, s = oracle.q8_0_to_split(blocks, rows * cols)
    assert np.array_equal(q, f["payload"])
    assert np.array_equal(s.view(np.uint32), f["scales"].view(np.uint32))


def test_q8_split_dequant_matches_block_dequant(oracle):
    n = 32 * 50
    blocks = oracle.q8_0_quantize(oracle.normal(3, n, 0, 0.05))
    q, s = oracle.q8_0_to_split(blocks, n)
    a = oracle.q8_split_dequant(q, s, n)
    b = oracle.q8_0_dequant(blocks, n)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # byte layout of the payload word: element i is byte (i & 3) of word i >> 2 (little-endian)
    words = q.view(np.uint32)
    i = 37
    assert np.array([(int(words[i >> 2]) >> (8 * (i & 3))) & 0xff], dtype=np.uint8).view(np.int8)[0] == q[i]


def test_q8_0_quantize_roundtrip(oracle):
    n = 32 * 400
    w = oracle.normal(5, n, 0.0, 0.02)
    w[:32] = 0.0  # an all-zero block: d = 0, q = 0
    blocks = oracle.q8_0_quantize(w)
    b = blocks.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    q = b[:, 2:].view(np.int8).astype(np.int32)
    assert np.all(q[0] == 0) and d[0] == 0
    amax = np.abs(w.reshape(-1, 32)).max(1)
    # the largest element maps to +-127 and no code is -128
    assert np.all(np.abs(q[1:]).max(1) == 127)
    assert q.min() >= -127
    deq = oracle.q8_0_dequant(blocks, n).reshape(-1, 32).astype(np.float64)
    err = np.abs(deq - w.reshape(-1, 32))
    # |q d - w| <= d/2 + 127 |d - amax/127| (fp16 rounding of d)
    bound = d / 2 + 127 * np.abs(d - amax / 127) + 1e-12
    assert np.all(err.max(1) <= bound * 1.0001)


# ------------------------------------------------------------------ GEMM --

def _deq(oracle, blocks, N, K):
    return oracle.q8_0_dequant(blocks, N * K).reshape(N, K).astype(np.float64)


@pytest.mark.parametrize("M,N,K", [(100, 100, 96), (37, 70, 64), (5, 3, 32)])
def test_gemm_oracle_vs_numpy(oracle, M, N, K):
    A = oracle.normal(1, M * K)
    blocks = oracle.q8_0_quantize(oracle.normal(2, N * K, 0, 0.02))
    W = _deq(oracle, blocks, N, K)
    want = A.reshape(M, K).astype(np.float64) @ W.T
    got64 = oracle.gemm_nt_q8_0(A, blocks, M, N, K, acc64=True).reshape(M, N)
    got32 = oracle.gemm_nt_q8_0(A, blocks, M, N, K, acc64=False).reshape(M, N)
    assert np.max(np.abs(got64 - want)) <= 1e-6 * rms(want)
    assert np.max(np.abs(got32 - want)) <= 1e-5 * rms(want)
    # a transposed operand would not match: A W (not A W^T) differs for N != K
    if N != K:
        assert want.shape == (M, N)


def test_gemm_oracle_modes_bias_batch_strides(oracle):
    M, N, K, batch = 33, 40, 64, 3
    lda, ldc = K + 4, N + 8
    sA, sC = M * lda + 12, M * ldc + 20
    A = oracle.normal(7, (batch - 1) * sA + M * lda)
    blocks = oracle.q8_0_quantize(oracle.normal(8, N * K, 0, 0.02))
    bias = oracle.normal(9, N, 0, 0.5)
    W = _deq(oracle, blocks, N, K)
    C0 = oracle.normal(10, (batch - 1) * sC + M * ldc)
    # mode 0 with bias
    C = C0.copy()
    oracle.gemm_nt_q8_0(A, blocks, M, N, K, bias=bias, C=C, mode=0, lda=lda, ldc=ldc, batch=batch, sA=sA, sC=sC)
    C1 = C0.copy()
    oracle.gemm_nt_q8_0(A, blocks, M, N, K, bias=bias, C=C1, mode=1, lda=lda, ldc=ldc, batch=batch, sA=sA, sC=sC)
    for z in range(batch):
        a = A[z * sA: z * sA + M * lda].reshape(M, lda)[:, :K].astype(np.float64)
        want = a @ W.T
        got = C[z * sC: z * sC + M * ldc].reshape(M, ldc)
        assert np.allclose(got[:, :N], want + bias, rtol=0, atol=1e-5)
        # mode 1 accumulates without bias
        got1 = C1[z * sC: z * sC + M * ldc].reshape(M, ldc)
        base = C0[z * sC: z * sC + M * ldc].reshape(M, ldc)
        assert np.allclose(got1[:, :N], base[:, :N] + want, rtol=0, atol=1e-5)
        # padding columns untouched
        assert np.array_equal(got[:, N:], base[:, N:])


def test_gemm_oracle_linearity(oracle):
    M, N, K = 16, 24, 64
    A1, A2 = oracle.normal(1, M * K), oracle.normal(2, M * K)
    blocks = oracle.q8_0_quantize(oracle.normal(3, N * K, 0, 0.02))
    c1 = oracle.gemm_nt_q8_0(A1, blocks, M, N, K)
    c2 = oracle.gemm_nt_q8_0(A2, blocks, M, N, K)
    c12 = oracle.gemm_nt_q8_0((2 * A1 - 3 * A2).astype(np.float32), blocks, M, N, K)
    assert np.allclose(c12, 2 * c1 - 3 * c2, atol=1e-5)


def test_gemm_oracle_split_general_k(oracle):
    """Split layout with K % 32 != 0: scales index the flat element (gemm_nt_q8_v.comp:37-43)."""
    M, N, K = 9, 11, 100
    A = oracle.normal(4, M * K)
    payload = oracle.uniform_int(5, -127, 127, N * K).astype(np.int8)
    scales = oracle.normal(6, (N * K + 31) // 32, 0.01, 0.002)
    C = oracle.gemm_nt_q8_split(A, payload, scales, M, N, K).reshape(M, N)
    fl = np.arange(N * K)
    W = (payload.astype(np.float64) * scales[fl >> 5]).reshape(N, K)
    want = A.reshape(M, K).astype(np.float64) @ W.T
    assert np.allclose(C, want, atol=1e-5)


def test_gemm_rows_matches_full(oracle):
    M, N, K = 50, 64, 96
    A = oracle.normal(1, M * K)
    blocks = oracle.q8_0_quantize(oracle.normal(2, N * K, 0, 0.02))
    full = oracle.gemm_nt_q8_0(A, blocks, M, N, K).reshape(M, N)
    rows = np.array([0, 7, 49, 13])
    part = oracle.gemm_rows(A, blocks, M, N, K, rows)
    assert np.array_equal(part, full[rows])


# ------------------------------------------------------------- attention --

def _np_attention(q, k, v, Tq, Tk, C, heads, causal=False, kv_len=None):
    hd = C // heads
    scale = np.float64(np.float32(1.0) / np.sqrt(np.float32(hd)))
    q = q.reshape(Tq, heads, hd).astype(np.float64)
    k = k.reshape(Tk, heads, hd).astype(np.float64)
    v = v.reshape(Tk, heads, hd).astype(np.float64)
    out = np.zeros((Tq, heads, hd))
    L = Tk if kv_len is None else kv_len
    for h in range(heads):
        s = q[:, h] @ k[:L, h].T * scale
        if causal:
            s = np.where(np.arange(L)[None, :] > np.arange(Tq)[:, None], -np.inf, s)
        with np.errstate(invalid="ignore"):
            m = s.max(1, keepdims=True)
            m = np.where(np.isfinite(m), m, 0)
            p = np.exp(s - m)
            l = p.sum(1, keepdims=True)
            out[:, h] = np.where(l > 0, (p @ v[:L, h]) / np.where(l > 0, l, 1), 0)
    return out.reshape(Tq, C)


@pytest.mark.parametrize("Tq,Tk,C,heads,causal", [
    (32, 32, 320, 5, True), (32, 77, 1280, 20, False), (64, 64, 320, 8, True), (48, 96, 512, 8, False),
    (20, 300, 128, 2, True)])
def test_attention_oracle_vs_numpy(oracle, Tq, Tk, C, heads, causal):
    """The reference test's shapes (fused_attn_test.cpp:74-79) plus a Tk >= 256 case."""
    q = oracle.normal(1, Tq * C)
    k = oracle.normal(2, Tk * C)
    v = oracle.normal(3, Tk * C)
    got = oracle.fused_attention(q, k, v, Tq, Tk, C, heads, causal).reshape(Tq, C)
    want = _np_attention(q, k, v, Tq, Tk, C, heads, causal)
    assert np.max(np.abs(got - want)) <= 1e-6 * max(rms(want), 1e-12)


def test_attention_oracle_special_cases(oracle):
    C, heads = 128, 2
    # Tk = 1: the output is the single V row
    q, k, v = oracle.normal(1, 5 * C), oracle.normal(2, C), oracle.normal(3, C)
    o = oracle.fused_attention(q, k, v, 5, 1, C, heads).reshape(5, C)
    assert np.allclose(o, np.tile(v, (5, 1)), atol=1e-6)
    # constant scores (zero keys): the output is the mean of V
    k0 = np.zeros(7 * C, dtype=np.float32)
    v7 = oracle.normal(4, 7 * C)
    o = oracle.fused_attention(q, k0, v7, 5, 7, C, heads).reshape(5, C)
    assert np.allclose(o, np.tile(v7.reshape(7, C).mean(0), (5, 1)), atol=1e-6)
    # causal: row 0 sees only key 0
    k7 = oracle.normal(5, 7 * C)
    o = oracle.fused_attention(oracle.normal(6, 7 * C), k7, v7, 7, 7, C, heads, causal=True).reshape(7, C)
    assert np.allclose(o[0], v7[:C], atol=1e-6)


def test_attention_oracle_kv_len_is_prefix_slicing(oracle):
    batch, Tq, Tk, C, heads = 3, 10, 77, 128, 2
    q = oracle.normal(1, batch * Tq * C)
    k = oracle.normal(2, batch * Tk * C)
    v = oracle.normal(3, batch * Tk * C)
    kv_len = np.array([1, 40, 0], dtype=np.int32)
    got = oracle.fused_attention_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, kv_len=kv_len)
    for b in range(batch):
        L = kv_len[b]
        if L == 0:
            assert np.all(got[b] == 0)
            continue
        kb = k[b * Tk * C: b * Tk * C + L * C]
        vb = v[b * Tk * C: b * Tk * C + L * C]
        want = oracle.fused_attention(q[b * Tq * C:(b + 1) * Tq * C].copy(), kb.copy(), vb.copy(), Tq, L, C, heads)
        assert np.array_equal(got[b].reshape(-1), want)


def test_attention_oracle_rows_and_fp16(oracle):
    batch, Tq, Tk, C, heads = 2, 40, 50, 128, 2
    q = oracle.normal(1, batch * Tq * C).astype(np.float16)
    k = oracle.normal(2, batch * Tk * C).astype(np.float16)
    v = oracle.normal(3, batch * Tk * C).astype(np.float16)
    full = oracle.fused_attention_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=1)
    rows = np.array([3, 39, 0])
    part = oracle.fused_attention_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=1, rows=rows)
    assert np.array_equal(part, full[:, rows])
    want = np.stack([_np_attention(q[b * Tq * C:(b + 1) * Tq * C].astype(np.float32),
                                   k[b * Tk * C:(b + 1) * Tk * C].astype(np.float32),
                                   v[b * Tk * C:(b + 1) * Tk * C].astype(np.float32), Tq, Tk, C, heads)
                     for b in range(batch)])
    assert np.max(np.abs(full - want)) <= 1e-6 * rms(want)
    o16 = oracle.fused_attention_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=1, out_dtype=1)
    assert np.array_equal(o16, full.astype(np.float16))


def test_attention_f32_baseline_matches_fp64(oracle):
    batch, Tq, Tk, C, heads = 2, 33, 150, 128, 2
    q = oracle.normal(1, batch * Tq * C)
    k = oracle.normal(2, batch * Tk * C)
    v = oracle.normal(3, batch * Tk * C)
    kv_len = np.array([150, 77], dtype=np.int32)
    got = oracle.fused_attention_f32(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, kv_len=kv_len)
    want = oracle.fused_attention_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, kv_len=kv_len)
    assert np.max(np.abs(got - want.reshape(-1))) <= 1e-5 * rms(want)


# ------------------------------------------------------------------ glue --

def test_layernorm_gelu_geglu(oracle):
    rows, d = 6, 320
    x = oracle.normal(1, rows * d, 0.3, 2.0)
    g, b = oracle.normal(2, d), oracle.normal(3, d)
    y = oracle.layernorm(x, g, b, rows, d).reshape(rows, d)
    xx = x.reshape(rows, d).astype(np.float64)
    want = (xx - xx.mean(1, keepdims=True)) / np.sqrt(xx.var(1, keepdims=True) + 1e-5) * g + b
    assert np.allclose(y, want, atol=2e-5)
    for t in [-6.0, -1.3, -0.1, 0.0, 0.2, 1.0, 3.7, 9.0]:
        exact = 0.5 * t * (1 + math.erf(t / math.sqrt(2)))
        assert abs(oracle.gelu_erf(t) - exact) <= 1.5e-7 * abs(t) + 1e-6
    F = 40
    h = oracle.normal(4, rows * 2 * F)
    gg = oracle.geglu(h, rows, F).reshape(rows, F)
    hh = h.reshape(rows, 2 * F).astype(np.float64)
    ge = 0.5 * hh[:, F:] * (1 + np.vectorize(math.erf)(hh[:, F:] / math.sqrt(2)))
    assert np.allclose(gg, hh[:, :F] * ge, atol=1e-5)


def _block_weights(oracle, C, Cc, F, seed=100):
    w, s = {}, seed
    for nm in ("norm1", "norm2", "norm3"):
        w[nm + "_w"] = oracle.normal(s, C, 1.0, 0.1); w[nm + "_b"] = oracle.normal(s + 1, C, 0.0, 0.1); s += 2
    for nm, (n, k) in {"attn1_q": (C, C), "attn1_k": (C, C), "attn1_v": (C, C), "attn1_out": (C, C),
                       "attn2_q": (C, C), "attn2_k": (C, Cc), "attn2_v": (C, Cc), "attn2_out": (C, C),
                       "ff_up": (2 * F, C), "ff_down": (C, F)}.items():
        w[nm] = oracle.q8_0_quantize(oracle.normal(s, n * k, 0.0, 0.08)); s += 1
    for nm, n in {"attn1_out_b": C, "attn2_out_b": C, "ff_up_b": 2 * F, "ff_down_b": C}.items():
        w[nm] = oracle.normal(s, n, 0.0, 0.02); s += 1
    return w


def test_block_composition(oracle):
    """oracle.sdxl_block vs an independent numpy fp64 block (dequantised weights,
    softmax attention, erf GELU via math.erf): pins the order of the block
    (sdvkgen.cpp:1739-1763), the GEGLU halves and the key-padding mask."""
    B, T, C, H, Tc, Cc, F = 2, 24, 64, 2, 7, 96, 96
    w = _block_weights(oracle, C, Cc, F)
    x = oracle.normal(1, B * T * C)
    ctx = oracle.normal(2, B * Tc * Cc)
    kl = np.array([7, 3], np.int32)
    got = oracle.sdxl_block(w, x, ctx, batch=B, tokens=T, channels=C, heads=H, ctx_tokens=Tc, ctx_channels=Cc,
                            ff_inner=F, ctx_len=kl).reshape(B * T, C)

    def deq(nm, n, k):
        return oracle.q8_0_dequant(w[nm], n * k).astype(np.float64).reshape(n, k)

    def ln(a, g, b):
        return (a - a.mean(1, keepdims=True)) / np.sqrt(a.var(1, keepdims=True) + 1e-5) * g + b

    def attn(q, k, v, tk, lens):
        o = np.zeros((B * T, C))
        hd = C // H
        for b in range(B):
            L = tk if lens is None else int(lens[b])
            for h in range(H):
                cs = slice(h * hd, (h + 1) * hd)
                qq = q[b * T:(b + 1) * T, cs]
                kk, vv = k[b * tk:b * tk + L, cs], v[b * tk:b * tk + L, cs]
                s = qq @ kk.T / math.sqrt(hd)
                p = np.exp(s - s.max(1, keepdims=True))
                o[b * T:(b + 1) * T, cs] = (p @ vv) / p.sum(1, keepdims=True)
        return o

    X = x.astype(np.float64).reshape(B * T, C)
    Cx = ctx.astype(np.float64).reshape(B * Tc, Cc)
    n = ln(X, w["norm1_w"], w["norm1_b"])
    a = attn(n @ deq("attn1_q", C, C).T, n @ deq("attn1_k", C, C).T, n @ deq("attn1_v", C, C).T, T, None)
    X = X + a @ deq("attn1_out", C, C).T + w["attn1_out_b"]
    n = ln(X, w["norm2_w"], w["norm2_b"])
    a = attn(n @ deq("attn2_q", C, C).T, Cx @ deq("attn2_k", C, Cc).T, Cx @ deq("attn2_v", C, Cc).T, Tc, kl)
    X = X + a @ deq("attn2_out", C, C).T + w["attn2_out_b"]
    n = ln(X, w["norm3_w"], w["norm3_b"])
    hh = n @ deq("ff_up", 2 * F, C).T + w["ff_up_b"]
    g = hh[:, :F] * (0.5 * hh[:, F:] * (1 + np.vectorize(math.erf)(hh[:, F:] / math.sqrt(2))))
    X = X + g @ deq("ff_down", C, F).T + w["ff_down_b"]
    delta_ref = X - x.reshape(B * T, C)
    delta = got - x.reshape(B * T, C)
    # fp32 restatement vs fp64 (relative to the RMS of the block's update)
    e = np.max(np.abs(delta - delta_ref)) / np.sqrt(np.mean(delta_ref ** 2))
    print(f"block oracle vs fp64: {e:.2e}")
    assert e <= 2e-5


# ------------------------------------------------------------------ NN GEMM --

def nn_numpy(payload, scales, B, M, N, K, lda=0, ldb=0, z=0, sA=0, sB=0):
    """float64 numpy: deq(A)[m, k] = int8(payload[fl]) * scales[fl >> 5], fl = z*sA + m*lda + k."""
    lda, ldb = lda or K, ldb or N
    fl = z * sA + np.arange(M)[:, None] * lda + np.arange(K)[None, :]
    A = payload.view(np.int8)[fl].astype(np.float64) * scales[fl >> 5].astype(np.float64)
    Bm = B[z * sB + np.arange(K)[:, None] * ldb + np.arange(N)[None, :]].astype(np.float64)
    return A @ Bm


def nn_inputs(oracle, M, N, K, seed, lda=0, ldb=0, batch=1, sA=0, sB=0):
    lda_e, ldb_e = lda or K, ldb or N
    na = (batch - 1) * sA + (M - 1) * lda_e + K
    nb = (batch - 1) * sB + (K - 1) * ldb_e + N
    payload = oracle.uniform_int(seed, -127, 127, na).astype(np.int8)
    scales = oracle.normal(seed + 1, (na + 31) // 32, 0.01, 0.004)
    B = oracle.normal(seed + 2, nb)
    return payload, scales, B


@pytest.mark.parametrize("M,N,K", [(1, 4, 4), (7, 12, 36), (64, 64, 64), (100, 68, 288), (33, 200, 96)])
def test_gemm_nn_oracle_vs_numpy(oracle, M, N, K):
    payload, scales, B = nn_inputs(oracle, M, N, K, 40)
    got = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K).reshape(M, N)
    want = nn_numpy(payload, scales, B, M, N, K)
    assert np.max(np.abs(got - want)) <= 1e-6 * max(1.0, np.max(np.abs(want)))
    f32 = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K, acc64=False).reshape(M, N)
    assert np.max(np.abs(f32 - want)) <= 1e-4 * max(1.0, np.max(np.abs(want)))


def test_gemm_nn_is_transposed_nt(oracle):
    """NN(W, B) = NT(B^T, W)^T: the same weight (split layout, rows of K with
    K % 32 == 0 so flat scale blocks are per row) through the pinned NT oracle."""
    M, N, K = 48, 40, 96
    payload, scales, B = nn_inputs(oracle, M, N, K, 50)
    nn = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K).reshape(M, N)
    Bt = np.ascontiguousarray(B.reshape(K, N).T).reshape(-1)
    nt = oracle.gemm_nt_q8_split(Bt, payload, scales, N, M, K).reshape(N, M)
    assert np.max(np.abs(nn - nt.T)) <= 1e-5 * np.max(np.abs(nn))


def test_gemm_nn_modes_batch_strides(oracle):
    """Batch z offsets A, B and C; lda / ldb / ldc padding (lda % 32 != 0, so a
    scale block straddles two rows); padding columns of C untouched; mode 1
    adds onto C."""
    M, N, K, batch = 20, 24, 40, 3
    lda, ldb, ldc = 44, 28, 30
    sA, sB, sC = M * lda + 12, K * ldb + 8, M * ldc + 5
    payload, scales, B = nn_inputs(oracle, M, N, K, 60, lda=lda, ldb=ldb, batch=batch, sA=sA, sB=sB)
    C0 = oracle.normal(63, (batch - 1) * sC + M * ldc)
    got = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K, C=C0.copy(), lda=lda, ldb=ldb, ldc=ldc, batch=batch,
                                  sA=sA, sB=sB, sC=sC)
    acc = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K, C=C0.copy(), mode=1, lda=lda, ldb=ldb, ldc=ldc,
                                  batch=batch, sA=sA, sB=sB, sC=sC)
    for z in range(batch):
        g = got[z * sC: z * sC + M * ldc].reshape(M, ldc)
        a = acc[z * sC: z * sC + M * ldc].reshape(M, ldc)
        c0 = C0[z * sC: z * sC + M * ldc].reshape(M, ldc)
        want = nn_numpy(payload, scales, B, M, N, K, lda=lda, ldb=ldb, z=z, sA=sA, sB=sB)
        assert np.max(np.abs(g[:, :N] - want)) <= 1e-5 * np.max(np.abs(want))
        assert np.array_equal(g[:, N:], c0[:, N:])
        assert np.max(np.abs(a[:, :N] - c0[:, :N] - want)) <= 1e-5 * np.max(np.abs(want)) + 1e-6
    assert np.array_equal(got[M * ldc: sC], C0[M * ldc: sC])


def test_gemm_nn_linearity(oracle):
    M, N, K = 16, 36, 64
    payload, scales, B1 = nn_inputs(oracle, M, N, K, 70)
    B2 = oracle.normal(74, K * N)
    c1 = oracle.gemm_nn_q8_split(payload, scales, B1, M, N, K)
    c2 = oracle.gemm_nn_q8_split(payload, scales, B2, M, N, K)
    c12 = oracle.gemm_nn_q8_split(payload, scales, (2.0 * B1 - 3.0 * B2).astype(np.float32), M, N, K)
    assert np.max(np.abs(c12 - (2.0 * c1 - 3.0 * c2))) <= 1e-5 * np.max(np.abs(c12))
