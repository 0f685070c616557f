"""GPU parity for the fused attention against the CPU oracle (fp64 online softmax,
tests/fused_attn_test.cpp:25-61 semantics).

Bar: max |O_gpu - O_ref| <= 2e-3 x RMS(O_ref) for fp32 outputs. fp16 outputs
add their own storage rounding (half an fp16 ulp of |O|), stated per element.
"""
from pathlib import Path

import numpy as np
import pytest

from helpers import REL_RMS_TOL, assert_parity, fp16_half_ulp, rms
from sdvk_amd import MI_ATTN_PREC_AUTO, MI_ATTN_PREC_FP16, MI_ATTN_PREC_SPLIT, MI_F16, MI_F32, ops
from sdvk_amd.hip import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"


def run_ref_api(q, k, v, Tq, Tk, C, heads, causal):
    """The reference call shape: fusedAttention on fp32 [T, C] buffers."""
    dq, dk, dv = (DeviceBuffer.from_array(x.astype(np.float32)) for x in (q, k, v))
    do = DeviceBuffer(max(Tq * C * 4, 4))
    ops.fused_attention(ops.FusedAttnArgs(dq, dk, dv, do, Tq, Tk, C, heads, causal))
    synchronize()
    return do.download(np.float32, Tq * C).reshape(Tq, C)


def run_ex(q, k, v, *, batch, Tq, Tk, C, heads, in_dtype, out_dtype, kv_len=None, causal=False, **kw):
    dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
    osz = 4 if out_dtype == MI_F32 else 2
    do = DeviceBuffer(batch * Tq * C * osz)
    dl = DeviceBuffer.from_array(np.asarray(kv_len, dtype=np.int32)) if kv_len is not None else None
    ops.fused_attention_ex(dq, dk, dv, do, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, causal=causal,
                           in_dtype=in_dtype, out_dtype=out_dtype, kv_len=dl, **kw)
    synchronize()
    return do.download(np.float32 if out_dtype == MI_F32 else np.float16, batch * Tq * C).reshape(batch, Tq, C)


def test_reference_test_shapes(gpu):
    """tests/fused_attn_test.cpp:74-79 (incl. hd = 40 and causal), fp32 API."""
    f = np.load(GOLDEN / "attn_ref_shapes.npz")
    for i in range(4):
        Tq, Tk, C, heads, causal = (int(x) for x in f[f"s{i}_shape"])
        print(f"[case] ref shape Tq={Tq} Tk={Tk} C={C} heads={heads} causal={causal}", flush=True)
        got = run_ref_api(f[f"s{i}_q"], f[f"s{i}_k"], f[f"s{i}_v"], Tq, Tk, C, heads, bool(causal))
        want = f[f"s{i}_o"].reshape(Tq, C)
        e = assert_parity(got, want, what=f"shape {i}")
        print(f"  err/rms = {e:.3e}", flush=True)


@pytest.mark.parametrize("Tq,Tk,C,heads,causal", [
    (100, 300, 128, 2, False), (100, 300, 128, 2, True), (257, 513, 640, 10, True), (1, 1, 64, 1, False),
    (300, 256, 320, 5, False), (129, 64, 1280, 20, True), (50, 1000, 40, 1, False)])
def test_fp32_api_tiled_sizes(gpu, oracle, Tq, Tk, C, heads, causal):
    """Tk >= 256 (the reference's tiled kernel, never numerically checked there)."""
    print(f"[case] fp32 Tq={Tq} Tk={Tk} C={C} heads={heads} causal={causal}", flush=True)
    q, k, v = oracle.normal(1, Tq * C), oracle.normal(2, Tk * C), oracle.normal(3, Tk * C)
    want = oracle.fused_attention(q, k, v, Tq, Tk, C, heads, causal).reshape(Tq, C)
    got = run_ref_api(q, k, v, Tq, Tk, C, heads, causal)
    assert_parity(got, want, what="fp32 api")


@pytest.mark.parametrize("Tq,Tk,C,heads", [(70, 90, 74, 2), (33, 40, 21, 3), (64, 100, 320, 8)])
def test_general_head_dims(gpu, oracle, Tq, Tk, C, heads):
    """hd not a multiple of 8 (scalar staging path) and hd = 40."""
    q, k, v = oracle.normal(4, Tq * C), oracle.normal(5, Tk * C), oracle.normal(6, Tk * C)
    want = oracle.fused_attention(q, k, v, Tq, Tk, C, heads, False).reshape(Tq, C)
    assert_parity(run_ref_api(q, k, v, Tq, Tk, C, heads, False), want, what=f"hd={C // heads}")


def test_special_cases(gpu, oracle):
    C, heads = 128, 2
    # Tk = 1: O = the V row (fp32 inputs travel as fp16 hi + lo: V to ~2^-22)
    q, k, v = oracle.normal(1, 5 * C), oracle.normal(2, C), oracle.normal(3, C)
    got = run_ref_api(q, k, v, 5, 1, C, heads, False)
    assert np.allclose(got, np.tile(v, (5, 1)), rtol=1e-6, atol=1e-7)
    # Tk = 0: no keys, O = 0 (the reference's l == 0 guard)
    got = run_ref_api(q, np.zeros(C, np.float32), np.zeros(C, np.float32), 5, 0, C, heads, False)
    assert np.all(got == 0)
    # kv_len = 0 for one batch item, full for the other
    batch, Tq, Tk = 2, 40, 77
    q = oracle.normal(4, batch * Tq * C).astype(np.float16)
    k = oracle.normal(5, batch * Tk * C).astype(np.float16)
    v = oracle.normal(6, batch * Tk * C).astype(np.float16)
    got = run_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=MI_F16, out_dtype=MI_F32,
                 kv_len=[0, 77])
    assert np.all(got[0] == 0)
    want = oracle.fused_attention_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=1,
                                     kv_len=np.array([0, 77], np.int32))
    assert_parity(got[1], want[1], what="kv_len full")


def test_outlier_key_in_either_lane_half(gpu, oracle):
    """One key per tile scores far above the others (s * log2(e) / 8 ~ 35
    above them): the running max must take both lane halves of a tile into
    account (keys 8j + 0..3 sit in one lane of a query, 8j + 4..7 in its
    partner), or exp2 of that key overflows fp16. Both halves, fp16 path."""
    B, Tq, Tk, C, heads = 1, 64, 192, 128, 2
    rng = np.random.default_rng(11)
    q = (rng.standard_normal(Tq * C) * 0.1 + 1.0).astype(np.float16)
    k = (rng.standard_normal((Tk, C)) * 0.1).astype(np.float16)
    v = rng.standard_normal(Tk * C).astype(np.float16)
    k[5] = 3.0      # tile 0: a key of the upper lane half
    k[64 + 2] = 3.0  # tile 1: a key of the lower lane half
    k[128 + 70 - 64] = 2.5
    k = k.reshape(-1)
    got = run_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=MI_F16, out_dtype=MI_F32)
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=1)
    assert_parity(got, want, what="outlier keys")


def _sample_rows(Tq, n, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, Tq - 1, 127, 128], rng.integers(0, Tq, n)])).astype(np.uint32)


@pytest.mark.parametrize("heads,T", [(10, 4096), (20, 1024)])
def test_config2_self_attention(gpu, oracle, heads, T):
    """batch 2, no mask, fp16 [B, T, H*64], scale 1/8."""
    print(f"[case] self-attn B=2 H={heads} T={T}", flush=True)
    B, C = 2, heads * 64
    q = oracle.normal(3, B * T * C).astype(np.float16)
    k = oracle.normal(4, B * T * C).astype(np.float16)
    v = oracle.normal(5, B * T * C).astype(np.float16)
    rows = _sample_rows(T, 40, heads)
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=T, Tk=T, C=C, heads=heads, in_dtype=1, rows=rows,
                                     threads=oracle.max_threads())
    got32 = run_ex(q, k, v, batch=B, Tq=T, Tk=T, C=C, heads=heads, in_dtype=MI_F16, out_dtype=MI_F32)
    e = assert_parity(got32[:, rows], want, what="fp16 in / fp32 out")
    got16 = run_ex(q, k, v, batch=B, Tq=T, Tk=T, C=C, heads=heads, in_dtype=MI_F16, out_dtype=MI_F16)
    g16 = got16[:, rows].astype(np.float64)
    bound = REL_RMS_TOL * rms(want) + fp16_half_ulp(want)
    assert np.all(np.abs(g16 - want) <= bound), "fp16 output beyond parity + storage rounding"
    print(f"  err/rms = {e:.3e} (fp32 out); fp16-out max err/rms = {np.abs(g16 - want).max() / rms(want):.3e}",
          flush=True)


@pytest.mark.parametrize("heads,T", [(10, 4096), (20, 1024)])
def test_config3_cross_attention(gpu, oracle, heads, T):
    """77 context tokens, key-padding lengths U{1..77} (seed 7)."""
    print(f"[case] cross-attn B=2 H={heads} T={T}", flush=True)
    B, C, Tk = 2, heads * 64, 77
    q = oracle.normal(3, B * T * C).astype(np.float16)
    k = oracle.normal(4, B * Tk * C).astype(np.float16)
    v = oracle.normal(5, B * Tk * C).astype(np.float16)
    kv_len = oracle.uniform_int(7, 1, 77, B)
    rows = _sample_rows(T, 60, heads + 1)
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=T, Tk=Tk, C=C, heads=heads, in_dtype=1,
                                     kv_len=kv_len, rows=rows, threads=oracle.max_threads())
    got = run_ex(q, k, v, batch=B, Tq=T, Tk=Tk, C=C, heads=heads, in_dtype=MI_F16, out_dtype=MI_F32,
                 kv_len=kv_len)
    e = assert_parity(got[:, rows], want, what="cross")
    print(f"  kv_len={kv_len.tolist()} err/rms = {e:.3e}", flush=True)


@pytest.mark.parametrize("nw", ["2", "4"])
@pytest.mark.parametrize("B,Tq,Tk,C,heads,causal,kv_len", [
    (2, 300, 1000, 128, 2, False, None),
    (2, 200, 300, 128, 2, True, None),
    (2, 130, 77, 640, 10, False, [77, 13]),
    (1, 1024, 1024, 1280, 20, False, None),
])
def test_two_and_four_wave_workgroups(gpu, oracle, tune, nw, B, Tq, Tk, C, heads, causal, kv_len):
    """The fp16 kernel's 64-query (2-wave) and 128-query (4-wave) workgroups,
    pinned with the attn_nw override, each against the oracle (the default rule takes
    4 waves unless Tq <= 64)."""
    print(f"[case] nw={nw} B={B} Tq={Tq} Tk={Tk} C={C} H={heads} causal={causal} kv_len={kv_len}", flush=True)
    tune("attn_nw", nw)
    q = oracle.normal(21, B * Tq * C).astype(np.float16)
    k = oracle.normal(22, B * Tk * C).astype(np.float16)
    v = oracle.normal(23, B * Tk * C).astype(np.float16)
    kl = np.asarray(kv_len, dtype=np.int32) if kv_len is not None else None
    rows = _sample_rows(Tq, 40, 5) if Tq > 512 else None
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=1, causal=causal,
                                     kv_len=kl, rows=rows, threads=oracle.max_threads())
    for out_dtype, prec in ((MI_F32, MI_ATTN_PREC_AUTO), (MI_F32, MI_ATTN_PREC_FP16), (MI_F16, MI_ATTN_PREC_AUTO)):
        got = run_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=MI_F16, out_dtype=out_dtype,
                     kv_len=kl, causal=causal, precision=prec)
        g = (got[:, rows] if rows is not None else got).astype(np.float64)
        w = want.reshape(g.shape)
        if out_dtype == MI_F32:
            # fp32 out: the default computes P in two parts (a tenth of the bar); one fp16 P product to the bar
            tol = REL_RMS_TOL / 10 if prec == MI_ATTN_PREC_AUTO else REL_RMS_TOL
            assert_parity(g, w, tol=tol, what=f"nw={nw} precision={prec}",
                          label="" if prec == MI_ATTN_PREC_AUTO else "[precision=fp16]")
        else:
            bound = REL_RMS_TOL * rms(w) + fp16_half_ulp(w)
            assert np.all(np.abs(g - w) <= bound), f"nw={nw}: fp16 output beyond parity + storage rounding"


@pytest.mark.parametrize("B,Tq,Tk,C,heads,kv_len,ws,odt", [
    (2, 4096, 77, 640, 10, [77, 40], False, MI_F16),
    (2, 4096, 4096, 640, 10, None, True, MI_F16),
    (2, 300, 1000, 128, 2, None, False, MI_F32),
    (1, 200, 130, 80, 2, [1], False, MI_F16),
    (2, 1024, 1024, 1280, 20, None, False, MI_F16),
])
def test_burst_build_equals_interleaved_build(gpu, oracle, tune, B, Tq, Tk, C, heads, kv_len, ws, odt):
    """The fp16 kernel's burst build (three waves per SIMD, the rule's choice
    for grids of more than two workgroups per CU) computes the interleaved
    build's bits: the same operations in the same order per tile. Pinned with
    attn_simd_waves on key padding, partial tiles, hd = 40, the key-split
    workspace entry and both output types; the interleaved result is checked
    against the oracle on sampled rows."""
    print(f"[case] burst vs interleaved B={B} Tq={Tq} Tk={Tk} C={C} H={heads} kv_len={kv_len} ws={ws}", flush=True)
    q = oracle.normal(31, B * Tq * C).astype(np.float16)
    k = oracle.normal(32, B * Tk * C).astype(np.float16)
    v = oracle.normal(33, B * Tk * C).astype(np.float16)
    kl = np.asarray(kv_len, dtype=np.int32) if kv_len is not None else None
    dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
    dl = DeviceBuffer.from_array(kl) if kl is not None else None
    kw = dict(batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=MI_F16, out_dtype=odt, kv_len=dl,
              precision=MI_ATTN_PREC_FP16)
    outs = []
    for waves in ("2", "3"):
        tune("attn_simd_waves", waves)
        do = DeviceBuffer(B * Tq * C * (2 if odt == MI_F16 else 4))
        n = ops.fused_attention_ws_bytes(**kw) if ws else 0
        ops.fused_attention_ws(dq, dk, dv, do, DeviceBuffer(n) if n else None, **kw)
        synchronize()
        outs.append(do.download(np.float16 if odt == MI_F16 else np.float32, B * Tq * C))
    assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8)), "burst build differs from interleaved"
    rows = _sample_rows(Tq, 24, 7) if Tq > 512 else None
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=1, kv_len=kl,
                                     rows=rows, threads=oracle.max_threads())
    g = outs[0].reshape(B, Tq, C).astype(np.float64)
    g = g[:, rows] if rows is not None else g
    w = want.reshape(g.shape)
    bound = REL_RMS_TOL * rms(w) + (fp16_half_ulp(w) if odt == MI_F16 else 0.0)
    assert np.all(np.abs(g - w) <= bound), "interleaved build beyond parity"


@pytest.mark.parametrize("B,H,T,Tk,causal,ws,prec", [(1, 20, 1024, 1024, False, False, MI_ATTN_PREC_AUTO),
                                                      (1, 20, 1024, 1024, False, False, MI_ATTN_PREC_SPLIT),
                                                      (2, 10, 4096, 4096, False, True, MI_ATTN_PREC_SPLIT),
                                                      (1, 8, 1024, 1024, True, False, MI_ATTN_PREC_AUTO),
                                                      (2, 4, 300, 77, False, False, MI_ATTN_PREC_SPLIT)])
def test_precise_mode(gpu, oracle, B, H, T, Tk, causal, ws, prec):
    """MI_ATTN_PREC_SPLIT (and MI_ATTN_PREC_AUTO with fp32 output, which
    picks it): P's fp16 residual as a second PV product on every tile, held to
    a tenth of the bar (sampled rows against the oracle), through the plain
    entry, the key-split workspace entry and the fp32 reference-layout entry
    (batch 1, whose fp32 output takes the same mode by default)."""
    print(f"[case] precise B={B} H={H} T={T} Tk={Tk} causal={causal} ws={ws} precision={prec}", flush=True)
    C = H * 64
    q = oracle.normal(21, B * T * C).astype(np.float16)
    k = oracle.normal(22, B * Tk * C).astype(np.float16)
    v = oracle.normal(23, B * Tk * C).astype(np.float16)
    rows = _sample_rows(T, 40, 7) if T > 512 else np.arange(T, dtype=np.uint32)
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=T, Tk=Tk, C=C, heads=H, causal=causal, in_dtype=1,
                                     rows=rows, threads=oracle.max_threads()).astype(np.float64)
    kw = dict(batch=B, Tq=T, Tk=Tk, C=C, heads=H, causal=causal, in_dtype=MI_F16, out_dtype=MI_F32, precision=prec)
    dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
    do = DeviceBuffer(B * T * C * 4)
    if ws:
        n = ops.fused_attention_ws_bytes(**kw)
        assert n > 0, "the shape has no key-split plan"
        ops.fused_attention_ws(dq, dk, dv, do, DeviceBuffer(n), **kw)
    else:
        ops.fused_attention_ex(dq, dk, dv, do, **kw)
    synchronize()
    got = do.download(np.float32, B * T * C).reshape(B, T, C)[:, rows].astype(np.float64)
    e = assert_parity(got, want, tol=REL_RMS_TOL / 10, what="precise")
    print(f"  err/rms = {e:.3e}", flush=True)
    if B == 1:
        got32 = run_ref_api(q, k, v, T, Tk, C, H, causal)[rows].astype(np.float64)
        e32 = assert_parity(got32, want.reshape(got32.shape), tol=REL_RMS_TOL / 10, what="precise, reference layout")
        print(f"  reference layout err/rms = {e32:.3e}", flush=True)


def test_strided_layouts_and_scale(gpu, oracle):
    """Token strides > C (e.g. fused QKV buffers), batch strides with gaps, custom scale."""
    B, Tq, Tk, C, heads = 2, 150, 200, 128, 2
    ldq, ldk, ldv = 3 * C, 3 * C, 3 * C
    sq, sk = Tq * ldq + 64, Tk * ldk + 64
    base = oracle.normal(9, B * max(sq, sk) + 3 * C).astype(np.float16)
    qv = base[: B * sq]
    kv = base[C: C + B * sk]
    vv = base[2 * C: 2 * C + B * sk]
    dq, dk, dv = DeviceBuffer.from_array(qv), DeviceBuffer.from_array(kv), DeviceBuffer.from_array(vv)
    do = DeviceBuffer(B * Tq * C * 4)
    scale = 0.07
    ops.fused_attention_ex(dq, dk, dv, do, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=MI_F16,
                           out_dtype=MI_F32, ldq=ldq, ldk=ldk, ldv=ldv, sq=sq, sk=sk, sv=sk, scale=scale)
    synchronize()
    got = do.download(np.float32, B * Tq * C).reshape(B, Tq, C)
    hd = C // heads
    for b in range(B):
        Q = qv[b * sq: b * sq + Tq * ldq].reshape(Tq, ldq)[:, :C].astype(np.float64)
        K = kv[b * sk: b * sk + Tk * ldk].reshape(Tk, ldk)[:, :C].astype(np.float64)
        V = vv[b * sk: b * sk + Tk * ldv].reshape(Tk, ldv)[:, :C].astype(np.float64)
        want = np.zeros((Tq, C))
        for h in range(heads):
            s = Q[:, h * hd:(h + 1) * hd] @ K[:, h * hd:(h + 1) * hd].T * np.float64(np.float32(scale))
            p = np.exp(s - s.max(1, keepdims=True))
            want[:, h * hd:(h + 1) * hd] = (p @ V[:, h * hd:(h + 1) * hd]) / p.sum(1, keepdims=True)
        assert_parity(got[b], want, what=f"strided b={b}")


@pytest.mark.parametrize("C,heads", [(128, 2), (80, 2)])
def test_staged_and_direct_output_stores_agree(gpu, oracle, tune, C, heads):
    """Output rows go through LDS (16-byte stores of whole rows) when the rows and head columns are 16-byte
    aligned, else straight from the MFMA layout: both give the same bits, in both kernels (fp16 and fp32
    inputs), for both output types, with a partial last row block and key padding. The attn_direct_store override
    forces the direct stores; an output 8 bytes off 16-byte alignment takes them by itself (fp16)."""
    B, Tq, Tk = 2, 130, 150
    kv_len = np.array([150, 61], dtype=np.int32)
    dl = DeviceBuffer.from_array(kv_len)
    for in_dtype, idt in ((MI_F16, np.float16), (MI_F32, np.float32)):
        q = oracle.normal(21, B * Tq * C).astype(idt)
        k = oracle.normal(22, B * Tk * C).astype(idt)
        v = oracle.normal(23, B * Tk * C).astype(idt)
        dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
        for out_dtype, odt in ((MI_F16, np.float16), (MI_F32, np.float32)):
            n = B * Tq * C
            do = DeviceBuffer(n * odt().itemsize + 16)
            outs = []
            for direct, off in ((False, 0), (True, 0), (False, 8)):
                if off and odt is np.float32:
                    continue
                print(f"[case] C={C} in={in_dtype} out={out_dtype} direct={direct} offset={off}", flush=True)
                if direct:
                    tune("attn_direct_store", "1")
                else:
                    tune("attn_direct_store", None)
                ops.fused_attention_ex(dq, dk, dv, do.value + off, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads,
                                       in_dtype=in_dtype, out_dtype=out_dtype, kv_len=dl)
                synchronize()
                outs.append(do.download(odt, n, offset=off))
            tune("attn_direct_store", None)
            for o in outs[1:]:
                assert np.array_equal(o.view(np.uint8), outs[0].view(np.uint8)), "staged and direct stores differ"
            want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads,
                                             in_dtype=oracle.OR_F16 if in_dtype == MI_F16 else oracle.OR_F32,
                                             kv_len=kv_len).reshape(-1).astype(np.float64)
            got = outs[0].astype(np.float64)
            if odt is np.float16:
                assert np.all(np.abs(got - want) <= REL_RMS_TOL * rms(want) + fp16_half_ulp(want))
            else:
                assert_parity(got, want, what="staged store")


def test_key_split_workspace_entry(gpu, oracle, tune):
    """mi_fused_attention_ws: the key-split plan of the last partial round of query blocks (2 x 10 heads x
    4096, 640 blocks against 512 resident: 128 blocks in 2 key ranges, one per CU) against the oracle on
    sampled rows, its repeat bit for bit, and agreement with mi_fused_attention_ex; a workspace below the
    plan's size (and none) runs mi_fused_attention_ex's plan exactly; the 4-range plan of 2 x 9 heads;
    forced plans on small shapes (uneven pieces, partial query block, hd = 40) against the oracle."""
    tune("attn_split", None)
    B, H, T = 2, 10, 4096
    C = H * 64
    kw = dict(batch=B, Tq=T, Tk=T, C=C, heads=H, in_dtype=MI_F16, out_dtype=MI_F16)
    nws = ops.fused_attention_ws_bytes(**kw)
    assert nws == 128 * 2 * (128 * 64 + 2 * 128) * 4, nws
    q, k, v = (oracle.normal(31 + i, B * T * C).astype(np.float16) for i in range(3))
    dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
    ws = DeviceBuffer(nws)
    outs = []
    for w in (ws, ws, None, DeviceBuffer(nws - 16)):
        print(f"[case] key split workspace {w.nbytes if w is not None else 0} B", flush=True)
        do = DeviceBuffer(B * T * C * 2)
        ops.fused_attention_ws(dq, dk, dv, do, w, **kw)
        synchronize()
        outs.append(do.download(np.float16, B * T * C))
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16)), "split plan does not repeat"
    assert np.array_equal(outs[2].view(np.uint16), outs[3].view(np.uint16)), "small workspace changed the plan"
    # the split blocks are the grid's last 128 (b = 1, heads 6..9): sample rows of both halves
    rows = np.unique(np.concatenate([np.arange(0, T, 151), np.arange(T - 40, T)])).astype(np.uint32)
    want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=T, Tk=T, C=C, heads=H, in_dtype=oracle.OR_F16,
                                     rows=rows, threads=oracle.max_threads()).astype(np.float64)
    for o in (outs[0], outs[2]):
        got = o.reshape(B, T, C)[:, rows].astype(np.float64)
        assert np.all(np.abs(got - want) <= REL_RMS_TOL * rms(want) + fp16_half_ulp(want))
    # everywhere (not only the sampled rows): split and unsplit each within the bar of the exact result
    a0, a2 = outs[0].astype(np.float64), outs[2].astype(np.float64)
    d = np.abs(a0 - a2)
    print(f"  split vs unsplit max |diff| / RMS = {d.max() / rms(want):.2e}", flush=True)
    assert np.all(d <= 2 * REL_RMS_TOL * rms(want) + 2 * fp16_half_ulp(np.maximum(np.abs(a0), np.abs(a2))))
    # 2 x 9 heads: 576 blocks, the last 64 in 4 key ranges
    H9 = 9
    kw9 = dict(batch=B, Tq=T, Tk=T, C=H9 * 64, heads=H9, in_dtype=MI_F16, out_dtype=MI_F32)
    n9 = ops.fused_attention_ws_bytes(**kw9)
    assert n9 == 64 * 4 * (128 * 64 + 2 * 128) * 4, n9
    print("[case] key split 2 x 9 heads, 4 ranges", flush=True)
    q9, k9, v9 = (oracle.normal(41 + i, B * T * H9 * 64).astype(np.float16) for i in range(3))
    d9 = [DeviceBuffer.from_array(x) for x in (q9, k9, v9)]
    o9 = DeviceBuffer(B * T * H9 * 64 * 4)
    ops.fused_attention_ws(*d9, o9, DeviceBuffer(n9), **kw9)
    synchronize()
    got9 = o9.download(np.float32, B * T * H9 * 64).reshape(B, T, H9 * 64)[:, rows].astype(np.float64)
    want9 = oracle.fused_attention_ex(q9, k9, v9, batch=B, Tq=T, Tk=T, C=H9 * 64, heads=H9, in_dtype=oracle.OR_F16,
                                      rows=rows, threads=oracle.max_threads()).astype(np.float64)
    assert_parity(got9, want9, what="2 x 9 heads key split")
    for (B, Tq, Tk, C, heads, split, odt) in [(2, 300, 1000, 128, 2, "3:3", MI_F32), (1, 200, 130, 80, 2, "1:2", MI_F32),
                                             (1, 256, 512, 128, 2, "2:4", MI_F16)]:
        print(f"[case] forced split {split} B={B} Tq={Tq} Tk={Tk} C={C} heads={heads}", flush=True)
        tune("attn_split", split)
        tune("attn_nw", "4")
        kw = dict(batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=MI_F16, out_dtype=odt)
        nws = ops.fused_attention_ws_bytes(**kw)
        assert nws > 0
        q, k, v = (oracle.normal(41 + i, B * n * C).astype(np.float16) for i, n in enumerate((Tq, Tk, Tk)))
        dq, dk, dv = (DeviceBuffer.from_array(x) for x in (q, k, v))
        osz = 4 if odt == MI_F32 else 2
        do = DeviceBuffer(B * Tq * C * osz)
        ops.fused_attention_ws(dq, dk, dv, do, DeviceBuffer(nws), **kw)
        synchronize()
        got = do.download(np.float32 if odt == MI_F32 else np.float16, B * Tq * C).astype(np.float64)
        want = oracle.fused_attention_ex(q, k, v, batch=B, Tq=Tq, Tk=Tk, C=C, heads=heads,
                                         in_dtype=oracle.OR_F16).reshape(-1).astype(np.float64)
        if odt == MI_F32:
            assert_parity(got, want, what=f"forced split {split}")
        else:
            assert np.all(np.abs(got - want) <= REL_RMS_TOL * rms(want) + fp16_half_ulp(want))
    tune("attn_split", None)
    tune("attn_nw", None)
