"""Cases run on the kernel emulator, one child process per case (a fault in
an emulated kernel ends that process with the emulator's report, not the
test session).

    python tests/kemu/cases.py '<json: {"case": name, ...params}>'

Each case calls the emulation build of the C-ABI on guarded buffers and
compares with the CPU oracle to the same bar as the GPU parity tests; it
also checks that nothing outside the logical output changed (padding
columns, batch gaps). Test infrastructure only.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))     # tests/ (helpers)
sys.path.insert(0, str(HERE))

import ctypes  # noqa: E402

import emu as kemu  # noqa: E402
from helpers import assert_parity, fp16_half_ulp, q8_weights, rms  # noqa: E402
from oracle import binding as ob  # noqa: E402
from sdvk_amd._lib import (MI_ATTN_PREC_FP16, MI_ATTN_PREC_SPLIT, MI_BLOCK_FP16_ACTIVATIONS,  # noqa: E402
                           MI_BLOCK_FP16_ATTENTION,
                           MI_BLOCK_FUSED_EPILOGUES, MI_BLOCK_JOINT_QKV, MI_F16, MI_F32, MiAttnArgs, MiBlockDims,
                           MiBlockWeights)
from test_gpu_block import BLOCK_TOL, make_weights  # noqa: E402
import gguf_writer as gw  # noqa: E402
from sdvk_amd._lib import MiGgufTensorInfo  # noqa: E402

SENTINEL = np.float32(12345.0)


_EMU = None


def _tune(name, value):
    """mi_tuning_set on the emulation build (value None clears the override)."""
    st = _EMU.lib.mi_tuning_set(name.encode(), None if value is None else str(value).encode())
    assert st == 0, f"mi_tuning_set({name}, {value}): status {st}"


def _set_cfg(cfg):
    _tune("gemm_cfg", cfg)


def _logical_mask(M, N, ldc, batch, sC, size):
    mask = np.zeros(size, dtype=bool)
    for z in range(batch):
        for m in range(M):
            s = z * sC + m * ldc
            mask[s:s + N] = True
    return mask


def _workspace(E, nbytes, front):
    """(pointer, bytes) of a guarded workspace filled with NaN, or (None, 0)."""
    if not nbytes:
        return None, 0, None
    b = E.buf(nbytes=nbytes, front=front).fill(0xFF)
    return b.ptr, nbytes, b


def gemm_nt(E, *, M, N, K, layout="q8_0", cfg=None, mode=0, bias=True, batch=1, lda=0, ldc=0, sA=0, sC=0,
            seed=1, front=False, order=0, tol=2e-3, bias_off=0, ws=True, a_off=0):
    """mi_gemm_nt_q8_0[_ws] / mi_gemm_nt_q8_split[_ws] against the oracle;
    bias_off shifts the bias pointer by that many floats (an unaligned bias),
    a_off the A pointer (an A that is only 4-byte aligned); ws: through the
    workspace entry with the workspace the library asks for (K splits)."""
    _set_cfg(cfg)
    E.order(order)
    lda_e, ldc_e = lda or K, ldc or N
    a_el = (batch - 1) * sA + (M - 1) * lda_e + K
    c_el = (batch - 1) * sC + (M - 1) * ldc_e + N
    A = ob.normal(seed, a_el)
    if K % 32:  # split layout only: int8 values and flat-index scales drawn directly
        assert layout == "split", "the 34-byte block layout needs K % 32 == 0"
        blocks = None
        q = ob.uniform_int(seed + 1, -127, 127, N * K).astype(np.int8)
        payload = np.concatenate([q, np.zeros((-q.size) % 4, np.int8)]).view(np.uint32)
        scales = ob.normal(seed + 4, (N * K + 31) // 32, 0.01, 0.002)
    else:
        blocks = q8_weights(ob, seed + 1, N, K)
    b = ob.normal(seed + 2, N, 0.0, 0.02) if bias else None
    C0 = ob.normal(seed + 3, c_el) if mode in (1, 2) else np.full(c_el, SENTINEL, dtype=np.float32)
    dA, dC = E.buf(np.concatenate([np.zeros(a_off, np.float32), A]), front=front), E.buf(C0, front=front)
    dA.ptr += 4 * a_off
    dB = E.buf(np.concatenate([np.zeros(bias_off, np.float32), b]), front=front) if bias else None
    if dB is not None and bias_off:
        dB.ptr += 4 * bias_off
    # mode 2 (C += acc + bias) = C0 + the mode-0 product with bias
    omode, oC = (0, np.zeros_like(C0)) if mode == 2 else (mode, C0.copy())
    wsp, wsn, _keep = _workspace(E, E.lib.mi_gemm_nt_q8_workspace_bytes(M, N, K, batch) if ws else 0, front)
    sfx, extra = ("_ws", (wsp, wsn)) if ws else ("", ())
    if layout == "q8_0":
        dW = E.buf(blocks, front=front)
        E.call("mi_gemm_nt_q8_0" + sfx, dA.ptr, dW.ptr, dB.ptr if dB else None, dC.ptr, M, N, K, mode, lda, ldc,
               batch, sA, sC, *extra, None)
        want = ob.gemm_nt_q8_0(A, blocks, M, N, K, bias=b, C=oC, mode=omode, lda=lda, ldc=ldc, batch=batch,
                               sA=sA, sC=sC, threads=ob.max_threads())
    else:
        if blocks is not None:
            payload, scales = ob.q8_0_to_split(blocks, N * K)
        dP, dS = E.buf(payload, front=front), E.buf(scales, front=front)
        E.call("mi_gemm_nt_q8_split" + sfx, dA.ptr, dP.ptr, dS.ptr, dB.ptr if dB else None, dC.ptr, M, N, K, mode,
               lda, ldc, batch, sA, sC, *extra, None)
        want = ob.gemm_nt_q8_split(A, payload, scales, M, N, K, bias=b, C=oC, mode=omode, lda=lda, ldc=ldc,
                                   batch=batch, sA=sA, sC=sC, threads=ob.max_threads())
    if mode == 2:
        want = want + C0
    got = dC.get(np.float32, c_el)
    mask = _logical_mask(M, N, ldc_e, batch, sC, c_el)
    assert np.array_equal(got[~mask], C0[~mask]), "elements outside the logical output changed"
    if mode in (1, 2):
        return assert_parity(got[mask] - C0[mask], want[mask] - C0[mask], tol=tol, what=f"gemm_nt mode {mode}")
    return assert_parity(got[mask], want[mask], tol=tol, what="gemm_nt")


def gemm_geglu(E, *, M, F, K, cfg=None, bias=True, lda=0, ldg=0, seed=1, front=False, order=0, tol=2e-3):
    """mi_gemm_nt_q8_0_geglu: against the separate path on the same build
    (mi_gemm_nt_q8_0 into [M, 2F], then mi_geglu) to fp32 rounding, and
    against the oracle's GEMM + GEGLU."""
    _set_cfg(cfg)
    E.order(order)
    lda_e, ldg_e = lda or K, ldg or F
    a_el, g_el = (M - 1) * lda_e + K, (M - 1) * ldg_e + F
    A = ob.normal(seed, a_el)
    blocks = q8_weights(ob, seed + 1, 2 * F, K)
    b = ob.normal(seed + 2, 2 * F, 0.0, 0.5) if bias else None
    dA, dW = E.buf(A, front=front), E.buf(blocks, front=front)
    dB = E.buf(b, front=front) if bias else None
    dG = E.buf(np.full(g_el, SENTINEL, np.float32), front=front)
    E.call("mi_gemm_nt_q8_0_geglu", dA.ptr, dW.ptr, dB.ptr if dB else None, dG.ptr, M, F, K, lda, ldg, None)
    got = dG.get(np.float32, g_el)
    mask = _logical_mask(M, F, ldg_e, 1, 0, g_el)
    assert np.array_equal(got[~mask], np.full((~mask).sum(), SENTINEL, np.float32)), "padding of G changed"
    got = got[mask].reshape(M, F)
    # separate path on the same build: same MFMA sums (no K split), fp32 epilogue arithmetic
    _tune("gemm_cfg", cfg.split(":")[0] if cfg else None)
    dH, dY = E.buf(nbytes=M * 2 * F * 4), E.buf(nbytes=M * F * 4)
    E.call("mi_gemm_nt_q8_0", dA.ptr, dW.ptr, dB.ptr if dB else None, dH.ptr, M, 2 * F, K, 0, lda, 0, 1, 0, 0, None)
    E.call("mi_geglu", dH.ptr, dY.ptr, M, F, None)
    sep = dY.get(np.float32, M * F).reshape(M, F)
    d_sep = float(np.max(np.abs(got - sep)) / max(rms(sep), 1e-30))
    h = ob.gemm_nt_q8_0(A, blocks, M, 2 * F, K, bias=b, lda=lda, threads=ob.max_threads())
    want = ob.geglu(h, M, F).reshape(M, F)
    # GEGLU multiplies two GEMM outputs: the GEMM bar (tol x RMS(h) on v and g)
    # propagates to |dG| <= tol RMS(h) (|gelu(g)| + |v gelu'(g)|) per element
    h2 = h.reshape(M, 2 * F).astype(np.float64)
    v, g = h2[:, :F], h2[:, F:]
    from math import erf as _erf
    cdf = 0.5 * (1.0 + np.vectorize(_erf)(g / np.sqrt(2.0)))
    dgelu = cdf + g * np.exp(-0.5 * g * g) / np.sqrt(2.0 * np.pi)
    bound = tol * rms(h2) * (np.abs(g * cdf) + np.abs(v * dgelu)) + 1e-6 * np.abs(want)
    assert np.all(np.isfinite(got)), "gemm_geglu: non-finite output"
    worst = float(np.max(np.abs(got - want) / bound))
    assert worst <= 1.0, f"gemm_geglu: error {worst:.2f} x the propagated GEMM bound"
    e = float(np.max(np.abs(got - want)) / rms(want))
    if cfg is None or ":" not in cfg:  # no K split in the separate path: same sums
        assert d_sep <= 2e-6, f"fused vs separate GEGLU: {d_sep:.3e} x RMS"
    return e


def gemm_nn(E, *, M, N, K, mode=0, batch=1, lda=0, ldb=0, ldc=0, sA=0, sB=0, sC=0, seed=1, front=False,
            order=0, tol=2e-3, kernel=None, ws=True):
    """mi_gemm_nn_q8_split against the oracle (flat-index scales). kernel="general"
    forces the untiled kernel (the nn_kernel override) on shapes the tiled one would take."""
    E.order(order)
    _tune("nn_kernel", kernel or None)
    lda_e, ldb_e, ldc_e = lda or K, ldb or N, ldc or N
    a_el = (batch - 1) * sA + (M - 1) * lda_e + K
    b_el = (batch - 1) * sB + (K - 1) * ldb_e + N if K else N
    c_el = (batch - 1) * sC + (M - 1) * ldc_e + N
    n_a = (a_el + 31) // 32 * 32
    w = ob.normal(seed, n_a, 0.0, 0.02)
    payload, scales = ob.q8_0_to_split(ob.q8_0_quantize(w), n_a)
    payload = payload.view(np.uint8)[:a_el]
    payload = np.concatenate([payload, np.zeros((-a_el) % 4, np.uint8)]).view(np.uint32)
    scales = scales[: (a_el + 31) // 32]
    B = ob.normal(seed + 1, b_el)
    C0 = ob.normal(seed + 3, c_el) if mode == 1 else np.full(c_el, SENTINEL, dtype=np.float32)
    dP, dS, dB, dC = (E.buf(payload, front=front), E.buf(scales, front=front), E.buf(B, front=front),
                      E.buf(C0, front=front))
    wsp, wsn, _keep = _workspace(E, E.lib.mi_gemm_nn_q8_workspace_bytes(M, N, K, batch) if ws else 0, front)
    sfx, extra = ("_ws", (wsp, wsn)) if ws else ("", ())
    E.call("mi_gemm_nn_q8_split" + sfx, dP.ptr, dS.ptr, dB.ptr, dC.ptr, M, N, K, mode, lda, ldb, ldc, batch, sA, sB,
           sC, *extra, None)
    want = ob.gemm_nn_q8_split(payload, scales, B, M, N, K, C=C0.copy(), mode=mode, lda=lda, ldb=ldb, ldc=ldc,
                               batch=batch, sA=sA, sB=sB, sC=sC, threads=ob.max_threads())
    got = dC.get(np.float32, c_el)
    mask = _logical_mask(M, N, ldc_e, batch, sC, c_el)
    assert np.array_equal(got[~mask], C0[~mask]), "elements outside the logical output changed"
    if mode == 1:
        return assert_parity(got[mask] - C0[mask], want[mask] - C0[mask], tol=tol, what="gemm_nn mode 1")
    return assert_parity(got[mask], want[mask], tol=tol, what="gemm_nn")


def attention(E, *, batch=1, Tq, Tk, C, heads, causal=False, f16_in=False, f16_out=False, kv_len=None, seed=1,
              front=False, order=0, tol=2e-3, nw=None, outliers=None, direct_store=False, split=None,
              precise=False, precision=None, simd_waves=None):
    """mi_fused_attention_ex (contiguous [batch, T, C]) against the oracle;
    split "<rest>:<pieces>": through mi_fused_attention_ws with that key-split
    plan forced (the attn_split override) and the workspace the library asks
    for; nw pins the fp16 kernel's workgroup size (attn_nw); outliers: key
    indices whose scores stand far above the rest (q ~ 1, k ~ 0.1 N(0, 1),
    those keys 3.0), so that a running max that misses them overflows;
    direct_store: output stores straight from the MFMA layout
    (attn_direct_store) instead of whole rows through LDS; precision: the
    mi_attn_args field, by default MI_ATTN_PREC_FP16 (one fp16 P product);
    precise: MI_ATTN_PREC_SPLIT (P's fp16 residual as a second PV product on
    every tile); simd_waves "2" | "3": the interleaved or the burst build of
    the fp16 kernel (attn_simd_waves)."""
    E.order(order)
    _tune("attn_nw", nw)
    _tune("attn_simd_waves", simd_waves)
    _tune("attn_direct_store", "1" if direct_store else None)
    _tune("attn_split", split)
    if precision is None:
        precision = MI_ATTN_PREC_SPLIT if precise else MI_ATTN_PREC_FP16
    idt = np.float16 if f16_in else np.float32
    q = ob.normal(seed, batch * Tq * C).astype(idt)
    k = ob.normal(seed + 1, batch * Tk * C).astype(idt)
    v = ob.normal(seed + 2, batch * Tk * C).astype(idt)
    if outliers:
        q = (q.astype(np.float32) * np.float32(0.1) + np.float32(1.0)).astype(idt)
        kk = (k.astype(np.float32) * np.float32(0.1)).reshape(batch, Tk, C)
        kk[:, outliers, :] = 3.0
        k = kk.reshape(-1).astype(idt)
    odt = np.float16 if f16_out else np.float32
    n_out = batch * Tq * C
    dq, dk, dv = E.buf(q, front=front), E.buf(k, front=front), E.buf(v, front=front)
    do = E.buf(np.full(n_out, 7.0, dtype=odt), front=front)
    dl = E.buf(np.asarray(kv_len, dtype=np.int32), front=front) if kv_len is not None else None
    x = MiAttnArgs(q=dq.ptr, k=dk.ptr, v=dv.ptr, out=do.ptr, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads,
                   causal=1 if causal else 0, in_dtype=MI_F16 if f16_in else MI_F32,
                   out_dtype=MI_F16 if f16_out else MI_F32, kv_len=dl.ptr if dl else None, precision=precision)
    if split:
        nws = E.lib.mi_fused_attention_ws_bytes(ctypes.byref(x))
        assert nws > 0, f"attention: split {split} planned no workspace"
        dws = E.buf(nbytes=nws, front=front).fill(0xFF)  # NaN bytes: every partial read must have been written
        E.call("mi_fused_attention_ws", ctypes.byref(x), dws.ptr, nws, None)
        _tune("attn_split", None)
    else:
        E.call("mi_fused_attention_ex", ctypes.byref(x), None)
    got = do.get(odt, n_out).astype(np.float64)
    want = ob.fused_attention_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, causal=causal,
                                 in_dtype=ob.OR_F16 if f16_in else ob.OR_F32, out_dtype=ob.OR_F32, kv_len=kv_len,
                                 threads=ob.max_threads()).reshape(-1).astype(np.float64)
    assert np.all(np.isfinite(got)), "attention: non-finite output"
    if f16_out:
        bound = tol * rms(want) + fp16_half_ulp(want)
        assert np.all(np.abs(got - want) <= bound), "attention: fp16 output beyond tol x RMS + half an ulp"
        return float(np.max(np.abs(got - want)) / rms(want))
    return assert_parity(got, want, tol=tol, what="attention")


# ---- full-size shapes with sampled workgroups ----------------------------------
# The benchmark's shapes at their real size, with only a few workgroups
# emulated (kemu_set_sample): the first one and the one that takes the last
# tile in the kernel's order (the bottom-right corner), with every K split and
# batch of those tiles. Inputs are the full tensors on guarded buffers, so the
# grids, tile counts, split choices and offsets are those of the GPU run;
# every element the sampled workgroups wrote is compared with the oracle's
# rows, and the written region must consist of whole 32-aligned MFMA tiles.

def _block_of_tile(t: int, nb: int) -> int:
    """blockIdx.x that the kernels' XCD swizzle (8 contiguous chunks of the
    tile order, chunk i on blockIdx.x % 8 == i) maps to linear tile t."""
    per, rem = divmod(nb, 8)
    if t < rem * (per + 1):
        xcd, local = divmod(t, per + 1)
    else:
        xcd, local = rem + (t - rem * (per + 1)) // per, (t - rem * (per + 1)) % per
    return local * 8 + xcd


def _probe_grid(E, spec_none: str, call) -> tuple[str, tuple[int, int, int]]:
    """Launches with no workgroup emulated and returns the main launch's grid."""
    E.sample(spec_none)
    call()
    return E.last_launch()


def _whole_tiles(mask: np.ndarray, what: str) -> None:
    """Runs of written elements along rows and along columns start at a
    multiple of 32 and span a multiple of 32 unless they end at the edge."""
    for m in (mask, mask.T):
        pad = np.zeros((m.shape[0], 1), dtype=np.int8)
        d = np.diff(np.concatenate([pad, m.astype(np.int8), pad], axis=1), axis=1)
        _, s = np.nonzero(d == 1)
        _, e = np.nonzero(d == -1)
        bad = (s % 32 != 0) | (((e - s) % 32 != 0) & (e != m.shape[1]))
        assert not bad.any(), f"{what}: written region is not whole 32-aligned tiles ({int(bad.sum())} runs)"


def gemm_full(E, *, M, N, K, cfg=None, layout="q8_0", seed=1, order=0, tol=2e-3, ws=True):
    """mi_gemm_nt_q8_0[_ws] / _split[_ws] at a full benchmark shape, sampled
    workgroups (with ws: the K-split plan the benchmark runs; the reduce pass
    runs whole over a zeroed workspace, so unsampled tiles read back as 0)."""
    _set_cfg(cfg)
    E.order(order)
    A = ob.normal(seed, M * K)
    blocks = q8_weights(ob, seed + 1, N, K)
    dA, dC = E.buf(A), E.buf(np.zeros(M * N, np.float32))
    nws = E.lib.mi_gemm_nt_q8_workspace_bytes(M, N, K, 1) if ws else 0
    dws = E.buf(nbytes=nws).fill(0) if nws else None
    sfx, extra = ("_ws", (dws.ptr if dws else None, nws)) if ws else ("", ())
    if layout == "q8_0":
        dW = E.buf(blocks)
        call = lambda: E.call("mi_gemm_nt_q8_0" + sfx, dA.ptr, dW.ptr, None, dC.ptr, M, N, K, 0, 0, 0, 1, 0, 0,
                              *extra, None)
    else:
        payload, scales = ob.q8_0_to_split(blocks, N * K)
        dP, dS = E.buf(payload), E.buf(scales)
        call = lambda: E.call("mi_gemm_nt_q8_split" + sfx, dA.ptr, dP.ptr, dS.ptr, None, dC.ptr, M, N, K, 0, 0, 0, 1,
                              0, 0, *extra, None)
    helpers = "gemm_fill|-|-|-;splitk_reduce|-|-|-"  # the K == 0 fill and the split reduce pass
    kern, grid = _probe_grid(E, f"gemm_q8_kernel|-|-|-;{helpers}", call)
    assert not np.any(dC.get(np.float32, M * N)), "a launch with no workgroup wrote C"
    xs = sorted({0, _block_of_tile(grid[0] - 1, grid[0])})
    x = ",".join(map(str, xs))
    print(f"  {kern} grid {grid}, blockIdx.x {xs}", flush=True)
    E.sample(f"gemm_q8_kernel|{x}|*|*;gemm_fill|-|-|-")
    before = E.lib.kemu_blocks_run()
    call()
    ran = E.lib.kemu_blocks_run() - before
    # a split plan's reduce pass runs whole: a capped grid over the [M, N / 4] units
    reduce = min(max(-(-(M * N // 4) // 256), 1), 1024) if grid[1] > 1 else 0
    assert ran == len(xs) * grid[1] * grid[2] + reduce, \
        f"{ran} workgroups ran, expected {len(xs)} x {grid[1]} x {grid[2]} + {reduce} (reduce)"
    got = dC.get(np.float32, M * N).reshape(M, N)
    mask = got != 0
    assert mask.any(), "the sampled workgroups wrote nothing"
    _whole_tiles(mask, f"gemm {kern} {grid}")
    rows = np.flatnonzero(mask.any(axis=1))
    want = ob.gemm_rows(A, blocks, M, N, K, rows, threads=ob.max_threads())
    sub = mask[rows]
    e = assert_parity(got[rows][sub], want[sub], tol=tol, what=f"gemm full {kern} grid {grid}")
    # the corner tile is among those written
    assert mask[M - 1, N - 1], "the bottom-right tile was not sampled"
    return e


def gemm_nn_full(E, *, M, N, K, seed=1, order=0, tol=2e-3):
    """mi_gemm_nn_q8_split at a full SDXL conv shape, sampled workgroups (the
    first and last column tiles of the last row tile, every K split)."""
    E.order(order)
    _tune("nn_kernel", None)
    w = ob.normal(seed, M * K, 0.0, 0.02)
    payload, scales = ob.q8_0_to_split(ob.q8_0_quantize(w), M * K)
    B = ob.normal(seed + 1, K * N)
    dP, dS, dB, dC = E.buf(payload), E.buf(scales), E.buf(B), E.buf(np.zeros(M * N, np.float32))
    nws = E.lib.mi_gemm_nn_q8_workspace_bytes(M, N, K, 1)
    dws = E.buf(nbytes=nws).fill(0) if nws else None
    call = lambda: E.call("mi_gemm_nn_q8_split_ws", dP.ptr, dS.ptr, dB.ptr, dC.ptr, M, N, K, 0, 0, 0, 0, 1, 0, 0, 0,
                          dws.ptr if dws else None, nws, None)
    kern, grid = _probe_grid(E, "gemm_nn_q8_tiled_kernel|-|-|-;gemm_nn_q8_kernel|-|-|-;splitk_reduce|-|-|-",
                             call)
    print(f"  {kern} grid {grid}", flush=True)
    E.sample("gemm_nn_q8_tiled_kernel|0,-1|-1|*;gemm_nn_q8_kernel|0,-1|-1|*")
    call()
    got = dC.get(np.float32, M * N).reshape(M, N)
    mask = got != 0
    assert mask.any() and mask[M - 1, N - 1], "the sampled workgroups did not write the corner tile"
    _whole_tiles(mask, f"gemm_nn {kern} {grid}")
    rows = np.flatnonzero(mask.any(axis=1))
    want = ob.gemm_nn_q8_split(payload.reshape(M, -1)[rows].reshape(-1), scales.reshape(M, -1)[rows].reshape(-1),
                               B, len(rows), N, K, threads=ob.max_threads()).reshape(len(rows), N)
    sub = mask[rows]
    return assert_parity(got[rows][sub], want[sub], tol=tol, what=f"gemm_nn full {kern} grid {grid}")


def attention_full(E, *, batch, Tq, Tk, C, heads, masked=False, nw=None, seed=1, order=0, tol=2e-3,
                   simd_waves=None):
    """fp16 mi_fused_attention_ex at a full benchmark shape, sampled workgroups
    (the first and the last in the kernel's order)."""
    E.order(order)
    _tune("attn_nw", nw)
    _tune("attn_simd_waves", simd_waves)
    _tune("attn_direct_store", None)
    q = ob.normal(seed, batch * Tq * C).astype(np.float16)
    k = ob.normal(seed + 1, batch * Tk * C).astype(np.float16)
    v = ob.normal(seed + 2, batch * Tk * C).astype(np.float16)
    kv_len = ob.uniform_int(seed + 6, 1, Tk, batch).astype(np.int32) if masked else None
    sentinel = np.float16(7.0)
    dq, dk, dv = E.buf(q), E.buf(k), E.buf(v)
    do = E.buf(np.full(batch * Tq * C, sentinel, np.float16))
    dl = E.buf(kv_len) if masked else None
    x = MiAttnArgs(q=dq.ptr, k=dk.ptr, v=dv.ptr, out=do.ptr, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, causal=0,
                   in_dtype=MI_F16, out_dtype=MI_F16, kv_len=dl.ptr if dl else None)
    call = lambda: E.call("mi_fused_attention_ex", ctypes.byref(x), None)
    kern, grid = _probe_grid(E, "attn_f16_kernel|-|-|-;attn_kernel|-|-|-", call)
    xs = sorted({0, _block_of_tile(grid[0] - 1, grid[0])})
    xl = ",".join(map(str, xs))
    print(f"  {kern} grid {grid}, blockIdx.x {xs}", flush=True)
    E.sample(f"attn_f16_kernel|{xl}|*|*;attn_kernel|{xl}|*|*")
    call()
    hd = C // heads
    got = do.get(np.float16, batch * Tq * C).reshape(batch, Tq, heads, hd)
    mask = got != sentinel
    head_written = mask.any(axis=3)
    assert head_written.any() and head_written[batch - 1, Tq - 1, heads - 1], "last query tile not sampled"
    assert np.array_equal(mask, np.repeat(head_written[..., None], hd, axis=3)), "partially written head rows"
    for b in range(batch):
        for h in range(heads):
            r = np.flatnonzero(head_written[b, :, h])
            if r.size:
                assert r[0] % 32 == 0 and (r.size % 32 == 0 or r[-1] == Tq - 1) and np.all(np.diff(r) == 1), \
                    f"written query rows of (batch {b}, head {h}) are not whole tiles"
    rows = np.flatnonzero(head_written.any(axis=(0, 2)))
    want = ob.fused_attention_ex(q, k, v, batch=batch, Tq=Tq, Tk=Tk, C=C, heads=heads, in_dtype=ob.OR_F16,
                                 out_dtype=ob.OR_F32, kv_len=kv_len, rows=rows,
                                 threads=ob.max_threads()).reshape(batch, len(rows), heads, hd)
    sel = mask[:, rows]
    g = got[:, rows].astype(np.float64)[sel]
    w = want.astype(np.float64)[sel]
    bound = tol * rms(w) + fp16_half_ulp(w)
    assert np.all(np.abs(g - w) <= bound), f"attention full {kern} grid {grid}: beyond tol x RMS + half an ulp"
    return float(np.max(np.abs(g - w)) / rms(w))


def block(E, *, B, T, C, H, Tc, Cc, F, masked=False, blocks=2, order=0, front=False, fused=False, qkv_joint=False,
          half=False, hattn=False):
    """Two applications of one SDXL transformer block: uncached
    (mi_sdxl_block_forward) vs context K / V projected once (mi_block_ctx_kv,
    mi_sdxl_block_forward_kv), against the oracle's block; cached and fresh
    runs must be bit-identical (same GEMM plans, fixed summation order). With
    fused / qkv_joint / half (fp16 activations): one block with those flags
    against the plain block, bit for bit (every flag combination computes the
    same sums). hattn (MI_BLOCK_FP16_ATTENTION, fp16 Q / K / V and attention
    inputs): against the oracle to the block bar, and the other flags against
    the block with that flag alone."""
    E.order(order)
    base = MI_BLOCK_FP16_ATTENTION if hattn else 0
    flags = ((MI_BLOCK_FUSED_EPILOGUES if fused else 0) | (MI_BLOCK_JOINT_QKV if qkv_joint else 0) |
             (MI_BLOCK_FP16_ACTIVATIONS if half else 0) | base)
    w = make_weights(ob, C, Cc, F, seed=500)
    dw = {k: E.buf(v, front=front) for k, v in w.items()}
    ptrs = {k: b.ptr for k, b in dw.items()}
    if qkv_joint:  # to_q / to_k / to_v back to back: the block takes one projection GEMM
        joint = E.buf(np.concatenate([w["attn1_q"], w["attn1_k"], w["attn1_v"]]), front=front)
        dw["_joint"] = joint
        nb = w["attn1_q"].nbytes
        ptrs.update(attn1_q=joint.ptr, attn1_k=joint.ptr + nb, attn1_v=joint.ptr + 2 * nb)
    bw = MiBlockWeights(*[ptrs[f[0]] for f in MiBlockWeights._fields_])
    # the same weights stored apart (three projection GEMMs)
    bw_apart = MiBlockWeights(*[dw[f[0]].ptr for f in MiBlockWeights._fields_])
    dims = MiBlockDims(B, T, C, H, Tc, Cc, F, flags)
    plain = MiBlockDims(B, T, C, H, Tc, Cc, F, base)
    x = ob.normal(3, B * T * C)
    ctx = ob.normal(4, B * Tc * Cc).astype(np.float16).astype(np.float32)
    kl = ob.uniform_int(8, 1, Tc, B) if masked else None
    dc = E.buf(ctx, front=front)
    dl = E.buf(np.asarray(kl, np.int32), front=front) if kl is not None else None
    ws_bytes = E.lib.mi_block_workspace_bytes(ctypes.byref(dims))
    kv_bytes = E.lib.mi_block_ctx_kv_bytes(ctypes.byref(dims))
    ws, kv = E.buf(nbytes=ws_bytes, front=front).fill(0xFF), E.buf(nbytes=kv_bytes, front=front).fill(0xFF)
    dx_fresh, dx_cached = E.buf(x, front=front), E.buf(x, front=front)
    for _ in range(blocks):
        E.call("mi_sdxl_block_forward", ctypes.byref(bw), ctypes.byref(dims), dx_fresh.ptr, dc.ptr,
               dl.ptr if dl else None, ws.ptr, ws_bytes, None)
    E.call("mi_block_ctx_kv", ctypes.byref(bw), ctypes.byref(dims), dc.ptr, kv.ptr, kv_bytes, None)
    for _ in range(blocks):
        E.call("mi_sdxl_block_forward_kv", ctypes.byref(bw), ctypes.byref(dims), dx_cached.ptr, kv.ptr, kv_bytes,
               dl.ptr if dl else None, ws.ptr, ws_bytes, None)
    fresh, cached = dx_fresh.get(np.float32), dx_cached.get(np.float32)
    want = x
    for _ in range(blocks):
        want = ob.sdxl_block(w, want, ctx, batch=B, tokens=T, channels=C, heads=H, ctx_tokens=Tc, ctx_channels=Cc,
                             ff_inner=F, ctx_len=kl, threads=ob.max_threads())
    assert np.all(np.isfinite(cached)) and np.all(np.isfinite(fresh)), "block: non-finite output"
    e = float(np.max(np.abs(fresh - want)) / rms(want - x))
    assert e <= blocks * BLOCK_TOL, f"block vs oracle: {e:.3e} x RMS(update)"
    assert np.array_equal(cached, fresh), \
        f"cached vs fresh K / V differ by {float(np.max(np.abs(cached - fresh))):.3e}"
    if flags != base:
        # one block with the flags vs the plain block (weights apart, separate epilogues)
        outs = []
        for wts, dd in ((bw, dims), (bw_apart, plain)):
            d1 = E.buf(x, front=front)
            E.call("mi_sdxl_block_forward", ctypes.byref(wts), ctypes.byref(dd), d1.ptr, dc.ptr,
                   dl.ptr if dl else None, ws.ptr, ws_bytes, None)
            outs.append(d1.get(np.float32))
        assert np.array_equal(outs[0], outs[1]), \
            f"flags {flags:#x} vs plain block differ by {float(np.max(np.abs(outs[0] - outs[1]))):.3e}"
    return e


def gemm_f16o(E, *, M, N, K, cfg=None, seed=1, order=0, front=False, ldc=0):
    """mi_gemm_nt_q8_0_f16o (fp16 output, A fp32 and fp16) against the RNE
    rounding of mi_gemm_nt_q8_0's fp32 output, bit for bit."""
    _set_cfg(cfg)
    E.order(order)
    a16 = ob.normal(seed, M * K).astype(np.float16)
    blocks = q8_weights(ob, seed + 1, N, K)
    bias = ob.normal(seed + 2, N, 0.0, 0.02)
    dW, dB = E.buf(blocks, front=front), E.buf(bias, front=front)
    dA32, dA16 = E.buf(a16.astype(np.float32), front=front), E.buf(a16, front=front)
    dC = E.buf(np.zeros(M * N, np.float32), front=front)
    E.call("mi_gemm_nt_q8_0", dA32.ptr, dW.ptr, dB.ptr, dC.ptr, M, N, K, 0, 0, 0, 1, 0, 0, None)
    want16 = dC.get(np.float32).astype(np.float16)
    ld = ldc or N
    for a_dtype, dA in ((0, dA32), (1, dA16)):
        dH = E.buf(np.full((M - 1) * ld + N, np.float16(7.0), np.float16), front=front)
        E.call("mi_gemm_nt_q8_0_f16o", dA.ptr, a_dtype, dW.ptr, dB.ptr, dH.ptr, M, N, K, 0, ldc, None)
        got = dH.get(np.float16).reshape(-1)
        rows = np.stack([got[m * ld:m * ld + N] for m in range(M)]).reshape(-1)
        assert np.array_equal(rows.view(np.uint16), want16.view(np.uint16)), \
            f"f16o (a_dtype {a_dtype}) differs from the rounded fp32 GEMM"
        if ld > N:  # the padding columns stay untouched
            pad = np.concatenate([got[m * ld + N:(m + 1) * ld] for m in range(M - 1)])
            assert np.all(pad == np.float16(7.0)), "f16o wrote past N"
    want = ob.gemm_nt_q8_0(a16.astype(np.float32), blocks, M, N, K, bias=bias, threads=ob.max_threads())
    return assert_parity(want16.astype(np.float32), want, what="gemm f16o")


def gemm_f16a(E, *, M, N, K, mode=0, cfg=None, seed=1, order=0, front=False):
    """mi_gemm_nt_q8_0_f16a (fp16 A) against mi_gemm_nt_q8_0_ws on the same
    values as fp32, bit for bit, with the workspace the library asks for."""
    _set_cfg(cfg)
    E.order(order)
    a16 = ob.normal(seed, M * K).astype(np.float16)
    blocks = q8_weights(ob, seed + 1, N, K)
    bias = ob.normal(seed + 2, N, 0.0, 0.02)
    C0 = ob.normal(seed + 3, M * N)
    dW, dB = E.buf(blocks, front=front), E.buf(bias, front=front)
    nws = E.lib.mi_gemm_nt_q8_workspace_bytes(M, N, K, 1)
    wsp, wsn, _keep = _workspace(E, nws, front)
    outs = []
    for entry, A in (("mi_gemm_nt_q8_0_f16a", a16), ("mi_gemm_nt_q8_0_ws", a16.astype(np.float32))):
        dA, dC = E.buf(A, front=front), E.buf(C0, front=front)
        E.call(entry, dA.ptr, dW.ptr, dB.ptr, dC.ptr, M, N, K, mode, 0, 0, 1, 0, 0, wsp, wsn, None)
        outs.append(dC.get(np.float32))
    assert np.array_equal(outs[0], outs[1]), "fp16-A GEMM differs from the fp32 GEMM on the same values"
    want = ob.gemm_nt_q8_0(a16.astype(np.float32), blocks, M, N, K, bias=None if mode == 1 else bias,
                           threads=ob.max_threads())
    return assert_parity(outs[0] - (C0 if mode else 0), want, what="gemm f16a")


def routing(E, *, table, order=0):
    """Host routing (tile / split choice, attention workgroup size): each
    entry [op, dims, grid, threads] is launched with no workgroup emulated and
    its main launch must have that grid and block size."""
    E.order(order)
    E.lib.mi_tuning_reset()
    E.sample("*|-|-|-")
    bad = []
    for op, dims, grid, threads in table:
        if op in ("gemm", "gemm_ws"):
            M, N, K = dims
            A, W, C = E.buf(nbytes=M * K * 4), E.buf(nbytes=N * K // 32 * 34), E.buf(nbytes=M * N * 4)
            if op == "gemm":
                E.call("mi_gemm_nt_q8_0", A.ptr, W.ptr, None, C.ptr, M, N, K, 0, 0, 0, 1, 0, 0, None)
            else:
                n = E.lib.mi_gemm_nt_q8_workspace_bytes(M, N, K, 1)
                ws = E.buf(nbytes=max(n, 16))
                E.call("mi_gemm_nt_q8_0_ws", A.ptr, W.ptr, None, C.ptr, M, N, K, 0, 0, 0, 1, 0, 0, ws.ptr, n, None)
        elif op in ("nn", "nn_ws"):
            M, N, K = dims
            P, S, B, C = E.buf(nbytes=M * K), E.buf(nbytes=M * K // 32 * 4), E.buf(nbytes=K * N * 4), \
                E.buf(nbytes=M * N * 4)
            if op == "nn":
                E.call("mi_gemm_nn_q8_split", P.ptr, S.ptr, B.ptr, C.ptr, M, N, K, 0, 0, 0, 0, 1, 0, 0, 0, None)
            else:
                n = E.lib.mi_gemm_nn_q8_workspace_bytes(M, N, K, 1)
                ws = E.buf(nbytes=max(n, 16))
                E.call("mi_gemm_nn_q8_split_ws", P.ptr, S.ptr, B.ptr, C.ptr, M, N, K, 0, 0, 0, 0, 1, 0, 0, 0, ws.ptr,
                       n, None)
        else:
            b, h, tq, tk = dims
            C = 64 * h
            q, k, v = E.buf(nbytes=b * tq * C * 2), E.buf(nbytes=b * tk * C * 2), E.buf(nbytes=b * tk * C * 2)
            o = E.buf(nbytes=b * tq * C * 2)
            x = MiAttnArgs(q=q.ptr, k=k.ptr, v=v.ptr, out=o.ptr, batch=b, Tq=tq, Tk=tk, C=C, heads=h, causal=0,
                           in_dtype=MI_F16, out_dtype=MI_F16, kv_len=None)
            E.call("mi_fused_attention_ex", ctypes.byref(x), None)
        kern, g = E.last_launch()
        got = [list(g), E.last_block_threads()]
        if got != [list(grid), threads]:
            bad.append(f"{op} {dims}: {kern} grid {got[0]} x {got[1]} threads, expected {list(grid)} x {threads}")
    E.sample("")
    assert not bad, "\n".join(bad)
    return 0.0


def block_full(E, *, fused=False, qkv_joint=False, cached=False, order=0, half=False, hattn=False):
    """The config-4 block (level 2: 2 x 1024 tokens, C 1280, 20 heads, context
    2 x 77 x 2048, FF 1280 -> 2 x 5120 -> 1280) at full size with the first and
    last workgroup of every grid dimension of every launch emulated: a bounds
    check of the workspace carve-up, the joint Q / K / V placement, the cached
    context K / V buffer and every kernel's offsets at the real sizes (the
    tensors the skipped workgroups would write stay unwritten, so no values
    are compared here; the small-shape block cases compare them)."""
    E.order(order)
    B, T, C, H, Tc, Cc, F = 2, 1024, 1280, 20, 77, 2048, 5120
    w = make_weights(ob, C, Cc, F, seed=500)
    dw = {k: E.buf(v) for k, v in w.items()}
    ptrs = {k: b.ptr for k, b in dw.items()}
    if qkv_joint:
        joint = E.buf(np.concatenate([w["attn1_q"], w["attn1_k"], w["attn1_v"]]))
        dw["_joint"] = joint
        nb = w["attn1_q"].nbytes
        ptrs.update(attn1_q=joint.ptr, attn1_k=joint.ptr + nb, attn1_v=joint.ptr + 2 * nb)
    bw = MiBlockWeights(*[ptrs[f[0]] for f in MiBlockWeights._fields_])
    flags = ((MI_BLOCK_FUSED_EPILOGUES if fused else 0) | (MI_BLOCK_JOINT_QKV if qkv_joint else 0) |
             (MI_BLOCK_FP16_ACTIVATIONS if half else 0) | (MI_BLOCK_FP16_ATTENTION if hattn else 0))
    dims = MiBlockDims(B, T, C, H, Tc, Cc, F, flags)
    dx = E.buf(ob.normal(3, B * T * C))
    dc = E.buf(ob.normal(4, B * Tc * Cc).astype(np.float16).astype(np.float32))
    dl = E.buf(ob.uniform_int(8, 1, Tc, B).astype(np.int32))
    ws_bytes = E.lib.mi_block_workspace_bytes(ctypes.byref(dims))
    kv_bytes = E.lib.mi_block_ctx_kv_bytes(ctypes.byref(dims))
    ws, kv = E.buf(nbytes=ws_bytes).fill(0), E.buf(nbytes=kv_bytes).fill(0)
    E.sample("*|0,-1|0,-1|0,-1")
    before = E.lib.kemu_launches()
    if cached:
        E.call("mi_block_ctx_kv", ctypes.byref(bw), ctypes.byref(dims), dc.ptr, kv.ptr, kv_bytes, None)
        E.call("mi_sdxl_block_forward_kv", ctypes.byref(bw), ctypes.byref(dims), dx.ptr, kv.ptr, kv_bytes, dl.ptr,
               ws.ptr, ws_bytes, None)
    else:
        E.call("mi_sdxl_block_forward", ctypes.byref(bw), ctypes.byref(dims), dx.ptr, dc.ptr, dl.ptr, ws.ptr,
               ws_bytes, None)
    n = E.lib.kemu_launches() - before
    print(f"  {n} launches, workspace {ws_bytes} B, context K/V {kv_bytes} B", flush=True)
    assert n >= 8, f"only {n} launches"
    return 0.0


def q8(E, *, n, seed=1, front=False, order=0):
    """Q8_0 decode (fp32 bit-exact, fp16 = RNE of it), repack to the split
    layout and its decode, and the device quantiser, against the oracle."""
    E.order(order)
    w = ob.normal(seed, n, 0.0, 0.02)
    if n >= 64:
        w[:32] = 0.0                                   # an all-zero block
        w[32:64] = np.arange(32, dtype=np.float32) - 15.5
    blocks = ob.q8_0_quantize(w)
    db = E.buf(blocks, front=front)
    want = ob.q8_0_dequant(blocks, n)
    o32, o16 = E.buf(nbytes=n * 4, front=front), E.buf(nbytes=n * 2, front=front)
    E.call("mi_q8_0_dequant", db.ptr, o32.ptr, MI_F32, n, None)
    E.call("mi_q8_0_dequant", db.ptr, o16.ptr, MI_F16, n, None)
    assert np.array_equal(o32.get(np.uint32, n), want.view(np.uint32)), "q8_0 dequant fp32"
    assert np.array_equal(o16.get(np.uint16, n), want.astype(np.float16).view(np.uint16)), "q8_0 dequant fp16"
    dp, ds = E.buf(nbytes=n, front=front), E.buf(nbytes=n // 32 * 4, front=front)
    E.call("mi_q8_0_to_split", db.ptr, dp.ptr, ds.ptr, n, None)
    payload, scales = ob.q8_0_to_split(blocks, n)
    assert np.array_equal(dp.get(np.int8, n), payload.view(np.int8)[:n]), "to_split payload"
    assert np.array_equal(ds.get(np.uint32, n // 32), scales.view(np.uint32)), "to_split scales"
    E.call("mi_q8_split_dequant", dp.ptr, ds.ptr, o32.ptr, MI_F32, n, None)
    assert np.array_equal(o32.get(np.uint32, n), want.view(np.uint32)), "split dequant"
    dw, dq = E.buf(w, front=front), E.buf(nbytes=n // 32 * 34, front=front)
    E.call("mi_q8_0_quantize", dw.ptr, dq.ptr, n, None)
    assert np.array_equal(dq.get(np.uint8, n // 32 * 34), blocks), "quantize"
    return 0.0


def glue(E, *, rows, d, affine=True, seed=1, front=False, order=0):
    """LayerNorm (also in place), GEGLU (F = d / 2) and the residual add
    against the oracle, to the GPU tests' bars."""
    E.order(order)
    x = ob.normal(seed, rows * d, 0.5, 3.0)
    g = ob.normal(seed + 1, d, 1.0, 0.2) if affine else None
    b = ob.normal(seed + 2, d, 0.0, 0.2) if affine else None
    want = ob.layernorm(x, g, b, rows, d)
    dx, dy = E.buf(x, front=front), E.buf(nbytes=x.nbytes, front=front)
    dg, dbb = (E.buf(g, front=front), E.buf(b, front=front)) if affine else (None, None)
    E.call("mi_layernorm", dx.ptr, dg.ptr if dg else None, dbb.ptr if dbb else None, dy.ptr, rows, d, 1e-5, None)
    assert np.max(np.abs(dy.get(np.float32) - want)) <= 4e-6, "layernorm"
    E.call("mi_layernorm", dx.ptr, dg.ptr if dg else None, dbb.ptr if dbb else None, dx.ptr, rows, d, 1e-5, None)
    assert np.max(np.abs(dx.get(np.float32) - want)) <= 4e-6, "layernorm in place"
    if d % 2 == 0:
        F = d // 2
        h = ob.normal(seed + 3, rows * 2 * F, 0.0, 2.0)
        dh, dg2 = E.buf(h, front=front), E.buf(nbytes=rows * F * 4, front=front)
        E.call("mi_geglu", dh.ptr, dg2.ptr, rows, F, None)
        wg = ob.geglu(h, rows, F)
        assert np.all(np.abs(dg2.get(np.float32) - wg) <= 2e-6 * (1 + np.abs(wg))), "geglu"
    a1, a2 = ob.normal(seed + 4, rows * d), ob.normal(seed + 5, rows * d)
    d1, d2 = E.buf(a1, front=front), E.buf(a2, front=front)
    E.call("mi_add_inplace", d1.ptr, d2.ptr, rows * d, None)
    assert np.array_equal(d1.get(np.float32), ob.add(a1, a2)), "add"
    return 0.0


def gguf_upload(E, *, big_rows=10240, big_cols=1280, order=0, front=False):
    """mi_gguf_upload_raw / _f32 / _q8_split of every tensor of the sample
    checkpoint plus a Q8_0 weight that crosses the 8 MiB staging buffers
    several times, each into a guarded buffer of exactly the tensor's size,
    against the host readers (mi_gguf_read_*, whose parity with the
    reference's Gguf.cpp is tests/test_gguf.py). Copies run deferred, so a
    staging buffer refilled before its copy was waited for is caught."""
    import tempfile
    E.order(order)
    blocks = ob.q8_0_quantize(ob.normal(5, big_rows * big_cols, 0.0, 0.02))
    spec = gw.sample_spec()
    spec.tensors.append(gw.Tensor(gw.PREFIX + "big.weight", (big_cols, big_rows), gw.T_Q8_0, blocks.tobytes()))
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "sample.gguf"
        gw.write(path, spec)
        h = ctypes.c_void_p()
        E.call("mi_gguf_open", str(path).encode(), gw.PREFIX.encode(), ctypes.byref(h))
        ver, n, off, size = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        E.call("mi_gguf_info", h, ctypes.byref(ver), ctypes.byref(n), ctypes.byref(off), ctypes.byref(size))
        checked, big_seen = 0, False
        for i in range(n.value):
            t = MiGgufTensorInfo()
            E.call("mi_gguf_tensor", h, i, ctypes.byref(t))
            raw = np.zeros(max(t.nbytes, 1), np.uint8)
            E.call("mi_gguf_read_raw", h, i, raw.ctypes.data, t.nbytes)
            d_raw = E.buf(nbytes=t.nbytes, front=front).fill(0xA5)
            E.call("mi_gguf_upload_raw", h, i, d_raw.ptr, t.nbytes, None)
            if E.status("mi_gguf_read_f32", h, i, None, 0) != 2:  # decodable type
                host = np.zeros(max(t.n_elems, 1), np.float32)
                E.call("mi_gguf_read_f32", h, i, host.ctypes.data, t.n_elems)
                d_f = E.buf(nbytes=t.n_elems * 4, front=front).fill(0xA5)
                E.call("mi_gguf_upload_f32", h, i, d_f.ptr, t.n_elems, None)
            else:
                d_f = None
            q8 = t.type == gw.T_Q8_0
            if q8:
                nb = t.n_elems // 32
                hq, hs = np.zeros(nb * 32, np.int8), np.zeros(nb, np.float32)
                E.call("mi_gguf_read_q8_split", h, i, hq.ctypes.data, hs.ctypes.data)
                d_q = E.buf(nbytes=nb * 32, front=front).fill(0xA5)
                d_s = E.buf(nbytes=nb * 4, front=front).fill(0xA5)
                E.call("mi_gguf_upload_q8_split", h, i, d_q.ptr, d_s.ptr, None)
            E.lib.kemu_sync()
            name = t.name.decode()
            assert np.array_equal(d_raw.get(np.uint8, t.nbytes), raw[: t.nbytes]), f"upload_raw {name}"
            if d_f is not None:
                assert np.array_equal(d_f.get(np.uint32, t.n_elems), host[: t.n_elems].view(np.uint32)), \
                    f"upload_f32 {name}"
            if q8:
                assert np.array_equal(d_q.get(np.int8, nb * 32), hq), f"upload_q8_split payload {name}"
                assert np.array_equal(d_s.get(np.uint32, nb), hs.view(np.uint32)), f"upload_q8_split scales {name}"
            checked += 1
            big_seen |= name == "big.weight" and t.nbytes == blocks.nbytes
        E.lib.mi_gguf_close(h)
    assert checked == n.value and checked >= 3 and big_seen
    return 0.0


CASES = {"gemm_nt": gemm_nt, "gemm_geglu": gemm_geglu, "gemm_f16a": gemm_f16a, "gemm_f16o": gemm_f16o, "gemm_nn": gemm_nn,
         "attention": attention, "block": block,
         "gguf_upload": gguf_upload, "q8": q8, "glue": glue, "gemm_full": gemm_full, "gemm_nn_full": gemm_nn_full,
         "attention_full": attention_full, "block_full": block_full, "routing": routing}


def main(argv):
    spec = json.loads(argv[1])
    name = spec.pop("case")
    schedules = spec.pop("schedules", [spec.pop("order", 0)])
    global _EMU
    E = _EMU = kemu.Emu()
    ob.build()
    for order in schedules:
        e = CASES[name](E, order=order, **spec)
        print(f"OK {name} order={order} err/rms={e:.3e} launches={E.lib.kemu_launches()}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
