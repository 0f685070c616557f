"""Shared test helpers: the parity bar and input builders."""
from __future__ import annotations

import numpy as np

# max |got - ref| <= 2e-3 x RMS(ref) for the fp16-MFMA
# GEMM and attention vs the reference's fp32 math.
REL_RMS_TOL = 2e-3


def rms(x: np.ndarray) -> float:
    x = np.asarray(x, dtype=np.float64)
    return float(np.sqrt(np.mean(x * x))) if x.size else 0.0


def err_vs_rms(got: np.ndarray, ref: np.ndarray) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    r = rms(ref)
    return float(np.max(np.abs(got - ref)) / r) if r > 0 else float(np.max(np.abs(got - ref)))


def assert_parity(got, ref, tol=REL_RMS_TOL, what=""):
    e = err_vs_rms(got, ref)
    assert np.all(np.isfinite(np.asarray(got, dtype=np.float64))), f"{what}: non-finite output"
    assert e <= tol, f"{what}: max|err| = {e:.3e} x RMS > {tol:.1e}"
    return e


def fp16_half_ulp(x: np.ndarray) -> np.ndarray:
    """Half an fp16 ulp at |x| (storage-rounding floor of an fp16 output)."""
    ax = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(ax, 2.0 ** -14)))
    return 0.5 * 2.0 ** (e - 10)


def q8_weights(oracle, seed: int, N: int, K: int, std: float = 0.02) -> np.ndarray:
    """Q8_0 blocks of an N x K weight drawn from N(0, std^2)."""
    w = oracle.normal(seed, N * K, 0.0, std)
    return oracle.q8_0_quantize(w)


def split_from_blocks(oracle, blocks: np.ndarray, n: int):
    payload, scales = oracle.q8_0_to_split(blocks, n)
    return payload, scales


def residual_split_ulps(C: int, F: int) -> float:
    """Bound, in ulp of max|x|, on fused vs separate residual epilogues of one
    block: each of the three residual GEMMs (two out-projections with K = C,
    FF-down with K = F) adds at most one partial per 64-wide K step into x
    with atomics, each rounding by at most half an ulp of |x|, where the
    separate path rounds once; 2 ulp more for the changed LayerNorm inputs
    downstream."""
    steps = lambda k: -(-k // 64)  # noqa: E731
    return 0.5 * (2 * (steps(C) + 1) + steps(F) + 1) + 2.0


def split_order_ulps(blocks: int) -> float:
    """Bound, in ulp of max|x|, on two runs of the same block path whose K-split
    GEMMs add their partials with atomics in a different order: a GEMM output
    then differs in its last bits, which can move each of the block's three
    residual adds (x + sublayer) by one ulp of |x|, plus at most one more ulp
    per add from the changed LayerNorm inputs downstream; per block applied."""
    return 2.0 * 3 * blocks
