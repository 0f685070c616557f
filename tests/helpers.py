"""Shared test helpers: the parity bar and input builders."""
from __future__ import annotations

import os

import numpy as np

# max |got - ref| <= 2e-3 x RMS(ref) for the fp16-MFMA
# GEMM and attention vs the reference's fp32 math.
REL_RMS_TOL = 2e-3


def rms(x: np.ndarray) -> float:
    x = np.asarray(x, dtype=np.float64)
    return float(np.sqrt(np.mean(x * x))) if x.size else 0.0


# Worst parity error of this session per test function, {module::function:
# (err, bar, test id)}; tests/conftest.py prints it in the terminal summary
# (visible under -q).
WORST: dict[str, tuple[float, float, str]] = {}


def record(e: float, tol: float = REL_RMS_TOL, label: str = "") -> float:
    """Notes an error (relative to its bar `tol`) for the end-of-session summary;
    `label` keeps a mode apart from the test function's default path."""
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    mod = (test.rsplit("/", 1)[-1].replace(".py", "").split("[")[0] if test else "?") + label
    prev = WORST.get(mod)
    if prev is None or e / tol > prev[0] / prev[1]:
        WORST[mod] = (float(e), float(tol), test)
    return e


def err_vs_rms(got: np.ndarray, ref: np.ndarray, note: bool = True) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    r = rms(ref)
    e = float(np.max(np.abs(got - ref)) / r) if r > 0 else float(np.max(np.abs(got - ref)))
    return record(e) if note and np.isfinite(e) else e


def assert_parity(got, ref, tol=REL_RMS_TOL, what="", label=""):
    e = err_vs_rms(got, ref, note=False)
    if np.isfinite(e):
        record(e, tol, label)
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
