"""GPU parity for the Q8 NN GEMM (mi_gemm_nn_q8_split, gemm_nn_q8_v.comp)
against the CPU oracle (or_gemm_nn_q8_split, pinned in tests/test_oracle.py).

Bar: max |C_gpu - C_ref| <= 2e-3 x RMS(C_ref) (fp16-MFMA kernel vs the
reference's fp32 shader math), on full outputs, or on sampled rows at the
SDXL conv shapes (every output row is independent).
"""
import numpy as np
import pytest

from helpers import REL_RMS_TOL, assert_parity, err_vs_rms, q8_weights
from sdvk_amd import ops
from sdvk_amd.hip import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu


def split_weight(oracle, seed, M, K):
    """A [M, K] weight from N(0, 0.02^2), Q8_0-quantised, in the split layout."""
    return oracle.q8_0_to_split(q8_weights(oracle, seed, M, K), M * K)


def run_nn(payload, scales, B, M, N, K, C0=None, csize=None, ws=False, **kw):
    """ws: through mi_gemm_nn_q8_split_ws with the workspace the library asks for (K splits)."""
    dq, ds, dB = DeviceBuffer.from_array(payload), DeviceBuffer.from_array(scales), DeviceBuffer.from_array(B)
    dC = DeviceBuffer.from_array(C0) if C0 is not None else DeviceBuffer(csize * 4)
    if ws:
        n = ops.gemm_nn_workspace_bytes(M, N, K, kw.get("batch", 1))
        kw["workspace"] = DeviceBuffer(n) if n else None
    ops.gemm_nn_q8(dq, ds, dB, dC, M, N, K, **kw)
    synchronize()
    return dC.download(np.float32, C0.size if C0 is not None else csize)


@pytest.mark.parametrize("M,N,K", [(1, 4, 32), (70, 68, 96), (64, 64, 64), (130, 200, 288), (320, 1028, 320)])
def test_nn_shapes_and_accumulate(gpu, oracle, M, N, K):
    print(f"[case] nn M={M} N={N} K={K}", flush=True)
    payload, scales = split_weight(oracle, M + 3, M, K)
    B = oracle.normal(N + 5, K * N)
    want = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K, threads=oracle.max_threads())
    got = run_nn(payload, scales, B, M, N, K, csize=M * N)
    e = assert_parity(got, want, what=f"{M}x{N}x{K} mode0")
    C0 = oracle.normal(9, M * N)
    got1 = run_nn(payload, scales, B, M, N, K, C0=C0, mode=1)
    assert_parity(got1 - C0, want, what="mode1")
    print(f"  err/rms = {e:.3e}", flush=True)


def test_nn_batch_strides_and_flat_scales(gpu, oracle):
    """Batch z offsets A, B and C; lda / ldb / ldc padding; lda % 32 != 0 so a
    scale block straddles two weight rows (the flat index, gemm_nn_q8_v.comp:23-28);
    K % 32 != 0; padding of C untouched."""
    M, N, K, batch = 60, 132, 100, 3
    lda, ldb, ldc = 108, 140, 150
    sA, sB, sC = M * lda + 12, K * ldb + 8, M * ldc + 7
    print(f"[case] nn batch={batch} strides lda={lda} ldb={ldb} ldc={ldc}", flush=True)
    na = (batch - 1) * sA + (M - 1) * lda + K
    # one flat N(0, 0.02^2) weight array quantised in flat blocks of 32: rows of
    # lda elements start mid-block, so the scales are the flat ones
    payload, scales = oracle.q8_0_to_split(q8_weights(oracle, 21, 1, (na + 31) // 32 * 32), (na + 31) // 32 * 32)
    B = oracle.normal(23, (batch - 1) * sB + (K - 1) * ldb + N)
    C0 = oracle.normal(24, (batch - 1) * sC + M * ldc)
    kw = dict(lda=lda, ldb=ldb, ldc=ldc, batch=batch, sA=sA, sB=sB, sC=sC)
    want = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K, C=C0.copy(), threads=oracle.max_threads(), **kw)
    got = run_nn(payload, scales, B, M, N, K, C0=C0, **kw)
    for z in range(batch):
        g = got[z * sC: z * sC + M * ldc].reshape(M, ldc)
        w = want[z * sC: z * sC + M * ldc].reshape(M, ldc)
        assert_parity(g[:, :N], w[:, :N], what=f"batch {z}")
        assert np.array_equal(g[:, N:], C0[z * sC: z * sC + M * ldc].reshape(M, ldc)[:, N:])
    assert np.array_equal(got[M * ldc: sC], C0[M * ldc: sC])


@pytest.mark.parametrize("kernel", ["tiled", "general"])
@pytest.mark.parametrize("mode", [0, 1])
def test_nn_tiled_strides_and_k_splits(gpu, oracle, tune, kernel, mode):
    """The tiled kernel (K % 64 == 0, lda and sA multiples of 16) with batch /
    leading dimensions, and with K split across workgroups through the
    workspace (64 x 64 x 1024: one tile, four splits summed in order by the
    reduce pass); the nn_kernel=general override runs the same cases on the untiled
    kernel."""
    if kernel == "general":
        tune("nn_kernel", "general")
    else:
        tune("nn_kernel", None)
    M, N, K, batch = 70, 36, 256, 3
    lda, ldb, ldc = 272, 40, 44
    sA, sB, sC = 19056, 10248, 3100
    print(f"[case] nn {kernel} mode={mode} batch={batch} strides", flush=True)
    na = (batch - 1) * sA + (M - 1) * lda + K
    payload, scales = oracle.q8_0_to_split(q8_weights(oracle, 61, 1, (na + 31) // 32 * 32), (na + 31) // 32 * 32)
    B = oracle.normal(62, (batch - 1) * sB + (K - 1) * ldb + N)
    C0 = oracle.normal(63, (batch - 1) * sC + M * ldc)
    kw = dict(lda=lda, ldb=ldb, ldc=ldc, batch=batch, sA=sA, sB=sB, sC=sC, mode=mode)
    want = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K, C=C0.copy(), threads=oracle.max_threads(), **kw)
    got = run_nn(payload, scales, B, M, N, K, C0=C0, ws=True, **kw)
    for z in range(batch):
        g = got[z * sC: z * sC + M * ldc].reshape(M, ldc)
        w = want[z * sC: z * sC + M * ldc].reshape(M, ldc)
        c0 = C0[z * sC: z * sC + M * ldc].reshape(M, ldc)
        if mode == 1:
            assert_parity(g[:, :N] - c0[:, :N], w[:, :N] - c0[:, :N], what=f"{kernel} batch {z} mode 1")
        else:
            assert_parity(g[:, :N], w[:, :N], what=f"{kernel} batch {z}")
        assert np.array_equal(g[:, N:], c0[:, N:])
    M, N, K = 64, 64, 1024
    payload, scales = split_weight(oracle, 64, M, K)
    B = oracle.normal(65, K * N)
    C0 = oracle.normal(66, M * N)
    want = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K, C=C0.copy(), mode=mode, threads=oracle.max_threads())
    got = run_nn(payload, scales, B, M, N, K, C0=C0, mode=mode, ws=True)
    if mode == 1:
        assert_parity(got - C0, want - C0, what=f"{kernel} K split mode 1")
    else:
        assert_parity(got, want, what=f"{kernel} K split")


# SDXL 1024^2 conv shapes: level-0 3x3 (320 -> 320 over a 4096-pixel chunk of the
# 128 x 128 latent), level-1 3x3 (640 -> 640, 64 x 64), level-2 3x3 (1280 -> 1280,
# 32 x 32), a 1x1 shortcut (640 -> 1280, 32 x 32)
CONV_SHAPES = [(320, 4096, 320 * 9), (640, 4096, 640 * 9), (1280, 1024, 1280 * 9), (1280, 1024, 640)]


@pytest.mark.parametrize("M,N,K", CONV_SHAPES)
def test_nn_conv_shapes_sampled_rows(gpu, oracle, M, N, K):
    print(f"[case] nn conv M={M} N={N} K={K}", flush=True)
    payload, scales = split_weight(oracle, 31, M, K)
    B = oracle.normal(32, K * N)
    got = run_nn(payload, scales, B, M, N, K, csize=M * N, ws=True).reshape(M, N)
    rng = np.random.default_rng(M + N + K)
    rows = np.unique(np.concatenate([[0, M - 1, min(63, M - 1), min(64, M - 1)], rng.integers(0, M, 24)]))
    # the oracle on the selected weight rows only (rows of C depend on rows of A)
    sub_p = payload.reshape(M, K)[rows].reshape(-1)
    sub_s = scales.reshape(M, K // 32)[rows].reshape(-1)
    want = oracle.gemm_nn_q8_split(sub_p, sub_s, B, len(rows), N, K, threads=oracle.max_threads()).reshape(-1, N)
    e = err_vs_rms(got[rows], want)
    print(f"  err/rms = {e:.3e} over {len(rows)} rows", flush=True)
    assert e <= REL_RMS_TOL


def test_nn_reference_dispatch_names(gpu, oracle):
    """Engine::dispatch("gemm_nn_q8_v", {Aq, B, C, S}, Pg) (vk_engine.cpp:57,63)."""
    M, N, K = 96, 64, 128
    payload, scales = split_weight(oracle, 41, M, K)
    B = oracle.normal(42, K * N)
    want = oracle.gemm_nn_q8_split(payload, scales, B, M, N, K)
    dq, ds, dB = DeviceBuffer.from_array(payload), DeviceBuffer.from_array(scales), DeviceBuffer.from_array(B)
    for name in ("gemm_nn_q8_v", "gemm_nn_q8"):
        dC = DeviceBuffer(M * N * 4)
        ops.dispatch(name, [dq, dB, dC, ds], ops.Pg(M, N, K))
        synchronize()
        assert_parity(dC.download(np.float32, M * N), want, what=name)


def test_nn_rejections(gpu, oracle):
    payload, scales = split_weight(oracle, 51, 8, 64)
    dq, ds = DeviceBuffer.from_array(payload), DeviceBuffer.from_array(scales)
    dB, dC = DeviceBuffer(64 * 16 * 4), DeviceBuffer(8 * 16 * 4)
    for bad in (dict(N=14), dict(K=62), dict(mode=2), dict(batch=0)):
        args = dict(M=8, N=16, K=64)
        args.update({k: v for k, v in bad.items() if k in args})
        kw = {k: v for k, v in bad.items() if k not in args}
        with pytest.raises(ops.MiError):
            ops.gemm_nn_q8(dq, ds, dB, dC, args["M"], args["N"], args["K"], **kw)
    with pytest.raises(ops.MiError):  # B not 16-byte aligned
        ops.gemm_nn_q8(dq, ds, dB.value + 4, dC, 8, 16, 64)
    with pytest.raises(ops.MiError):  # C aliases B
        ops.gemm_nn_q8(dq, ds, dB, dB, 8, 16, 64)
    synchronize()
