"""GPU parity of the candidate Q8_0 GEMM builds that the tile rules do not
choose until measured faster, against the CPU oracle (the same bar and cases as
the other tile configurations, tests/test_gpu_gemm.py): the row-stationary
kernel with row-coalesced A loads and the quad transpose (gemm_cfg 7..10:
256 x 256 / 192 / 160 / 128 tiles) and the 4-wave 256 x 256 LDS kernel
(gemm_cfg 11, one wave per SIMD, no K split), and the 4-wave 256 x 128 and
128 x 256 LDS builds (12, 13: 128 x 64 / 64 x 128 per wave), and the 8-wave
192 x 256 LDS build (14: 96 x 64 per wave)."""
import numpy as np
import pytest

from helpers import REL_RMS_TOL, assert_parity, err_vs_rms, q8_weights
from sdvk_amd import ops
from sdvk_amd.hip import DeviceBuffer, synchronize
from test_gpu_gemm import run_q8_0, workspace

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg", ["7", "7:2", "8", "9:3", "10", "11", "12", "12:2", "13", "13:3", "14", "14:2"])
@pytest.mark.parametrize("M,N,K", [(300, 200, 640), (1030, 130, 256), (257, 512, 128)])
def test_coalesced_rows_config(gpu, oracle, tune, cfg, M, N, K):
    print(f"[case] cfg={cfg} M={M} N={N} K={K}", flush=True)
    tune("gemm_cfg", cfg)
    A = oracle.normal(11, M * K)
    blocks = q8_weights(oracle, 12, N, K)
    bias = oracle.normal(13, N, 0.0, 0.02)
    want = oracle.gemm_nt_q8_0(A, blocks, M, N, K, bias=bias, threads=oracle.max_threads()).reshape(M, N)
    got = run_q8_0(A, blocks, M, N, K, bias=bias, ws=True).reshape(M, N)
    assert_parity(got, want, what=f"cfg {cfg} mode0")
    C0 = oracle.normal(14, M * N)
    got1 = run_q8_0(A, blocks, M, N, K, C0=C0, mode=1, ws=True).reshape(M, N)
    assert_parity(got1 - C0.reshape(M, N), want - bias, what=f"cfg {cfg} mode1")
    payload, scales = oracle.q8_0_to_split(blocks, N * K)
    dC = DeviceBuffer(M * N * 4)
    ops.gemm_nt_q8_bias(DeviceBuffer.from_array(A), DeviceBuffer.from_array(payload), dC,
                        DeviceBuffer.from_array(scales), DeviceBuffer.from_array(bias), M, N, K,
                        workspace=workspace(M, N, K))
    synchronize()
    assert_parity(dC.download(np.float32, M * N).reshape(M, N), want, what=f"cfg {cfg} split layout")


@pytest.mark.parametrize("cfg", ["7", "11", "12", "13", "14", "15"])
def test_candidate_config_baseline_shape(gpu, oracle, tune, cfg):
    M, N, K = 9216, 1280, 1280
    print(f"[case] cfg={cfg} baseline M={M} N={N} K={K}", flush=True)
    tune("gemm_cfg", cfg)
    A = oracle.normal(1, M * K)
    blocks = q8_weights(oracle, 2, N, K)
    got = run_q8_0(A, blocks, M, N, K).reshape(M, N)
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([[0, M - 1, 255, 256], rng.integers(0, M, 64)]))
    want = oracle.gemm_rows(A, blocks, M, N, K, rows, threads=oracle.max_threads())
    e = err_vs_rms(got[rows], want)
    print(f"  err/rms = {e:.3e}", flush=True)
    assert e <= REL_RMS_TOL
