"""Determinism on the GPU: every sum has a fixed order, so a call repeats bit
for bit (the reference's plain-store epilogues, gemm_nt_q8_v.comp:115-127,
are deterministic too).

  * every BASELINE GEMM shape (configs 0 and 1), twice through the entry
    without a workspace and twice through the workspace entry (K splits
    summed in split order): each pair bit-identical;
  * without a workspace, every LDS tile build the planner can pick gives the
    same bits (same MFMA instruction, same K order), and the 34-byte-block and
    split-layout entries agree;
  * every attention shape of configs 2-3 twice: bit-identical;
  * the config-4 block twice, plain and with every flag: bit-identical.
"""
import numpy as np
import pytest

from helpers import q8_weights
from sdvk_amd import MI_F16, ops
from sdvk_amd.hip import DeviceBuffer, synchronize
from test_gpu_block import make_weights, to_device

pytestmark = pytest.mark.gpu

BASELINE_SHAPES = [(9216, 1280, 1280), (8192, 640, 640), (8192, 5120, 640), (8192, 640, 2560),
                   (2048, 1280, 1280), (2048, 10240, 1280), (2048, 1280, 5120), (154, 640, 2048),
                   (154, 1280, 2048)]


@pytest.mark.parametrize("M,N,K", BASELINE_SHAPES)
def test_gemm_repeats_bit_for_bit(gpu, oracle, M, N, K):
    print(f"[case] determinism gemm M={M} N={N} K={K}", flush=True)
    dA = DeviceBuffer.from_array(oracle.normal(1, M * K))
    dW = DeviceBuffer.from_array(q8_weights(oracle, 2, N, K))
    dB = DeviceBuffer.from_array(oracle.normal(3, N, 0.0, 0.02))
    nws = ops.gemm_workspace_bytes(M, N, K)
    ws = DeviceBuffer(nws) if nws else None
    outs = []
    for use_ws in (False, False, True, True):
        dC = DeviceBuffer(M * N * 4)
        dC.fill_zero()
        ops.gemm_nt_q8_0(dA, dW, dC, M, N, K, bias=dB, workspace=ws if use_ws else None)
        synchronize()
        outs.append(dC.download(np.float32, M * N))
    assert np.array_equal(outs[0], outs[1]), "two calls without a workspace differ"
    assert np.array_equal(outs[2], outs[3]), "two calls with a workspace differ"
    if nws == 0:
        assert np.array_equal(outs[0], outs[2]), "no split planned, yet the workspace entry differs"
    print(f"  split workspace {nws} B; ws vs plain max |diff| {float(np.max(np.abs(outs[2] - outs[0]))):.3e}",
          flush=True)


def test_unsplit_sums_do_not_depend_on_the_tile_build(gpu, oracle, tune):
    M, N, K = 700, 520, 640
    A = oracle.normal(5, M * K)
    blocks = q8_weights(oracle, 6, N, K)
    payload, scales = oracle.q8_0_to_split(blocks, N * K)
    dA, dW = DeviceBuffer.from_array(A), DeviceBuffer.from_array(blocks)
    dP, dS = DeviceBuffer.from_array(payload), DeviceBuffer.from_array(scales)
    ref = None
    for cfg in ("0", "1", "2", "3", "4", "5", "6"):
        tune("gemm_cfg", cfg)
        for layout in ("blocks", "split"):
            dC = DeviceBuffer(M * N * 4)
            if layout == "blocks":
                ops.gemm_nt_q8_0(dA, dW, dC, M, N, K)
            else:
                ops.gemm_nt_q8(dA, dP, dC, dS, M, N, K)
            synchronize()
            got = dC.download(np.float32, M * N)
            if ref is None:
                ref = got
            d = float(np.max(np.abs(got - ref)))
            print(f"  cfg {cfg:>2} {layout:<6} max |diff| vs cfg 0 = {d:.3e}", flush=True)
            assert np.array_equal(got, ref), f"cfg {cfg} ({layout}) differs from cfg 0"


@pytest.mark.parametrize("B,H,Tq,Tk,masked", [(2, 10, 4096, 4096, False), (2, 20, 1024, 1024, False),
                                               (2, 10, 4096, 77, True), (2, 20, 1024, 77, True)])
def test_attention_repeats_bit_for_bit(gpu, oracle, B, H, Tq, Tk, masked):
    print(f"[case] determinism attention B={B} H={H} Tq={Tq} Tk={Tk}", flush=True)
    C = 64 * H
    q = DeviceBuffer.from_array(oracle.normal(1, B * Tq * C).astype(np.float16))
    k = DeviceBuffer.from_array(oracle.normal(2, B * Tk * C).astype(np.float16))
    v = DeviceBuffer.from_array(oracle.normal(3, B * Tk * C).astype(np.float16))
    kl = DeviceBuffer.from_array(oracle.uniform_int(7, 1, Tk, B).astype(np.int32)) if masked else None
    outs = []
    for _ in range(2):
        o = DeviceBuffer(B * Tq * C * 2)
        ops.fused_attention_ex(q, k, v, o, batch=B, Tq=Tq, Tk=Tk, C=C, heads=H, in_dtype=MI_F16, out_dtype=MI_F16,
                               kv_len=kl)
        synchronize()
        outs.append(o.download(np.uint16, B * Tq * C))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("flags", [0, ops.MI_BLOCK_FUSED_EPILOGUES | ops.MI_BLOCK_JOINT_QKV])
def test_block_repeats_bit_for_bit(gpu, oracle, flags):
    B, T, C, H, Tc, Cc, F = 2, 1024, 1280, 20, 77, 2048, 5120
    print(f"[case] determinism block config 4 flags={flags}", flush=True)
    w = make_weights(oracle, C, Cc, F, seed=400)
    dev, bw = to_device(w)
    if flags & ops.MI_BLOCK_JOINT_QKV:
        joint = DeviceBuffer.from_array(np.concatenate([w["attn1_q"], w["attn1_k"], w["attn1_v"]]))
        nb = w["attn1_q"].nbytes
        bw = ops.BlockWeights(**dict(dev, attn1_q=joint.value, attn1_k=joint.value + nb,
                                     attn1_v=joint.value + 2 * nb))
    dims = ops.BlockDims(B, T, C, H, Tc, Cc, F, flags)
    x = oracle.normal(1, B * T * C)
    dc = DeviceBuffer.from_array(oracle.normal(6, B * Tc * Cc).astype(np.float16).astype(np.float32))
    dl = DeviceBuffer.from_array(oracle.uniform_int(8, 1, Tc, B).astype(np.int32))
    ws = DeviceBuffer(ops.block_workspace_bytes(dims))
    outs = []
    for _ in range(2):
        dx = DeviceBuffer.from_array(x)
        ops.sdxl_block_forward(bw, dims, dx, dc, ws, ctx_len=dl)
        synchronize()
        outs.append(dx.download(np.float32, x.size))
    assert np.all(np.isfinite(outs[0])) and np.array_equal(outs[0], outs[1])


def test_nn_gemm_repeats_bit_for_bit(gpu, oracle):
    M, N, K = 320, 4096, 2880
    payload, scales = oracle.q8_0_to_split(q8_weights(oracle, 31, M, K), M * K)
    dq, ds = DeviceBuffer.from_array(payload), DeviceBuffer.from_array(scales)
    dB = DeviceBuffer.from_array(oracle.normal(32, K * N))
    ws = DeviceBuffer(ops.gemm_nn_workspace_bytes(M, N, K))
    outs = []
    for _ in range(2):
        dC = DeviceBuffer(M * N * 4)
        ops.gemm_nn_q8(dq, ds, dB, dC, M, N, K, workspace=ws)
        synchronize()
        outs.append(dC.download(np.float32, M * N))
    assert np.array_equal(outs[0], outs[1])
