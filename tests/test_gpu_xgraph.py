"""GPU: the hot-path calls captured into a HIP graph (stream capture of the
C-ABI launches) and replayed give the eager results.

The sequence holds a GEMM without K splits, a K-split GEMM (partials in a
workspace, then the reduce pass), a K-split tiled NN GEMM (the same), a
key-padded fp16 attention and a key-split fp16 attention (pieces in a
workspace, then the merge pass; the split forced with the attn_split override). The graph is replayed three times with eager work
and a synchronisation between the replays; every replay must equal the eager
results bit for bit (every sum has a fixed order).
"""
import numpy as np
import pytest

from helpers import q8_weights
from sdvk_amd import MI_F16, MI_F32, hip, ops
from sdvk_amd.hip import DeviceBuffer

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(gpu, oracle, tune):
    print("[case] graph capture / replay of GEMM, split-K GEMM, NN GEMM, attention", flush=True)
    st = hip.Stream()
    M1, N1, K1 = 2048, 1280, 1280            # no K split
    M2, N2, K2 = 154, 640, 2048              # K split through the workspace
    M3, N3, K3 = 320, 1024, 640              # tiled NN GEMM with K splits
    B, T, Tk, H = 2, 130, 77, 2
    C = H * 64
    A1 = DeviceBuffer.from_array(oracle.normal(1, M1 * K1))
    W1 = DeviceBuffer.from_array(q8_weights(oracle, 2, N1, K1))
    A2 = DeviceBuffer.from_array(oracle.normal(3, M2 * K2))
    W2 = DeviceBuffer.from_array(q8_weights(oracle, 4, N2, K2))
    pay, sc = oracle.q8_0_to_split(q8_weights(oracle, 5, M3, K3), M3 * K3)
    P3, S3 = DeviceBuffer.from_array(pay), DeviceBuffer.from_array(sc)
    B3 = DeviceBuffer.from_array(oracle.normal(6, K3 * N3))
    q = DeviceBuffer.from_array(oracle.normal(7, B * T * C).astype(np.float16))
    k = DeviceBuffer.from_array(oracle.normal(8, B * Tk * C).astype(np.float16))
    v = DeviceBuffer.from_array(oracle.normal(9, B * Tk * C).astype(np.float16))
    kv_len = DeviceBuffer.from_array(np.array([77, 30], dtype=np.int32))
    Ts, Tks, Hs = 256, 512, 2
    qs = DeviceBuffer.from_array(oracle.normal(10, Ts * Hs * 64).astype(np.float16))
    ks = DeviceBuffer.from_array(oracle.normal(11, Tks * Hs * 64).astype(np.float16))
    vs = DeviceBuffer.from_array(oracle.normal(12, Tks * Hs * 64).astype(np.float16))
    skw = dict(batch=1, Tq=Ts, Tk=Tks, C=Hs * 64, heads=Hs, in_dtype=MI_F16, out_dtype=MI_F16)
    tune("attn_nw", "4")
    tune("attn_split", "2:4")
    ws4 = DeviceBuffer(ops.fused_attention_ws_bytes(**skw))
    assert ws4.nbytes > 0, "the forced key split has no workspace"
    outs = [DeviceBuffer(M1 * N1 * 4), DeviceBuffer(M2 * N2 * 4), DeviceBuffer(M3 * N3 * 4),
            DeviceBuffer(B * T * C * 4), DeviceBuffer(Ts * Hs * 64 * 2)]
    ws2 = DeviceBuffer(ops.gemm_workspace_bytes(M2, N2, K2))
    ws3 = DeviceBuffer(ops.gemm_nn_workspace_bytes(M3, N3, K3))
    assert ws2.nbytes > 0 and ws3.nbytes > 0, "the shapes no longer split K"

    def sequence():
        ops.gemm_nt_q8_0(A1, W1, outs[0], M1, N1, K1, stream=st)
        ops.gemm_nt_q8_0(A2, W2, outs[1], M2, N2, K2, workspace=ws2, stream=st)
        ops.gemm_nn_q8(P3, S3, B3, outs[2], M3, N3, K3, workspace=ws3, stream=st)
        ops.fused_attention_ex(q, k, v, outs[3], batch=B, Tq=T, Tk=Tk, C=C, heads=H, in_dtype=MI_F16,
                               out_dtype=MI_F32, kv_len=kv_len, stream=st)
        ops.fused_attention_ws(qs, ks, vs, outs[4], ws4, stream=st, **skw)

    def read():
        st.synchronize()
        return [o.download(np.float32, o.nbytes // 4) for o in outs]

    sequence()
    eager = read()
    for o in outs:
        o.fill_zero(st)
    st.synchronize()

    g = hip.Graph(st)
    g.begin()
    sequence()
    g.end()
    # capture records, it does not run: the outputs are still zero
    assert all(not np.any(x) for x in read()), "the capture ran the kernels"

    other = DeviceBuffer(M1 * N1 * 4)
    for rep in range(3):
        for o in outs:
            o.fill_zero(st)
        g.launch()
        got = read()
        ops.gemm_nt_q8_0(A1, W1, other, M1, N1, K1, stream=st)  # eager work between replays
        st.synchronize()
        for i, what in enumerate(("GEMM", "K-split GEMM", "K-split NN GEMM", "attention", "key-split attention")):
            assert np.array_equal(got[i], eager[i]), f"replay {rep}: {what} differs from eager"
        print(f"  replay {rep} ok", flush=True)
