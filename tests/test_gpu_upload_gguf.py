"""GPU side of the GGUF path: mi_gguf_upload_* place a checkpoint's tensors in
device memory in the layouts the GEMM entries read (sdvkgen.cpp:549-611), and
a weight loaded from a file through each layout multiplies exactly like the
same weight given to the GEMM directly.

Bars: uploads are byte- / bit-exact against the host readers (whose parity
with the reference's Gguf.cpp is tests/test_gguf.py); the GEMM checks use the
north-star bar (max |err| <= 2e-3 x RMS) against the oracle, and the two
layouts must agree bit for bit (both dequantise w = fp16(fp32(d) * q)).
"""
from __future__ import annotations

import numpy as np
import pytest

import gguf_writer as gw
from helpers import assert_parity
from sdvk_amd import ops
from sdvk_amd.gguf import GgufFile
from sdvk_amd.hip import DeviceBuffer, Stream, synchronize

pytestmark = pytest.mark.gpu


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def sample(tmp_path_factory):
    path = tmp_path_factory.mktemp("gguf_gpu") / "sample.gguf"
    gw.write(path, gw.sample_spec())
    return path


def test_uploads_match_host_readers(gpu, sample):
    print("[case] gguf sample uploads", flush=True)
    with GgufFile() as g:
        assert g.open(str(sample), [], gw.PREFIX)
        st = Stream()
        for t in g.tensors():
            raw = g.readRaw(t)
            d = DeviceBuffer(t.nbytes)
            g.upload_raw(t, d, st)
            st.synchronize()
            assert np.array_equal(d.download(np.uint8, t.nbytes), raw), t.name
            host = g.readFloat(t.name, [])
            if host.size:
                f = DeviceBuffer(host.nbytes)
                g.upload_f32(t, f, st)
                st.synchronize()
                assert np.array_equal(bits(f.download(np.float32, host.size)), bits(host)), t.name
            ok, q, s = g.readQ8(t.name, [])
            if ok and s.size:
                dq, ds = DeviceBuffer(q.nbytes), DeviceBuffer(s.nbytes)
                g.upload_q8_split(t, dq, ds, st)
                st.synchronize()
                nb = s.size
                assert np.array_equal(dq.download(np.int8, nb * 32), q[: nb * 32]), t.name
                assert np.array_equal(bits(ds.download(np.float32, nb)), bits(s)), t.name


def test_large_tensor_streams_through_staging(gpu, oracle, tmp_path):
    """A 10240 x 1280 Q8_0 weight (13.9 MB stored, 52 MB as fp32) crosses the
    8 MiB staging buffers several times in every upload."""
    N, K = 10240, 1280
    print(f"[case] gguf large Q8_0 {N}x{K}", flush=True)
    blocks = oracle.q8_0_quantize(oracle.normal(5, N * K, 0.0, 0.02))
    path = tmp_path / "big.gguf"
    gw.write(path, gw.GgufSpec(tensors=[gw.Tensor("ff.weight", (K, N), gw.T_Q8_0, blocks.tobytes())]))
    with GgufFile() as g:
        assert g.open(str(path), [])
        t = g.find("ff.weight")
        assert (t.rows, t.cols) == (N, K)
        d = DeviceBuffer(t.nbytes)
        g.upload_raw(t, d)
        f = DeviceBuffer(N * K * 4)
        g.upload_f32(t, f)
        dq, ds = DeviceBuffer(N * K), DeviceBuffer(N * K // 32 * 4)
        g.upload_q8_split(t, dq, ds)
        synchronize()
        assert np.array_equal(d.download(np.uint8, t.nbytes), blocks)
        want = oracle.q8_0_dequant(blocks, N * K)
        assert np.array_equal(bits(f.download(np.float32, N * K)), bits(want))
        payload, scales = oracle.q8_0_to_split(blocks, N * K)
        assert np.array_equal(dq.download(np.int8, N * K), payload)
        assert np.array_equal(bits(ds.download(np.float32, N * K // 32)), bits(scales))


def test_file_weight_through_both_gemm_layouts(gpu, oracle, tmp_path, tune):
    """A Q8_0 linear weight [N, K] read from a GGUF file feeds mi_gemm_nt_q8_0
    as 34-byte blocks and mi_gemm_nt_q8_split as payload + scales."""
    tune("gemm_cfg", "1")  # one tile config, no K split: both entries sum in the same order
    M, N, K = 300, 640, 1280
    print(f"[case] gguf weight -> gemm M={M} N={N} K={K}", flush=True)
    blocks = oracle.q8_0_quantize(oracle.normal(6, N * K, 0.0, 0.02))
    path = tmp_path / "lin.gguf"
    gw.write(path, gw.GgufSpec(tensors=[gw.Tensor("proj.weight", (K, N), gw.T_Q8_0, blocks.tobytes())]))
    A = oracle.normal(7, M * K)
    dA = DeviceBuffer.from_array(A)
    with GgufFile() as g:
        assert g.open(str(path), [])
        t = g.find("proj.weight")
        dW = DeviceBuffer(t.nbytes)
        g.upload_raw(t, dW)
        dq, ds = DeviceBuffer(N * K), DeviceBuffer(N * K // 32 * 4)
        g.upload_q8_split(t, dq, ds)
    synchronize()
    c1, c2 = DeviceBuffer(M * N * 4), DeviceBuffer(M * N * 4)
    ops.gemm_nt_q8_0(dA, dW, c1, M, N, K)
    ops.gemm_nt_q8(dA, dq, c2, ds, M, N, K)
    synchronize()
    got1, got2 = c1.download(np.float32, M * N), c2.download(np.float32, M * N)
    want = oracle.gemm_nt_q8_0(A, blocks, M, N, K, threads=oracle.max_threads())
    assert_parity(got1, want, what="blocks layout")
    assert np.array_equal(got1, got2)
