"""Writes the golden fixtures in tests/golden/.

q8_0_reference.npz  -- Q8_0 blocks (random N(0,0.02) weights quantised by the
    oracle's generator plus known-answer blocks: q in {-128,-127,-1,0,1,127},
    d = +-0, subnormal, min normal, 1, max finite, inf, nan) and what the
    REFERENCE'S OWN GGUF reader returns for them (GgufFile::readFloat and
    ::readQ8, src/Modules/Model/Gguf.cpp:514-557, compiled from
    /root/reference into oracle/_ref by oracle/Makefile). Requires oracle/_ref.
gemm_bench_case.npz -- the reference GEMM harness's correctness case
    (tests/gemm_q8_bench.cpp:59-80: M=N=100, K=96, A = i8/127, B int8,
    scales 0.01) with our portable generator, expected C in fp64.
attn_ref_shapes.npz -- the reference attention test's four shapes
    (tests/fused_attn_test.cpp:74-79) with inputs on an fp16-exact grid
    (k/2048, |k| <= 2048) and the fp64 online-softmax outputs.

gguf_sample_ref.npz -- the sample checkpoint of tests/gguf_writer.py
    (sample_spec: every metadata type, F32 / F16 / BF16 / Q4_0 / Q8_0 / Q4_K
    tensors) and what the REFERENCE'S OWN GgufFile returns for it opened with
    the UNet prefix: tensor table, data offset, readFloat and readQ8Into per
    tensor (Gguf.cpp:290-583). Requires oracle/_ref.

Run from the repo root: python tests/golden/gen_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import binding as ob  # noqa: E402

sys.path.insert(0, str(ROOT / "tests"))
import gguf_writer as gw  # noqa: E402

OUT = Path(__file__).resolve().parent


def kat_blocks() -> np.ndarray:
    ds = [0x0000, 0x8000, 0x0001, 0x03ff, 0x0400, 0x3c00, 0xbc00, 0x7bff, 0x2e66, 0x7c00, 0xfc00, 0x7e00]
    qs = np.array([-128, -127, -1, 0, 1, 127] * 5 + [42, -42], dtype=np.int8)
    out = []
    for i, d in enumerate(ds):
        blk = np.zeros(34, dtype=np.uint8)
        blk[0], blk[1] = d & 0xff, d >> 8
        blk[2:] = np.roll(qs, i).view(np.uint8)
        out.append(blk)
    return np.concatenate(out)


def gen_q8() -> None:
    rows, cols = 16, 96
    w = ob.normal(101, rows * cols, 0.0, 0.02)
    blocks = np.concatenate([ob.q8_0_quantize(w), kat_blocks()])  # 12 KAT blocks = 4 rows of 96
    rows += 4
    res = ob.ref_q8_0_decode(blocks, rows, cols)
    if res is None:
        raise SystemExit("oracle/_ref/libgguf_ref.so missing: build it with `make -C oracle` "
                         "where /root/reference is present")
    f, q, s, q2, s2 = res
    assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32))
    np.savez_compressed(OUT / "q8_0_reference.npz", blocks=blocks, rows=rows, cols=cols, dequant=f,
                        payload=q, scales=s)


def gen_gemm() -> None:
    M, N, K = 100, 100, 96
    A = (ob.uniform_int(201, -127, 127, M * K).astype(np.float32) / np.float32(127.0)).astype(np.float32)
    B = ob.uniform_int(202, -127, 127, N * K).astype(np.int8)
    S = np.full((N * K + 31) // 32, 0.01, dtype=np.float32)
    C = ob.gemm_nt_q8_split(A, B, S, M, N, K, acc64=True)
    np.savez_compressed(OUT / "gemm_bench_case.npz", M=M, N=N, K=K, A=A, B=B, S=S, C=C)


def gen_attn() -> None:
    shapes = [(32, 32, 320, 5, 1), (32, 77, 1280, 20, 0), (64, 64, 320, 8, 1), (48, 96, 512, 8, 0)]
    data = {}
    for i, (Tq, Tk, C, heads, causal) in enumerate(shapes):
        def grid(seed, n):
            return (ob.uniform_int(seed, -2048, 2048, n).astype(np.float32) / np.float32(2048.0)).astype(np.float16)
        q, k, v = grid(300 + 3 * i, Tq * C), grid(301 + 3 * i, Tk * C), grid(302 + 3 * i, Tk * C)
        o = ob.fused_attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), Tq, Tk, C, heads,
                               bool(causal))
        data[f"s{i}_shape"] = np.array([Tq, Tk, C, heads, causal])
        data[f"s{i}_q"], data[f"s{i}_k"], data[f"s{i}_v"], data[f"s{i}_o"] = q, k, v, o
    np.savez_compressed(OUT / "attn_ref_shapes.npz", **data)


def gen_gguf() -> None:
    import tempfile

    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "sample.gguf"
        data = gw.write(path, gw.sample_spec())
        r = ob.RefGguf(path, gw.PREFIX)
        if not r.ok:
            raise SystemExit(f"reference reader rejects the sample: {r.error}")
        out = {"file_bytes": np.frombuffer(data, dtype=np.uint8), "data_offset": r.data_offset()}
        table = r.tensors()
        out["names"] = np.array([t[0] for t in table])
        for i, (name, ty, dims, off, nb, _) in enumerate(table):
            out[f"t{i}_tob"] = np.array([ty, off, nb], dtype=np.uint64)
            out[f"t{i}_dims"] = np.array(dims, dtype=np.uint64)
            n = int(np.prod(dims))
            f, _ = r.read_float(name, n)
            if f is not None:
                out[f"t{i}_float"] = f
            q, sc, _ = r.read_q8(name, n, True)
            if q is not None:
                out[f"t{i}_q"], out[f"t{i}_s"] = q, sc
        r.close()
    np.savez_compressed(OUT / "gguf_sample_ref.npz", **out)


if __name__ == "__main__":
    if ob.ref_lib() is None:
        raise SystemExit("oracle/_ref/libgguf_ref.so missing: build it with `make -C oracle` "
                         "where /root/reference is present")
    gen_q8()
    gen_gemm()
    gen_attn()
    gen_gguf()
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)
