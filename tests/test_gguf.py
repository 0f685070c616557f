"""GGUF reader parity (no GPU): libmi_sdvk.so's mi_gguf_* entries (through the
sdvk_amd.gguf.GgufFile mirror) against

  * the reference's own ofc::GgufFile (src/Modules/Model/Gguf.cpp, compiled
    from /root/reference into oracle/_ref by oracle/Makefile) on the same files:
    table, metadata, getters, readRaw / readFloat / readQ8 / readQ8Into,
    bit-exact, and the same accept / reject verdict on malformed files;
  * independent numpy decodes of the payloads the writer put in (these need
    no reference build);
  * tests/golden/gguf_sample_ref.npz, the reference's decode of the sample file
    (travels where /root/reference does not);
  * the ggdims rules of sdvkgen.cpp:151-176 on hand-computed shapes.
"""
from __future__ import annotations

import math
import struct
from pathlib import Path

import numpy as np
import pytest

import gguf_writer as gw
from oracle import binding as ob
from sdvk_amd import _lib
from sdvk_amd.gguf import GgufFile

GOLDEN = Path(__file__).parent / "golden"
needs_ref = pytest.mark.skipif(ob.ref_lib() is None, reason="oracle/_ref (the reference's Gguf.cpp) not built here")


@pytest.fixture(scope="module")
def sample(tmp_path_factory):
    path = tmp_path_factory.mktemp("gguf") / "sample.gguf"
    gw.write(path, gw.sample_spec())
    return path


def bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def open_ours(path, prefix=""):
    g = GgufFile()
    err = []
    assert g.open(str(path), err, prefix), err
    return g


# ---------------------------------------------------------------- vs reference --

@needs_ref
@pytest.mark.parametrize("prefix", ["", gw.PREFIX])
def test_table_and_data_match_reference(sample, prefix):
    g, r = open_ours(sample, prefix), ob.RefGguf(sample, prefix)
    assert r.ok, r.error
    assert g.version() == r.version() == 3
    assert g.dataOffset() == r.data_offset()
    rt = r.tensors()
    assert len(g.tensors()) == len(rt) > 0
    for t, (name, ty, dims, off, nb, shape) in zip(g.tensors(), rt):
        assert (t.name, t.type, t.dims, t.offset, t.nbytes) == (name, ty, dims, off, nb)
        assert t.shape() == shape                      # GgufTensor::shape, Gguf.cpp:96-102
        raw = g.readRaw(t)
        assert raw is not None and np.array_equal(raw, r.read_raw(t.index, t.nbytes))
        ours = g.readFloat(t.name, [])
        ref, ref_err = r.read_float(t.name, t.nElems())
        if ref is None:
            assert ours.size == 0, f"{name}: reference rejects ({ref_err}) but ours decoded"
        else:
            assert np.array_equal(bits(ours), bits(ref)), name
        ok, q, s = g.readQ8(t.name, [])
        for into in (False, True):
            rq, rs, _ = r.read_q8(t.name, t.nElems(), into)
            assert ok == (rq is not None), name
            if ok:
                nb = t.nElems() // 32
                assert np.array_equal(q[: nb * 32], rq[: nb * 32]) and np.array_equal(bits(s), bits(rs)), name


@needs_ref
def test_metadata_and_getters_match_reference(sample):
    g, r = open_ours(sample), ob.RefGguf(sample)
    keys = [k for k, _, _ in gw.sample_spec().meta] + ["no.such.key"]
    for k in keys:
        m, rm = g.meta(k), r.meta(k)
        assert (m is None) == (rm is None), k
        if m is None:
            continue
        assert (m.type, m.u, m.b, m.s, m.arrType) == (rm["type"], rm["u"], rm["b"], rm["s"], rm["arr_type"]), k
        assert struct.pack("<d", m.f) == struct.pack("<d", rm["f"]), k
        if m.arrType in (gw.F32, gw.F64):
            assert [struct.pack("<d", x) for x in m.items] == [struct.pack("<d", x) for x in rm["items"]], k
        else:
            assert m.items == rm["items"], k
        for kind, fn, dflt in (("u64", g.getU64, 17), ("i64", g.getI64, -17), ("f64", g.getF64, 0.5),
                               ("f32", g.getF32, 0.25), ("str", g.getStr, "dflt")):
            a, b = fn(k, dflt), r.get(kind, k, dflt)
            if isinstance(a, float) and math.isnan(a):
                assert math.isnan(b), (k, kind)
            else:
                assert a == b, (k, kind, a, b)


def malformed_cases():
    """(id, bytes): files the reader must reject, or accept, exactly like the reference."""
    base = gw.sample_spec()
    good = gw.build(base)
    cases = [("sample", good)]
    s = gw.sample_spec()
    s.magic = b"GGUX"
    cases.append(("bad_magic", gw.build(s)))
    for v in (1, 2, 4):
        s = gw.sample_spec()
        s.version = v
        cases.append((f"version{v}", gw.build(s)))
    # cuts inside the header, the metadata and the tensor table
    head_end = 24
    kv_end = head_end + sum(len(gw._string(k)) + 4 + len(gw._value(t, v)) for k, t, v in base.meta)
    for cut in (3, 12, 30, kv_end - 5, kv_end + 9, kv_end + 40):
        cases.append((f"truncated{cut}", good[:cut]))
    s = gw.sample_spec()
    s.n_tensors = (1 << 24) + 1
    cases.append(("implausible_count", gw.build(s)))
    for nd in (0, 5):
        s = gw.GgufSpec(tensors=[gw.Tensor("x", (1,) * max(nd, 0), gw.T_F32, b"\0" * 4)])
        cases.append((f"ndims{nd}", gw.build(s)))
    s = gw.GgufSpec(tensors=[gw.Tensor("x", (4,), gw.T_F32, b"\0" * 16), gw.Tensor("x", (4,), gw.T_F32, b"\0" * 16)])
    cases.append(("duplicate", gw.build(s)))
    for name, t, v in (("align3", gw.U32, 3), ("align0", gw.U32, 0), ("align_f32", gw.F32, 64.0),
                       ("align_str", gw.STR, "64"), ("align_u8", gw.U8, 16), ("align_bool", gw.BOOL, True)):
        s = gw.GgufSpec(meta=[("general.alignment", t, v)], tensors=[gw.Tensor("x", (8,), gw.T_F32, b"\0" * 32)])
        cases.append((name, gw.build(s)))
    s = gw.GgufSpec(meta=[("general.alignment", gw.U32, 1 << 20)], tensors=[gw.Tensor("x", (8,), gw.T_F32, b"\1" * 32)])
    cases.append(("data_offset_past_eof", gw.build(s)[:200]))
    cases.append(("huge_string", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", (1 << 30) + 1) + b"k"))
    cases.append(("huge_array", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw._string("k")
                  + struct.pack("<IIQ", gw.ARR, gw.U8, (1 << 32) + 1)))
    cases.append(("unknown_kv_type", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw._string("k") + struct.pack("<II", 13, 0)))
    cases.append(("nested_array", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw._string("k")
                  + struct.pack("<IIQ", gw.ARR, gw.ARR, 1) + struct.pack("<IQ", gw.U8, 0)))
    cases.append(("empty_file", b""))
    return cases


@needs_ref
@pytest.mark.parametrize("case", malformed_cases(), ids=lambda c: c[0])
def test_accept_reject_matches_reference(tmp_path, case):
    name, data = case
    path = tmp_path / f"{name}.gguf"
    path.write_bytes(data)
    ours, err = GgufFile(), []
    ok = ours.open(str(path), err)
    r = ob.RefGguf(path)
    assert ok == r.ok, f"{name}: ours {'accepts' if ok else 'rejects: ' + err[0]}, reference " \
                       f"{'accepts' if r.ok else 'rejects: ' + str(r.error)}"
    if ok:
        assert [t.name for t in ours.tensors()] == [t[0] for t in r.tensors()]
        assert ours.dataOffset() == r.data_offset()


@needs_ref
def test_tensor_data_past_end_of_file(tmp_path):
    """The table may point past the file: open succeeds, reads fail (readRaw's read error)."""
    s = gw.GgufSpec(tensors=[gw.Tensor("ok", (8,), gw.T_F32, b"\0" * 32),
                             gw.Tensor("far", (64,), gw.T_Q8_0, b"", offset=1 << 20)])
    path = tmp_path / "far.gguf"
    gw.write(path, s)
    g, r = open_ours(path), ob.RefGguf(path)
    assert r.ok
    assert g.readFloat("far", []).size == 0 and r.read_float("far", 64)[0] is None
    assert not g.readQ8("far", [])[0] and r.read_q8("far", 64, True)[0] is None
    assert g.readFloat("ok", []).size == 8 and r.read_float("ok", 8)[0].size == 8


# ------------------------------------------------------ independent decodes --

def test_decodes_against_numpy(sample):
    """Each payload decodes to what the writer encoded: F32 / F16 / BF16 bit
    patterns, Q8_0 fp32(d) * q, Q4_0 d * (nibble - 8) with byte i's low nibble
    at element 2i (Gguf.cpp:499-511), a partial trailing Q8_0 block -> zeros."""
    spec = gw.sample_spec()
    g = open_ours(sample)
    for t in spec.tensors:
        raw = np.frombuffer(t.data, dtype=np.uint8)
        n = int(np.prod(t.dims))
        got = g.readFloat(t.name, [])
        if t.type == gw.T_F32:
            want = raw.view("<f4")
        elif t.type == gw.T_F16:
            want = raw.view("<f2").astype(np.float32)
        elif t.type == gw.T_BF16:
            want = (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
        elif t.type == gw.T_Q8_0:
            blk = raw.reshape(-1, 34)
            nb = n // 32
            d = blk[:nb, :2].copy().view("<f2").astype(np.float32)
            want = np.zeros(n, dtype=np.float32)
            want[: nb * 32] = (d * blk[:nb, 2:].view(np.int8).astype(np.float32)).reshape(-1)
            ok, q, s = g.readQ8(t.name, [])
            assert ok and np.array_equal(q[: nb * 32], blk[:nb, 2:].view(np.int8).reshape(-1))
            assert np.array_equal(bits(s), bits(d.reshape(-1)))
        elif t.type == gw.T_Q4_0:
            blk = raw.reshape(-1, 18)
            d = blk[:, :2].copy().view("<f2").astype(np.float32)
            nib = np.empty((blk.shape[0], 32), dtype=np.int32)
            nib[:, 0::2] = blk[:, 2:] & 0x0F
            nib[:, 1::2] = blk[:, 2:] >> 4
            want = (d * (nib - 8).astype(np.float32)).reshape(-1)
        else:
            assert got.size == 0  # no decoder for this type (Q4_K)
            continue
        assert np.array_equal(bits(got), bits(want)), t.name


def test_q4_0_nibble_order_known_answer(tmp_path):
    """Byte 0x21 in block 0 with d = 1: element 0 = 1 - 8, element 1 = 2 - 8."""
    nib = np.zeros((1, 32), dtype=np.uint8)
    nib[0, 0], nib[0, 1] = 1, 2
    path = tmp_path / "q4.gguf"
    gw.write(path, gw.GgufSpec(tensors=[gw.Tensor("w", (32,), gw.T_Q4_0, gw.q4_0_bytes(np.array([1.0]), nib))]))
    got = open_ours(path).readFloat("w", [])
    assert got[0] == -7.0 and got[1] == -6.0 and np.all(got[2:] == -8.0)
    assert gw.q4_0_bytes(np.array([1.0]), nib)[2] == 0x21


def test_logical_dims_ggdims_rules(sample):
    """sdvkgen.cpp:151-176: orig_shape wins (rows = first, cols = product of the
    rest), else 1-D (n, 1), 2-D (dims[1], dims[0]), N-D (last dim, product of
    the others). The orig_shape key is looked up by the (prefix-stripped) name."""
    g = open_ours(sample, gw.PREFIX)
    want = {"a.weight": (3, 64), "b.bias": (96, 1), "c.weight": (3, 64), "conv.weight": (8, 32 * 3 * 3),
            "g.weight": (4, 3 * 3 * 32), "i.weight": (40, 1), "e.weight": (5, 96)}
    for name, rc in want.items():
        t = g.find(name)
        assert (t.rows, t.cols) == rc, name
    full = open_ours(sample)  # no prefix: the key comfy.gguf.orig_shape.conv.weight no longer names the tensor
    t = full.find(gw.PREFIX + "conv.weight")
    assert (t.rows, t.cols) == (8, 3 * 3 * 32)


def test_errors_and_missing(sample, tmp_path):
    g = open_ours(sample)
    err = []
    assert g.readFloat("nope", err).size == 0 and "not found" in err[0]
    err = []
    assert g.readFloat("cond_stage_model.h.weight", err).size == 0 and "unsupported" in err[0]
    err = []
    ok, _, _ = g.readQ8(gw.PREFIX + "a.weight", err)
    assert not ok and "not Q8_0" in err[0]
    assert g.find("nope") is None and g.meta("nope") is None
    assert g.getU64("general.architecture", 5) == 5 and g.getStr("sdxl.u8", "x") == "x"
    bad = GgufFile()
    err = []
    assert not bad.open(str(tmp_path / "missing.gguf"), err) and "cannot open" in err[0]
    lib = _lib.load()
    assert lib.mi_gguf_open(None, None, None) == _lib.MI_ERR_INVALID_ARG
    assert lib.mi_gguf_tensor(g._h, 10**6, None) == _lib.MI_ERR_NOT_FOUND


def test_prefix_filters_and_strips(sample):
    g = open_ours(sample, gw.PREFIX)
    names = [t.name for t in g.tensors()]
    assert names == [t.name[len(gw.PREFIX):] for t in gw.sample_spec().tensors if t.name.startswith(gw.PREFIX)]
    assert g.find("a.weight") is not None and g.find(gw.PREFIX + "a.weight") is None


def test_golden_reference_decode(tmp_path):
    """The reference reader's results on the sample file, recorded by
    tests/golden/gen_golden.py where /root/reference is present."""
    f = np.load(GOLDEN / "gguf_sample_ref.npz")
    path = tmp_path / "sample.gguf"
    data = gw.write(path, gw.sample_spec())
    assert np.array_equal(np.frombuffer(data, dtype=np.uint8), f["file_bytes"]), "sample file bytes changed"
    g = open_ours(path, gw.PREFIX)
    names = [str(x) for x in f["names"]]
    assert [t.name for t in g.tensors()] == names
    assert g.dataOffset() == int(f["data_offset"])
    for i, name in enumerate(names):
        t = g.find(name)
        assert (t.type, t.offset, t.nbytes) == tuple(int(x) for x in f[f"t{i}_tob"])
        assert t.dims == tuple(int(x) for x in f[f"t{i}_dims"])
        if f"t{i}_float" in f:
            assert np.array_equal(bits(g.readFloat(name, [])), f[f"t{i}_float"].view(np.uint32)), name
        if f"t{i}_q" in f:
            ok, q, s = g.readQ8(name, [])
            nb = t.nElems() // 32
            assert ok and np.array_equal(q[: nb * 32], f[f"t{i}_q"][: nb * 32]) and np.array_equal(bits(s), f[f"t{i}_s"].view(np.uint32))
