"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/mi_sdvk.h declares, and rejects bad arguments before touching HIP."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from sdvk_amd import _lib, ops

HEADER = Path(__file__).resolve().parents[1] / "include" / "mi_sdvk.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for n in ["mi_gemm_nt_q8_0", "mi_gemm_nt_q8_split", "mi_fused_attention", "mi_fused_attention_ex",
              "mi_fused_attn_supported", "mi_q8_0_dequant", "mi_q8_split_dequant", "mi_q8_0_to_split",
              "mi_status_string", "mi_last_error", "mi_version"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"libmi_sdvk.so does not export {name}"
        assert name in _lib.SIGNATURES, f"no ctypes signature for {name}"


def test_attn_args_struct_layout():
    # mi_attn_args: 4 pointers, 5 u32, 3 i32, 8 u64, 1 pointer, 1 float, 1 i32 (precision)
    assert ctypes.sizeof(_lib.MiAttnArgs) == 4 * 8 + 5 * 4 + 3 * 4 + 8 * 8 + 8 + 4 + 4


def test_status_strings():
    lib = _lib.load()
    assert lib.mi_status_string(0) == b"ok"
    assert lib.mi_status_string(2) == b"unsupported shape"
    assert lib.mi_status_string(99) == b"unknown status"
    assert lib.mi_version() >= 100


@pytest.mark.parametrize("C,heads,ok", [(640, 10, True), (1280, 20, True), (320, 8, True), (320, 5, True),
                                        (64, 1, True), (65, 1, False), (100, 3, False), (0, 1, False),
                                        (128, 0, False), (130, 2, False)])
def test_fused_attn_supported_predicate(C, heads, ok):
    """fused_attn.cpp:34-38: heads | C and 1 <= C/heads <= 64."""
    assert ops.fused_attn_supported(C, heads) is ok


def test_errors_are_returned_not_raised_through_the_abi():
    lib = _lib.load()
    # null pointers -> MI_ERR_INVALID_ARG, detail in mi_last_error
    st = lib.mi_gemm_nt_q8_0(None, None, None, None, 8, 8, 32, 0, 0, 0, 1, 0, 0, None)
    assert st == _lib.MI_ERR_INVALID_ARG
    assert b"null" in lib.mi_last_error()
    # empty problem is a no-op
    assert lib.mi_gemm_nt_q8_0(None, None, None, None, 0, 8, 32, 0, 0, 0, 1, 0, 0, None) == _lib.MI_OK
    # K % 32 != 0 on the block entry: unsupported (checked before any device work)
    fake = 1 << 20
    st = lib.mi_gemm_nt_q8_0(fake, fake * 2, None, fake * 3, 8, 8, 48, 0, 0, 0, 1, 0, 0, None)
    assert st == _lib.MI_ERR_UNSUPPORTED
    # misaligned A
    st = lib.mi_gemm_nt_q8_0(fake + 4, fake * 2, None, fake * 3, 8, 8, 32, 0, 0, 0, 1, 0, 0, None)
    assert st == _lib.MI_ERR_ALIGNMENT
    # C overlapping A
    st = lib.mi_gemm_nt_q8_0(fake, fake * 2, None, fake + 64, 8, 8, 32, 0, 0, 0, 1, 0, 0, None)
    assert st == _lib.MI_ERR_ALIASING
    # bad mode (0 store, 1 accumulate, 2 accumulate + bias)
    for entry_mode in (3, 7):
        st = lib.mi_gemm_nt_q8_split(fake, fake * 2, fake * 4, None, fake * 3, 8, 8, 32, entry_mode, 0, 0, 1, 0, 0,
                                     None)
        assert st == _lib.MI_ERR_INVALID_ARG
        st = lib.mi_gemm_nt_q8_0(fake, fake * 2, None, fake * 3, 8, 8, 32, entry_mode, 0, 0, 1, 0, 0, None)
        assert st == _lib.MI_ERR_INVALID_ARG
    # GEGLU GEMM: K must be a positive multiple of 32; G must not overlap A
    assert lib.mi_gemm_nt_q8_0_geglu(fake, fake * 2, None, fake * 3, 8, 8, 48, 0, 0, None) == _lib.MI_ERR_UNSUPPORTED
    assert lib.mi_gemm_nt_q8_0_geglu(fake, fake * 2, None, fake * 3, 8, 8, 0, 0, 0, None) == _lib.MI_ERR_UNSUPPORTED
    assert lib.mi_gemm_nt_q8_0_geglu(fake, fake * 2, None, fake + 64, 8, 8, 32, 0, 0, None) == _lib.MI_ERR_ALIASING
    assert lib.mi_gemm_nt_q8_0_geglu(None, None, None, None, 0, 8, 32, 0, 0, None) == _lib.MI_OK
    # the split entry takes any K (the scalar gemm_nt_q8 does, gemm_nt_q8.comp:52-80) and an A that is only
    # 4-byte aligned; a 2-byte-aligned A is an alignment error
    st = lib.mi_gemm_nt_q8_split(fake + 2, fake * 2, fake * 4, None, fake * 3, 8, 8, 30, 0, 0, 0, 1, 0, 0, None)
    assert st == _lib.MI_ERR_ALIGNMENT
    # workspace entries: a workspace overlapping an operand, or misaligned
    st = lib.mi_gemm_nt_q8_0_ws(fake, fake * 2, None, fake * 3, 8, 8, 32, 0, 0, 0, 1, 0, 0, fake * 3 + 16, 4096,
                                None)
    assert st == _lib.MI_ERR_ALIASING
    st = lib.mi_gemm_nt_q8_0_ws(fake, fake * 2, None, fake * 3, 8, 8, 32, 0, 0, 0, 1, 0, 0, fake * 5 + 4, 4096, None)
    assert st == _lib.MI_ERR_ALIGNMENT
    # the workspace a plan needs: none for a grid that fills the GPU, split planes for a small one
    assert lib.mi_gemm_nt_q8_workspace_bytes(8192, 5120, 640, 1) == 0
    assert lib.mi_gemm_nt_q8_workspace_bytes(154, 640, 2048, 1) == 8 * 154 * 640 * 4
    assert lib.mi_gemm_nt_q8_workspace_bytes(154, 640, 2048, 2) == 2 * 4 * 154 * 640 * 4
    assert lib.mi_gemm_nn_q8_workspace_bytes(1280, 1024, 640, 1) == 2 * 1280 * 1024 * 4
    assert lib.mi_gemm_nn_q8_workspace_bytes(1280, 1024, 100, 1) == 0  # K % 64 != 0: the untiled kernel
    # unsupported attention head dim: the reference exit(1)s; here an error code
    st = lib.mi_fused_attention(fake, fake * 2, fake * 3, fake * 4, 8, 8, 130, 1, 0, None)
    assert st == _lib.MI_ERR_UNSUPPORTED
    # attention output aliasing q
    st = lib.mi_fused_attention(fake, fake * 2, fake * 3, fake, 8, 8, 128, 2, 0, None)
    assert st == _lib.MI_ERR_ALIASING
    # dequant: n not a multiple of 32
    assert lib.mi_q8_0_dequant(fake, fake * 2, 0, 33, None) == _lib.MI_ERR_UNSUPPORTED
    assert lib.mi_q8_0_dequant(fake, fake * 2, 7, 32, None) == _lib.MI_ERR_INVALID_ARG


def test_attention_workspace_entry_plans_and_errors():
    """mi_fused_attention_ws_bytes / mi_fused_attention_ws on the host side: the
    key-split plan's size for self-attention L1 (640 query blocks of 128 for
    2 x 256 resident: the last 128 in 2 key ranges, one per CU, 128 x 64 fp32 O rows plus
    a max and a sum per query and piece), none for the shapes without a plan,
    and the workspace's own argument errors, all before any device work."""
    import ctypes
    lib = _lib.load()
    fake = 1 << 24

    def args(B, H, Tq, Tk, causal=0, kv_len=None):
        x = _lib.MiAttnArgs()
        C = 64 * H
        x.q, x.k, x.v, x.out = fake, fake * 4, fake * 8, fake * 12
        x.batch, x.Tq, x.Tk, x.C, x.heads, x.causal = B, Tq, Tk, C, H, causal
        x.in_dtype = x.out_dtype = _lib.MI_F16
        x.ldq = x.ldk = x.ldv = x.ldo = C
        x.sq, x.so, x.sk, x.sv = Tq * C, Tq * C, Tk * C, Tk * C
        x.kv_len = kv_len
        return x

    assert lib.mi_fused_attention_ws_bytes(None) == 0
    l1 = args(2, 10, 4096, 4096)
    assert lib.mi_fused_attention_ws_bytes(ctypes.byref(l1)) == 128 * 2 * (128 * 64 + 2 * 128) * 4
    # 2 x 9 heads: 576 blocks, the last 64 in 4 ranges; 2 x 12 heads: 768, the last 256 (one per CU) unsplit
    assert lib.mi_fused_attention_ws_bytes(ctypes.byref(args(2, 9, 4096, 4096))) == 64 * 4 * (128 * 64 + 2 * 128) * 4
    for other in (args(2, 20, 1024, 1024), args(2, 12, 4096, 4096), args(2, 10, 4096, 77),
                  args(2, 10, 4096, 4096, causal=1),
                  args(2, 10, 4096, 4096, kv_len=fake * 16)):
        assert lib.mi_fused_attention_ws_bytes(ctypes.byref(other)) == 0
    need = 128 * 2 * (128 * 64 + 2 * 128) * 4
    # a workspace overlapping the output, or not 16-byte aligned
    st = lib.mi_fused_attention_ws(ctypes.byref(l1), fake * 12 + 64, need, None)
    assert st == _lib.MI_ERR_ALIASING
    st = lib.mi_fused_attention_ws(ctypes.byref(l1), fake * 20 + 8, need, None)
    assert st == _lib.MI_ERR_ALIGNMENT


def test_python_mirror_raises_mi_error():
    with pytest.raises(ops.MiError) as e:
        ops.fused_attention(ops.FusedAttnArgs(1 << 20, 2 << 20, 3 << 20, 4 << 20, 8, 8, 130, 1))
    assert e.value.status == _lib.MI_ERR_UNSUPPORTED
    with pytest.raises(ValueError):
        ops.dispatch("gemm_nt_q8_v_b", [1, 2, 3, 4], ops.Pg(8, 8, 32))  # 5 bindings expected
    with pytest.raises(ValueError):
        ops.dispatch("no_such_kernel", [], None)


def test_c_and_cpp_callers_link_and_run(tmp_path):
    """include/mi_sdvk.h compiles as C99 and C++17, and a C++ program linked
    against libmi_sdvk.so makes the host-side calls (no GPU work): status text,
    argument rejection through the return value, the GGUF reader."""
    import shutil
    import subprocess
    import sys

    sys.path.insert(0, str(Path(__file__).resolve().parent))
    import gguf_writer as gw
    from sdvk_amd.gguf import GgufFile

    if not shutil.which("gcc") or not shutil.which("g++"):
        pytest.skip("no host C/C++ compiler")
    here = Path(__file__).resolve().parent / "cabi"
    inc = HEADER.parent
    lib = Path(_lib.LIB_PATH)
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-c", str(here / "abi_c.c"), f"-I{inc}", "-o",
                    str(tmp_path / "abi_c.o")], check=True)
    exe = tmp_path / "abi_host"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", str(here / "abi_host.cpp"), f"-I{inc}", str(lib),
                    f"-Wl,-rpath,{lib.parent}", "-o", str(exe)], check=True)
    sample = tmp_path / "sample.gguf"
    gw.write(sample, gw.sample_spec())
    out = subprocess.run([str(exe), str(sample), gw.PREFIX], check=True, capture_output=True, text=True).stdout
    lines = dict(l.split(" ", 1) for l in out.strip().splitlines() if not l.startswith("tensor "))
    assert lines["status2"] == "unsupported shape"
    assert lines["null_gemm"] == f"{_lib.MI_ERR_INVALID_ARG} reason"
    assert lines["attn_supported"] == "1 0"
    assert lines["open"] == "0" and lines["arch"] == "sdxl"
    assert lines["find_missing"] == str(_lib.MI_ERR_NOT_FOUND)
    g = GgufFile()
    assert g.open(str(sample), [], gw.PREFIX)
    tens = [l.split() for l in out.splitlines() if l.startswith("tensor ")]
    assert [t[1] for t in tens] == [t.name for t in g.tensors()]
    for row, t in zip(tens, g.tensors()):
        assert (int(row[2]), int(row[3]), int(row[4]), int(row[5])) == (t.type, t.nbytes, t.rows, t.cols)
        f = g.readFloat(t.name, [])
        want = float(np.sum(f[np.isfinite(f)], dtype=np.float64)) if f.size else 0.0
        assert abs(float(row[6]) - want) <= 1e-6 * max(1.0, abs(want))


def test_tuning_overrides_are_bounded():
    """mi_tuning_set accepts the documented ranges only: GEMM builds 0..6 with
    1..64 K splits, attention key-split plans of 1..64 pieces, 2 or 4 attention
    waves per workgroup, 2 or 3 per SIMD, and rejects the rest."""
    lib = _lib.load()
    try:
        for name, value in [(b"gemm_cfg", b"6"), (b"gemm_cfg", b"0:64"), (b"attn_split", b"2:8"),
                            (b"attn_split", b"0"), (b"attn_nw", b"2"), (b"attn_simd_waves", b"3"),
                            (b"attn_simd_waves", b"2")]:
            assert lib.mi_tuning_set(name, value) == 0, (name, value)
        for name, value in [(b"gemm_cfg", b"7"), (b"gemm_cfg", b"1:65"), (b"attn_split", b"2:65"),
                            (b"attn_split", b"2:0"), (b"attn_nw", b"3"), (b"attn_simd_waves", b"4"),
                            (b"no_such_knob", b"1")]:
            assert lib.mi_tuning_set(name, value) != 0, (name, value)
    finally:
        lib.mi_tuning_reset()
