"""numpy front end of the CPU oracle (oracle/liboracle.so) and of the reference
GGUF reader compiled into oracle/_ref/libgguf_ref.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libgguf_ref.so"
OR_F32, OR_F16 = 0, 1

_lib = None
_ref = None

_vp, _u32, _u64, _i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32


def build() -> None:
    """Builds liboracle.so (and _ref when /root/reference is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.or_fp16_to_fp32.restype = ctypes.c_float
        L.or_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.or_fp32_to_fp16.restype = ctypes.c_uint16
        L.or_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.or_gelu_erf.restype = ctypes.c_float
        L.or_gelu_erf.argtypes = [ctypes.c_float]
        L.or_fill_normal.argtypes = [_u64, ctypes.c_float, ctypes.c_float, _vp, _u64]
        L.or_fill_uniform_int.argtypes = [_u64, _i32, _i32, _vp, _u64]
        L.or_q8_0_quantize.argtypes = [_vp, _u64, _vp]
        L.or_q8_0_dequant.argtypes = [_vp, _u64, _vp]
        L.or_q8_0_to_split.argtypes = [_vp, _u64, _vp, _vp]
        L.or_q8_split_dequant.argtypes = [_vp, _vp, _u64, _vp]
        L.or_gemm_nn_q8_split.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                          _u64, _u64, _u64, ctypes.c_int, ctypes.c_int]
        L.or_gemm_nt_q8_split.argtypes = [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32,
                                          _u32, _u64, _u64, ctypes.c_int, ctypes.c_int]
        L.or_gemm_nt_q8_0.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                      _u64, _u64, ctypes.c_int, ctypes.c_int]
        L.or_gemm_nt_q8_0_rows.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp, _u32,
                                           ctypes.c_int]
        L.or_fused_attention.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, ctypes.c_int]
        L.or_fused_attention_ex.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, ctypes.c_int,
                                            _u64, _u64, _u64, _u64, _u64, _u64, _u64, _u64, ctypes.c_int,
                                            ctypes.c_int, _vp, _vp, _u32, ctypes.c_int]
        L.or_fused_attention_f32.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp, _u32,
                                             ctypes.c_int]
        L.or_layernorm.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, ctypes.c_float]
        L.or_geglu.argtypes = [_vp, _vp, _u32, _u32]
        L.or_add.argtypes = [_vp, _vp, _vp, _u64]
        L.or_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def ref_lib() -> ctypes.CDLL | None:
    """The reference's own Gguf.cpp (None when it was not built here)."""
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            return None
        R = ctypes.CDLL(str(REF_LIB))
        R.ref_fp16_to_fp32.restype = ctypes.c_float
        R.ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        R.ref_q8_0_decode.restype = ctypes.c_int
        R.ref_q8_0_decode.argtypes = [ctypes.c_char_p, _vp, _u64, _u64, _vp, _vp, _vp, _vp, _vp]
        cp, i32 = ctypes.c_char_p, ctypes.c_int
        R.ref_gguf_open.restype = _vp
        R.ref_gguf_open.argtypes = [cp, cp, cp, i32]
        R.ref_gguf_close.argtypes = [_vp]
        R.ref_gguf_version.restype = ctypes.c_uint32
        R.ref_gguf_version.argtypes = [_vp]
        R.ref_gguf_count.restype = _u64
        R.ref_gguf_count.argtypes = [_vp]
        R.ref_gguf_data_offset.restype = _u64
        R.ref_gguf_data_offset.argtypes = [_vp]
        R.ref_gguf_tensor.argtypes = [_vp, _u64, cp, i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
        R.ref_gguf_read_float.restype = ctypes.c_int64
        R.ref_gguf_read_float.argtypes = [_vp, cp, _vp, _u64, cp, i32]
        R.ref_gguf_read_q8.argtypes = [_vp, cp, _vp, _vp, i32, cp, i32]
        R.ref_gguf_read_raw.argtypes = [_vp, _u64, _vp, _u64]
        R.ref_gguf_meta.argtypes = [_vp, cp, _vp, _vp, _vp, _vp, cp, i32, _vp, _vp]
        R.ref_gguf_meta_array.argtypes = [_vp, cp, _vp, _vp, _u64]
        R.ref_gguf_meta_str_item.argtypes = [_vp, cp, _u64, cp, i32]
        R.ref_gguf_get_u64.restype = _u64
        R.ref_gguf_get_u64.argtypes = [_vp, cp, _u64]
        R.ref_gguf_get_i64.restype = ctypes.c_int64
        R.ref_gguf_get_i64.argtypes = [_vp, cp, ctypes.c_int64]
        R.ref_gguf_get_f64.restype = ctypes.c_double
        R.ref_gguf_get_f64.argtypes = [_vp, cp, ctypes.c_double]
        R.ref_gguf_get_f32.restype = ctypes.c_float
        R.ref_gguf_get_f32.argtypes = [_vp, cp, ctypes.c_float]
        R.ref_gguf_get_str.argtypes = [_vp, cp, cp, cp, i32]
        _ref = R
    return _ref


def _p(a) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def max_threads() -> int:
    return int(lib().or_max_threads())


# ---------------------------------------------------------------- generators --

def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().or_fill_normal(seed, mean, std, _p(out), n)
    return out


def uniform_int(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().or_fill_uniform_int(seed, lo, hi, _p(out), n)
    return out


# ---------------------------------------------------------------------- Q8_0 --

def q8_0_quantize(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    assert w.size % 32 == 0
    blocks = np.empty(w.size // 32 * 34, dtype=np.uint8)
    lib().or_q8_0_quantize(_p(w), w.size, _p(blocks))
    return blocks


def q8_0_dequant(blocks: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().or_q8_0_dequant(_p(np.ascontiguousarray(blocks)), n, _p(out))
    return out


def q8_0_to_split(blocks: np.ndarray, n: int) -> tuple[np.ndarray, np.ndarray]:
    payload = np.empty(n, dtype=np.int8)
    scales = np.empty(n // 32, dtype=np.float32)
    lib().or_q8_0_to_split(_p(np.ascontiguousarray(blocks)), n, _p(payload), _p(scales))
    return payload, scales


def q8_split_dequant(payload: np.ndarray, scales: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().or_q8_split_dequant(_p(np.ascontiguousarray(payload)), _p(np.ascontiguousarray(scales)), n, _p(out))
    return out


def ref_q8_0_decode(blocks: np.ndarray, rows: int, cols: int):
    """Runs the reference GgufFile readers on a one-tensor GGUF file."""
    R = ref_lib()
    if R is None:
        return None
    n = rows * cols
    out = np.empty(n, dtype=np.float32)
    q = np.empty(n, dtype=np.int8)
    s = np.empty(n // 32, dtype=np.float32)
    q2 = np.empty(n, dtype=np.int8)
    s2 = np.empty(n // 32, dtype=np.float32)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "t.gguf").encode()
        st = R.ref_q8_0_decode(path, _p(np.ascontiguousarray(blocks)), rows, cols, _p(out), _p(q), _p(s),
                               _p(q2), _p(s2))
    if st != 0:
        raise RuntimeError(f"reference GGUF decode failed: {st}")
    return out, q, s, q2, s2


class RefGguf:
    """The reference's ofc::GgufFile (Gguf.hpp:90-140) opened on a file, with its
    table, metadata and decoders returned as numpy / Python values. Test
    infrastructure: the checker for libmi_sdvk.so's mi_gguf_* entries."""

    def __init__(self, path, prefix: str = ""):
        R = ref_lib()
        if R is None:
            raise RuntimeError("oracle/_ref/libgguf_ref.so is not built")
        self.R = R
        err = ctypes.create_string_buffer(512)
        self.h = R.ref_gguf_open(str(path).encode(), prefix.encode() if prefix else None, err, 512)
        self.error = None if self.h else err.value.decode()

    def close(self):
        if self.h:
            self.R.ref_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def ok(self) -> bool:
        return bool(self.h)

    def version(self) -> int:
        return int(self.R.ref_gguf_version(self.h))

    def data_offset(self) -> int:
        return int(self.R.ref_gguf_data_offset(self.h))

    def tensors(self) -> list:
        """[(name, type, dims, offset, nbytes, shape)] in table order."""
        out = []
        for i in range(int(self.R.ref_gguf_count(self.h))):
            name = ctypes.create_string_buffer(4096)
            t, nd = ctypes.c_uint32(), ctypes.c_uint32()
            dims = (ctypes.c_uint64 * 4)()
            off, nb, r, c = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
            assert self.R.ref_gguf_tensor(self.h, i, name, 4096, ctypes.byref(t), ctypes.byref(nd), dims,
                                          ctypes.byref(off), ctypes.byref(nb), ctypes.byref(r), ctypes.byref(c)) == 0
            out.append((name.value.decode(), t.value, tuple(dims[: nd.value]), off.value, nb.value, (r.value, c.value)))
        return out

    def read_raw(self, index: int, nbytes: int):
        out = np.empty(nbytes, dtype=np.uint8)
        st = self.R.ref_gguf_read_raw(self.h, index, _p(out), nbytes)
        return out if st == 0 else None

    def read_float(self, name: str, n: int):
        """(values or None, error text)."""
        out = np.empty(max(n, 1), dtype=np.float32)
        err = ctypes.create_string_buffer(512)
        k = self.R.ref_gguf_read_float(self.h, name.encode(), _p(out), out.size, err, 512)
        return (out[:k], "") if k >= 0 else (None, err.value.decode())

    def read_q8(self, name: str, n: int, into: bool):
        q = np.empty(max(n, 1), dtype=np.int8)
        s = np.empty(max(n // 32, 1), dtype=np.float32)
        err = ctypes.create_string_buffer(512)
        st = self.R.ref_gguf_read_q8(self.h, name.encode(), _p(q), _p(s), 1 if into else 0, err, 512)
        return (q[:n], s[: n // 32], "") if st == 0 else (None, None, err.value.decode())

    def meta(self, key: str):
        """None, or dict(type, u, f, b, s, arr_type, items)."""
        t, ar, n = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
        u, f, b = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_int()
        s = ctypes.create_string_buffer(1 << 16)
        if self.R.ref_gguf_meta(self.h, key.encode(), ctypes.byref(t), ctypes.byref(u), ctypes.byref(f),
                                ctypes.byref(b), s, 1 << 16, ctypes.byref(ar), ctypes.byref(n)) != 0:
            return None
        items: tuple = ()
        if t.value == 9 and n.value:
            if ar.value == 8:
                lst = []
                for i in range(n.value):
                    sb = ctypes.create_string_buffer(1 << 16)
                    self.R.ref_gguf_meta_str_item(self.h, key.encode(), i, sb, 1 << 16)
                    lst.append(sb.value.decode("utf-8", "replace"))
                items = tuple(lst)
            else:
                uu = np.zeros(n.value, dtype=np.uint64)
                ff = np.zeros(n.value, dtype=np.float64)
                self.R.ref_gguf_meta_array(self.h, key.encode(), _p(uu), _p(ff), n.value)
                if ar.value in (6, 12):
                    items = tuple(float(x) for x in ff)
                elif ar.value == 7:
                    items = tuple(bool(x) for x in uu)
                else:
                    items = tuple(int(x) for x in uu)
        return dict(type=t.value, u=u.value, f=f.value, b=bool(b.value), s=s.value.decode("utf-8", "replace"),
                    arr_type=ar.value, items=items)

    def get(self, kind: str, key: str, default):
        k = key.encode()
        if kind == "u64":
            return int(self.R.ref_gguf_get_u64(self.h, k, default))
        if kind == "i64":
            return int(self.R.ref_gguf_get_i64(self.h, k, default))
        if kind == "f64":
            return float(self.R.ref_gguf_get_f64(self.h, k, default))
        if kind == "f32":
            return float(self.R.ref_gguf_get_f32(self.h, k, default))
        out = ctypes.create_string_buffer(1 << 16)
        self.R.ref_gguf_get_str(self.h, k, default.encode(), out, 1 << 16)
        return out.value.decode("utf-8", "replace")


# ---------------------------------------------------------------------- GEMM --

def gemm_nt_q8_0(A: np.ndarray, blocks: np.ndarray, M: int, N: int, K: int, *, bias=None, C=None,
                 mode: int = 0, lda: int = 0, ldc: int = 0, batch: int = 1, sA: int = 0, sC: int = 0,
                 acc64: bool = True, threads: int = 1) -> np.ndarray:
    ldc_e = ldc or N
    if C is None:
        C = np.zeros(((batch - 1) * sC + (M - 1) * ldc_e + N) if batch > 1 else M * ldc_e, dtype=np.float32)
    lib().or_gemm_nt_q8_0(_p(A), _p(blocks), _p(bias), _p(C), M, N, K, mode, lda, ldc, batch, sA, sC,
                          1 if acc64 else 0, threads)
    return C


def gemm_nt_q8_split(A, payload, scales, M, N, K, *, bias=None, C=None, mode=0, lda=0, ldc=0, batch=1,
                     sA=0, sC=0, acc64=True, threads=1) -> np.ndarray:
    ldc_e = ldc or N
    if C is None:
        C = np.zeros(((batch - 1) * sC + (M - 1) * ldc_e + N) if batch > 1 else M * ldc_e, dtype=np.float32)
    lib().or_gemm_nt_q8_split(_p(A), _p(payload), _p(scales), _p(bias), _p(C), M, N, K, mode, lda, ldc,
                              batch, sA, sC, 1 if acc64 else 0, threads)
    return C


def gemm_nn_q8_split(payload, scales, B, M, N, K, *, C=None, mode=0, lda=0, ldb=0, ldc=0, batch=1, sA=0, sB=0,
                     sC=0, acc64=True, threads=1) -> np.ndarray:
    """C[M,N] (=|+=) deq(A)[M,K] . B[K,N] (gemm_nn_q8_v.comp), C flat with ldc / sC."""
    ldc_e = ldc or N
    if C is None:
        C = np.zeros(((batch - 1) * sC + (M - 1) * ldc_e + N) if batch > 1 else M * ldc_e, dtype=np.float32)
    lib().or_gemm_nn_q8_split(_p(np.ascontiguousarray(payload)), _p(np.ascontiguousarray(scales)),
                              _p(np.ascontiguousarray(B)), _p(C), M, N, K, mode, lda, ldb, ldc, batch, sA, sB, sC,
                              1 if acc64 else 0, threads)
    return C


def gemm_rows(A, blocks, M, N, K, rows, *, bias=None, lda=0, threads=1) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    C = np.zeros(len(rows) * N, dtype=np.float32)
    lib().or_gemm_nt_q8_0_rows(_p(A), _p(blocks), _p(bias), _p(C), M, N, K, lda, 0, _p(rows), len(rows),
                               threads)
    return C.reshape(len(rows), N)


# ----------------------------------------------------------------- attention --

def fused_attention(q, k, v, Tq, Tk, C, heads, causal=False) -> np.ndarray:
    out = np.zeros(Tq * C, dtype=np.float32)
    lib().or_fused_attention(_p(q), _p(k), _p(v), _p(out), Tq, Tk, C, heads, 1 if causal else 0)
    return out


def fused_attention_ex(q, k, v, *, batch, Tq, Tk, C, heads, causal=False, in_dtype=OR_F32,
                       out_dtype=OR_F32, kv_len=None, rows=None, threads=1) -> np.ndarray:
    """Contiguous [batch, T, C] inputs; returns [batch, nrows, C] (all rows when rows is None)."""
    nr = Tq if rows is None else len(rows)
    odt = np.float32 if out_dtype == OR_F32 else np.float16
    out = np.zeros(batch * nr * C, dtype=odt)
    kl = None if kv_len is None else np.ascontiguousarray(kv_len, dtype=np.int32)
    rw = None if rows is None else np.ascontiguousarray(rows, dtype=np.uint32)
    lib().or_fused_attention_ex(_p(q), _p(k), _p(v), _p(out), batch, Tq, Tk, C, heads, 1 if causal else 0,
                                C, C, C, C, Tq * C, Tk * C, Tk * C, nr * C, in_dtype, out_dtype, _p(kl), _p(rw),
                                nr, threads)
    return out.reshape(batch, nr, C)


def fused_attention_f32(q, k, v, *, batch, Tq, Tk, C, heads, kv_len=None, q_rows=None, threads=1):
    out = np.zeros(batch * Tq * C, dtype=np.float32)
    kl = None if kv_len is None else np.ascontiguousarray(kv_len, dtype=np.int32)
    lib().or_fused_attention_f32(_p(q), _p(k), _p(v), _p(out), batch, Tq, Tk, C, heads, _p(kl),
                                 Tq if q_rows is None else q_rows, threads)
    return out


# ---------------------------------------------------------------------- glue --

def layernorm(x, gamma, beta, rows, d, eps=1e-5):
    y = np.empty(rows * d, dtype=np.float32)
    lib().or_layernorm(_p(x), _p(gamma), _p(beta), _p(y), rows, d, eps)
    return y


def gelu_erf(x: float) -> float:
    return float(lib().or_gelu_erf(x))


def geglu(h, rows, F):
    y = np.empty(rows * F, dtype=np.float32)
    lib().or_geglu(_p(h), _p(y), rows, F)
    return y


def add(a, b):
    c = np.empty_like(a, dtype=np.float32)
    lib().or_add(_p(np.ascontiguousarray(a, np.float32)), _p(np.ascontiguousarray(b, np.float32)), _p(c), a.size)
    return c


# ----------------------------------------------------------- transformer block --

BLOCK_FIELDS = ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "norm3_w", "norm3_b",
                "attn1_q", "attn1_k", "attn1_v", "attn1_out", "attn1_out_b",
                "attn2_q", "attn2_k", "attn2_v", "attn2_out", "attn2_out_b",
                "ff_up", "ff_up_b", "ff_down", "ff_down_b")


def sdxl_block(w: dict, x, ctx, *, batch, tokens, channels, heads, ctx_tokens, ctx_channels, ff_inner,
               ctx_len=None, threads=1):
    """One SDXL BasicTransformerBlock on the oracle's primitives, in the order of
    sdvkgen.cpp:1739-1763 (crossAttention :1283-1290, geglu :1709-1720):
    LN1 -> self-attention -> add -> LN2 -> cross-attention on ctx -> add -> LN3
    -> GEGLU FF -> add. Linear weights are Q8_0 blocks [out, in]; x is
    [batch * tokens, channels], ctx [batch * ctx_tokens, ctx_channels].
    GEMMs accumulate in fp64, attention is the fp64 online softmax."""
    rows, crow, C = batch * tokens, batch * ctx_tokens, channels
    x = np.array(x, dtype=np.float32, copy=True)

    def lin(a, wq, bias, m, n, k):
        return gemm_nt_q8_0(np.ascontiguousarray(a, np.float32), wq, m, n, k, bias=bias, threads=threads)

    def attn(a_q, a_kv, prefix, m_kv, tk, k_in, kl):
        q = lin(a_q, w[prefix + "_q"], None, rows, C, C)
        k = lin(a_kv, w[prefix + "_k"], None, m_kv, C, k_in)
        v = lin(a_kv, w[prefix + "_v"], None, m_kv, C, k_in)
        o = fused_attention_ex(q, k, v, batch=batch, Tq=tokens, Tk=tk, C=C, heads=heads, kv_len=kl,
                               threads=threads).reshape(-1)
        return lin(o, w[prefix + "_out"], w[prefix + "_out_b"], rows, C, C)

    n = layernorm(x, w["norm1_w"], w["norm1_b"], rows, C)
    x = add(x, attn(n, n, "attn1", rows, tokens, C, None))
    n = layernorm(x, w["norm2_w"], w["norm2_b"], rows, C)
    x = add(x, attn(n, np.ascontiguousarray(ctx, np.float32), "attn2", crow, ctx_tokens, ctx_channels, ctx_len))
    n = layernorm(x, w["norm3_w"], w["norm3_b"], rows, C)
    h = lin(n, w["ff_up"], w["ff_up_b"], rows, 2 * ff_inner, C)
    g = geglu(h, rows, ff_inner)
    x = add(x, lin(g, w["ff_down"], w["ff_down_b"], rows, C, ff_inner))
    return x
