"""ctypes binding of libmi_sdvk.so (declarations in include/mi_sdvk.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback for any operator.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from . import hip

LIB_PATH = Path(__file__).resolve().parent / "libmi_sdvk.so"

(MI_OK, MI_ERR_INVALID_ARG, MI_ERR_UNSUPPORTED, MI_ERR_ALIGNMENT, MI_ERR_ALIASING, MI_ERR_HIP, MI_ERR_IO,
 MI_ERR_NOT_FOUND) = range(8)
MI_F32, MI_F16 = 0, 1
MI_ATTN_PREC_AUTO, MI_ATTN_PREC_FP16, MI_ATTN_PREC_SPLIT = 0, 1, 2

# Every function declared in include/mi_sdvk.h, with its ctypes signature.
_u32, _u64, _i32, _vp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32, ctypes.c_void_p


class MiAttnArgs(ctypes.Structure):
    """Mirror of mi_attn_args (include/mi_sdvk.h)."""
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp),
        ("batch", _u32), ("Tq", _u32), ("Tk", _u32), ("C", _u32), ("heads", _u32),
        ("causal", _i32), ("in_dtype", _i32), ("out_dtype", _i32),
        ("ldq", _u64), ("ldk", _u64), ("ldv", _u64), ("ldo", _u64),
        ("sq", _u64), ("sk", _u64), ("sv", _u64), ("so", _u64),
        ("kv_len", _vp),
        ("scale", ctypes.c_float),
        ("precision", _i32),
    ]


class MiBlockWeights(ctypes.Structure):
    """Mirror of mi_block_weights (include/mi_sdvk.h)."""
    _fields_ = [(n, _vp) for n in (
        "norm1_w", "norm1_b", "norm2_w", "norm2_b", "norm3_w", "norm3_b",
        "attn1_q", "attn1_k", "attn1_v", "attn1_out", "attn1_out_b",
        "attn2_q", "attn2_k", "attn2_v", "attn2_out", "attn2_out_b",
        "ff_up", "ff_up_b", "ff_down", "ff_down_b")]


class MiBlockDims(ctypes.Structure):
    """Mirror of mi_block_dims (include/mi_sdvk.h)."""
    _fields_ = [(n, _u32) for n in ("batch", "tokens", "channels", "heads", "ctx_tokens", "ctx_channels",
                                    "ff_inner", "flags")]


MI_BLOCK_FUSED_EPILOGUES, MI_BLOCK_JOINT_QKV, MI_BLOCK_FP16_ACTIVATIONS, MI_BLOCK_FP16_ATTENTION = 1, 2, 4, 8


class MiGgufTensorInfo(ctypes.Structure):
    """Mirror of mi_gguf_tensor_info (include/mi_sdvk.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("type", _u32), ("n_dims", _u32), ("dims", _u64 * 4),
                ("offset", _u64), ("nbytes", _u64), ("n_elems", _u64), ("rows", _u64), ("cols", _u64)]


class MiGgufMetaInfo(ctypes.Structure):
    """Mirror of mi_gguf_meta_info (include/mi_sdvk.h)."""
    _fields_ = [("type", _u32), ("arr_type", _u32), ("u", _u64), ("f", ctypes.c_double), ("b", _i32),
                ("str", ctypes.POINTER(ctypes.c_char)), ("str_len", _u64), ("arr_len", _u64)]


SIGNATURES = {
    "mi_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "mi_last_error": (ctypes.c_char_p, []),
    "mi_version": (ctypes.c_int, []),
    "mi_tuning_set": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p]),
    "mi_tuning_reset": (None, []),
    "mi_q8_0_dequant": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _u64, _vp]),
    "mi_q8_split_dequant": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int, _u64, _vp]),
    "mi_q8_0_to_split": (ctypes.c_int, [_vp, _vp, _vp, _u64, _vp]),
    "mi_q8_0_quantize": (ctypes.c_int, [_vp, _vp, _u64, _vp]),
    "mi_gemm_nt_q8_0": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                       _u64, _u64, _vp]),
    "mi_gemm_nt_q8_split": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32,
                                           _u32, _u64, _u64, _vp]),
    "mi_gemm_nt_q8_workspace_bytes": (_u64, [_u32, _u32, _u32, _u32]),
    "mi_gemm_nt_q8_0_ws": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                          _u64, _u64, _vp, _u64, _vp]),
    "mi_gemm_nt_q8_0_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                               _u64, _u64, _vp]),
    "mi_gemm_noalloc_init": (ctypes.c_int, []),
    "mi_gemm_nt_q8_split_ws": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32,
                                              _u32, _u64, _u64, _vp, _u64, _vp]),
    "mi_gemm_nt_q8_0_geglu": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "mi_gemm_nt_q8_0_geglu_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "mi_gemm_nt_q8_0_f16a": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u64, _u64,
                                            _vp, _u64, _vp]),
    "mi_gemm_nt_q8_0_f16o": (ctypes.c_int, [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "mi_gemm_nn_q8_split": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                           _u64, _u64, _u64, _vp]),
    "mi_gemm_nn_q8_workspace_bytes": (_u64, [_u32, _u32, _u32, _u32]),
    "mi_gemm_nn_q8_split_ws": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                              _u64, _u64, _u64, _vp, _u64, _vp]),
    "mi_fused_attn_supported": (ctypes.c_int, [_u32, _u32]),
    "mi_fused_attention": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, ctypes.c_int, _vp]),
    "mi_fused_attention_ex": (ctypes.c_int, [ctypes.POINTER(MiAttnArgs), _vp]),
    "mi_fused_attention_ws_bytes": (ctypes.c_uint64, [ctypes.POINTER(MiAttnArgs)]),
    "mi_fused_attention_ws": (ctypes.c_int, [ctypes.POINTER(MiAttnArgs), _vp, ctypes.c_uint64, _vp]),
    "mi_layernorm": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, ctypes.c_float, _vp]),
    "mi_layernorm_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, _u32, ctypes.c_float, _vp]),
    "mi_geglu": (ctypes.c_int, [_vp, _vp, _u32, _u32, _vp]),
    "mi_geglu_f16": (ctypes.c_int, [_vp, _vp, _u32, _u32, _vp]),
    "mi_add_inplace": (ctypes.c_int, [_vp, _vp, _u64, _vp]),
    "mi_block_workspace_bytes": (_u64, [ctypes.POINTER(MiBlockDims)]),
    "mi_sdxl_block_forward": (ctypes.c_int, [ctypes.POINTER(MiBlockWeights), ctypes.POINTER(MiBlockDims), _vp, _vp,
                                             _vp, _vp, _u64, _vp]),
    "mi_block_ctx_kv_bytes": (_u64, [ctypes.POINTER(MiBlockDims)]),
    "mi_block_ctx_kv": (ctypes.c_int, [ctypes.POINTER(MiBlockWeights), ctypes.POINTER(MiBlockDims), _vp, _vp, _u64,
                                       _vp]),
    "mi_sdxl_block_forward_kv": (ctypes.c_int, [ctypes.POINTER(MiBlockWeights), ctypes.POINTER(MiBlockDims), _vp,
                                                _vp, _u64, _vp, _vp, _u64, _vp]),
    "mi_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "mi_gguf_close": (None, [_vp]),
    "mi_gguf_info": (ctypes.c_int, [_vp, ctypes.POINTER(_u32), ctypes.POINTER(_u64), ctypes.POINTER(_u64),
                                    ctypes.POINTER(_u64)]),
    "mi_gguf_tensor": (ctypes.c_int, [_vp, _u64, ctypes.POINTER(MiGgufTensorInfo)]),
    "mi_gguf_find": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]),
    "mi_gguf_meta": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(MiGgufMetaInfo)]),
    "mi_gguf_meta_array": (ctypes.c_int, [_vp, ctypes.c_char_p, _u64, _u64, _vp, _vp, _vp]),
    "mi_gguf_read_raw": (ctypes.c_int, [_vp, _u64, _vp, _u64]),
    "mi_gguf_read_f32": (ctypes.c_int, [_vp, _u64, _vp, _u64]),
    "mi_gguf_read_q8_split": (ctypes.c_int, [_vp, _u64, _vp, _vp]),
    "mi_gguf_upload_raw": (ctypes.c_int, [_vp, _u64, _vp, _u64, _vp]),
    "mi_gguf_upload_f32": (ctypes.c_int, [_vp, _u64, _vp, _u64, _vp]),
    "mi_gguf_upload_q8_split": (ctypes.c_int, [_vp, _u64, _vp, _vp, _vp]),
}

_lib = None


class MiError(RuntimeError):
    def __init__(self, status: int, fn: str, detail: str):
        self.status = status
        super().__init__(f"{fn}: {status_string(status)} ({detail})")


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built: run `python -m sdvk_amd.build` "
                              "(or __graft_entry__.build()); there is no fallback path")
        hip.lib()  # bind ROCm's HIP runtime first so the library reuses it
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def status_string(status: int) -> str:
    return load().mi_status_string(status).decode()


def call(name: str, *args) -> None:
    """Calls `name`; raises MiError with mi_last_error() on a non-OK status."""
    lib = load()
    st = getattr(lib, name)(*args)
    if st != MI_OK:
        raise MiError(st, name, lib.mi_last_error().decode())


def ptr(x) -> int | None:
    """Device address of a DeviceBuffer / int / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.value
