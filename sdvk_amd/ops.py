"""Host-side mirror of sdvk's operator surface for the Q8 GEMM / fused attention.

Names, argument meaning and error behaviour follow the reference
(paths relative to the sdvk source root):

  FusedAttnArgs, fused_attn_supported, fused_attention
      src/Modules/GPU/fused_attn.hpp:13-28, fused_attn.cpp:34-61
  gemm_nt_q8 / gemm_nt_q8_bias (split int8 + fp32-scale layout)
      src/Modules/Diffusion/sdvkgen.cpp:917-936
  gemm_nn_q8 (weights-left GEMM of the conv paths, gemm_nn_q8_v.comp)
      sdvkgen.cpp:944-948
  Pg push layout + dispatch(kernel_name, bufs, push)
      sdvkgen.cpp:901-903, vk_engine.cpp:1143-1180, KERNELS[] :55-63,123-124
  layernorm / geglu / add2 (block glue)
      sdvkgen.cpp:1094-1103, :1709-1720, :1746,1751,1762
  BlockWeights / BlockDims / sdxl_block_forward (one transformer block)
      sdvkgen.cpp:1739-1763 with crossAttention :1283-1290
  block_ctx_kv / sdxl_block_forward_kv (the block with cached context K / V)

Where the reference calls exit(1) (unsupported attention shape, binding-count
mismatch) these raise MiError / ValueError instead. Every call goes to
libmi_sdvk.so; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

from . import _lib
from ._lib import (MI_ATTN_PREC_AUTO, MI_ATTN_PREC_FP16, MI_ATTN_PREC_SPLIT, MI_BLOCK_FP16_ACTIVATIONS,
                   MI_BLOCK_FP16_ATTENTION, MI_BLOCK_FUSED_EPILOGUES, MI_BLOCK_JOINT_QKV, MI_F16, MI_F32, MiAttnArgs,
                   MiBlockDims, MiBlockWeights, MiError, call, ptr)

__all__ = [
    "MiError", "MI_F32", "MI_F16", "MI_ATTN_PREC_AUTO", "MI_ATTN_PREC_FP16", "MI_ATTN_PREC_SPLIT",
    "tuning", "tuning_set", "tuning_reset", "MI_BLOCK_FUSED_EPILOGUES", "MI_BLOCK_FP16_ACTIVATIONS",
    "MI_BLOCK_FP16_ATTENTION", "MI_BLOCK_JOINT_QKV", "FusedAttnArgs", "fused_attn_supported", "fused_attention",
    "fused_attention_ex", "gemm_nt_q8", "gemm_nt_q8_bias", "gemm_nt_q8_0", "gemm_nt_q8_0_geglu", "gemm_nn_q8",
    "gemm_nt_q8_0_f16a", "gemm_nt_q8_0_f16o", "gemm_nt_q8_0_geglu_f16", "layernorm_f16", "geglu_f16",
    "gemm_workspace_bytes", "gemm_nn_workspace_bytes",
    "q8_0_dequant",
    "q8_split_dequant", "q8_0_to_split", "q8_0_quantize", "Pg", "dispatch", "KERNELS", "layernorm", "geglu", "add2",
    "BlockWeights", "BlockDims", "block_workspace_bytes", "sdxl_block_forward", "block_ctx_kv_bytes", "block_ctx_kv",
    "sdxl_block_forward_kv",
]


def _s(stream) -> Optional[int]:
    if stream is None:
        return None
    return stream.handle.value if hasattr(stream, "handle") else int(stream)


# ---------------------------------------------------------------- plan overrides --

def tuning_set(name: str, value: Optional[str]) -> None:
    """mi_tuning_set: pins one plan choice process-wide (None clears it)."""
    call("mi_tuning_set", name.encode(), None if value is None else str(value).encode())


def tuning_reset() -> None:
    """mi_tuning_reset: every plan choice back to the built-in rules."""
    _lib.load().mi_tuning_reset()


class tuning:
    """Context manager: `with ops.tuning(gemm_cfg="1:2"):` sets the overrides
    for the block and clears them on exit."""

    def __init__(self, **overrides):
        self.overrides = {k: v for k, v in overrides.items()}

    def __enter__(self):
        for k, v in self.overrides.items():
            tuning_set(k, v)
        return self

    def __exit__(self, *exc):
        for k in self.overrides:
            tuning_set(k, None)
        return False


# ------------------------------------------------------------------ attention --

@dataclass
class FusedAttnArgs:
    """fused_attn.hpp:13-23: fp32 [T, C] buffers, heads interleaved inside C."""
    q: object = None
    k: object = None
    v: object = None
    out: object = None
    Tq: int = 0
    Tk: int = 0
    C: int = 0
    heads: int = 1
    causal: bool = False


def fused_attn_supported(C: int, heads: int) -> bool:
    """fused_attn.cpp:34-38: heads divides C and 1 <= C/heads <= 64."""
    return bool(_lib.load().mi_fused_attn_supported(C, heads))


def fused_attention(a: FusedAttnArgs, stream=None) -> None:
    """fused_attn.cpp:40-61. Raises MiError(MI_ERR_UNSUPPORTED) where the
    reference prints and exits."""
    call("mi_fused_attention", ptr(a.q), ptr(a.k), ptr(a.v), ptr(a.out), a.Tq, a.Tk, a.C, a.heads,
         1 if a.causal else 0, _s(stream))


def fused_attention_ex(q, k, v, out, *, batch: int, Tq: int, Tk: int, C: int, heads: int,
                       causal: bool = False, in_dtype: int = MI_F32, out_dtype: int = MI_F32,
                       ldq: int = 0, ldk: int = 0, ldv: int = 0, ldo: int = 0, sq: int = 0,
                       sk: int = 0, sv: int = 0, so: int = 0, kv_len=None, scale: float = 0.0,
                       precision: int = MI_ATTN_PREC_AUTO, stream=None) -> None:
    """Batched / strided / fp16 / key-padded form (mi_fused_attention_ex)."""
    x = _attn_args(q, k, v, out, batch, Tq, Tk, C, heads, causal, in_dtype, out_dtype, ldq, ldk, ldv, ldo, sq, sk,
                   sv, so, kv_len, scale, precision)
    call("mi_fused_attention_ex", ctypes.byref(x), _s(stream))


def _attn_args(q, k, v, out, batch, Tq, Tk, C, heads, causal, in_dtype, out_dtype, ldq, ldk, ldv, ldo, sq, sk, sv, so,
               kv_len, scale, precision=MI_ATTN_PREC_AUTO) -> MiAttnArgs:
    return MiAttnArgs(q=ptr(q), k=ptr(k), v=ptr(v), out=ptr(out), batch=batch, Tq=Tq, Tk=Tk, C=C,
                      heads=heads, causal=1 if causal else 0, in_dtype=in_dtype, out_dtype=out_dtype,
                      ldq=ldq, ldk=ldk, ldv=ldv, ldo=ldo, sq=sq, sk=sk, sv=sv, so=so,
                      kv_len=ptr(kv_len), scale=scale, precision=precision)


def fused_attention_ws_bytes(*, batch: int, Tq: int, Tk: int, C: int, heads: int, causal: bool = False,
                             in_dtype: int = MI_F32, out_dtype: int = MI_F32, kv_len=None,
                             precision: int = MI_ATTN_PREC_AUTO) -> int:
    """Workspace mi_fused_attention_ws uses for this call's key-split plan (0: no split); contiguous tensors
    with 16-byte aligned rows assumed (the plan does not depend on the addresses otherwise)."""
    x = _attn_args(0x1000, 0x2000_0000_000, 0x4000_0000_000, 0x6000_0000_000, batch, Tq, Tk, C, heads, causal,
                   in_dtype, out_dtype, 0, 0, 0, 0, 0, 0, 0, 0, kv_len, 0.0, precision)
    return int(_lib.load().mi_fused_attention_ws_bytes(ctypes.byref(x)))


def fused_attention_ws(q, k, v, out, workspace, *, batch: int, Tq: int, Tk: int, C: int, heads: int,
                       causal: bool = False, in_dtype: int = MI_F32, out_dtype: int = MI_F32, ldq: int = 0,
                       ldk: int = 0, ldv: int = 0, ldo: int = 0, sq: int = 0, sk: int = 0, sv: int = 0, so: int = 0,
                       kv_len=None, scale: float = 0.0, precision: int = MI_ATTN_PREC_AUTO, stream=None) -> None:
    """mi_fused_attention_ws: fused_attention_ex with a workspace for the key-split plan."""
    x = _attn_args(q, k, v, out, batch, Tq, Tk, C, heads, causal, in_dtype, out_dtype, ldq, ldk, ldv, ldo, sq, sk,
                   sv, so, kv_len, scale, precision)
    wp, wn = _ws(workspace)
    call("mi_fused_attention_ws", ctypes.byref(x), wp, wn, _s(stream))


# ------------------------------------------------------------------------ GEMM --

def _ws(workspace):
    """(pointer, bytes) of an optional workspace buffer."""
    return (ptr(workspace), getattr(workspace, "nbytes", 0)) if workspace is not None else (None, 0)


def gemm_workspace_bytes(M: int, N: int, K: int, batch: int = 1) -> int:
    """Workspace the *_ws NT GEMM entries use for this shape's K-split plan (0: no split)."""
    return int(_lib.load().mi_gemm_nt_q8_workspace_bytes(M, N, K, batch))


def gemm_nn_workspace_bytes(M: int, N: int, K: int, batch: int = 1) -> int:
    """Workspace mi_gemm_nn_q8_split_ws uses for this shape's K-split plan (0: no split)."""
    return int(_lib.load().mi_gemm_nn_q8_workspace_bytes(M, N, K, batch))


def gemm_nt_q8(A, Bq, C, Bs, M: int, N: int, K: int, *, mode: int = 0, lda: int = 0, ldc: int = 0,
               batch: int = 1, sA: int = 0, sC: int = 0, workspace=None, stream=None) -> None:
    """sdvkgen.cpp:917-926 gemmNtQ8: C = A . deq(Bq, Bs)^T on the split layout (any K)."""
    if workspace is not None:
        call("mi_gemm_nt_q8_split_ws", ptr(A), ptr(Bq), ptr(Bs), None, ptr(C), M, N, K, mode, lda, ldc,
             batch, sA, sC, *_ws(workspace), _s(stream))
        return
    call("mi_gemm_nt_q8_split", ptr(A), ptr(Bq), ptr(Bs), None, ptr(C), M, N, K, mode, lda, ldc,
         batch, sA, sC, _s(stream))


def gemm_nt_q8_0_geglu(A, W, G, M: int, F: int, K: int, *, bias=None, lda: int = 0, ldg: int = 0,
                       stream=None) -> None:
    """linear(ff_up) + geglu (sdvkgen.cpp:1709-1720) in one GEMM: W has 2F Q8_0 rows (value, then gate),
    G[M, F] = (A.W[:F]^T + b[:F]) * gelu(A.W[F:]^T + b[F:])."""
    call("mi_gemm_nt_q8_0_geglu", ptr(A), ptr(W), ptr(bias), ptr(G), M, F, K, lda, ldg, _s(stream))


def gemm_nn_q8(Aq, As, B, C, M: int, N: int, K: int, *, mode: int = 0, lda: int = 0, ldb: int = 0, ldc: int = 0,
               batch: int = 1, sA: int = 0, sB: int = 0, sC: int = 0, workspace=None, stream=None) -> None:
    """sdvkgen.cpp:944-948 gemmNnQ8: C[M,N] = deq(Aq, As)[M,K] . B[K,N] (the conv paths' weights-left GEMM)."""
    if workspace is not None:
        call("mi_gemm_nn_q8_split_ws", ptr(Aq), ptr(As), ptr(B), ptr(C), M, N, K, mode, lda, ldb, ldc, batch, sA,
             sB, sC, *_ws(workspace), _s(stream))
        return
    call("mi_gemm_nn_q8_split", ptr(Aq), ptr(As), ptr(B), ptr(C), M, N, K, mode, lda, ldb, ldc, batch, sA, sB, sC,
         _s(stream))


def gemm_nt_q8_bias(A, Bq, C, Bs, bias, M: int, N: int, K: int, *, mode: int = 0, lda: int = 0,
                    ldc: int = 0, batch: int = 1, sA: int = 0, sC: int = 0, workspace=None, stream=None) -> None:
    """sdvkgen.cpp:928-936 gemmNtQ8Bias: as gemm_nt_q8, + bias[n] in mode 0."""
    if workspace is not None:
        call("mi_gemm_nt_q8_split_ws", ptr(A), ptr(Bq), ptr(Bs), ptr(bias), ptr(C), M, N, K, mode, lda,
             ldc, batch, sA, sC, *_ws(workspace), _s(stream))
        return
    call("mi_gemm_nt_q8_split", ptr(A), ptr(Bq), ptr(Bs), ptr(bias), ptr(C), M, N, K, mode, lda,
         ldc, batch, sA, sC, _s(stream))


def gemm_nt_q8_0(A, W, C, M: int, N: int, K: int, *, bias=None, mode: int = 0, lda: int = 0,
                 ldc: int = 0, batch: int = 1, sA: int = 0, sC: int = 0, workspace=None, stream=None) -> None:
    """North-star entry: W is the raw stream of 34-byte GGUF Q8_0 blocks. With a workspace
    (gemm_workspace_bytes) small grids may split K (mi_gemm_nt_q8_0_ws)."""
    if workspace is not None:
        call("mi_gemm_nt_q8_0_ws", ptr(A), ptr(W), ptr(bias), ptr(C), M, N, K, mode, lda, ldc, batch, sA,
             sC, *_ws(workspace), _s(stream))
        return
    call("mi_gemm_nt_q8_0", ptr(A), ptr(W), ptr(bias), ptr(C), M, N, K, mode, lda, ldc, batch, sA,
         sC, _s(stream))


def gemm_nt_q8_0_f16a(A, W, C, M: int, N: int, K: int, *, bias=None, mode: int = 0, lda: int = 0, ldc: int = 0,
                      batch: int = 1, sA: int = 0, sC: int = 0, workspace=None, stream=None) -> None:
    """gemm_nt_q8_0 with fp16 activations A (mi_gemm_nt_q8_0_f16a; extension): the same bits as the fp32
    entry given A's fp16 values as fp32."""
    call("mi_gemm_nt_q8_0_f16a", ptr(A), ptr(W), ptr(bias), ptr(C), M, N, K, mode, lda, ldc, batch, sA, sC,
         *_ws(workspace), _s(stream))


def gemm_nt_q8_0_f16o(A, W, C, M: int, N: int, K: int, *, a_dtype: int = MI_F32, bias=None, lda: int = 0,
                      ldc: int = 0, stream=None) -> None:
    """C (fp16) = fp16(A . W^T + bias), the unsplit fp32 result rounded once (mi_gemm_nt_q8_0_f16o; extension);
    A fp32 or fp16 (a_dtype)."""
    call("mi_gemm_nt_q8_0_f16o", ptr(A), a_dtype, ptr(W), ptr(bias), ptr(C), M, N, K, lda, ldc, _s(stream))


def gemm_nt_q8_0_geglu_f16(A, W, G, M: int, F: int, K: int, *, bias=None, lda: int = 0, ldg: int = 0,
                           stream=None) -> None:
    """gemm_nt_q8_0_geglu with fp16 A and fp16 G (mi_gemm_nt_q8_0_geglu_f16; extension)."""
    call("mi_gemm_nt_q8_0_geglu_f16", ptr(A), ptr(W), ptr(bias), ptr(G), M, F, K, lda, ldg, _s(stream))


# ------------------------------------------------------------------ Q8_0 utils --

def q8_0_dequant(blocks, out, n: int, out_dtype: int = MI_F32, stream=None) -> None:
    """Gguf.cpp:514-523 on the device (fp32 bit-exact)."""
    call("mi_q8_0_dequant", ptr(blocks), ptr(out), out_dtype, n, _s(stream))


def q8_split_dequant(payload, scales, out, n: int, out_dtype: int = MI_F32, stream=None) -> None:
    call("mi_q8_split_dequant", ptr(payload), ptr(scales), ptr(out), out_dtype, n, _s(stream))


def q8_0_quantize(w, blocks, n: int, stream=None) -> None:
    """sdvkgen.cpp:533-544 quantization rule on the device (fp32 -> 34-byte Q8_0 blocks)."""
    call("mi_q8_0_quantize", ptr(w), ptr(blocks), n, _s(stream))


def q8_0_to_split(blocks, payload, scales, n: int, stream=None) -> None:
    """Gguf.cpp:559-583 (readQ8Into) on the device."""
    call("mi_q8_0_to_split", ptr(blocks), ptr(payload), ptr(scales), n, _s(stream))


# ------------------------------------------------------------------ block glue --

def layernorm(x, gamma, beta, y, rows: int, d: int, eps: float = 1e-5, stream=None) -> None:
    """layernorm_fwd (two-pass mean / variance, affine when gamma/beta are given)."""
    call("mi_layernorm", ptr(x), ptr(gamma), ptr(beta), ptr(y), rows, d, eps, _s(stream))


def layernorm_f16(x, gamma, beta, y, rows: int, d: int, eps: float = 1e-5, stream=None) -> None:
    """layernorm with y stored as fp16 (mi_layernorm_f16; extension)."""
    call("mi_layernorm_f16", ptr(x), ptr(gamma), ptr(beta), ptr(y), rows, d, eps, _s(stream))


def geglu_f16(h, y, rows: int, F: int, stream=None) -> None:
    """geglu with y stored as fp16 (mi_geglu_f16; extension)."""
    call("mi_geglu_f16", ptr(h), ptr(y), rows, F, _s(stream))


def geglu(h, y, rows: int, F: int, stream=None) -> None:
    """y = h[:, :F] * gelu_erf(h[:, F:]) for h = [rows, 2F]."""
    call("mi_geglu", ptr(h), ptr(y), rows, F, _s(stream))


def add2(x, a, n: int, stream=None) -> None:
    """x += a (n floats, in place)."""
    call("mi_add_inplace", ptr(x), ptr(a), n, _s(stream))


@dataclass
class BlockDims:
    batch: int
    tokens: int
    channels: int
    heads: int
    ctx_tokens: int
    ctx_channels: int
    ff_inner: int
    flags: int = 0   # MI_BLOCK_FUSED_EPILOGUES | MI_BLOCK_JOINT_QKV

    def c(self) -> MiBlockDims:
        return MiBlockDims(self.batch, self.tokens, self.channels, self.heads, self.ctx_tokens,
                           self.ctx_channels, self.ff_inner, self.flags)


@dataclass
class BlockWeights:
    """Device buffers of one block (diffusers names); linear weights are Q8_0 blocks [out, in]."""
    norm1_w: object
    norm1_b: object
    norm2_w: object
    norm2_b: object
    norm3_w: object
    norm3_b: object
    attn1_q: object
    attn1_k: object
    attn1_v: object
    attn1_out: object
    attn1_out_b: object
    attn2_q: object
    attn2_k: object
    attn2_v: object
    attn2_out: object
    attn2_out_b: object
    ff_up: object
    ff_up_b: object
    ff_down: object
    ff_down_b: object

    def c(self) -> MiBlockWeights:
        return MiBlockWeights(*[ptr(getattr(self, f[0])) for f in MiBlockWeights._fields_])


def block_workspace_bytes(dims: BlockDims) -> int:
    return int(_lib.load().mi_block_workspace_bytes(ctypes.byref(dims.c())))


def sdxl_block_forward(w: BlockWeights, dims: BlockDims, x, ctx, workspace, *, ctx_len=None,
                       workspace_bytes: Optional[int] = None, stream=None) -> None:
    """One SDXL BasicTransformerBlock, x [batch*tokens, channels] updated in place."""
    nbytes = workspace_bytes if workspace_bytes is not None else getattr(workspace, "nbytes", 0)
    wc, dc = w.c(), dims.c()
    call("mi_sdxl_block_forward", ctypes.byref(wc), ctypes.byref(dc), ptr(x), ptr(ctx), ptr(ctx_len),
         ptr(workspace), nbytes, _s(stream))


def block_ctx_kv_bytes(dims: BlockDims) -> int:
    """Bytes of one block's cached cross-attention K and V."""
    return int(_lib.load().mi_block_ctx_kv_bytes(ctypes.byref(dims.c())))


def block_ctx_kv(w: BlockWeights, dims: BlockDims, ctx, kv, *, stream=None) -> None:
    """K = ctx . attn2_k^T, V = ctx . attn2_v^T into kv, once per sampling job
    (crossAttention recomputes them every call, sdvkgen.cpp:1283-1290)."""
    wc, dc = w.c(), dims.c()
    call("mi_block_ctx_kv", ctypes.byref(wc), ctypes.byref(dc), ptr(ctx), ptr(kv), getattr(kv, "nbytes", 0),
         _s(stream))


def sdxl_block_forward_kv(w: BlockWeights, dims: BlockDims, x, kv, workspace, *, ctx_len=None,
                          workspace_bytes: Optional[int] = None, stream=None) -> None:
    """sdxl_block_forward with the cross-attention K / V of block_ctx_kv."""
    nbytes = workspace_bytes if workspace_bytes is not None else getattr(workspace, "nbytes", 0)
    wc, dc = w.c(), dims.c()
    call("mi_sdxl_block_forward_kv", ctypes.byref(wc), ctypes.byref(dc), ptr(x), ptr(kv), getattr(kv, "nbytes", 0),
         ptr(ctx_len), ptr(workspace), nbytes, _s(stream))


# --------------------------------------------- reference kernel-name dispatch --

@dataclass
class Pg:
    """sdvkgen.cpp:901-903 / gemm_q8_bench.cpp:19-21 push layout (48 bytes)."""
    M: int
    N: int
    K: int
    mode: int = 0
    sA: int = 0
    sB: int = 0
    sC: int = 0
    batch: int = 1
    lda: int = 0
    ldb: int = 0
    ldc: int = 0
    pad: int = 0


# name -> number of bindings (vk_engine.cpp:55-63,123-124)
KERNELS = {
    "gemm_nt_q8": 4, "gemm_nt_q8_v": 4, "gemm_nt_q8_v_bm128": 4, "gemm_nt_q8_v_bk32": 4,
    "gemm_nt_q8_v_bm128_bk32": 4, "gemm_nt_q8_v_b": 5, "gemm_nt_q8_v_bm128_b": 5,
    "gemm_nn_q8_v": 4, "gemm_nn_q8": 4,
    "fused_attn": 4, "fused_attn_tiled": 4,
}


def dispatch(kernel: str, bufs: Sequence, push, stream=None) -> None:
    """Engine::dispatch(kernelName, {BufRef...}, push) for the kernels this
    library replaces. Tile-size variants (_bm128, _bk32) all map to the same
    MFMA kernel; the grid is chosen here, so no gx/gy/gz arguments."""
    if kernel not in KERNELS:
        raise ValueError(f"unknown kernel {kernel}")
    if len(bufs) != KERNELS[kernel]:
        raise ValueError(f"kernel {kernel} expects {KERNELS[kernel]} bindings, got {len(bufs)}")
    if kernel.startswith("gemm_nn_q8"):
        Aq, B, C, S = bufs  # binding order {Aq, B, C, S} (vk_engine.cpp:57,63)
        pc: Pg = push
        call("mi_gemm_nn_q8_split", ptr(Aq), ptr(S), ptr(B), ptr(C), pc.M, pc.N, pc.K, pc.mode, pc.lda, pc.ldb,
             pc.ldc, max(pc.batch, 1), pc.sA, pc.sB, pc.sC, _s(stream))
    elif kernel.startswith("gemm_nt_q8"):
        A, Bq, C, S = bufs[:4]
        bias = bufs[4] if len(bufs) == 5 else None
        pc: Pg = push
        call("mi_gemm_nt_q8_split", ptr(A), ptr(Bq), ptr(S), ptr(bias), ptr(C), pc.M, pc.N, pc.K,
             pc.mode, pc.lda, pc.ldc, max(pc.batch, 1), pc.sA, pc.sC, _s(stream))
    else:
        q, k, v, o = bufs
        a: FusedAttnArgs = push
        fused_attention(FusedAttnArgs(q, k, v, o, a.Tq, a.Tk, a.C, a.heads, a.causal), stream)
