"""Writes GGUF v2 / v3 container files for tests (our own writer: the container
layout of Gguf.cpp:290-416 -- magic, version, counts, typed metadata pairs,
tensor table, data section aligned to general.alignment -- plus switches that
produce the malformed variants the reader must reject).

Tensor payloads are given as raw bytes; the helpers below build them for the
element / block types the reader decodes (F32, F16, BF16, Q4_0, Q8_0).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Any

import numpy as np

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}

# ggml tensor types
T_F32, T_F16, T_Q4_0, T_Q8_0, T_Q4_K, T_BF16 = 0, 1, 2, 8, 12, 30


@dataclass
class Tensor:
    name: str
    dims: tuple            # ggml order: dims[0] fastest
    type: int
    data: bytes
    offset: int | None = None   # None: next aligned position


@dataclass
class GgufSpec:
    tensors: list = field(default_factory=list)
    meta: list = field(default_factory=list)   # (key, type, value); arrays: (key, ARR, (elem_type, [items]))
    version: int = 3
    magic: bytes = b"GGUF"
    alignment: int = 32    # used to place data; write general.alignment yourself to change the reader's rule
    n_tensors: int | None = None  # override the header counts (malformed files)
    n_kv: int | None = None


def _string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _scalar(t: int, v: Any) -> bytes:
    if t == STR:
        return _string(v)
    if t == BOOL:
        return struct.pack("<B", 1 if v else 0)
    return struct.pack(_FMT[t], v)


def _value(t: int, v: Any) -> bytes:
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_scalar(et, x) for x in items)
    return _scalar(t, v)


def build(spec: GgufSpec) -> bytes:
    head = spec.magic + struct.pack("<I", spec.version)
    head += struct.pack("<QQ", len(spec.tensors) if spec.n_tensors is None else spec.n_tensors,
                        len(spec.meta) if spec.n_kv is None else spec.n_kv)
    kv = b"".join(_string(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in spec.meta)
    # data offsets: each tensor at the next multiple of the alignment
    offsets, pos = [], 0
    for t in spec.tensors:
        if t.offset is None:
            pos = (pos + spec.alignment - 1) // spec.alignment * spec.alignment
            offsets.append(pos)
            pos += len(t.data)
        else:
            offsets.append(t.offset)
    table = b""
    for t, off in zip(spec.tensors, offsets):
        table += _string(t.name) + struct.pack("<I", len(t.dims)) + b"".join(struct.pack("<Q", d) for d in t.dims)
        table += struct.pack("<IQ", t.type, off)
    out = bytearray(head + kv + table)
    while len(out) % spec.alignment:
        out.append(0)
    base = len(out)
    end = max([o + len(t.data) for t, o in zip(spec.tensors, offsets)] or [0])
    out.extend(b"\0" * end)
    for t, off in zip(spec.tensors, offsets):
        out[base + off: base + off + len(t.data)] = t.data
    return bytes(out)


def write(path, spec: GgufSpec) -> bytes:
    data = build(spec)
    with open(path, "wb") as f:
        f.write(data)
    return data


# ---- payload builders ---------------------------------------------------------------

def f32_bytes(x: np.ndarray) -> bytes:
    return np.ascontiguousarray(x, dtype="<f4").tobytes()


def f16_bytes(x: np.ndarray) -> bytes:
    return np.ascontiguousarray(x, dtype="<f2").tobytes()


def bf16_bytes(x: np.ndarray) -> bytes:
    """Truncating fp32 -> bf16 (upper 16 bits), so the decode is exact."""
    u = np.ascontiguousarray(x, dtype="<f4").view("<u4") >> 16
    return u.astype("<u2").tobytes()


def q8_0_bytes(d: np.ndarray, q: np.ndarray) -> bytes:
    """Blocks {fp16 d, int8 q[32]} from per-block scales d (fp16-representable) and int8 q."""
    nb = d.size
    blk = np.empty((nb, 34), dtype=np.uint8)
    blk[:, :2] = np.asarray(d, dtype="<f2").view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = np.asarray(q, dtype=np.int8).reshape(nb, 32).view(np.uint8)
    return blk.tobytes()


def q4_0_bytes(d: np.ndarray, nib: np.ndarray) -> bytes:
    """Blocks {fp16 d, uint8 qs[16]}; nib is (nb, 32) nibbles 0..15, packed two per
    byte: byte i = nib[2i] | nib[2i + 1] << 4."""
    nb = d.size
    nib = np.asarray(nib, dtype=np.uint8).reshape(nb, 32)
    blk = np.empty((nb, 18), dtype=np.uint8)
    blk[:, :2] = np.asarray(d, dtype="<f2").view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = nib[:, 0::2] | (nib[:, 1::2] << 4)
    return blk.tobytes()


# ---- the sample checkpoint used by the tests and the golden fixture --------------

PREFIX = "model.diffusion_model."


def _special_f16() -> np.ndarray:
    """fp16 patterns the decoders must keep exact: zeros, subnormals, min normal,
    max finite, infinities, a NaN."""
    bits = np.array([0x0000, 0x8000, 0x0001, 0x03ff, 0x0400, 0x3c00, 0xbc00, 0x7bff, 0xfbff, 0x7c00, 0xfc00,
                     0x7e00], dtype=np.uint16)
    return bits.view(np.float16)


def sample_spec(seed: int = 7) -> GgufSpec:
    """A small checkpoint-shaped file: every metadata value type (scalars and
    arrays), F32 / F16 / BF16 / Q4_0 / Q8_0 tensors in 1-D, 2-D, 3-D and 4-D, a
    4-D conv weight tagged with comfy.gguf.orig_shape and one without, a Q8_0
    tensor whose element count is not a multiple of 32, a type the reader does
    not decode (Q4_K), tensors outside the UNet prefix, general.alignment 64."""
    rng = np.random.default_rng(seed)
    sp = GgufSpec(alignment=64)
    sp.meta = [
        ("general.architecture", STR, "sdxl"),
        ("general.alignment", U32, 64),
        ("general.name", STR, "mi-sdvk sample é"),
        ("sdxl.u8", U8, 200), ("sdxl.i8", I8, -5), ("sdxl.u16", U16, 60000), ("sdxl.i16", I16, -3000),
        ("sdxl.u32", U32, 4_000_000_000), ("sdxl.i32", I32, -2_000_000_000), ("sdxl.f32", F32, 1.5),
        ("sdxl.bool", BOOL, True), ("sdxl.u64", U64, (1 << 63) + 5), ("sdxl.i64", I64, -7),
        ("sdxl.f64", F64, -2.25), ("sdxl.f32_nan", F32, float("nan")),
        ("arr.u8", ARR, (U8, [1, 2, 255])), ("arr.i8", ARR, (I8, [-1, 2, -128])),
        ("arr.u16", ARR, (U16, [65535, 0])), ("arr.i16", ARR, (I16, [-32768, 7])),
        ("arr.u32", ARR, (U32, [4_294_967_295, 1])), ("arr.i32", ARR, (I32, [-1, 5])),
        ("arr.u64", ARR, (U64, [(1 << 64) - 1, 3])), ("arr.i64", ARR, (I64, [-(1 << 63), 9])),
        ("arr.f32", ARR, (F32, [0.5, -1.0, 3.25])), ("arr.f64", ARR, (F64, [1e300, -0.0])),
        ("arr.bool", ARR, (BOOL, [True, False, True])), ("arr.str", ARR, (STR, ["a", "bé", ""])),
        ("arr.empty", ARR, (U32, [])),
        ("comfy.gguf.orig_shape.conv.weight", ARR, (I32, [8, 32, 3, 3])),
    ]
    t = []
    t.append(Tensor(PREFIX + "a.weight", (64, 3), T_F32, f32_bytes(rng.standard_normal(192).astype(np.float32))))
    h = np.concatenate([_special_f16(), rng.standard_normal(84).astype(np.float16)])
    t.append(Tensor(PREFIX + "b.bias", (96,), T_F16, f16_bytes(h)))
    t.append(Tensor(PREFIX + "c.weight", (32, 2, 3), T_BF16, bf16_bytes(rng.standard_normal(192).astype(np.float32))))
    d4 = np.concatenate([_special_f16()[:4], rng.uniform(0.001, 0.1, 4).astype(np.float16)])
    t.append(Tensor(PREFIX + "d.weight", (64, 4), T_Q4_0, q4_0_bytes(d4, rng.integers(0, 16, (8, 32)))))
    d8 = np.concatenate([_special_f16(), (rng.standard_normal(3) * 0.01).astype(np.float16)])
    q8 = rng.integers(-128, 128, (15, 32)).astype(np.int8)
    q8[0, :6] = [-128, -127, -1, 0, 1, 127]
    t.append(Tensor(PREFIX + "e.weight", (96, 5), T_Q8_0, q8_0_bytes(d8, q8)))
    t.append(Tensor(PREFIX + "f.bias", (64,), T_Q8_0,
                    q8_0_bytes(np.array([0.01, -0.02], dtype=np.float16), rng.integers(-127, 128, (2, 32)))))
    t.append(Tensor(PREFIX + "conv.weight", (3, 3, 32, 8), T_Q8_0,
                    q8_0_bytes((rng.uniform(0.001, 0.01, 72)).astype(np.float16), rng.integers(-127, 128, (72, 32)))))
    t.append(Tensor(PREFIX + "g.weight", (3, 3, 32, 4), T_Q8_0,
                    q8_0_bytes((rng.uniform(0.001, 0.01, 36)).astype(np.float16), rng.integers(-127, 128, (36, 32)))))
    t.append(Tensor(PREFIX + "i.weight", (40,), T_Q8_0,  # 40 elements: one whole block + a partial one
                    q8_0_bytes(np.array([0.5, 0.25], dtype=np.float16), rng.integers(-127, 128, (2, 32)))))
    # Q4_K has no decoder here; the reader counts one byte per element for it
    t.append(Tensor("cond_stage_model.h.weight", (256, 2), T_Q4_K, bytes(rng.integers(0, 256, 512, dtype=np.uint8))))
    t.append(Tensor("first_stage_model.j.bias", (16,), T_F32, f32_bytes(np.arange(16, dtype=np.float32))))
    sp.tensors = t
    return sp
