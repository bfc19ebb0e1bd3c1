"""GGUF images for the loader tests, assembled byte by byte from ggml's
published GGUF specification (versions 1-3):

    u32 magic "GGUF" | u32 version | tensor count | metadata count   (u64; u32 in v1)
    metadata: string key | u32 value type | value
    tensor infos: string name | u32 n_dims | dims, innermost first (u64; u32 in v1)
                  | u32 ggml type | u64 offset from the data section
    zero padding to the alignment (general.alignment, default 32) | tensor data,
    each tensor starting at an aligned offset

with string = length (u64; u32 in v1) + UTF-8 bytes. This is test
infrastructure (the reference writes its files with candle's
gguf_file::write, tools/quantize-moonshine/src/main.rs:163-166)."""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


def _count(version: int, n: int) -> bytes:
    return struct.pack("<I" if version == 1 else "<Q", n)


def _string(version: int, s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return _count(version, len(b)) + b


def _value(version: int, vtype: int, val) -> bytes:
    if vtype == STRING:
        return _string(version, val)
    if vtype == ARRAY:
        etype, items = val
        return struct.pack("<I", etype) + _count(version, len(items)) + b"".join(
            _value(version, etype, v) for v in items)
    return struct.pack(_FMT[vtype], val)


def gguf_bytes(metadata=(), tensors=(), *, version: int = 3, alignment: int | None = None) -> bytes:
    """metadata: (key, value type, value) triples (ARRAY value = (element
    type, items)); tensors: (name, shape outermost first, ggml type, bytes)."""
    md = list(metadata)
    if alignment is not None:
        md.append(("general.alignment", U32, alignment))
    align = alignment or 32
    out = bytearray(struct.pack("<II", 0x46554747, version))
    out += _count(version, len(tensors)) + _count(version, len(md))
    for key, vtype, val in md:
        out += _string(version, key) + struct.pack("<I", vtype) + _value(version, vtype, val)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off = (off + len(data) + align - 1) // align * align
    for (name, shape, gtype, _), o in zip(tensors, offsets):
        out += _string(version, name) + struct.pack("<I", len(shape))
        for d in reversed(shape):
            out += struct.pack("<I" if version == 1 else "<Q", d)
        out += struct.pack("<IQ", gtype, o)
    out += b"\0" * ((-len(out)) % align)
    base = len(out)
    for (_, _, _, data), o in zip(tensors, offsets):
        out += b"\0" * (base + o - len(out))
        out += bytes(data)
    return bytes(out)
