"""Minimal GGUF v3 writer for the tests (written from the published GGUF v3
format: header, typed metadata, tensor records, aligned data section).

Metadata values are given as (value_type, value) pairs so that every GGUF
value type can be exercised; arrays as (ARRAY, (element_type, [values])).
Tensors are (name, ggml_type, dims, raw_bytes) with dims in file order
(dims[0] = the contiguous row length, as GGUF stores ne[0] first).
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _scalar(t, v):
    if t == STRING:
        return _str(v)
    return struct.pack(_FMT[t], v)


def _value(t, v):
    if t != ARRAY:
        return _scalar(t, v)
    et, vals = v
    return struct.pack("<IQ", et, len(vals)) + b"".join(_scalar(et, x) for x in vals)


def gguf_bytes(metadata, tensors, alignment=32, version=3, set_alignment_key=False):
    """The file as bytes. Tensor data offsets are aligned to `alignment`; with
    set_alignment_key the general.alignment key announces it (else readers
    assume 32)."""
    md = list(metadata)
    if set_alignment_key:
        md.append(("general.alignment", U32, alignment))
    out = bytearray(struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(md)))
    for key, t, v in md:
        out += _str(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += len(data)
    for (name, gtype, dims, _), o in zip(tensors, offsets):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gtype, o)
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    base = len(out)
    for (_, _, _, data), o in zip(tensors, offsets):
        out += b"\0" * (base + o - len(out))
        out += bytes(np.asarray(data, np.uint8).tobytes() if not isinstance(data, (bytes, bytearray)) else data)
    return bytes(out)


def write_gguf(path, metadata, tensors, **kw):
    data = gguf_bytes(metadata, tensors, **kw)
    with open(path, "wb") as f:
        f.write(data)
    return len(data)
