"""A GGUF v3 writer for tests: the published layout, written from its
definition (magic "GGUF", u32 version 3, u64 tensor count, u64 metadata
count; typed key/value pairs; tensor infos; padding to the alignment; the
data section), so the reader's table can be checked against what was put in."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}


def _string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t in _SCALAR:
        return struct.pack(_SCALAR[t], v)
    if t == STRING:
        return _string(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    raise ValueError(t)


def write_gguf(path, kvs, tensors, alignment: int | None = None, version: int = 3):
    """kvs: [(key, type, value)] (ARRAY value: (element type, items));
    tensors: [(name, dims, type, bytes)].  Tensor data is laid out in order,
    each start padded to the alignment (32 unless given; given values are
    also written as general.alignment).  Returns (data_offset, offsets,
    info_end), info_end the file offset where the tensor infos end."""
    align = alignment or 32
    kv = list(kvs)
    if alignment is not None:
        kv.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, t, v in kv:
        head += _string(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += -(-len(data) // align) * align
    for (name, dims, t, _), o in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, o)
    data_offset = -(-len(head) // align) * align
    with open(path, "wb") as fh:
        fh.write(head + b"\0" * (data_offset - len(head)))
        for (_, _, _, data), o in zip(tensors, offsets):
            fh.write(bytes(data))
            pad = -(-len(data) // align) * align - len(data)
            fh.write(b"\0" * pad)
    return data_offset, offsets, len(head)


def as_bytes(a: np.ndarray) -> bytes:
    return np.ascontiguousarray(a).tobytes()
