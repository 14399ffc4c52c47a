"""A minimal GGUF writer for the tests, written from the GGUF specification
(ggml docs/gguf.md): header, typed key/value metadata, tensor infos, data
aligned to ``general.alignment``.  Used to build the files the parser and the
upload path are tested on; it also writes deliberately broken variants.
"""
from __future__ import annotations

import struct

import numpy as np

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = \
    range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i",
        FLOAT32: "<f", BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def gstr(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def kv_bytes(key: str, vtype: int, value, elem_type: int | None = None) -> bytes:
    out = gstr(key) + struct.pack("<I", vtype)
    if vtype == STRING:
        return out + gstr(value)
    if vtype == ARRAY:
        out += struct.pack("<IQ", elem_type, len(value))
        if elem_type == STRING:
            return out + b"".join(gstr(v) for v in value)
        return out + b"".join(struct.pack(_FMT[elem_type], v) for v in value)
    return out + struct.pack(_FMT[vtype], value)


def build(kvs, tensors, alignment: int = 32, version: int = 3, magic: bytes = b"GGUF",
          offsets=None, pad_data: bool = True) -> bytes:
    """kvs: [(key, type, value[, elem_type])]; tensors: [(name, ggml_type,
    ne tuple, data bytes)].  Tensor data is laid out in order, each start
    aligned; `offsets` overrides the recorded offsets (broken files)."""
    meta = b"".join(kv_bytes(*kv) for kv in kvs)
    data = b""
    offs = []
    for _, _, _, raw in tensors:
        pad = (-len(data)) % alignment
        data += b"\0" * pad
        offs.append(len(data))
        data += bytes(raw)
    if offsets is not None:
        offs = offsets
    infos = b""
    for (name, gtype, ne, _), off in zip(tensors, offs):
        infos += gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        infos += struct.pack("<IQ", gtype, off)
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs)) + meta + infos
    if pad_data:
        head += b"\0" * ((-len(head)) % alignment)
    return head + data


def write(path, kvs, tensors, **kw) -> bytes:
    b = build(kvs, tensors, **kw)
    with open(path, "wb") as f:
        f.write(b)
    return b


def f32_tensor(a: np.ndarray) -> bytes:
    return np.ascontiguousarray(a, dtype="<f4").tobytes()
