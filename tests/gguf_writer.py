"""A small GGUF writer for the tests (the public GGUF layout, versions 2/3,
little-endian): header, typed metadata, tensor infos, aligned data section.

Values are given with explicit GGUF types so every type can be exercised:
``("key", UINT32, 7)``, ``("key", ARRAY, (FLOAT32, [1.0, 2.0]))``,
``("key", ARRAY, (ARRAY, [(INT8, [1]), (STRING, ["a"])]))``.
"""
from __future__ import annotations

import struct

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
FMT = {UINT8: "B", INT8: "b", UINT16: "H", INT16: "h", UINT32: "I", INT32: "i", FLOAT32: "f", BOOL: "?",
       UINT64: "Q", INT64: "q", FLOAT64: "d"}


def gstr(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t in FMT:
        return struct.pack("<" + FMT[t], v)
    if t == STRING:
        return gstr(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        if et in FMT:
            return out + struct.pack(f"<{len(items)}{FMT[et]}", *items)
        return out + b"".join(value(et, x) for x in items)
    raise ValueError(f"unknown GGUF type {t}")


def kv(key: str, t: int, v) -> bytes:
    return gstr(key) + struct.pack("<I", t) + value(t, v)


def tensor_info(name: str, ne, ggml_type: int, offset: int) -> bytes:
    return gstr(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) + struct.pack("<IQ", ggml_type,
                                                                                                      offset)


def build(kvs, tensors, alignment: int = 32, version: int = 3, set_alignment_key: bool = None) -> bytes:
    """kvs: [(key, type, value)]; tensors: [(name, ne, ggml_type, data_bytes)].
    Tensor data is laid out in order, each at the next multiple of ``alignment``
    (which is written as general.alignment unless it is 32 or
    set_alignment_key is False)."""
    kvs = list(kvs)
    if set_alignment_key is None:
        set_alignment_key = alignment != 32
    if set_alignment_key:
        kvs.append(("general.alignment", UINT32, alignment))
    offsets, pos = [], 0
    for _, _, _, data in tensors:
        pos = (pos + alignment - 1) // alignment * alignment
        offsets.append(pos)
        pos += len(data)
    head = struct.pack("<4sIQQ", b"GGUF", version, len(tensors), len(kvs))
    head += b"".join(kv(*x) for x in kvs)
    head += b"".join(tensor_info(n, ne, t, o) for (n, ne, t, _), o in zip(tensors, offsets))
    head += b"\0" * ((-len(head)) % alignment)
    body = bytearray()
    for (_, _, _, data), o in zip(tensors, offsets):
        body += b"\0" * (o - len(body))
        body += data
    return bytes(head) + bytes(body)
