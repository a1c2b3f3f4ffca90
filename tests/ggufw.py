"""Minimal GGUF v3 writer for the loader tests (from the published GGUF layout:
magic, version, tensor count, key count, typed key/values, tensor directory,
aligned data region)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)


def _str(s: bytes) -> bytes:
    return struct.pack("<Q", len(s)) + s


def _scalar(t: int, v) -> bytes:
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}
    if t == STR:
        return _str(v.encode())
    return struct.pack(fmt[t], v)


def _value(t: int, v) -> bytes:
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_scalar(et, x) for x in items)
    return _scalar(t, v)


def write(path, kvs, tensors, alignment=32, magic=b"GGUF", truncate=None):
    """kvs: list of (key, type, value); tensors: list of (name, dims, type, bytes).
    Returns the data-region offset of each tensor."""
    head = bytearray(magic + struct.pack("<IQQ", 3, len(tensors), len(kvs)))
    for k, t, v in kvs:
        head += _str(k.encode()) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, dims, ty, data in tensors:
        head += _str(name.encode()) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, off)
        offs.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    head += b"\0" * ((-len(head)) % alignment)
    body = bytearray()
    for (_, _, _, data), o in zip(tensors, offs):
        body += b"\0" * (o - len(body))
        body += data
    blob = bytes(head + body)
    if truncate is not None:
        blob = blob[:truncate]
    with open(path, "wb") as f:
        f.write(blob)
    return offs, len(head)
