"""A GGUF (version 3) writer for the tests: builds files from Python values per the public GGUF specification
(little-endian header, key/value table, tensor directory, data section aligned to general.alignment)."""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def _s(b) -> bytes:
    if isinstance(b, str):
        b = b.encode()
    return struct.pack("<Q", len(b)) + b


def value(t: int, v, et: int | None = None) -> bytes:
    """Type tag + payload of one metadata value (et: element type of an array)."""
    if t == STR:
        return struct.pack("<I", STR) + _s(v)
    if t == ARR:
        out = struct.pack("<IIQ", ARR, et, len(v))
        for x in v:
            out += _s(x) if et == STR else struct.pack(_FMT[et], x)
        return out
    return struct.pack("<I", t) + struct.pack(_FMT[t], v)


def build(kv: list, tensors: list, alignment: int = 32, version: int = 3, pad_byte: bytes = b"\0") -> bytes:
    """kv: [(key, type, value[, elem type])]; tensors: [(name, type, ne tuple, data bytes)] laid out in order,
    each at an aligned offset. A general.alignment entry in kv is honoured as given (the caller keeps it equal
    to `alignment`)."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kv))
    for item in kv:
        key, t, v = item[:3]
        head += _s(key) + value(t, v, item[3] if len(item) > 3 else None)
    offs, off = [], 0
    for name, typ, ne, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, typ, ne, data), o in zip(tensors, offs):
        head += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", typ, o)
    start = (len(head) + alignment - 1) // alignment * alignment
    out = bytearray(head + pad_byte * (start - len(head)))
    for (name, typ, ne, data), o in zip(tensors, offs):
        out += b"\0" * (start + o - len(out))
        out += data
    return bytes(out)
