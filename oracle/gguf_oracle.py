"""CPU oracle of the GGUF reader: TEST INFRASTRUCTURE ONLY (tests/ use it as the checker; the product never does).

A plain-Python restatement of the reference's parse (src/gguf.cpp:113-194 of avallavall/qwen27-engine):
magic 'GGUF' (0x46554747 little-endian), version 3 only, u64 tensor and key counts; per key a u64-length string,
a u32 value type and the value (scalars of types 0..12, strings, arrays of one element type; integer and bool
arrays -> ARR_INT, f32 / f64 arrays -> ARR_FLOAT, string arrays -> ARR_STRING; nested arrays are an error);
per tensor: name, u32 n_dims (1..4), n_dims u64 extents, u32 ggml type, u64 offset; nbytes = elements / block
size * block bytes; the data section starts at the end of the directory rounded up to general.alignment (32 by
default); every tensor must end inside the file. Errors raise GGUFError with the reference's message.
Pinned in tests/test_gguf.py by a hand-assembled known-answer file, writer round trips and one case per error.
"""
from __future__ import annotations

import struct

INT, FLOAT, BOOL, STRING, ARR_INT, ARR_FLOAT, ARR_STRING = range(7)

# ggml type -> (block bytes, block size), src/gguf.cpp:36-62
BLOCK = {0: (4, 1), 1: (2, 1), 30: (2, 1), 10: (84, 256), 12: (144, 256), 14: (210, 256), 16: (66, 256),
         17: (74, 256), 18: (98, 256), 21: (110, 256), 22: (82, 256), 23: (136, 256), 29: (56, 256)}

# gguf value type -> struct format of a scalar, src/gguf.cpp:87-104
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}
_STR, _ARR = 8, 9


class GGUFError(Exception):
    pass


class _Cur:
    def __init__(self, b: bytes):
        self.b, self.p = b, 0

    def get(self, fmt: str):
        n = struct.calcsize(fmt)
        if self.p + n > len(self.b):
            raise GGUFError("gguf: truncated file")
        v = struct.unpack_from(fmt, self.b, self.p)[0]
        self.p += n
        return v

    def str(self) -> bytes:
        n = self.get("<Q")
        if self.p + n > len(self.b):
            raise GGUFError("gguf: truncated string")
        s = self.b[self.p:self.p + n]
        self.p += n
        return s


def _scalar(c: _Cur, t: int):
    if t not in _SCALAR:
        raise GGUFError(f"gguf: bad value type {t}")
    v = c.get(_SCALAR[t])
    if t in (6, 12):
        return False, float(v)
    if t == 10 and v >= 1 << 63:  # u64 stored in int64 (src/gguf.cpp:96)
        v -= 1 << 64
    return True, int(v)


def parse(data: bytes, path: str = "<bytes>"):
    """Returns (kv, tensors, data_start): kv maps key bytes -> (kind, value) with the last value of a repeated key,
    tensors is a list of dicts (name, n_dims, ne, type, offset, nbytes, data_off) in file order."""
    c = _Cur(data)
    if c.get("<I") != 0x46554747:
        raise GGUFError(f"not a GGUF file: {path}")
    version = c.get("<I")
    if version != 3:
        raise GGUFError(f"GGUF version {version} not supported")
    n_tensors, n_kv = c.get("<Q"), c.get("<Q")
    kv = {}
    for _ in range(n_kv):
        key = c.str()
        t = c.get("<I")
        if t == _STR:
            kv[key] = (STRING, c.str())
        elif t == _ARR:
            et, n = c.get("<I"), c.get("<Q")
            if et == _STR:
                kv[key] = (ARR_STRING, [c.str() for _ in range(n)])
            else:
                vals = [_scalar(c, et)[1] for _ in range(n)]
                kv[key] = (ARR_FLOAT if et in (6, 12) else ARR_INT, vals)
        else:
            isint, v = _scalar(c, t)
            kv[key] = ((BOOL if t == 7 else INT) if isint else FLOAT, v)
    tensors = []
    for _ in range(n_tensors):
        name = c.str()
        n_dims = c.get("<I")
        if n_dims < 1 or n_dims > 4:
            raise GGUFError(f"bad n_dims for {name.decode('utf-8', 'replace')}")
        ne = [c.get("<Q") for _ in range(n_dims)] + [1] * (4 - n_dims)
        typ = c.get("<I")
        off = c.get("<Q")
        if typ not in BLOCK:
            raise GGUFError(f"unknown ggml type {typ}")
        bb, bs = BLOCK[typ]
        n = ne[0] * ne[1] * ne[2] * ne[3]
        tensors.append(dict(name=name, n_dims=n_dims, ne=tuple(ne), type=typ, offset=off, nbytes=n // bs * bb))
    align = 32
    if b"general.alignment" in kv:
        kind, v = kv[b"general.alignment"]
        if kind in (INT, BOOL):
            align = v
        elif kind == ARR_INT and len(v) == 1:
            align = v[0]
        else:
            raise GGUFError("key is not an int: general.alignment")
    data_start = (c.p + align - 1) // align * align
    for t in tensors:
        if data_start + t["offset"] + t["nbytes"] > len(data):
            raise GGUFError(f"tensor out of file: {t['name'].decode('utf-8', 'replace')}")
        t["data_off"] = data_start + t["offset"]
    return kv, tensors, data_start
