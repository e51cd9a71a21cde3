"""The reference engine's GGUF reader (src/gguf.h, src/gguf.cpp) over the C ABI (q27h_gguf_*), and the staged
host -> HBM upload of tensor rows (q27h_copy_h2d_staged, the transfer of src/qmat.h:34).

Same names and meaning as the C++ class: GGUF(path) maps and parses the file (raising Q27Error with the
reference's message on a malformed file), tensor() raises for a missing name, find() returns None, kv() raises
for a missing key, get_int / get_float / get_str convert as the reference does.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import GTensorC, GValueC, Q27Error, check, lib

F32, F16, Q2_K, Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ1_M, BF16 = (
    0, 1, 10, 12, 14, 16, 17, 18, 21, 22, 23, 29, 30)
INT, FLOAT, BOOL, STRING, ARR_INT, ARR_FLOAT, ARR_STRING = range(7)


def gtype_name(t: int) -> str:
    return lib().q27h_gtype_name(t).decode()


def gtype_block_bytes(t: int) -> int:
    b = lib().q27h_gtype_block_bytes(t)
    if b == 0:
        raise Q27Error(-5, f"unknown ggml type {t}")
    return b


def gtype_block_size(t: int) -> int:
    gtype_block_bytes(t)
    return lib().q27h_gtype_block_size(t)


@dataclass
class GTensor:
    """src/gguf.h:21-30. `data` is the host address of the tensor's bytes inside the mapping."""
    name: str
    type: int
    n_dims: int
    ne: tuple
    offset: int
    nbytes: int
    data: int
    _owner: object = None
    _index: int = -1

    def rows(self) -> int:
        return self.ne[1] * self.ne[2] * self.ne[3]

    def row_bytes(self) -> int:
        return self.ne[0] // gtype_block_size(self.type) * gtype_block_bytes(self.type)

    def array(self) -> np.ndarray:
        """The tensor's bytes as a read-only numpy view of the mapping (valid while its GGUF is open)."""
        if self.nbytes == 0:
            return np.zeros(0, np.uint8)
        a = np.ctypeslib.as_array((C.c_uint8 * self.nbytes).from_address(self.data))
        a.flags.writeable = False
        return a


@dataclass
class GValue:
    """src/gguf.h:33-41"""
    kind: int
    i: int = 0
    f: float = 0.0
    s: str = ""
    ai: tuple = ()
    af: tuple = ()
    as_: tuple = ()


class GGUF:
    """src/gguf.h:43-70"""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().q27h_gguf_open(str(path).encode(), C.byref(h)))
        self._h = h
        self.path = str(path)
        self._tensors = None
        self._keys = None

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().q27h_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _tensor_at(self, i: int) -> GTensor:
        t = GTensorC()
        check(lib().q27h_gguf_tensor(self._h, i, C.byref(t)))
        name = C.string_at(t.name, t.name_len).decode("utf-8", "surrogateescape")
        return GTensor(name, t.type, t.n_dims, tuple(t.ne), t.offset, t.nbytes, t.data or 0, self, i)

    def tensors(self) -> list:
        if self._tensors is None:
            self._tensors = [self._tensor_at(i) for i in range(lib().q27h_gguf_n_tensors(self._h))]
        return self._tensors

    def find(self, name: str):
        i = lib().q27h_gguf_find(self._h, name.encode("utf-8", "surrogateescape"))
        return None if i < 0 else self.tensors()[i]

    def tensor(self, name: str) -> GTensor:
        t = self.find(name)
        if t is None:
            raise Q27Error(-7, f"missing tensor {name}")
        return t

    def _key_index(self) -> dict:
        if self._keys is None:
            sp, n = C.c_void_p(), C.c_size_t()
            keys = {}
            for i in range(lib().q27h_gguf_n_kv(self._h)):
                check(lib().q27h_gguf_key(self._h, i, C.byref(sp), C.byref(n)))
                keys[C.string_at(sp.value, n.value).decode("utf-8", "surrogateescape")] = i
            self._keys = keys
        return self._keys

    def keys(self) -> list:
        return list(self._key_index())

    def has(self, key: str) -> bool:
        return key in self._key_index()

    def kv(self, key: str) -> GValue:
        i = self._key_index().get(key)
        if i is None:
            raise Q27Error(-7, f"missing key {key}")
        v = GValueC()
        check(lib().q27h_gguf_kv_at(self._h, i, C.byref(v)))
        out = GValue(v.kind, v.i, v.f)
        if v.kind == STRING:
            out.s = C.string_at(v.s, v.s_len).decode("utf-8", "surrogateescape")
        elif v.kind == ARR_INT:
            out.ai = tuple(v.ai[j] for j in range(v.n))
        elif v.kind == ARR_FLOAT:
            out.af = tuple(v.af[j] for j in range(v.n))
        elif v.kind == ARR_STRING:
            sp, n = C.c_void_p(), C.c_size_t()
            items = []
            for j in range(v.n):
                check(lib().q27h_gguf_kv_str_at(self._h, i, j, C.byref(sp), C.byref(n)))
                items.append(C.string_at(sp.value, n.value).decode("utf-8", "surrogateescape"))
            out.as_ = tuple(items)
        return out

    # src/gguf.cpp:203-222
    def get_int(self, key: str) -> int:
        v = self.kv(key)
        if v.kind in (INT, BOOL):
            return v.i
        if v.kind == ARR_INT and len(v.ai) == 1:
            return v.ai[0]
        raise Q27Error(-5, f"key is not an int: {key}")

    def get_float(self, key: str) -> float:
        v = self.kv(key)
        if v.kind == FLOAT:
            return v.f
        if v.kind == INT:
            return float(v.i)
        raise Q27Error(-5, f"key is not a float: {key}")

    def get_str(self, key: str) -> str:
        v = self.kv(key)
        if v.kind != STRING:
            raise Q27Error(-5, f"key is not a string: {key}")
        return v.s


def copy_h2d_staged(dst, src_addr: int, nbytes: int, threads: int = 0, s=None) -> None:
    """q27h_copy_h2d_staged: host bytes at src_addr -> device tensor / address dst on stream s."""
    from .ops import _ptr, _stream

    check(lib().q27h_copy_h2d_staged(_ptr(dst), src_addr, nbytes, threads, _stream(s)))


def upload_rows(t: GTensor, dst, row0: int = 0, nrows: int | None = None, threads: int = 0, s=None) -> None:
    """Rows [row0, row0 + nrows) of tensor t (raw GGUF blocks) to device memory dst (the transfer of
    qmat_upload, src/qmat.h:34), read from t's open file with q27h_gguf_upload_rows."""
    from .ops import _ptr, _stream

    nrows = t.rows() - row0 if nrows is None else nrows
    g = t._owner
    if g is None or not getattr(g, "_h", None):
        raise Q27Error(-4, f"{t.name}: its GGUF is closed")
    check(lib().q27h_gguf_upload_rows(g._h, t._index, row0, nrows, _ptr(dst), threads, _stream(s)))
