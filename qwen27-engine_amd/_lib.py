"""Loading and building lib/libq27h.so, and the ctypes signatures of every C-ABI entry point."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libq27h.so")


class Q27Error(RuntimeError):
    """A non-zero status of a q27h_* call; .code is the Q27H_ERR_* value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (status {code})")
        self.code = code


_p, _i, _f, _sz, _i64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_int64


class GTensorC(C.Structure):
    """q27h_gtensor"""
    _fields_ = [("name", C.c_char_p), ("name_len", C.c_size_t), ("type", C.c_int), ("n_dims", C.c_int),
                ("ne", C.c_int64 * 4), ("offset", C.c_uint64), ("nbytes", C.c_uint64), ("data", C.c_void_p)]


class GValueC(C.Structure):
    """q27h_gvalue"""
    _fields_ = [("kind", C.c_int), ("i", C.c_int64), ("f", C.c_double), ("s", C.c_void_p), ("s_len", C.c_size_t),
                ("n", C.c_uint64), ("ai", C.POINTER(C.c_int64)), ("af", C.POINTER(C.c_double))]


# name -> argument types (all return int status unless listed in _RESTYPE)
SIGNATURES = {
    "q27h_rmsnorm": [_p, _p, _p, _i, _i, _f, _p, _i],
    "q27h_add": [_p, _p, _p, _i, _p],
    "q27h_swiglu": [_p, _p, _p, _i, _p],
    "q27h_set_int": [_p, _i, _p],
    "q27h_rmsnorm_q8": [_p, _p, _p, _p, _p, _i, _i, _f, _p, _p],
    "q27h_sum_norm_q8": [_p, _p, _i, _i, _p, _p, _f, _p, _p, _p, _p, _p, _sz],
    "q27h_sum_norm_rows": [_p, _p, _i, _i, _p, _p, _f, _p, _p, _p, _p, _p],
    "q27h_add_norm_rows": [_p, _p, _p, _i, _i, _p, _f, _p, _p, _p, _p, _p],
    "q27h_quantize_q8_1": [_p, _p, _p, _i, _i, _p, _p],
    "q27h_swiglu_q8": [_p, _p, _p, _p, _i, _p, _p],
    "q27h_gated_rmsnorm_q8": [_p, _p, _p, _p, _p, _i, _f, _p, _p],
    "q27h_gated_rmsnorm": [_p, _p, _p, _p, _i, _i, _f, _p],
    "q27h_l2norm_heads": [_p, _i, _i, _i, _i, _f, _p],
    "q27h_gdn_gates": [_p, _p, _p, _p, _p, _p, _i, _i, _p],
    "q27h_gemv_bf16_pair": [_p, _p, _p, _p, _p, _i, _i, _i, _p],
    "q27h_gdn_conv": [_p, _p, _p, _p, _p, _i, _i, _i, _p],
    "q27h_gdn_step": [_p, _p, _p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _f, _i, _p, _i],
    "q27h_gdn_step_chunked": [_p, _p, _p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _f, _p],
    "q27h_gdn_prefill_exact": [_i],
    "q27h_gdn_conv_l2": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _p, _p, _p, _p, _p, _p, _i, _p, _p, _sz],
    "q27h_gdn_conv_prefill": [_p, _p, _p, _p, _p, _i, _i, _i, _f, _p, _p, _p, _p, _p, _p, _i, _p],
    "q27h_gdn_flip_plane": [_p, _p],
    "q27h_flip_plane_to": [_p, _p, _p],
    "q27h_to_bf16": [_p, _p, _sz, _p],
    "q27h_to_q8_wire": [_p, _p, _i, _p, _i, _i, _i, _p],
    "q27h_add_norm_rows_q8": [_p, _p, _p, _i, _i, _p, _f, _p, _p, _p, _p, _i, _p],
    "q27h_kv_cache_bytes": [_i, _i, _i],
    "q27h_attn_prep": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _f, _f, _i, _i, _i, _i, _p, _p, _sz, _p, _p],
    "q27h_get_rows_iq2_s": [_p, _i64, _p, _i, _p, _i, _p, _p],
    "q27h_get_rows_q4_k": [_p, _i64, _p, _i, _p, _i, _p, _p],
    "q27h_get_rows_q6_k": [_p, _i64, _p, _i, _p, _i, _p, _p],
    "q27h_get_rows_q8_0": [_p, _i64, _p, _i, _p, _i, _p, _p],
    "q27h_qmat_bytes": [_i, _i, _i],
    "q27h_qmat_repack": [_i, _i, _i, _p, _p, _p],
    "q27h_qgemv": [_i, _i, _i, _p, _p, _p, _p, _i, _p],
    "q27h_qgemv_f32": [_i, _i, _i, _p, _p, _p, _i, _p],
    "q27h_qgemv_waves": [_i, _i, _i],
    "q27h_gtype_block_bytes": [_i],
    "q27h_gtype_block_size": [_i],
    "q27h_gtype_name": [_i],
    "q27h_gguf_open": [C.c_char_p, C.POINTER(_p)],
    "q27h_gguf_close": [_p],
    "q27h_gguf_n_tensors": [_p],
    "q27h_gguf_find": [_p, C.c_char_p],
    "q27h_gguf_tensor": [_p, _i64, C.POINTER(GTensorC)],
    "q27h_gguf_n_kv": [_p],
    "q27h_gguf_key": [_p, _i64, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)],
    "q27h_gguf_kv": [_p, C.c_char_p, C.POINTER(GValueC)],
    "q27h_gguf_kv_at": [_p, _i64, C.POINTER(GValueC)],
    "q27h_gguf_kv_str_at": [_p, _i64, C.c_uint64, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)],
    "q27h_copy_h2d_staged": [_p, _p, _sz, _i, _p],
    "q27h_gguf_upload_rows": [_p, _i64, _i64, _i64, _p, _i, _p],
    "q27h_last_error": [],
    "q27h_abi_version": [],
}
_RESTYPE = {"q27h_kv_cache_bytes": _sz, "q27h_qmat_bytes": _sz, "q27h_last_error": C.c_char_p,
            "q27h_gtype_name": C.c_char_p, "q27h_gguf_close": None, "q27h_gguf_n_tensors": _i64, "q27h_gguf_find": _i64,
            "q27h_gguf_n_kv": _i64}

_lib = None


def build_library(arch: str = "gfx950", jobs: int = 8) -> str:
    """Compile csrc/*.hip for `arch` with hipcc into lib/libq27h.so (cross-compiles without a GPU)."""
    subprocess.run(["make", "-s", "-C", os.path.join(_HERE, "csrc"), f"-j{jobs}", f"ARCH={arch}"], check=True)
    return LIB_PATH


def lib():
    """The loaded library with ctypes signatures set. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Q27Error(-3, f"{LIB_PATH} is missing: build it with build_library() (or __graft_entry__.build())")
        # torch ships its own HIP runtime (same soname); loading it first makes the library bind to that one
        # instead of pulling a second runtime from /opt/rocm into the process
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, C.c_int)
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise Q27Error(status, lib().q27h_last_error().decode())
