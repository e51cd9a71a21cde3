"""ctypes binding of the CPU oracle (oracle/lib/libq27oracle.so): TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; the product
library never imports it. Every wrapper takes and returns numpy arrays; the C side follows the reference
kernels' float order (see q27_oracle.c).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "lib", "libq27oracle.so")

_f = C.c_float
_i = C.c_int
_p = C.c_void_p
_i64 = C.c_int64

_SIGS = {
    "q27o_expf": (_f, [_f]),
    "q27o_logf": (_f, [_f]),
    "q27o_sincos": (None, [_f, _p, _p]),
    "q27o_silu": (_f, [_f]),
    "q27o_sigmoid": (_f, [_f]),
    "q27o_softplus": (_f, [_f]),
    "q27o_f2h": (C.c_uint16, [_f]),
    "q27o_h2f": (_f, [C.c_uint16]),
    "q27o_f2bf": (C.c_uint16, [_f]),
    "q27o_bf2f": (_f, [C.c_uint16]),
    "q27o_rope_freqs": (None, [_f, _p]),
    "q27o_quantize_q8_1": (None, [_p, _p, _p, _i, _i, _p]),
    "q27o_rmsnorm": (None, [_p, _p, _p, _i, _i, _f, _i]),
    "q27o_add": (None, [_p, _p, _p, _i]),
    "q27o_swiglu": (None, [_p, _p, _p, _i]),
    "q27o_rmsnorm_q8": (None, [_p, _p, _p, _p, _p, _i, _i, _f, _p]),
    "q27o_sum_norm_q8": (None, [_p, _p, _i, _i, _p, _f, _p, _p, _p]),
    "q27o_sum_norm_rows": (None, [_p, _p, _i, _i, _p, _f, _p, _p, _p, _p]),
    "q27o_add_norm_rows": (None, [_p, _p, _p, _i, _i, _p, _f, _p, _p, _p, _p]),
    "q27o_swiglu_q8": (None, [_p, _p, _p, _p, _i, _p]),
    "q27o_gated_rmsnorm": (None, [_p, _p, _p, _p, _i, _i, _f]),
    "q27o_gated_rmsnorm_q8": (None, [_p, _p, _p, _p, _p, _i, _f, _p]),
    "q27o_l2norm_heads": (None, [_p, _i, _i, _i, _i, _f]),
    "q27o_gdn_gates": (None, [_p, _p, _p, _p, _p, _p, _i, _i]),
    "q27o_gdn_conv": (None, [_p, _p, _p, _i, _p, _i, _i, _i]),
    "q27o_gdn_conv_l2": (None, [_p, _p, _p, _i, _p, _i, _i, _i, _i, _f, _p, _p, _p, _p, _p, _p, _i]),
    "q27o_gdn_conv_prefill": (None, [_p, _p, _p, _i, _p, _i, _i, _i, _f, _p, _p, _p, _p, _p, _p, _i]),
    "q27o_kv_cache_bytes": (C.c_size_t, [_i, _i, _i]),
    "q27o_attn_prep": (None, [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _f, _f, _i, _i, _i, _i, _p, _p]),
    "q27o_get_rows_iq2_s": (None, [_p, _i64, _p, _i, _p, _i, _p]),
    "q27o_get_rows_q4_k": (None, [_p, _i64, _p, _i, _p, _i, _p]),
    "q27o_get_rows_q6_k": (None, [_p, _i64, _p, _i, _p, _i, _p]),
    "q27o_get_rows_q8_0": (None, [_p, _i64, _p, _i, _p, _i, _p]),
    "q27o_iq2s_grid": (C.POINTER(C.c_uint64), []),
    "q27o_qgemv_block_bytes": (_i, [_i]),
    "q27o_qgemv_waves": (_i, [_i, _i, _i]),
    "q27o_qgemv": (_i, [_i, _p, _i, _i, _p, _p, _p, _i]),
    "q27o_to_bf16": (None, [_p, _p, C.c_size_t]),
    "q27o_gemv_bf16_pair": (None, [_p, _p, _p, _p, _p, _i, _i, _i]),
    "q27o_to_q8_wire": (None, [_p, _p, _i, _p, _i, _i, _i]),
    "q27o_add_norm_rows_q8": (None, [_p, _p, _p, _i, _i, _p, C.c_float, _p, _p, _p, _p, _i]),
    "q27o_gdn_step": (_i, [_p, _p, _p, _i, _p, _p, _p, _i, _p, _i, _i, _i, C.c_float, _i, _i]),
    "q27o_gdn_step_parts": (_i, [_i, _p, _p, _p, _i, _p, _p, _p, _i, _p, _i, _i, _i, C.c_float, _i, _i]),
}

_lib = None


def build() -> None:
    """Compile the oracle with its Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous numpy arrays"
    return a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- scalar math
def expf(x: float) -> float:
    return lib().q27o_expf(x)


def logf(x: float) -> float:
    return lib().q27o_logf(x)


def sincos(theta: float):
    s, c = C.c_float(), C.c_float()
    lib().q27o_sincos(theta, C.byref(s), C.byref(c))
    return s.value, c.value


def silu(x):
    return lib().q27o_silu(x)


def f2h(x: float) -> int:
    return lib().q27o_f2h(x)


def h2f(h: int) -> float:
    return lib().q27o_h2f(h)


def f2bf(x: float) -> int:
    return lib().q27o_f2bf(x)


def rope_freqs(theta_scale: float) -> np.ndarray:
    out = np.zeros(32, np.float32)
    lib().q27o_rope_freqs(theta_scale, _ptr(out))
    return out


# ---------------------------------------------------------------- ops (numpy in, numpy out)
def quantize_q8_1(x, K, ncols, with_xs=False):
    x = _f32(x)
    xq = np.zeros(K * ncols, np.int8)
    xd = np.zeros(K * ncols // 32, np.float32)
    xs = np.zeros(K * ncols // 16, np.float32) if with_xs else None
    lib().q27o_quantize_q8_1(_ptr(x), _ptr(xq), _ptr(xd), K, ncols, _ptr(xs))
    return xq, xd, xs


def rmsnorm(x, w, n, rows, eps, ystride=0):
    x, w = _f32(x), _f32(w)
    ys = ystride or n
    y = np.zeros(rows * ys, np.float32)
    lib().q27o_rmsnorm(_ptr(x), _ptr(w), _ptr(y), n, rows, eps, ystride)
    return y


def add(x, a):
    x, a = _f32(x), _f32(a)
    y = np.zeros_like(x)
    lib().q27o_add(_ptr(x), _ptr(a), _ptr(y), x.size)
    return y


def swiglu(g, u):
    g, u = _f32(g), _f32(u)
    y = np.zeros_like(g)
    lib().q27o_swiglu(_ptr(g), _ptr(u), _ptr(y), g.size)
    return y


def rmsnorm_q8(x, w, n, rows, eps, with_h=True, with_xs=False):
    x, w = _f32(x), _f32(w)
    h = np.zeros(rows * n, np.float32) if with_h else None
    xq = np.zeros(rows * n, np.int8)
    xd = np.zeros(rows * n // 32, np.float32)
    xs = np.zeros(rows * n // 16, np.float32) if with_xs else None
    lib().q27o_rmsnorm_q8(_ptr(x), _ptr(w), _ptr(h), _ptr(xq), _ptr(xd), n, rows, eps, _ptr(xs))
    return h, xq, xd, xs


def sum_norm_q8(x, partial, w, n, rows, eps, with_h=True):
    x = _f32(x).copy()
    partial, w = _f32(partial), _f32(w)
    h = np.zeros(rows * n, np.float32) if with_h else None
    xq = np.zeros(rows * n, np.int8)
    xd = np.zeros(rows * n // 32, np.float32)
    lib().q27o_sum_norm_q8(_ptr(x), _ptr(partial), n, rows, _ptr(w), eps, _ptr(h), _ptr(xq), _ptr(xd))
    return x, h, xq, xd


def sum_norm_rows(x, partial, w, n, M, eps, with_h=False, with_xs=True):
    x = _f32(x).copy()
    partial, w = _f32(partial), _f32(w)
    h = np.zeros(M * n, np.float32) if with_h else None
    xq = np.zeros(M * n, np.int8)
    xd = np.zeros(M * n // 32, np.float32)
    xs = np.zeros(M * n // 16, np.float32) if with_xs else None
    lib().q27o_sum_norm_rows(_ptr(x), _ptr(partial), n, M, _ptr(w), eps, _ptr(h), _ptr(xq), _ptr(xd), _ptr(xs))
    return x, h, xq, xd, xs


def add_norm_rows(x, partial, recv_bf16, w, n, M, eps, with_h=False, with_xs=True):
    x = _f32(x).copy()
    partial, w = _f32(partial), _f32(w)
    recv = None if recv_bf16 is None else np.ascontiguousarray(recv_bf16, dtype=np.uint16)
    h = np.zeros(M * n, np.float32) if with_h else None
    xq = np.zeros(M * n, np.int8)
    xd = np.zeros(M * n // 32, np.float32)
    xs = np.zeros(M * n // 16, np.float32) if with_xs else None
    lib().q27o_add_norm_rows(_ptr(x), _ptr(partial), _ptr(recv), n, M, _ptr(w), eps, _ptr(h), _ptr(xq), _ptr(xd), _ptr(xs))
    return x, h, xq, xd, xs


def swiglu_q8(g, u, with_xs=False):
    g, u = _f32(g), _f32(u)
    n = g.size
    xq = np.zeros(n, np.int8)
    xd = np.zeros(n // 32, np.float32)
    xs = np.zeros(n // 16, np.float32) if with_xs else None
    lib().q27o_swiglu_q8(_ptr(g), _ptr(u), _ptr(xq), _ptr(xd), n, _ptr(xs))
    return xq, xd, xs


def gated_rmsnorm(o, w, z, n, heads, eps):
    o, w, z = _f32(o), _f32(w), _f32(z)
    y = np.zeros(n * heads, np.float32)
    lib().q27o_gated_rmsnorm(_ptr(o), _ptr(w), _ptr(z), _ptr(y), n, heads, eps)
    return y


def gated_rmsnorm_q8(o, w, z, heads, eps, with_xs=False):
    o, w, z = _f32(o), _f32(w), _f32(z)
    xq = np.zeros(heads * 128, np.int8)
    xd = np.zeros(heads * 4, np.float32)
    xs = np.zeros(heads * 8, np.float32) if with_xs else None
    lib().q27o_gated_rmsnorm_q8(_ptr(o), _ptr(w), _ptr(z), _ptr(xq), _ptr(xd), heads, eps, _ptr(xs))
    return xq, xd, xs


def l2norm_heads(x, n, heads, T, stride, eps):
    x = _f32(x).copy()
    lib().q27o_l2norm_heads(_ptr(x), n, heads, T, stride, eps)
    return x


def gdn_gates(a, b, ssm_a, dt_bias, H, T):
    a, b, ssm_a, dt_bias = _f32(a), _f32(b), _f32(ssm_a), _f32(dt_bias)
    g = np.zeros(H * T, np.float32)
    beta = np.zeros(H * T, np.float32)
    lib().q27o_gdn_gates(_ptr(a), _ptr(b), _ptr(ssm_a), _ptr(dt_bias), _ptr(g), _ptr(beta), H, T)
    return g, beta


def gdn_conv(x, w, planes, in_plane, C_, T, snapshots):
    x, w = _f32(x), _f32(w)
    planes = _f32(planes).copy()
    y = np.zeros(T * C_, np.float32)
    lib().q27o_gdn_conv(_ptr(x), _ptr(w), _ptr(planes), in_plane, _ptr(y), C_, T, int(snapshots))
    return y, planes


def gdn_conv_l2(x, w, planes, in_plane, C_, T, snapshots, n_norm_heads, eps, a, b, ssm_a, dt_bias, H):
    x, w, a, b, ssm_a, dt_bias = map(_f32, (x, w, a, b, ssm_a, dt_bias))
    planes = _f32(planes).copy()
    y = np.zeros(T * C_, np.float32)
    g = np.zeros(T * H, np.float32)
    beta = np.zeros(T * H, np.float32)
    lib().q27o_gdn_conv_l2(_ptr(x), _ptr(w), _ptr(planes), in_plane, _ptr(y), C_, T, int(snapshots), n_norm_heads, eps,
                           _ptr(a), _ptr(b), _ptr(ssm_a), _ptr(dt_bias), _ptr(g), _ptr(beta), H)
    return y, planes, g, beta


def gdn_conv_prefill(x, w, planes, in_plane, C_, M, n_norm_heads, eps, a, b, ssm_a, dt_bias, H):
    x, w, a, b, ssm_a, dt_bias = map(_f32, (x, w, a, b, ssm_a, dt_bias))
    planes = _f32(planes).copy()
    y = np.zeros(M * C_, np.float32)
    g = np.zeros(M * H, np.float32)
    beta = np.zeros(M * H, np.float32)
    lib().q27o_gdn_conv_prefill(_ptr(x), _ptr(w), _ptr(planes), in_plane, _ptr(y), C_, M, n_norm_heads, eps, _ptr(a),
                                _ptr(b), _ptr(ssm_a), _ptr(dt_bias), _ptr(g), _ptr(beta), H)
    return y, planes, g, beta


def kv_cache_bytes(nkvh, n_ctx, q8):
    return lib().q27o_kv_cache_bytes(nkvh, n_ctx, int(q8))


def attn_prep(qg, k, v, q_norm, k_norm, kcache, vcache, pos0, T, eps, theta_scale, nqh, nkvh, n_ctx, q8, rope3=None,
              rdelta=None):
    """kcache / vcache: uint8 numpy arrays of kv_cache_bytes, updated in place. Returns qn."""
    qg, k, v, q_norm, k_norm = map(_f32, (qg, k, v, q_norm, k_norm))
    qn = np.zeros(T * nqh * 256, np.float32)
    r3 = None if rope3 is None else np.ascontiguousarray(rope3, dtype=np.int32)
    rd = None if rdelta is None else np.array([rdelta], np.int32)
    lib().q27o_attn_prep(_ptr(qg), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(qn), _ptr(kcache), _ptr(vcache),
                         pos0, T, eps, theta_scale, nqh, nkvh, n_ctx, int(q8), _ptr(r3), _ptr(rd))
    return qn


def get_rows(kind, table, row_bytes, ids, n, img=None):
    table = np.ascontiguousarray(table, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    img = None if img is None else _f32(img)
    y = np.zeros(ids.size * n, np.float32)
    getattr(lib(), "q27o_get_rows_" + kind)(_ptr(table), row_bytes, _ptr(ids), ids.size, _ptr(y), n, _ptr(img))
    return y


def iq2s_grid() -> np.ndarray:
    p = lib().q27o_iq2s_grid()
    return np.ctypeslib.as_array(p, shape=(1024,)).copy()


def qgemv(type_, raw, N, K, xq, xd, ncols):
    """Decode GEMV over raw GGUF rows (q27_oracle_qgemv.c): returns y [ncols][N] (f32)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xd = _f32(xd)
    y = np.zeros(ncols * N, np.float32)
    if lib().q27o_qgemv(type_, _ptr(raw), N, K, _ptr(xq), _ptr(xd), _ptr(y), ncols) != 0:
        raise ValueError("q27o_qgemv: bad type or shape")
    return y.reshape(ncols, N)


def qgemv_waves(type_, K, ncols):
    return int(lib().q27o_qgemv_waves(type_, K, ncols))


def gdn_step(q, k, v, stride, g, beta, planes, in_plane, H, HK, T, scale, snapshots, flip, parts=None):
    """Delta-rule recurrence (q27_oracle_gdn.c). q / k / v share the row stride; returns (o [T][H][128], planes).
    `parts` (8 or 16) overrides the contract's part count."""
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    planes = _f32(planes).copy()
    o = np.zeros(T * H * 128, np.float32)
    args = (_ptr(q), _ptr(k), _ptr(v), stride, _ptr(g), _ptr(beta), _ptr(planes), in_plane, _ptr(o), H, HK, T, scale,
            int(snapshots), int(flip))
    rc = lib().q27o_gdn_step(*args) if parts is None else lib().q27o_gdn_step_parts(parts, *args)
    if rc != 0:
        raise ValueError("q27o_gdn_step: bad shape")
    return o, planes


def wire_row_bytes(n, qb):
    return n + 2 * n // qb


def to_bf16(x):
    x = _f32(x)
    y = np.zeros(x.size, np.uint16)
    lib().q27o_to_bf16(_ptr(x), _ptr(y), x.size)
    return y


def to_q8_wire(partial, ef, first, n, M, qb):
    """Returns (wire uint8 [M][n + 2n/qb], ef after the call or None)."""
    partial = _f32(partial)
    ef = None if ef is None else _f32(ef).copy()
    wire = np.zeros(M * wire_row_bytes(n, qb), np.uint8)
    lib().q27o_to_q8_wire(_ptr(partial), _ptr(ef), int(first), _ptr(wire), n, M, qb)
    return wire, ef


def add_norm_rows_q8(x, own, recv, w, n, M, eps, qb, with_h=False, with_xs=True):
    x = _f32(x).copy()
    w = _f32(w)
    own = np.ascontiguousarray(own, dtype=np.uint8)
    recv = np.ascontiguousarray(recv, dtype=np.uint8)
    h = np.zeros(M * n, np.float32) if with_h else None
    xq = np.zeros(M * n, np.int8)
    xd = np.zeros(M * n // 32, np.float32)
    xs = np.zeros(M * n // 16, np.float32) if with_xs else None
    lib().q27o_add_norm_rows_q8(_ptr(x), _ptr(own), _ptr(recv), n, M, _ptr(w), eps, _ptr(h), _ptr(xq), _ptr(xd), _ptr(xs),
                                qb)
    return x, h, xq, xd, xs


def gemv_bf16_pair(Wa, Wb, x, N, K, T):
    """Wa, Wb: bf16 bit patterns (uint16) [N][K]; returns (ya [T][N], yb [T][N])."""
    Wa = np.ascontiguousarray(Wa, dtype=np.uint16)
    Wb = np.ascontiguousarray(Wb, dtype=np.uint16)
    x = _f32(x)
    ya = np.zeros(T * N, np.float32)
    yb = np.zeros(T * N, np.float32)
    lib().q27o_gemv_bf16_pair(_ptr(Wa), _ptr(Wb), _ptr(x), _ptr(ya), _ptr(yb), N, K, T)
    return ya.reshape(T, N), yb.reshape(T, N)
