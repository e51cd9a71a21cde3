"""The reference engine's launchers (src/ops.h, src/prefill.h, src/qmat.h) over torch device tensors.

Same names, argument order and defaults as the C++ declarations; tensors stand for device pointers (None for
nullptr), `s` is a HIP stream handle (int) and defaults to torch's current stream. Every function only
enqueues work. A bad shape or a failed launch raises Q27Error (the reference throws std::runtime_error).
"""
from __future__ import annotations

from ._lib import check, lib


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(s):
    if s is not None:
        return s
    import torch

    return torch.cuda.current_stream().cuda_stream


# ---------------------------------------------------------------- ops.h
def rmsnorm(x, w, y, n, rows, eps, s=None, ystride=0):
    check(lib().q27h_rmsnorm(_ptr(x), _ptr(w), _ptr(y), n, rows, eps, _stream(s), ystride))


def add(x, a, y, n, s=None):
    check(lib().q27h_add(_ptr(x), _ptr(a), _ptr(y), n, _stream(s)))


def swiglu(g, u, y, n, s=None):
    check(lib().q27h_swiglu(_ptr(g), _ptr(u), _ptr(y), n, _stream(s)))


def set_int(p, v, s=None):
    check(lib().q27h_set_int(_ptr(p), v, _stream(s)))


def get_rows_iq2_s(table, row_bytes, ids, T, y, n, s=None, img=None):
    check(lib().q27h_get_rows_iq2_s(_ptr(table), row_bytes, _ptr(ids), T, _ptr(y), n, _stream(s), _ptr(img)))


def get_rows_q4_k(table, row_bytes, ids, T, y, n, s=None, img=None):
    check(lib().q27h_get_rows_q4_k(_ptr(table), row_bytes, _ptr(ids), T, _ptr(y), n, _stream(s), _ptr(img)))


def get_rows_q6_k(table, row_bytes, ids, T, y, n, s=None, img=None):
    check(lib().q27h_get_rows_q6_k(_ptr(table), row_bytes, _ptr(ids), T, _ptr(y), n, _stream(s), _ptr(img)))


def get_rows_q8_0(table, row_bytes, ids, T, y, n, s=None, img=None):
    check(lib().q27h_get_rows_q8_0(_ptr(table), row_bytes, _ptr(ids), T, _ptr(y), n, _stream(s), _ptr(img)))


def gdn_gates(a, b, ssm_a, dt_bias, g, beta, H, T, s=None):
    check(lib().q27h_gdn_gates(_ptr(a), _ptr(b), _ptr(ssm_a), _ptr(dt_bias), _ptr(g), _ptr(beta), H, T, _stream(s)))


def gemv_bf16_pair(Wa, Wb, x, ya, yb, N, K, T, s=None):
    """src/ops.h:24-26: ya[t] = Wa x[t], yb[t] = Wb x[t] (Wa, Wb bf16 [N][K] as 16-bit tensors)."""
    check(lib().q27h_gemv_bf16_pair(_ptr(Wa), _ptr(Wb), _ptr(x), _ptr(ya), _ptr(yb), N, K, T, _stream(s)))


def gdn_conv(x, w, planes, in_plane, y, C, T, snapshots, s=None):
    check(lib().q27h_gdn_conv(_ptr(x), _ptr(w), _ptr(planes), _ptr(in_plane), _ptr(y), C, T, int(snapshots), _stream(s)))


def gdn_step(q, k, v, stride, g, beta, planes, in_plane, o, H, HK, T, scale, snapshots, s=None, flip=False):
    """src/ops.h:40-45: the gated delta rule over T tokens (flip: prefill, final state to the other plane)."""
    check(lib().q27h_gdn_step(_ptr(q), _ptr(k), _ptr(v), stride, _ptr(g), _ptr(beta), _ptr(planes), _ptr(in_plane),
                              _ptr(o), H, HK, T, scale, int(snapshots), _stream(s), int(flip)))


def gdn_step_chunked(q, k, v, stride, g, beta, planes, in_plane, o, H, HK, T, scale, s=None):
    """gdn_step's prefill (flip) mode in the chunked form on matrix cores (no counterpart in the reference)."""
    check(lib().q27h_gdn_step_chunked(_ptr(q), _ptr(k), _ptr(v), stride, _ptr(g), _ptr(beta), _ptr(planes),
                                      _ptr(in_plane), _ptr(o), H, HK, T, scale, _stream(s)))


def gdn_prefill_exact(on):
    """Process-wide: True = the GDN prefill path in the checker's bits (gdn_step's prefill sequential,
    gdn_conv_prefill's SiLU and L2 scale correctly rounded), False (the default) = the faster forms within the 1e-5
    fp32 bar (the chunked recurrence from 128 tokens on, the hardware-exp SiLU and rsq L2 scale of the conv). Returns
    the previous setting."""
    return bool(lib().q27h_gdn_prefill_exact(int(bool(on))))


def l2norm_heads(x, n, heads, T, stride, eps, s=None):
    check(lib().q27h_l2norm_heads(_ptr(x), n, heads, T, stride, eps, _stream(s)))


def gated_rmsnorm(o, w, z, y, n, heads, eps, s=None):
    check(lib().q27h_gated_rmsnorm(_ptr(o), _ptr(w), _ptr(z), _ptr(y), n, heads, eps, _stream(s)))


def kv_cache_bytes(nkvh, n_ctx, q8):
    return lib().q27h_kv_cache_bytes(nkvh, n_ctx, int(q8))


def attn_prep(qg, k, v, q_norm, k_norm, qn, kcache, vcache, pos0, T, eps, theta_scale, nqh, nkvh, n_ctx, q8, s=None,
              pf=None, pf_bytes=0, rope3=None, rdelta=None):
    check(lib().q27h_attn_prep(_ptr(qg), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(qn), _ptr(kcache),
                               _ptr(vcache), _ptr(pos0), T, eps, theta_scale, nqh, nkvh, n_ctx, int(q8), _stream(s),
                               _ptr(pf), pf_bytes, _ptr(rope3), _ptr(rdelta)))


def rmsnorm_q8(x, w, h, xq, xd, n, rows, eps, s=None, xs=None):
    check(lib().q27h_rmsnorm_q8(_ptr(x), _ptr(w), _ptr(h), _ptr(xq), _ptr(xd), n, rows, eps, _stream(s), _ptr(xs)))


def sum_norm_q8(x, partial, n, rows, ar, w, eps, h, xq, xd, s=None, pf=None, pf_bytes=0):
    check(lib().q27h_sum_norm_q8(_ptr(x), _ptr(partial), n, rows, _ptr(ar), _ptr(w), eps, _ptr(h), _ptr(xq), _ptr(xd),
                                 _stream(s), _ptr(pf), pf_bytes))


def swiglu_q8(g, u, xq, xd, n, s=None, xs=None):
    check(lib().q27h_swiglu_q8(_ptr(g), _ptr(u), _ptr(xq), _ptr(xd), n, _stream(s), _ptr(xs)))


def gated_rmsnorm_q8(o, w, z, xq, xd, heads, eps, s=None, xs=None):
    check(lib().q27h_gated_rmsnorm_q8(_ptr(o), _ptr(w), _ptr(z), _ptr(xq), _ptr(xd), heads, eps, _stream(s), _ptr(xs)))


def gdn_conv_l2(x, w, planes, in_plane, y, C, T, snapshots, n_norm_heads, eps, a, b, ssm_a, dt_bias, g, beta, H, s=None,
                pf=None, pf_bytes=0):
    check(lib().q27h_gdn_conv_l2(_ptr(x), _ptr(w), _ptr(planes), _ptr(in_plane), _ptr(y), C, T, int(snapshots),
                                 n_norm_heads, eps, _ptr(a), _ptr(b), _ptr(ssm_a), _ptr(dt_bias), _ptr(g), _ptr(beta), H,
                                 _stream(s), _ptr(pf), pf_bytes))


# ---------------------------------------------------------------- prefill.h
def gdn_conv_prefill(x, w, planes, in_plane, y, C, M, n_norm_heads, eps, a, b, ssm_a, dt_bias, g, beta, H, s=None):
    check(lib().q27h_gdn_conv_prefill(_ptr(x), _ptr(w), _ptr(planes), _ptr(in_plane), _ptr(y), C, M, n_norm_heads, eps,
                                      _ptr(a), _ptr(b), _ptr(ssm_a), _ptr(dt_bias), _ptr(g), _ptr(beta), H, _stream(s)))


def gdn_flip_plane(plane, s=None):
    check(lib().q27h_gdn_flip_plane(_ptr(plane), _stream(s)))


def flip_plane_to(dst, src, s=None):
    check(lib().q27h_flip_plane_to(_ptr(dst), _ptr(src), _stream(s)))


def wire_qb():
    """src/ops.cu:20-30: values per scale on the q8 wire from Q27_WIRE (q8: 32, q8b16: 16, bf16: 0; default 16)."""
    import os

    v = os.environ.get("Q27_WIRE")
    if v is None:
        return 16
    table = {"q8": 32, "q8b16": 16, "bf16": 0}
    if v not in table:
        raise ValueError("Q27_WIRE: bf16, q8 or q8b16")
    return table[v]


def to_bf16(x, y, n, s=None):
    """src/prefill.h:35: y (bf16 as uint16 / int16 / bfloat16 tensor) = bf16(x)."""
    check(lib().q27h_to_bf16(_ptr(x), _ptr(y), n, _stream(s)))


def to_q8_wire(partial, ef, first, wire, n, M, s=None, qb=None):
    """src/prefill.h:38: q8 wire rows of partial (+ ef unless first), ef <- rounding error (may be None)."""
    check(lib().q27h_to_q8_wire(_ptr(partial), _ptr(ef), int(first), _ptr(wire), n, M, wire_qb() if qb is None else qb,
                                _stream(s)))


def add_norm_rows_q8(x, own, recv, n, M, w, eps, h, xq, xd, xs, s=None, qb=None):
    """src/prefill.h:40-41: x += dequant(own) + dequant(recv), then RMSNorm * w -> h, q8_1, xs."""
    check(lib().q27h_add_norm_rows_q8(_ptr(x), _ptr(own), _ptr(recv), n, M, _ptr(w), eps, _ptr(h), _ptr(xq), _ptr(xd),
                                      _ptr(xs), wire_qb() if qb is None else qb, _stream(s)))


def sum_norm_rows(x, partial, n, M, ex, w, eps, h, xq, xd, xs, s=None):
    check(lib().q27h_sum_norm_rows(_ptr(x), _ptr(partial), n, M, _ptr(ex), _ptr(w), eps, _ptr(h), _ptr(xq), _ptr(xd),
                                   _ptr(xs), _stream(s)))


def add_norm_rows(x, partial, recv, n, M, w, eps, h, xq, xd, xs, s=None):
    check(lib().q27h_add_norm_rows(_ptr(x), _ptr(partial), _ptr(recv), n, M, _ptr(w), eps, _ptr(h), _ptr(xq), _ptr(xd),
                                   _ptr(xs), _stream(s)))


# ---------------------------------------------------------------- qmat.h
def quantize_q8_1(x, xq, xd, K, ncols, s=None, xs=None):
    check(lib().q27h_quantize_q8_1(_ptr(x), _ptr(xq), _ptr(xd), K, ncols, _stream(s), _ptr(xs)))


# Weight types of the decode GEMV: ggml type ids (src/gguf.h:12-14).
Q2_K, Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 10, 12, 14, 16, 17, 18, 21, 22, 23, 29
BLOCK_BYTES = {Q2_K: 84, Q4_K: 144, Q6_K: 210, IQ2_XXS: 66, IQ2_XS: 74, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ4_XS: 136,
               IQ1_M: 56}


class QMat:
    """A quantized weight matrix on the GPU in the tile layout (src/qmat.h:19-29): `buf` is a torch uint8 device
    tensor owning the repacked bytes."""

    def __init__(self, type, N, K, buf):
        self.type, self.N, self.K, self.buf = type, N, K, buf
        self.nb, self.ntiles, self.bytes = K // 256, N // 8, buf.numel()


def qmat_bytes(type, N, K):
    return int(lib().q27h_qmat_bytes(type, N, K))


def qmat_supported(type):
    return type in BLOCK_BYTES


def qmat_upload(raw, type, N, K, s=None):
    """Repack N raw GGUF rows (a torch uint8 tensor on the device, [N][K/256] blocks) into a new QMat
    (src/qmat.h:34, qmat_upload after its host-to-device copy)."""
    import torch

    nbytes = qmat_bytes(type, N, K)
    if nbytes == 0:
        check(lib().q27h_qmat_repack(type, N, K, None, None, _stream(s)))  # raises with the reason
    buf = torch.empty(nbytes, dtype=torch.uint8, device=raw.device)
    check(lib().q27h_qmat_repack(type, N, K, _ptr(raw), _ptr(buf), _stream(s)))
    return QMat(type, N, K, buf)


def qmat_free(m):
    m.buf = None


def qgemv(m, xq, xd, y, ncols, s=None):
    check(lib().q27h_qgemv(m.type, m.N, m.K, _ptr(m.buf), _ptr(xq), _ptr(xd), _ptr(y), ncols, _stream(s)))


def qgemv_f32(m, x, y, ncols, s=None):
    """quantize_q8_1 of x (f32 [ncols][K]) and qgemv in one launch (q27h_qgemv_f32)."""
    check(lib().q27h_qgemv_f32(m.type, m.N, m.K, _ptr(m.buf), _ptr(x), _ptr(y), ncols, _stream(s)))


def qgemv_waves(type_, K, ncols):
    return int(lib().q27h_qgemv_waves(type_, K, ncols))
