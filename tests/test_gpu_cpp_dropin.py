"""The C++ drop-in headers at run time: tests/cpp/libdropin_layer.so calls the q27:: functions exactly as
src/model.cu does -- a GDN layer (decode with snapshots, prefill in flip mode), the fused ops of an attention + FFN
prefill layer, and a decode GEMV whose weights are read with q27::GGUF and uploaded with qmat_upload -- and every
output is compared bit for bit with the oracle run through the same sequence. A bad shape must surface as the
reference's std::runtime_error (checked on the CPU)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import cfgdata as cd
from conftest import assert_bits_equal

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "tests", "cpp", "libdropin_layer.so")
E, D, KH, H = 5120, 128, cd.KH, cd.HV
CC = cd.C_CONV
EPS = np.float32(1e-6)


def say(msg):
    print(f"[gpu-cpp] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dl(q27):
    q27.lib()  # imports torch first: the helper must bind to the same HIP runtime as torch and the library
    if not os.path.exists(LIB):  # normally built by __graft_entry__.build(); a host-only compile of a few seconds
        import subprocess

        r = subprocess.run(["make", "-s", "-C", os.path.dirname(LIB)], capture_output=True, text=True)
        if r.returncode != 0:
            pytest.skip("tests/cpp helper not built: " + r.stderr[-300:])
    return C.CDLL(LIB)


def test_bad_shape_throws_runtime_error(dl):
    err = C.create_string_buffer(256)
    assert dl.dropin_bad_shape(err, 256) == 1
    assert b"n must be 5120" in err.value


def layer_inputs(r, T):
    f = lambda n, s=1.0: cd.normal(r, n, s)  # noqa: E731
    return dict(x=f(T * E), partial=f(T * E), w_norm=(1 + 0.1 * r.standard_normal(E)).astype(np.float32),
                conv_in=f(T * CC), conv_w=f(CC * 4, 0.5), conv_planes=f(4 * CC * 3), a=f(T * H, 2.0), b=f(T * H, 2.0),
                ssm_a=-np.abs(f(H)), dt_bias=f(H), ssm_planes=f(4 * H * D * D, 0.5),
                gnorm_w=(1 + 0.1 * r.standard_normal(D)).astype(np.float32), z=f(T * H * D))


@pytest.mark.gpu
@pytest.mark.parametrize("T,pin", [(4, 0), (1, 3), (3, 2)])
def test_gdn_decode_layer_through_cpp_headers(q27, oracle, dl, dev, T, pin):
    import torch

    say(f"C++ drop-in GDN decode layer T={T} plane={pin}")
    r = cd.rng(800 + T + pin)
    i = layer_inputs(r, T)
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    d = {k: up(v) for k, v in i.items()}
    plane = torch.tensor([pin], dtype=torch.int32, device=dev)
    h, xq, xd = torch.zeros(T * E, device=dev), torch.zeros(T * E, dtype=torch.int8, device=dev), torch.zeros(T * E // 32, device=dev)
    y, g, beta = torch.zeros(T * CC, device=dev), torch.zeros(T * H, device=dev), torch.zeros(T * H, device=dev)
    o = torch.zeros(T * H * D, device=dev)
    oxq, oxd = torch.zeros(T * H * D, dtype=torch.int8, device=dev), torch.zeros(T * H * D // 32, device=dev)
    bits = lambda a: (cd.to_bf16_values(a).view(np.uint32) >> 16).astype(np.uint16)  # noqa: E731
    w_alpha, w_beta = bits(cd.normal(r, H * E, 0.02)), bits(cd.normal(r, H * E, 0.02))
    ab = torch.zeros(2 * T * H, device=dev)
    dwa, dwb = up(w_alpha.view(np.int16)), up(w_beta.view(np.int16))  # kept alive: the call takes raw pointers
    err = C.create_string_buffer(512)
    p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = dl.dropin_gdn_decode(T, p(d["x"]), p(d["partial"]), p(d["w_norm"]), p(h), p(xq), p(xd),
                              p(dwa), p(dwb), p(ab), p(d["conv_in"]),
                              p(d["conv_w"]), p(d["conv_planes"]), p(plane), p(y), p(d["ssm_a"]),
                              p(d["dt_bias"]), p(g), p(beta), p(d["ssm_planes"]), p(o), p(d["gnorm_w"]), p(d["z"]),
                              p(oxq), p(oxd), s, err, 512)
    assert rc == 0, err.value
    torch.cuda.synchronize()
    ox, oh, oq, od = oracle.sum_norm_q8(i["x"], i["partial"], i["w_norm"], E, T, EPS)
    oa, ob_ = oracle.gemv_bf16_pair(w_alpha, w_beta, oh, H, E, T)
    oy, ocp, og, ob = oracle.gdn_conv_l2(i["conv_in"], i["conv_w"], i["conv_planes"], pin, CC, T, True, 2 * KH, EPS,
                                         oa.reshape(-1), ob_.reshape(-1), i["ssm_a"], i["dt_bias"], H)
    oo, osp = oracle.gdn_step(oy, oy[KH * D:], oy[2 * KH * D:], CC, og, ob, i["ssm_planes"], pin, H, KH, T,
                              np.float32(1.0) / np.sqrt(np.float32(D)), True, False)
    gq, gd, _ = oracle.gated_rmsnorm_q8(oo, i["gnorm_w"], i["z"], H * T, EPS)
    down = lambda t: t.cpu().numpy()  # noqa: E731
    assert_bits_equal(down(ab), np.concatenate([oa.reshape(-1), ob_.reshape(-1)]), "alpha / beta")
    for got, want, what in ((d["x"], ox, "x"), (h, oh, "h"), (xq, oq, "xq"), (xd, od, "xd"), (y, oy, "conv y"),
                            (d["conv_planes"], ocp, "conv planes"), (g, og, "g"), (beta, ob, "beta"), (o, oo, "o"),
                            (d["ssm_planes"], osp, "state planes"), (oxq, gq, "o xq"), (oxd, gd, "o xd")):
        assert_bits_equal(down(got), want, what)


@pytest.mark.gpu
@pytest.mark.parametrize("M,pin", [(300, 0), (2048, 1)])
def test_gdn_prefill_layer_through_cpp_headers(q27, oracle, dl, dev, M, pin):
    import torch

    say(f"C++ drop-in GDN prefill layer M={M} plane={pin}")
    r = cd.rng(900 + M)
    i = layer_inputs(r, M)
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    d = {k: up(v) for k, v in i.items()}
    plane = torch.tensor([pin], dtype=torch.int32, device=dev)
    y, g, beta = torch.zeros(M * CC, device=dev), torch.zeros(M * H, device=dev), torch.zeros(M * H, device=dev)
    o = torch.zeros(M * H * D, device=dev)
    oxq, oxd = torch.zeros(M * H * D, dtype=torch.int8, device=dev), torch.zeros(M * H * D // 32, device=dev)
    oxs = torch.zeros(M * H * D // 16, device=dev)
    err = C.create_string_buffer(512)
    p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    prev = q27.ops.gdn_prefill_exact(True)  # the sequential recurrence, bit for bit against the checker
    rc = dl.dropin_gdn_prefill(M, p(d["conv_in"]), p(d["conv_w"]), p(d["conv_planes"]), p(plane), p(y), p(d["a"]),
                               p(d["b"]), p(d["ssm_a"]), p(d["dt_bias"]), p(g), p(beta), p(d["ssm_planes"]), p(o),
                               p(d["gnorm_w"]), p(d["z"]), p(oxq), p(oxd), p(oxs), s, err, 512)
    torch.cuda.synchronize()
    q27.ops.gdn_prefill_exact(prev)
    assert rc == 0, err.value
    oy, ocp, og, ob = oracle.gdn_conv_prefill(i["conv_in"], i["conv_w"], i["conv_planes"], pin, CC, M, 2 * KH, EPS,
                                              i["a"], i["b"], i["ssm_a"], i["dt_bias"], H)
    oo, osp = oracle.gdn_step(oy, oy[KH * D:], oy[2 * KH * D:], CC, og, ob, i["ssm_planes"], pin, H, KH, M,
                              np.float32(1.0) / np.sqrt(np.float32(D)), False, True)
    gq, gd, gs = oracle.gated_rmsnorm_q8(oo, i["gnorm_w"], i["z"], H * M, EPS, with_xs=True)
    down = lambda t: t.cpu().numpy()  # noqa: E731
    for got, want, what in ((y, oy, "conv y"), (d["conv_planes"], ocp, "conv planes"), (g, og, "g"), (beta, ob, "beta"),
                            (o, oo, "o"), (d["ssm_planes"], osp, "state planes"), (oxq, gq, "o xq"), (oxd, gd, "o xd"),
                            (oxs, gs, "o xs")):
        assert_bits_equal(down(got), want, what)
    assert int(plane.item()) == 1 - pin  # gdn_flip_plane


@pytest.mark.gpu
def test_attn_ffn_prefill_through_cpp_headers(q27, oracle, dl, dev):
    import torch

    M, FF, n_ctx, pos0 = 96, 17408, 4096, 1000
    say(f"C++ drop-in attention + FFN prefill M={M}")
    r = cd.rng(950)
    kind = "iq2_s"
    bb, bv = cd.BLOCK[kind]
    row_bytes = E // bv * bb
    table = cd.random_table(r, kind, 4096, E)
    ids = r.integers(0, 4096, M).astype(np.int32)
    w_attn, w_ffn = cd.normal(r, E, 0.1, 1.0), cd.normal(r, E, 0.1, 1.0)
    qg, k, v = cd.normal(r, M * cd.NQH * 512), cd.normal(r, M * cd.NKVH * 256), cd.normal(r, M * cd.NKVH * 256)
    qw, kw = cd.normal(r, 256, 0.1, 1.0), cd.normal(r, 256, 0.1, 1.0)
    partial, gate, up, ao = cd.normal(r, M * E), cd.normal(r, M * FF, 2.0), cd.normal(r, M * FF, 2.0), cd.normal(r, M * 6144)
    upd = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    z = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt, device=dev)  # noqa: E731
    nb = q27.ops.kv_cache_bytes(cd.NKVH, n_ctx, True)
    dt_, dids, x = upd(table), upd(ids), z(M * E)
    h, xq, xd, xs = z(M * E), z(M * E, torch.int8), z(M * E // 32), z(M * E // 16)
    qn, kc, vc = z(M * cd.NQH * 256), z(nb, torch.uint8), z(nb, torch.uint8)
    xq2, xd2, xs2 = z(M * E, torch.int8), z(M * E // 32), z(M * E // 16)
    gq, gd, gs = z(M * FF, torch.int8), z(M * FF // 32), z(M * FF // 16)
    aq, ad = z(M * 6144, torch.int8), z(M * 6144 // 32)
    ins = [upd(a) for a in (w_attn, qg, k, v, qw, kw, partial, w_ffn, gate, up, ao)]
    dw_attn, dqg, dk, dv, dqw, dkw, dpartial, dw_ffn, dgate, dup, dao = ins
    dpos0 = upd(np.array([pos0], np.int32))  # kept alive: the call takes raw pointers
    p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    err = C.create_string_buffer(512)
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = dl.dropin_attn_prefill(M, p(dt_), C.c_int64(row_bytes), p(dids), p(x), p(dw_attn), p(h), p(xq), p(xd), p(xs),
                                p(dqg), p(dk), p(dv), p(dqw), p(dkw), p(qn), p(kc), p(vc), p(dpos0),
                                n_ctx, C.c_float(cd.THETA_SCALE), p(dpartial), p(dw_ffn), p(xq2), p(xd2), p(xs2), p(dgate),
                                p(dup), FF, p(gq), p(gd), p(gs), p(dao), p(aq), p(ad), s, err, 512)
    assert rc == 0, err.value
    torch.cuda.synchronize()
    ox = oracle.get_rows(kind, table, row_bytes, ids, E)
    oh, oq, od, os_ = oracle.rmsnorm_q8(ox, w_attn, E, M, EPS, with_h=True, with_xs=True)
    okc, ovc = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
    oqn = oracle.attn_prep(qg, k, v, qw, kw, okc, ovc, pos0, M, EPS, cd.THETA_SCALE, cd.NQH, cd.NKVH, n_ctx, True)
    ox2, _, oq2, od2, os2 = oracle.sum_norm_rows(ox, partial, w_ffn, E, M, EPS)
    ogq, ogd, ogs = oracle.swiglu_q8(gate, up, with_xs=True)
    oaq, oad, _ = oracle.quantize_q8_1(ao, 6144, M)
    down = lambda t: t.cpu().numpy()  # noqa: E731
    for got, want, what in ((x, ox2, "x"), (h, oh, "h"), (xq, oq, "attn xq"), (xd, od, "attn xd"), (xs, os_, "attn xs"),
                            (qn, oqn, "qn"), (kc, okc, "kcache"), (vc, ovc, "vcache"), (xq2, oq2, "ffn xq"),
                            (xd2, od2, "ffn xd"), (xs2, os2, "ffn xs"), (gq, ogq, "swiglu xq"), (gd, ogd, "swiglu xd"),
                            (gs, ogs, "swiglu xs"), (aq, oaq, "quantize xq"), (ad, oad, "quantize xd")):
        assert_bits_equal(down(got), want, what)


@pytest.mark.gpu
def test_gguf_gemv_through_cpp_headers(q27, oracle, dl, dev, tmp_path):
    import torch

    import gguf_writer as W

    say("C++ drop-in GGUF -> qmat_upload -> qgemv")
    r = cd.rng(960)
    N, K, nc = 1024, 5120, 4
    raw = cd.random_weights(r, cd.Q6_K, N, K)
    path = tmp_path / "m.gguf"
    path.write_bytes(W.build([("general.architecture", W.STR, "qwen35")],
                             [("blk.0.ffn_down.weight", cd.Q6_K, (K, N), raw.tobytes())]))
    xq, xd = cd.q8_activations(oracle, r, nc, K)
    scratch = torch.empty(raw.size, dtype=torch.uint8, device=dev)
    y = torch.zeros(nc * N, device=dev)
    err = C.create_string_buffer(512)
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    dxq, dxd = torch.from_numpy(xq).to(dev), torch.from_numpy(xd).to(dev)
    rc = dl.dropin_gguf_gemv(str(path).encode(), b"blk.0.ffn_down.weight", C.c_void_p(dxq.data_ptr()),
                             C.c_void_p(dxd.data_ptr()), C.c_void_p(y.data_ptr()), nc, C.c_void_p(scratch.data_ptr()),
                             C.c_size_t(raw.size), s, err, 512)
    assert rc == 0, err.value
    torch.cuda.synchronize()
    assert_bits_equal(y.cpu().numpy().reshape(nc, N), oracle.qgemv(cd.Q6_K, raw, N, K, xq, xd, nc), "gguf gemv")
    rc = dl.dropin_gguf_gemv(str(path).encode(), b"blk.0.missing", C.c_void_p(dxq.data_ptr()), C.c_void_p(dxd.data_ptr()),
                             C.c_void_p(y.data_ptr()), nc, C.c_void_p(scratch.data_ptr()), C.c_size_t(raw.size), s, err, 512)
    assert rc == 1 and err.value == b"missing tensor blk.0.missing"
