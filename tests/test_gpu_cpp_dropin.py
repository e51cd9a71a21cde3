"""The C++ drop-in headers at run time: tests/cpp/libdropin_layer.so calls q27::sum_norm_q8, gdn_conv_l2,
gdn_step, gated_rmsnorm_q8, gdn_conv_prefill and gdn_flip_plane exactly as src/model.cu does for a GDN layer
(decode with snapshots, and prefill in flip mode); every output is compared bit for bit with the oracle run through
the same sequence. A bad shape must surface as the reference's std::runtime_error (checked on the CPU)."""
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
    err = C.create_string_buffer(512)
    p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = dl.dropin_gdn_decode(T, p(d["x"]), p(d["partial"]), p(d["w_norm"]), p(h), p(xq), p(xd), p(d["conv_in"]),
                              p(d["conv_w"]), p(d["conv_planes"]), p(plane), p(y), p(d["a"]), p(d["b"]), p(d["ssm_a"]),
                              p(d["dt_bias"]), p(g), p(beta), p(d["ssm_planes"]), p(o), p(d["gnorm_w"]), p(d["z"]),
                              p(oxq), p(oxd), s, err, 512)
    assert rc == 0, err.value
    torch.cuda.synchronize()
    ox, oh, oq, od = oracle.sum_norm_q8(i["x"], i["partial"], i["w_norm"], E, T, EPS)
    oy, ocp, og, ob = oracle.gdn_conv_l2(i["conv_in"], i["conv_w"], i["conv_planes"], pin, CC, T, True, 2 * KH, EPS,
                                         i["a"], i["b"], i["ssm_a"], i["dt_bias"], H)
    oo, osp = oracle.gdn_step(oy, oy[KH * D:], oy[2 * KH * D:], CC, og, ob, i["ssm_planes"], pin, H, KH, T,
                              np.float32(1.0) / np.sqrt(np.float32(D)), True, False)
    gq, gd, _ = oracle.gated_rmsnorm_q8(oo, i["gnorm_w"], i["z"], H * T, EPS)
    down = lambda t: t.cpu().numpy()  # noqa: E731
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
    rc = dl.dropin_gdn_prefill(M, p(d["conv_in"]), p(d["conv_w"]), p(d["conv_planes"]), p(plane), p(y), p(d["a"]),
                               p(d["b"]), p(d["ssm_a"]), p(d["dt_bias"]), p(g), p(beta), p(d["ssm_planes"]), p(o),
                               p(d["gnorm_w"]), p(d["z"]), p(oxq), p(oxd), p(oxs), s, err, 512)
    assert rc == 0, err.value
    torch.cuda.synchronize()
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
