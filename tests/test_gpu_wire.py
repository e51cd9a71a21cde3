"""GPU parity of the two-card wire formats (q27h_to_bf16, q27h_to_q8_wire, q27h_add_norm_rows_q8 through the C ABI)
against the CPU oracle: bit-exact wire bytes, error-feedback rows, x, h, q8_1 and per-16 sums, for both wire widths
(q8b16, q8), first / carried / absent error feedback, and the prefill batch of 2048 rows."""
import sys

import numpy as np
import pytest

import cfgdata as cd
from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu
E, EPS = cd.E, cd.EPS


def say(msg):
    print(f"[gpu-wire] {msg}", flush=True)
    sys.stdout.flush()


def up(dev, a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("qb", [16, 32])
@pytest.mark.parametrize("M,ef_mode", [(2048, "carried"), (4, "first"), (7, "none"), (1, "carried")])
def test_to_q8_wire(q27, oracle, dev, qb, M, ef_mode):
    import torch

    say(f"to_q8_wire qb={qb} M={M} ef={ef_mode}")
    r = cd.rng(1000 + M + qb)
    p = cd.normal(r, M * E, 3.0)
    p[::97] *= 30
    p[E:E + 64] = 0  # zero blocks
    ef0 = None if ef_mode == "none" else cd.normal(r, M * E, 0.01)
    first = ef_mode == "first"
    rb = oracle.wire_row_bytes(E, qb)
    wire = torch.full((M * rb,), 0xAB, dtype=torch.uint8, device=dev)
    ef = None if ef0 is None else up(dev, ef0)
    q27.ops.to_q8_wire(up(dev, p), ef, first, wire, E, M, qb=qb)
    torch.cuda.synchronize()
    ow, oef = oracle.to_q8_wire(p, ef0, first, E, M, qb)
    assert_bits_equal(wire.cpu().numpy(), ow, "wire")
    if ef is not None:
        assert_bits_equal(ef.cpu().numpy(), oef, "ef")


@pytest.mark.parametrize("qb", [16, 32])
@pytest.mark.parametrize("M,with_h,with_xs", [(2048, False, True), (4, True, False), (3, True, True)])
def test_add_norm_rows_q8(q27, oracle, dev, qb, M, with_h, with_xs):
    import torch

    say(f"add_norm_rows_q8 qb={qb} M={M} h={with_h} xs={with_xs}")
    r = cd.rng(1100 + M + qb)
    x, w = cd.normal(r, M * E), cd.normal(r, E, 0.1, 1.0)
    own, _ = oracle.to_q8_wire(cd.normal(r, M * E, 2.0), None, True, E, M, qb)
    recv, _ = oracle.to_q8_wire(cd.normal(r, M * E, 2.0), None, True, E, M, qb)
    dx = up(dev, x)
    h = torch.zeros(M * E, device=dev) if with_h else None
    xq, xd = torch.zeros(M * E, dtype=torch.int8, device=dev), torch.zeros(M * E // 32, device=dev)
    xs = torch.zeros(M * E // 16, device=dev) if with_xs else None
    q27.ops.add_norm_rows_q8(dx, up(dev, own), up(dev, recv), E, M, up(dev, w), EPS, h, xq, xd, xs, qb=qb)
    torch.cuda.synchronize()
    ox, oh, oq, od, os_ = oracle.add_norm_rows_q8(x, own, recv, w, E, M, EPS, qb, with_h, with_xs)
    assert_bits_equal(dx.cpu().numpy(), ox, "x")
    assert_bits_equal(xq.cpu().numpy(), oq, "xq")
    assert_bits_equal(xd.cpu().numpy(), od, "xd")
    if with_h:
        assert_bits_equal(h.cpu().numpy(), oh, "h")
    if with_xs:
        assert_bits_equal(xs.cpu().numpy(), os_, "xs")


@pytest.mark.parametrize("n,offset", [(2048 * E, 0), (4 * E + 2, 0), (4098, 2)])
def test_to_bf16(q27, oracle, dev, n, offset):
    """Quad path (aligned, n % 4 == 0) and pair path (n % 4 == 2, or an 8-byte aligned x); specials and ties."""
    import torch

    say(f"to_bf16 n={n} offset={offset}")
    r = cd.rng(1200 + n)
    x = cd.normal(r, n + offset, 5.0)
    u = x.view(np.uint32)
    u[offset:offset + 16] = (u[offset:offset + 16] & 0xFFFF0000) | 0x8000
    x[offset + 16:offset + 22] = np.array([np.inf, -np.inf, 0.0, -0.0, 1e-40, 3.3e38], np.float32)
    dx = up(dev, x)
    y = torch.zeros(n + 2, dtype=torch.int16, device=dev)
    q27.ops.to_bf16(dx[offset:], y, n)
    torch.cuda.synchronize()
    got = y.cpu().numpy().view(np.uint16)
    assert_bits_equal(got[:n], oracle.to_bf16(x[offset:]), "bf16")
    assert got[n] == 0 and got[n + 1] == 0


@pytest.mark.parametrize("N,K,T", [(48, 5120, 4), (48, 5120, 1), (5, 1032, 3)])
def test_gemv_bf16_pair(q27, oracle, dev, N, K, T):
    """ssm_alpha / ssm_beta of the decode GDN layer (src/model.cu:776), and a K that is not a multiple of 512."""
    import torch

    say(f"gemv_bf16_pair N={N} K={K} T={T}")
    r = cd.rng(1300 + K + T)
    bits = lambda a: cd.to_bf16_values(a).view(np.uint32).__rshift__(16).astype(np.uint16)  # noqa: E731
    Wa, Wb = bits(cd.normal(r, N * K, 0.05)), bits(cd.normal(r, N * K, 0.05))
    x = cd.normal(r, T * K)
    ya, yb = torch.full((T * N,), float("nan"), device=dev), torch.full((T * N,), float("nan"), device=dev)
    q27.ops.gemv_bf16_pair(up(dev, Wa.view(np.int16)), up(dev, Wb.view(np.int16)), up(dev, x), ya, yb, N, K, T)
    torch.cuda.synchronize()
    oa, ob = oracle.gemv_bf16_pair(Wa, Wb, x, N, K, T)
    assert_bits_equal(ya.cpu().numpy(), oa.reshape(-1), "ya")
    assert_bits_equal(yb.cpu().numpy(), ob.reshape(-1), "yb")
