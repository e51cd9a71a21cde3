"""Pins of the oracle's wire formats of the two-card sum (to_bf16, to_q8_wire, add_norm_rows_q8) and of
gemv_bf16_pair (CPU only).

The reference ships no vectors for them (src/prefill.cu:338-406). Pins: bf16 rounding against an integer
restatement of round-to-nearest-even (and the specials); closed-form q8 blocks (zero, one-hot, exact ties);
the quantization error bound; the error-feedback identity (with ef carried, the sum of K dequantized rows stays
within one rounding step of K times the partial, while without it the error grows with K); and add_norm_rows_q8 ==
sum_norm_rows on the dequantized sum (the already pinned row engine). gemv_bf16_pair: one-hot rows, exact integer
dots and a float64 bound.
"""
import numpy as np
import pytest

E = 5120
EPS = 1e-6


def rnd(seed, n, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


def unpack(wire, n, M, qb):
    rb = n + 2 * n // qb
    w = wire.reshape(M, rb)
    q = w[:, :n].view(np.int8).astype(np.float32)
    d = w[:, n:].copy().view(np.float16).astype(np.float32)
    return q, d


def dequant(wire, n, M, qb):
    q, d = unpack(wire, n, M, qb)
    return (q.reshape(M, n // qb, qb) * d[:, :, None]).reshape(M, n)


def test_to_bf16_rne_and_specials(oracle):
    x = rnd(1, 4096, 3.0)
    x[:8] = np.array([0.0, -0.0, np.inf, -np.inf, 3.0e38, 1e-40, -1e-45, 1.0], np.float32)
    u = x.view(np.uint32).copy()
    u[8:16] = (u[8:16] & 0xFFFF0000) | 0x8000  # exact ties: to even
    u[16:24] = (u[16:24] & 0xFFFF0000) | 0x8001  # just above a tie: up
    x = u.view(np.float32)
    got = oracle.to_bf16(x)
    lo, hi = u & 0xFFFF, u >> 16
    want = (hi + ((lo > 0x8000) | ((lo == 0x8000) & (hi & 1 == 1)))).astype(np.uint16)
    finite = np.isfinite(x)
    assert np.array_equal(got[finite], want[finite])
    assert got[2] == 0x7F80 and got[3] == 0xFF80
    n = oracle.to_bf16(np.array([np.nan, -np.nan], np.float32))
    assert np.all((n & 0x7F80) == 0x7F80) and np.all((n & 0x7F) != 0)  # NaN stays NaN


@pytest.mark.parametrize("qb", [16, 32])
def test_q8_wire_closed_forms(oracle, qb):
    p = np.zeros(E, np.float32)
    p[qb + 3] = -2.5                            # block 1: one-hot
    p[2 * qb:3 * qb] = 1.5                      # block 2: constant
    p[3 * qb] = 127.0                           # block 3: d = 1 exactly, ties round away from zero
    p[3 * qb + 1:3 * qb + 5] = [2.5, -2.5, 0.5, -0.5]
    wire, ef = oracle.to_q8_wire(p, np.zeros(E, np.float32), True, E, 1, qb)
    q, d = unpack(wire, E, 1, qb)
    assert np.all(q[0, :qb] == 0) and d[0, 0] == 0                       # zero block
    assert q[0, qb + 3] == -127 and np.count_nonzero(q[0, qb:2 * qb]) == 1
    assert d[0, 1] == np.float32(np.float16(np.float32(2.5) / np.float32(127)))
    assert np.all(q[0, 2 * qb:3 * qb] == 127)
    assert list(q[0, 3 * qb:3 * qb + 5]) == [127, 3, -3, 1, -1] and d[0, 3] == 1.0
    assert np.all(ef[3 * qb + 1:3 * qb + 5] == np.float32([-0.5, 0.5, -0.5, 0.5]))  # y - 1 * q
    assert np.all(ef[:qb] == 0)


@pytest.mark.parametrize("qb", [16, 32])
def test_q8_wire_error_bound(oracle, qb):
    M = 3
    p = rnd(2, M * E, 4.0)
    p[::131] *= 40
    wire, ef = oracle.to_q8_wire(p, np.zeros(M * E, np.float32), True, E, M, qb)
    q, d = unpack(wire, E, M, qb)
    amax = np.abs(p.reshape(M, E // qb, qb)).max(-1)
    dd = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(d, dd.astype(np.float16).astype(np.float32))
    assert np.all(np.abs(q) <= 127)
    bound = (dd * (0.5 + 127 * 2.0 ** -11) * (1 + 1e-6))[:, :, None]
    assert np.all(np.abs(ef.reshape(M, E // qb, qb)) <= bound)
    # ef is the difference to what the wire carries
    assert np.allclose(p.reshape(M, E) - dequant(wire, E, M, qb), ef.reshape(M, E), rtol=0, atol=1e-6 * np.abs(p).max())


def test_q8_wire_error_feedback_does_not_accumulate(oracle):
    """Carried ef: sum_k dequant_k = K p + ef_0 - ef_K, so the accumulated error stays one rounding step; with
    first = True every time (no feedback) it grows with K."""
    qb, K = 16, 40
    p = rnd(3, E, 1.0)
    ef = np.zeros(E, np.float32)
    acc_fb = np.zeros(E, np.float64)
    acc_nofb = np.zeros(E, np.float64)
    for k in range(K):
        wire, ef = oracle.to_q8_wire(p, ef, k == 0, E, 1, qb)
        acc_fb += dequant(wire, E, 1, qb)[0]
        wire0, _ = oracle.to_q8_wire(p, None, True, E, 1, qb)
        acc_nofb += dequant(wire0, E, 1, qb)[0]
    err_fb = np.abs(acc_fb - K * p.astype(np.float64)).max()
    err_nofb = np.abs(acc_nofb - K * p.astype(np.float64)).max()
    step = np.abs(p).max() / 127
    assert err_fb <= 1.01 * step * (0.5 + 127 * 2.0 ** -11)
    assert err_nofb > 5 * err_fb


@pytest.mark.parametrize("qb", [16, 32])
def test_add_norm_rows_q8_equals_unfused(oracle, qb):
    M = 4
    x, w = rnd(4, M * E), (1 + 0.1 * rnd(5, E)).astype(np.float32)
    own, _ = oracle.to_q8_wire(rnd(6, M * E, 2.0), None, True, E, M, qb)
    recv, _ = oracle.to_q8_wire(rnd(7, M * E, 2.0), None, True, E, M, qb)
    partial = (dequant(own, E, M, qb) + dequant(recv, E, M, qb)).astype(np.float32).reshape(-1)  # exact products, one add
    got = oracle.add_norm_rows_q8(x, own, recv, w, E, M, EPS, qb, with_h=True, with_xs=True)
    want = oracle.sum_norm_rows(x, partial, w, E, M, EPS, with_h=True, with_xs=True)
    for g, wnt in zip(got, want):
        assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                              wnt.view(np.uint32) if wnt.dtype == np.float32 else wnt)


# ---------------------------------------------------------------- gemv_bf16_pair (src/ops.cu:377-393)
def bf16_bits(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_gemv_bf16_pair_one_hot_and_integer_exact(oracle):
    """One-hot rows pick single activations exactly; small-integer weights and activations make every partial sum
    an exact integer, so the result must equal the exact dot product (a wrong index or a dropped pair fails)."""
    N, K, T = 6, 5120, 3
    r = np.random.default_rng(8)
    x = r.standard_normal(T * K).astype(np.float32)
    Wa = np.zeros((N, K), np.float32)
    cols = r.integers(0, K, N)
    Wa[np.arange(N), cols] = 1.0
    Wb = r.integers(-3, 4, (N, K)).astype(np.float32)
    xi = r.integers(-4, 5, T * K).astype(np.float32)
    ya, _ = oracle.gemv_bf16_pair(bf16_bits(Wa), bf16_bits(Wb), x, N, K, T)
    assert np.array_equal(ya, x.reshape(T, K)[:, cols])
    _, yb = oracle.gemv_bf16_pair(bf16_bits(Wa), bf16_bits(Wb), xi, N, K, T)
    assert np.array_equal(yb, xi.reshape(T, K) @ Wb.T)


def test_gemv_bf16_pair_float64_bound(oracle):
    N, K, T = 48, 5120, 4
    r = np.random.default_rng(9)
    Wa, Wb = (r.standard_normal((N, K)) * 0.05).astype(np.float32), (r.standard_normal((N, K)) * 0.05).astype(np.float32)
    ba, bb = bf16_bits(Wa), bf16_bits(Wb)
    x = r.standard_normal(T * K).astype(np.float32)
    ya, yb = oracle.gemv_bf16_pair(ba, bb, x, N, K, T)
    fa = (ba.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    fb = (bb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x64 = x.reshape(T, K).astype(np.float64)
    for got, f in ((ya, fa), (yb, fb)):
        want = x64 @ f.T
        mag = np.abs(x64) @ np.abs(f).T
        assert np.all(np.abs(got - want) <= 1e-6 * mag + 1e-30)
