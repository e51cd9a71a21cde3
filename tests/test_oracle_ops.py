"""Pins of the oracle's fused ops (CPU only): closed forms, invariants, float64 bounds, the reference's own
fused == unfused identities (tools/test_fused.cu:55-102) and encode -> decode round trips for the GGUF blocks.

The reference ships no golden vectors for this path; each check below is chosen so that a plausible slip in
the restatement (a dropped term, a wrong index or sign, a swapped operand) fails it.
"""
import math

import numpy as np
import pytest

from conftest import assert_bits_equal

E = 5120
EPS = 1e-6


def rnd(seed, n, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


# ---------------------------------------------------------------- q8_1
def test_q8_1_closed_forms(oracle):
    x = np.zeros(128, np.float32)
    x[32 + 5] = -3.5                      # block 1: one-hot
    x[64:96] = np.arange(32) - 15.5       # block 2: amax 15.5 -> d = 15.5/127
    x[96:128] = np.float32(0.5)           # block 3: constant
    x[96] = 127.0                         # d = 1 exactly: y/d = y, ties k + 0.5 round away from zero
    x[97], x[98], x[99], x[100] = 2.5, -2.5, 0.5, -0.5
    xq, xd, xs = oracle.quantize_q8_1(x, 128, 1, with_xs=True)
    assert np.all(xq[:32] == 0) and xd[0] == 0 and np.all(xs[:2] == 0)
    assert xq[37] == -127 and np.count_nonzero(xq[32:64]) == 1
    assert xd[1] == np.float32(np.float16(np.float32(3.5) / np.float32(127)))
    assert xq[64] == -127 and xq[95] == 127
    assert list(xq[96:101]) == [127, 3, -3, 1, -1]
    assert xd[3] == 1.0
    assert xs[0] == 0 and xs[4] == np.float32(np.arange(16).sum() - 15.5 * 16) and xs[5] == np.float32(np.arange(16, 32).sum() - 15.5 * 16)


@pytest.mark.parametrize("scale", [1.0, 1e-3, 1e4])
def test_q8_1_bounds_random(oracle, scale):
    K, nc = 1024, 3
    x = rnd(1, K * nc, scale)
    x[::97] *= 50
    xq, xd, xs = oracle.quantize_q8_1(x, K, nc, with_xs=True)
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(1)
    d = amax / np.float32(127)
    assert np.array_equal(xd, d.astype(np.float16).astype(np.float32))     # stored scale = fp16 RNE of d
    q = xq.reshape(-1, 32).astype(np.float64)
    assert np.all(np.abs(q) <= 127) and np.all(np.abs(q).max(1) == 127)
    err = np.abs(q * d[:, None].astype(np.float64) - b)                     # quantized with the unrounded d
    assert np.all(err <= d[:, None] * (0.5 + 1e-5))
    s64 = x.astype(np.float64).reshape(-1, 16)
    assert np.all(np.abs(xs - s64.sum(1)) <= 1e-6 * np.abs(s64).sum(1) + 1e-30)


# ---------------------------------------------------------------- RMSNorm rows
def test_rmsnorm_q8_constant_row(oracle):
    for c in (1.0, 0.5, -2.0):
        x = np.full(E, c, np.float32)
        w = np.ones(E, np.float32)
        h, xq, xd, _ = oracle.rmsnorm_q8(x, w, E, 1, EPS)
        want = np.float32(c) * (np.float32(1) / np.sqrt(np.float32(c * c) + np.float32(EPS)))
        assert np.all(h == want)
        assert np.all(np.abs(xq) == 127)


def test_rmsnorm_q8_float64_bound_and_invariant(oracle):
    rows = 3
    x = rnd(2, rows * E)
    x[np.random.default_rng(3).choice(rows * E, 15, replace=False)] *= 50
    w = np.ones(E, np.float32)
    h, xq, xd, xs = oracle.rmsnorm_q8(x, w, E, rows, EPS, with_xs=True)
    x64 = x.astype(np.float64).reshape(rows, E)
    m = (x64 ** 2).mean(1, keepdims=True)
    h64 = x64 / np.sqrt(m + EPS)
    assert np.max(np.abs(h.reshape(rows, E) - h64) / (np.abs(h64) + 1e-30)) < 2e-6
    mh = (h.astype(np.float64).reshape(rows, E) ** 2).mean(1)
    assert np.allclose(mh, (m / (m + EPS)).ravel(), rtol=1e-5)


def test_rmsnorm_q8_equals_rmsnorm_then_quantize(oracle):
    # tools/test_fused.cu:68-74
    T = 4
    x = rnd(4, T * E, 3.0)
    w = rnd(5, E, 0.5)
    h, xq, xd, xs = oracle.rmsnorm_q8(x, w, E, T, EPS, with_xs=True)
    h2 = oracle.rmsnorm(x, w, E, T, EPS)
    q2, d2, s2 = oracle.quantize_q8_1(h2, E, T, with_xs=True)
    assert_bits_equal(h, h2, "h")
    assert_bits_equal(xq, q2, "xq")
    assert_bits_equal(xd, d2, "xd")
    assert_bits_equal(xs, s2, "xs")


def test_sum_norm_q8_equals_add_rmsnorm_quantize(oracle):
    # tools/test_fused.cu:55-66
    T = 4
    x0 = rnd(6, T * E, 3.0)
    part = rnd(7, T * E)
    w = rnd(8, E, 0.5)
    xa, ha, qa, da = oracle.sum_norm_q8(x0, part, w, E, T, EPS)
    xb = oracle.add(x0, part)
    hb = oracle.rmsnorm(xb, w, E, T, EPS)
    qb, db, _ = oracle.quantize_q8_1(hb, E, T)
    for got, want, what in ((xa, xb, "x"), (ha, hb, "h"), (qa, qb, "xq"), (da, db, "xd")):
        assert_bits_equal(got, want, what)


def test_sum_norm_rows_and_add_norm_rows(oracle):
    M = 5
    x0 = rnd(9, M * E)
    part = rnd(10, M * E)
    w = rnd(11, E, 0.2) + 1
    xa, ha, qa, da = oracle.sum_norm_q8(x0, part, w, E, M, EPS)
    xb, hb, qb, db, sb = oracle.sum_norm_rows(x0, part, w, E, M, EPS, with_h=True)
    for got, want, what in ((xb, xa, "x"), (hb, ha, "h"), (qb, qa, "xq"), (db, da, "xd")):
        assert_bits_equal(got, want, what)
    _, _, sq = oracle.quantize_q8_1(hb, E, M, with_xs=True)
    assert_bits_equal(sb, sq, "xs")
    xc, hc, qc, dc, sc = oracle.add_norm_rows(x0, part, None, w, E, M, EPS, with_h=True)
    for got, want, what in ((xc, xb, "x"), (hc, hb, "h"), (qc, qb, "xq"), (dc, db, "xd"), (sc, sb, "xs")):
        assert_bits_equal(got, want, what)
    # bf16 wire: x + (bf16(partial) + recv), each step one IEEE f32 rounding (numpy float32 arithmetic)
    recv = rnd(12, M * E).astype(np.float32)
    recv_bits = ((recv.view(np.uint32).astype(np.uint64) + 0x7FFF + ((recv.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    xr, _, _, _, _ = oracle.add_norm_rows(x0, part, recv_bits, w, E, M, EPS)
    pu = part.view(np.uint32).astype(np.uint64)
    pb = (((pu + 0x7FFF + ((pu >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    rb = (recv_bits.astype(np.uint32) << 16).view(np.float32)
    assert_bits_equal(xr, x0 + (pb + rb), "x (bf16 wire)")


# ---------------------------------------------------------------- SwiGLU
def test_swiglu_q8_equals_swiglu_then_quantize(oracle):
    n = 4 * 17408
    g = rnd(13, n, 2.0)
    u = rnd(14, n, 2.0)
    xq, xd, xs = oracle.swiglu_q8(g, u, with_xs=True)
    y = oracle.swiglu(g, u)
    q2, d2, s2 = oracle.quantize_q8_1(y, n, 1, with_xs=True)
    assert_bits_equal(xq, q2, "xq")
    assert_bits_equal(xd, d2, "xd")
    assert_bits_equal(xs, s2, "xs")
    g64 = g.astype(np.float64)
    y64 = g64 / (1 + np.exp(-g64)) * u
    assert np.max(np.abs(y - y64) / (np.abs(y64) + 1e-30)) < 1e-6
    assert np.all(oracle.swiglu(np.zeros(64, np.float32), u[:64]) == 0)


# ---------------------------------------------------------------- gated RMSNorm
def test_gated_rmsnorm_q8(oracle):
    heads = 4 * 48
    o = rnd(15, heads * 128)
    z = rnd(16, heads * 128)
    w = rnd(17, 128, 0.1) + 1
    xq, xd, xs = oracle.gated_rmsnorm_q8(o, w, z, heads, EPS, with_xs=True)
    y = oracle.gated_rmsnorm(o, w, z, 128, heads, EPS)
    q2, d2, s2 = oracle.quantize_q8_1(y, 128, heads, with_xs=True)
    assert_bits_equal(xq, q2, "xq")
    assert_bits_equal(xd, d2, "xd")
    assert_bits_equal(xs, s2, "xs")
    o64 = o.astype(np.float64).reshape(heads, 128)
    z64 = z.astype(np.float64).reshape(heads, 128)
    y64 = o64 / np.sqrt((o64 ** 2).mean(1, keepdims=True) + EPS) * w * (z64 / (1 + np.exp(-z64)))
    assert np.max(np.abs(y.reshape(heads, 128) - y64) / (np.abs(y64) + 1e-12)) < 3e-6
    # w = 1 and z = 100 (silu(100) == 100 in float): a plain 128-wide RMSNorm times 100
    y100 = oracle.gated_rmsnorm(o, np.ones(128, np.float32), np.full(heads * 128, 100, np.float32), 128, heads, EPS)
    r = oracle.rmsnorm(o, np.ones(128, np.float32), 128, heads, EPS)
    assert np.max(np.abs(y100 / 100 - r) / (np.abs(r) + 1e-12)) < 2e-6


# ---------------------------------------------------------------- L2 norm and the GDN input stage
def test_l2norm_heads_invariant(oracle):
    T, heads, C = 3, 32, 10240
    x = rnd(18, T * C)
    x[:128] = 0
    y = oracle.l2norm_heads(x, 128, heads, T, C, EPS)
    y3 = y.reshape(T, C)
    x3 = x.reshape(T, C).astype(np.float64)
    for t in range(T):
        for h in range(heads):
            S = (x3[t, 128 * h:128 * h + 128] ** 2).sum()
            got = (y3[t, 128 * h:128 * h + 128].astype(np.float64) ** 2).sum()
            assert abs(got - S / (S + EPS)) < 1e-5
    assert np.all(y[:128] == 0)
    assert np.array_equal(y3[:, 128 * heads:], x.reshape(T, C)[:, 128 * heads:])  # only the first `heads` heads change


def gdn_inputs(seed, T, KH=8, H=24):
    C = 2 * KH * 128 + H * 128
    r = np.random.default_rng(seed)
    f = lambda n, s=1.0: (r.standard_normal(n) * s).astype(np.float32)  # noqa: E731
    return dict(C=C, KH=KH, H=H, x=f(T * C), w=f(C * 4, 0.5), planes=f(4 * C * 3), ab=f(2 * T * H, 2.0), sa=f(H),
                dtb=f(H))


def test_gdn_conv_l2_equals_gates_conv_l2norm(oracle):
    # tools/test_fused.cu:76-102 (E = 5120, T = 4, KH = 8, H = 24)
    T = 4
    d = gdn_inputs(19, T)
    C, H, KH = d["C"], d["H"], d["KH"]
    a, b = d["ab"][:T * H], d["ab"][T * H:]
    y, st, g, beta = oracle.gdn_conv_l2(d["x"], d["w"], d["planes"], 0, C, T, True, 2 * KH, EPS, a, b, d["sa"], d["dtb"], H)
    g2, b2 = oracle.gdn_gates(a, b, d["sa"], d["dtb"], H, T)
    y2, st2 = oracle.gdn_conv(d["x"], d["w"], d["planes"], 0, C, T, True)
    y2 = oracle.l2norm_heads(y2, 128, 2 * KH, T, C, EPS)
    for got, want, what in ((y, y2, "y"), (st, st2, "state"), (g, g2, "g"), (beta, b2, "beta")):
        assert_bits_equal(got, want, what)


def test_gdn_conv_float64_and_gates(oracle):
    T = 4
    d = gdn_inputs(20, T, KH=2, H=4)
    C = d["C"]
    pin = 2
    y, st = oracle.gdn_conv(d["x"], d["w"], d["planes"], pin, C, T, True)
    P = d["planes"].reshape(4, C, 3).astype(np.float64)
    X = d["x"].reshape(T, C).astype(np.float64)
    W = d["w"].reshape(C, 4).astype(np.float64)
    hist = np.concatenate([P[pin].T, X], 0)  # rows: 3 state taps (oldest first), then the T inputs
    for t in range(T):
        s = (hist[t:t + 4].T * W).sum(1)
        want = s / (1 + np.exp(-s))
        assert np.max(np.abs(y.reshape(T, C)[t] - want)) < 1e-5
        assert np.array_equal(st.reshape(4, C, 3)[t], hist[t + 1:t + 4].T.astype(np.float32))  # snapshot of plane t
    a = d["ab"][:T * 4]
    b = d["ab"][T * 4:]
    g, beta = oracle.gdn_gates(a, b, d["sa"], d["dtb"], 4, T)
    a64 = (a.reshape(T, 4) + d["dtb"]).astype(np.float64)
    sp = np.where(a64 > 20, a64, np.log1p(np.exp(a64)))
    assert np.allclose(g.reshape(T, 4), sp * d["sa"], rtol=3e-6, atol=1e-7)
    assert np.allclose(beta, 1 / (1 + np.exp(-b.astype(np.float64))), rtol=3e-7)


def test_gdn_conv_prefill_equals_chained_decode(oracle):
    """Prefill over M rows == the decode conv applied in steps of <= 4 tokens with the state carried."""
    M, KH, H = 11, 2, 4
    d = gdn_inputs(21, M, KH, H)
    C = d["C"]
    a, b = d["ab"][:M * H], d["ab"][M * H:]
    pin = 1
    y, st, g, beta = oracle.gdn_conv_prefill(d["x"], d["w"], d["planes"], pin, C, M, 2 * KH, EPS, a, b, d["sa"], d["dtb"], H)
    planes = d["planes"].copy()
    ys = []
    cur = pin
    for t0 in range(0, M, 4):
        T = min(4, M - t0)
        yt, planes = oracle.gdn_conv(d["x"][t0 * C:(t0 + T) * C], d["w"], planes, cur, C, T, False)
        cur = T - 1
        ys.append(yt)
    y2 = oracle.l2norm_heads(np.concatenate(ys), 128, 2 * KH, M, C, EPS)
    assert_bits_equal(y, y2, "y")
    assert_bits_equal(st.reshape(4, C, 3)[0], planes.reshape(4, C, 3)[cur], "state after the batch (plane 0)")
    assert_bits_equal(st.reshape(4, C, 3)[1], d["planes"].reshape(4, C, 3)[1], "input plane untouched")
    g2, b2 = oracle.gdn_gates(a, b, d["sa"], d["dtb"], H, M)
    assert_bits_equal(g, g2, "g")
    assert_bits_equal(beta, b2, "beta")


def test_gdn_conv_prefill_short_batch_uses_state(oracle):
    M, KH, H = 2, 1, 2
    d = gdn_inputs(22, M, KH, H)
    C = d["C"]
    a, b = d["ab"][:M * H], d["ab"][M * H:]
    _, st, _, _ = oracle.gdn_conv_prefill(d["x"], d["w"], d["planes"], 0, C, M, 2 * KH, EPS, a, b, d["sa"], d["dtb"], H)
    P = d["planes"].reshape(4, C, 3)
    X = d["x"].reshape(M, C)
    want = np.stack([P[0][:, 2], X[0], X[1]], 1)  # last 3 inputs: old tap 3, then the two new rows
    assert np.array_equal(st.reshape(4, C, 3)[1], want)


# ---------------------------------------------------------------- attention input stage
NQH, NKVH = 24, 4
THETA_SCALE = float(np.float32(1e7) ** np.float32(-2.0 / 64))


def attn_inputs(seed, T):
    r = np.random.default_rng(seed)
    f = lambda n, s=1.0: (r.standard_normal(n) * s).astype(np.float32)  # noqa: E731
    return f(T * NQH * 512), f(T * NKVH * 256), f(T * NKVH * 256), f(256, 0.1) + 1, f(256, 0.1) + 1


def run_attn(oracle, T, pos0, n_ctx, q8, seed=23, rope3=None, rdelta=None):
    qg, k, v, qw, kw = attn_inputs(seed, T)
    nb = oracle.kv_cache_bytes(NKVH, n_ctx, q8)
    kc = np.zeros(nb, np.uint8)
    vc = np.zeros(nb, np.uint8)
    qn = oracle.attn_prep(qg, k, v, qw, kw, kc, vc, pos0, T, EPS, THETA_SCALE, NQH, NKVH, n_ctx, q8, rope3, rdelta)
    return qn, kc, vc, (qg, k, v, qw, kw)


def test_attn_prep_rotation(oracle):
    T, pos0, n_ctx = 3, 0, 16
    qn, kc, vc, (qg, k, v, qw, kw) = run_attn(oracle, T, pos0, n_ctx, False)
    qn = qn.reshape(T, NQH, 256)
    q = qg.reshape(T, NQH, 512)[:, :, :256].astype(np.float64)
    qs = q / np.sqrt((q ** 2).mean(2, keepdims=True) + EPS) * qw
    # position 0: identity (cos 0 = 1, sin 0 = 0)
    assert np.max(np.abs(qn[0] - qs[0]) / (np.abs(qs[0]) + 1e-12)) < 2e-6
    # rotation by theta_j = p * theta_scale^j of the pairs (j, j + 32), dims >= 64 untouched
    for t in range(T):
        th = t * np.array([THETA_SCALE ** j for j in range(32)])
        x0, x1 = qs[t, :, :32], qs[t, :, 32:64]
        want = np.concatenate([x0 * np.cos(th) - x1 * np.sin(th), x0 * np.sin(th) + x1 * np.cos(th), qs[t, :, 64:]], 1)
        assert np.max(np.abs(qn[t] - want)) < 5e-6
        n_in = x0 ** 2 + x1 ** 2
        n_out = qn[t, :, :32].astype(np.float64) ** 2 + qn[t, :, 32:64].astype(np.float64) ** 2
        assert np.max(np.abs(n_out - n_in) / (n_in + 1e-12)) < 1e-5
    # f16 cache: K rotated like q (through the k norm), V copied; rows pos0 .. pos0 + T - 1 of each KV head
    kcache = kc.view(np.float16).reshape(NKVH, n_ctx, 256)
    vcache = vc.view(np.float16).reshape(NKVH, n_ctx, 256)
    assert np.array_equal(vcache[:, :T], v.reshape(T, NKVH, 256).transpose(1, 0, 2).astype(np.float16))
    assert np.all(kcache[:, T:] == 0) and np.all(vcache[:, T:] == 0)
    k64 = k.reshape(T, NKVH, 256).astype(np.float64)
    ks = k64 / np.sqrt((k64 ** 2).mean(2, keepdims=True) + EPS) * kw
    assert np.max(np.abs(kcache[:, 0].astype(np.float64) - ks[0]) / (np.abs(ks[0]) + 1e-3)) < 1e-3


def test_attn_prep_long_positions_and_rdelta(oracle):
    T = 4
    qa, kca, vca, _ = run_attn(oracle, T, 150000, 180224, True)
    qb, kcb, vcb, _ = run_attn(oracle, T, 150003, 180224, True, rdelta=3)  # same angles, cache rows shifted by 3
    assert_bits_equal(qa, qb, "qn")
    ia = kca[:NKVH * 180224 * 256].reshape(NKVH, 180224, 256)
    ib = kcb[:NKVH * 180224 * 256].reshape(NKVH, 180224, 256)
    assert np.array_equal(ia[:, 150000:150004], ib[:, 150003:150007])
    # rope3 with t = h = w = p gives the plain positions
    rope3 = np.repeat(np.arange(150000, 150004, dtype=np.int32), 3)
    qc, kcc, _, _ = run_attn(oracle, T, 150000, 180224, True, rope3=rope3)
    assert_bits_equal(qc, qa, "qn (rope3 t=h=w)")
    assert np.array_equal(kcc, kca)


def test_attn_prep_q8_0_cache(oracle):
    T, n_ctx = 2, 8
    qn, kc, vc, (qg, k, v, qw, kw) = run_attn(oracle, T, 5, n_ctx, True)
    so = NKVH * n_ctx * 256
    vq = vc[:so].view(np.int8).reshape(NKVH, n_ctx, 256)
    vs = vc[so:].view(np.float16).reshape(NKVH, n_ctx, 8)
    vv = v.reshape(T, NKVH, 256).transpose(1, 0, 2).reshape(NKVH, T, 8, 32)
    amax = np.abs(vv).max(3)
    d = amax / np.float32(127)
    assert np.array_equal(vs[:, 5:7], d.astype(np.float16))
    q = vq[:, 5:7].reshape(NKVH, T, 8, 32).astype(np.float64)
    assert np.all(np.abs(q).max(3) == 127)
    assert np.all(np.abs(q * d[..., None] - vv) <= d[..., None] * (0.5 + 1e-5))
    assert np.all(vq[:, :5] == 0) and np.all(vq[:, 7:] == 0)
    # out-of-range cache rows are not written
    _, kz, vz, _ = run_attn(oracle, 2, n_ctx - 1, n_ctx, True)
    assert np.all(kz[:so].view(np.int8).reshape(NKVH, n_ctx, 256)[:, :n_ctx - 1] == 0)


# ---------------------------------------------------------------- gathers: encode -> decode round trips
def h16(x):
    return np.array([x], np.float16).view(np.uint16)[0]


def enc_q8_0(d, q):
    b = bytearray(34)
    b[0:2] = int(h16(d)).to_bytes(2, "little")
    b[2:34] = np.asarray(q, np.int8).tobytes()
    return bytes(b)


def enc_q4_k(d, dmin, sc, mn, q):
    """sc, mn: 8 six-bit values; q: 256 four-bit values in value order."""
    b = bytearray(144)
    b[0:2] = int(h16(d)).to_bytes(2, "little")
    b[2:4] = int(h16(dmin)).to_bytes(2, "little")
    s = bytearray(12)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    b[4:16] = s
    for j in range(4):
        for l in range(32):
            b[16 + 32 * j + l] = (q[64 * j + l] & 15) | ((q[64 * j + 32 + l] & 15) << 4)
    return bytes(b)


def enc_q6_k(d, sc, q):
    """sc: 16 int8 scales; q: 256 six-bit values (0..63) in value order."""
    b = bytearray(210)
    for half in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q[128 * half + l + 32 * i] for i in range(4))
            b[64 * half + l] = (q1 & 15) | ((q3 & 15) << 4)
            b[64 * half + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            b[128 + 32 * half + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b[192:208] = np.asarray(sc, np.int8).tobytes()
    b[208:210] = int(h16(d)).to_bytes(2, "little")
    return bytes(b)


def enc_iq2_s(d, scales4, gidx, signs):
    """scales4: 16 four-bit scales (two per 32-group); gidx: 32 ten-bit grid indices; signs: 32 sign bytes."""
    b = bytearray(82)
    b[0:2] = int(h16(d)).to_bytes(2, "little")
    for ib in range(8):
        qh = 0
        for l in range(4):
            gi = gidx[4 * ib + l]
            b[2 + 4 * ib + l] = gi & 0xFF
            qh |= ((gi >> 8) & 3) << (2 * l)
            b[34 + 4 * ib + l] = signs[4 * ib + l]
        b[66 + ib] = qh
        b[74 + ib] = (scales4[2 * ib] & 15) | ((scales4[2 * ib + 1] & 15) << 4)
    return bytes(b)


def test_get_rows_q8_0_closed_form(oracle):
    r = np.random.default_rng(24)
    n, vocab = 256, 6
    d = r.uniform(2 ** -10, 2 ** -4, (vocab, n // 32)).astype(np.float16)
    q = r.integers(-128, 128, (vocab, n), dtype=np.int8)
    table = b"".join(enc_q8_0(d[v, k], q[v, 32 * k:32 * k + 32]) for v in range(vocab) for k in range(n // 32))
    ids = np.array([3, 0, 5, 3, -2], np.int32)
    img = r.standard_normal((2, n)).astype(np.float32)
    y = oracle.get_rows("q8_0", np.frombuffer(table, np.uint8), n // 32 * 34, ids, n, img).reshape(-1, n)
    for t, i in enumerate(ids[:4]):
        want = q[i].astype(np.float32) * np.repeat(d[i].astype(np.float32), 32)
        assert np.array_equal(y[t], want)
    assert np.array_equal(y[4], img[1])


def test_get_rows_q4_k_roundtrip(oracle):
    r = np.random.default_rng(25)
    blocks, want = [], []
    for _ in range(4):
        d, dm = np.float16(r.uniform(1e-3, 1e-2)), np.float16(r.uniform(1e-3, 1e-2))
        sc, mn = r.integers(0, 64, 8), r.integers(0, 64, 8)
        q = r.integers(0, 16, 256)
        blocks.append(enc_q4_k(d, dm, sc, mn, q))
        g = np.arange(256) // 32
        want.append(np.float32(d) * sc[g].astype(np.float32) * q.astype(np.float32) - np.float32(dm) * mn[g].astype(np.float32))
    table = np.frombuffer(b"".join(blocks), np.uint8)
    y = oracle.get_rows("q4_k", table, 144 * 2, np.array([1, 0], np.int32), 512).reshape(2, 512)
    assert np.array_equal(y[0], np.concatenate(want[2:4]))
    assert np.array_equal(y[1], np.concatenate(want[0:2]))


def test_get_rows_q6_k_roundtrip(oracle):
    r = np.random.default_rng(26)
    blocks, want = [], []
    for _ in range(3):
        d = np.float16(r.uniform(1e-3, 1e-2))
        sc = r.integers(-128, 128, 16)
        q = r.integers(0, 64, 256)
        blocks.append(enc_q6_k(d, sc, q))
        want.append(np.float32(d) * sc[np.arange(256) // 16].astype(np.float32) * (q - 32).astype(np.float32))
    table = np.frombuffer(b"".join(blocks), np.uint8)
    y = oracle.get_rows("q6_k", table, 210, np.array([2, 0, 1], np.int32), 256).reshape(3, 256)
    for t, i in enumerate([2, 0, 1]):
        assert np.array_equal(y[t], want[i])


def test_get_rows_iq2_s_roundtrip(oracle):
    grid = oracle.iq2s_grid()
    r = np.random.default_rng(27)
    d = np.float16(r.uniform(1e-3, 1e-2))
    scales4 = r.integers(0, 16, 16)
    gidx = r.integers(0, 1024, 32)
    signs = r.integers(0, 256, 32)
    table = np.frombuffer(enc_iq2_s(d, scales4, gidx, signs), np.uint8)
    y = oracle.get_rows("iq2_s", table, 82, np.array([0], np.int32), 256)
    for i in range(256):
        ib, l, j = i // 32, (i % 32) // 8, i % 8
        db = np.float32(d) * (np.float32(0.5) + np.float32(scales4[2 * ib + (l >= 2)])) * np.float32(0.25)
        mag = np.float32((int(grid[gidx[4 * ib + l]]) >> (8 * j)) & 0xFF)
        sgn = np.float32(-1 if (signs[4 * ib + l] >> j) & 1 else 1)
        assert y[i] == db * mag * sgn, i


def test_iq2s_grid_table(oracle):
    g = oracle.iq2s_grid()
    assert len(g) == 1024 and len(set(g.tolist())) == 1024 and np.all(g[1:] > g[:-1])
    mags = {(int(v) >> (8 * j)) & 0xFF for v in g for j in range(8)}
    assert mags == {0x08, 0x19, 0x2B}
    assert int(g[0]) == 0x0808080808080808 and int(g[-1]) == 0x2B2B2B2B2B2B2B2B
