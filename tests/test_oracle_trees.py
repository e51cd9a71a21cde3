"""The oracle's summation trees, pinned by sums derived by hand (CPU only).

Each test feeds an input of tests/treepins.py, whose sums depend on the order of the float32 additions, and
checks an output that shows the sum (a norm scale through h / y / qn, or the q8_1 block sum xs) against the value
derived by hand for the reference's tree (src/ops.cu:34-50, 93-108, 279, 441-443, 605; src/common.cuh:80-86).
Each test also checks that the derived value differs from what a sequential sum, a reversed per-thread order or a
contiguous thread layout would give, so a mistake of that kind in the oracle fails here.

The products of a norm are `scale * v * w`, associated left to right as C does ((scale * v) * w,
src/ops.cu:66,103,282); rows of small integers, whose sums of squares are exact in any order, pin that association
against numpy's float32 arithmetic.
"""
import numpy as np
import pytest

import treepins as tp
from cfgdata import round_half_away

E = tp.N_ROW
f32 = np.float32


def expect_row(v, w, scale):
    return (f32(scale) * v) * w


def test_tree_sums_separate_the_orders():
    """The hand-derived sums differ from the other orders' sums, and each differs enough to change the scale at
    the eps the tests use."""
    for good, bad in [(tp.ROW_WARPS_SUM, tp.ROW_WARPS_SEQ), (tp.ROW_CROSS_SUM, tp.ROW_CROSS_SEQ),
                      (tp.ROW_KORDER_SUM, tp.ROW_KORDER_REV)]:
        assert good != bad
        tp.eps_separating(good, bad, E)
    for n in (128, 256):
        tp.eps_separating(tp.HEAD_WARPS_SUM[n], tp.HEAD_WARPS_SEQ[n], n)
    tp.eps_separating(tp.GATED_CROSS_SUM, tp.GATED_CROSS_SEQ, 128)
    tp.eps_separating(tp.L2_LANES_SUM, tp.L2_LANES_SEQ, 128, tp.l2_scale)
    tp.eps_separating(tp.L2_KORDER_SUM, tp.L2_KORDER_REV, 128, tp.l2_scale)


ROW_CASES = [("warps", tp.row_warps, tp.ROW_WARPS_SUM, tp.ROW_WARPS_SEQ),
             ("cross", tp.row_cross, tp.ROW_CROSS_SUM, tp.ROW_CROSS_SEQ),
             ("korder", tp.row_korder, tp.ROW_KORDER_SUM, tp.ROW_KORDER_REV)]


@pytest.mark.parametrize("name,make,t_good,t_bad", ROW_CASES, ids=[c[0] for c in ROW_CASES])
@pytest.mark.parametrize("m", [1.0, 2.0 ** -7])
def test_row_norm_tree(oracle, name, make, t_good, t_bad, m):
    """rmsnorm, rmsnorm_q8, sum_norm_q8, sum_norm_rows and add_norm_rows: h = scale * v with the scale of the
    hand-derived sum of squares, for two rows (the second is the first times 2)."""
    m2 = m * m
    eps = tp.eps_separating(t_good, t_bad, E, m2=m2)
    v1 = make(m)
    x = np.concatenate([v1, v1 * f32(2)])
    w = np.ones(E, np.float32)
    want = np.concatenate([expect_row(v1, w, tp.row_scale(t_good * m2, E, eps)),
                           expect_row(v1 * f32(2), w, tp.row_scale(t_good * m2 * 4, E, eps))])
    other = np.concatenate([expect_row(v1, w, tp.row_scale(t_bad * m2, E, eps)),
                            expect_row(v1 * f32(2), w, tp.row_scale(t_bad * m2 * 4, E, eps))])
    assert not np.array_equal(want, other)
    zero = np.zeros_like(x)
    assert np.array_equal(oracle.rmsnorm(x, w, E, 2, eps), want)
    assert np.array_equal(oracle.rmsnorm_q8(x, w, E, 2, eps)[0], want)
    assert np.array_equal(oracle.sum_norm_q8(x, zero, w, E, 2, eps)[1], want)
    assert np.array_equal(oracle.sum_norm_rows(x, zero, w, E, 2, eps, with_h=True)[1], want)
    assert np.array_equal(oracle.add_norm_rows(x, zero, None, w, E, 2, eps, with_h=True)[1], want)


def test_row_norm_products_associate_left(oracle):
    """h = (scale * v) * w. Integer rows |v| <= 8 have exact sums of squares in any order, so the scale is known."""
    r = np.random.default_rng(91)
    rows = 8
    x = r.integers(-8, 9, rows * E).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(E)).astype(np.float32)
    eps = 1e-6
    t = (x.astype(np.float64).reshape(rows, E) ** 2).sum(1)
    s = np.array([tp.row_scale(ti, E, eps) for ti in t], np.float32)[:, None]
    xr = x.reshape(rows, E)
    left = ((s * xr) * w).ravel()
    right = (s * (xr * w)).ravel()
    assert np.count_nonzero(left != right) > 1000
    h, xq, xd, _ = oracle.rmsnorm_q8(x, w, E, rows, eps)
    assert np.array_equal(h, left)
    assert np.array_equal(oracle.rmsnorm(x, w, E, rows, eps), left)
    b = left.reshape(-1, 32)
    d = np.abs(b).max(1) / f32(127)
    assert np.array_equal(xq.reshape(-1, 32).astype(np.float64), round_half_away(b / d[:, None]))


@pytest.mark.parametrize("case", ["warps", "cross"])
def test_gated_head_tree(oracle, case):
    """gated_rmsnorm(_q8): the scale of a 128-head from the 4-warp block_sum, y = ((scale * v) * w) * silu(z) with
    w = 1 and z = 64, where silu(64) = 64 exactly (e^-64 vanishes next to 1)."""
    if case == "warps":
        v, t_good, t_bad = tp.head_warps(128), tp.HEAD_WARPS_SUM[128], tp.HEAD_WARPS_SEQ[128]
    else:
        v, t_good, t_bad = tp.gated_cross(), tp.GATED_CROSS_SUM, tp.GATED_CROSS_SEQ
    eps = tp.eps_separating(t_good, t_bad, 128)
    w = np.ones(128, np.float32)
    z = np.full(128, 64.0, np.float32)
    want = ((tp.row_scale(t_good, 128, eps) * v) * w) * f32(64)
    other = ((tp.row_scale(t_bad, 128, eps) * v) * w) * f32(64)
    assert not np.array_equal(want, other)
    assert np.array_equal(oracle.gated_rmsnorm(v, w, z, 128, 1, eps), want)
    _, _, xs = oracle.gated_rmsnorm_q8(v, w, z, 1, eps, with_xs=True)
    # the second 16 of the head hold (scale * 1) * 64 sixteen times (or 0): its xs is 16 times that, exactly
    assert xs[1] == f32(16) * want[16]


def test_gated_products_associate_left(oracle):
    """((scale * v) * w) * silu(z) with integer heads (exact sums of squares) and z in [32, 64) (silu(z) == z)."""
    r = np.random.default_rng(92)
    heads = 256
    o = r.integers(-8, 9, heads * 128).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(128)).astype(np.float32)
    z = r.uniform(32, 64, heads * 128).astype(np.float32)
    eps = 1e-6
    t = (o.astype(np.float64).reshape(heads, 128) ** 2).sum(1)
    s = np.array([tp.row_scale(ti, 128, eps) for ti in t], np.float32)[:, None]
    ob, zb = o.reshape(heads, 128), z.reshape(heads, 128)
    left = (((s * ob) * w) * zb).ravel()
    assert np.count_nonzero(left != ((s * (ob * w)) * zb).ravel()) > 1000
    assert np.count_nonzero(left != ((s * ob) * (w * zb)).ravel()) > 1000
    assert np.array_equal(oracle.gated_rmsnorm(o, w, z, 128, heads, eps), left)
    xq, xd, xs = oracle.gated_rmsnorm_q8(o, w, z, heads, eps, with_xs=True)
    b = left.reshape(-1, 32)
    d = np.abs(b).max(1) / f32(127)
    assert np.array_equal(xq.reshape(-1, 32).astype(np.float64), round_half_away(b / d[:, None]))
    # xs sums the unrounded products, so it sees a one-ulp difference in any of them
    assert np.array_equal(xs, tp.butterfly16(left))


def test_attn_products_associate_left(oracle):
    """attn_prep's head norm: qn = (scale * v) * w at position 0 (the rotation is the identity there), with integer
    heads (exact sums of squares)."""
    r = np.random.default_rng(93)
    nqh, nkvh, T, n_ctx = 24, 4, 1, 4
    qg = r.integers(-8, 9, (T, nqh, 512)).astype(np.float32)
    k = r.integers(-8, 9, T * nkvh * 256).astype(np.float32)
    wq = (1 + 0.1 * r.standard_normal(256)).astype(np.float32)
    wk = (1 + 0.1 * r.standard_normal(256)).astype(np.float32)
    eps = 1e-6
    nb = oracle.kv_cache_bytes(nkvh, n_ctx, False)
    kc, vc = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
    qn = oracle.attn_prep(qg.ravel(), k, k, wq, wk, kc, vc, 0, T, eps, tp.f32(0.6), nqh, nkvh, n_ctx, False)
    q = qg[0, :, :256]
    s = np.array([tp.row_scale(t, 256, eps) for t in (q.astype(np.float64) ** 2).sum(1)], np.float32)[:, None]
    left = (s * q) * wq
    assert np.count_nonzero(left != s * (q * wq)) > 100
    assert np.array_equal(qn.reshape(nqh, 256), left)
    kh = k.reshape(nkvh, 256)
    sk = np.array([tp.row_scale(t, 256, eps) for t in (kh.astype(np.float64) ** 2).sum(1)], np.float32)[:, None]
    kcache = kc.view(np.float16).reshape(nkvh, n_ctx, 256)
    assert np.array_equal(kcache[:, 0], ((sk * kh) * wk).astype(np.float16))


L2_CASES = [("lanes", tp.l2_lanes, tp.L2_LANES_SUM, tp.L2_LANES_SEQ),
            ("korder", tp.l2_korder, tp.L2_KORDER_SUM, tp.L2_KORDER_REV)]


def l2_expect(v, t, eps):
    return (v * tp.l2_scale(t, 128, eps)) * (f32(1) / np.sqrt(f32(128)))


@pytest.mark.parametrize("name,make,t_good,t_bad", L2_CASES, ids=[c[0] for c in L2_CASES])
def test_l2_head_tree(oracle, name, make, t_good, t_bad):
    """l2norm_heads: out = (p * scale) * (1 / sqrt(128)), scale from the warp's strided lanes and butterfly."""
    eps = tp.eps_separating(t_good, t_bad, 128, tp.l2_scale)
    v = make()
    want = l2_expect(v, t_good, eps)
    assert not np.array_equal(want, l2_expect(v, t_bad, eps))
    # 3 rows of stride 384: heads 0 and 1 normed, head 2 untouched
    x = np.tile(np.concatenate([v, v * f32(0.5), v]), 3)
    got = oracle.l2norm_heads(x, 128, 2, 3, 384, eps).reshape(3, 3, 128)
    for t in range(3):
        assert np.array_equal(got[t, 0], want)
        assert np.array_equal(got[t, 1], l2_expect(v * f32(0.5), t_good * 0.25, eps))
        assert np.array_equal(got[t, 2], v)


@pytest.mark.parametrize("name,make,t_good,t_bad", L2_CASES, ids=[c[0] for c in L2_CASES])
@pytest.mark.parametrize("kind", ["conv_l2", "conv_prefill"])
def test_conv_l2_tree(oracle, name, make, t_good, t_bad, kind):
    """The L2 norm fused into gdn_conv_l2 / gdn_conv_prefill: conv weights (0, 0, 0, 1) and a zero state make the
    conv output the input itself, and inputs 32 and 2^17 pass SiLU unchanged (e^-32 vanishes next to 1); so the
    normed heads are the pattern in units of 32."""
    m = 32.0
    eps = tp.eps_separating(t_good, t_bad, 128, tp.l2_scale, m2=m * m)
    v = make(m)
    C, nk, H = 384, 2, 1
    T = 3
    x = np.tile(np.concatenate([v, v, np.full(128, m, np.float32)]), T)
    w = np.tile(np.array([0, 0, 0, 1], np.float32), C)
    planes = np.zeros(4 * C * 3, np.float32)
    gz = np.zeros(T * H, np.float32)
    one = np.ones(H, np.float32)
    if kind == "conv_l2":
        y = oracle.gdn_conv_l2(x, w, planes, 0, C, T, False, nk, eps, gz, gz, one, one, H)[0]
    else:
        y = oracle.gdn_conv_prefill(x, w, planes, 0, C, T, nk, eps, gz, gz, one, one, H)[0]
    want = l2_expect(v, t_good * m * m, eps)
    assert not np.array_equal(want, l2_expect(v, t_bad * m * m, eps))
    y = y.reshape(T, 3, 128)
    for t in range(T):
        assert np.array_equal(y[t, 0], want)
        assert np.array_equal(y[t, 1], want)
        assert np.array_equal(y[t, 2], np.full(128, m, np.float32))


def test_attn_head_tree(oracle):
    """attn_prep: the 256-head RMSNorm's 8-warp block_sum. At position 0 the rotation is the identity (cos 0 = 1,
    sin 0 = 0), so qn = (scale * v) * w for every dim."""
    n = 256
    t_good, t_bad = tp.HEAD_WARPS_SUM[n], tp.HEAD_WARPS_SEQ[n]
    eps = tp.eps_separating(t_good, t_bad, n)
    v = tp.head_warps(n)
    nqh, nkvh, T, n_ctx = 24, 4, 1, 4
    qg = np.zeros((T, nqh, 512), np.float32)
    qg[:, :, :256] = v
    k = np.tile(v, T * nkvh)
    w = np.ones(256, np.float32)
    nb = oracle.kv_cache_bytes(nkvh, n_ctx, False)
    kc, vc = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
    qn = oracle.attn_prep(qg.ravel(), k, k, w, w, kc, vc, 0, T, eps, tp.f32(0.6), nqh, nkvh, n_ctx, False)
    want = (tp.row_scale(t_good, n, eps) * v) * w
    assert not np.array_equal(want, (tp.row_scale(t_bad, n, eps) * v) * w)
    assert np.array_equal(qn.reshape(-1, nqh, 256)[0, 5], want)
    kcache = kc.view(np.float16).reshape(nkvh, n_ctx, 256)
    assert np.array_equal(kcache[2, 0], want.astype(np.float16))


def test_xs_butterfly(oracle):
    """quantize_q8_1's xs: the xor 8, 4, 2, 1 sums of tests/treepins.py, not the sequential ones."""
    x, want = tp.xs_blocks()
    assert not np.array_equal(want, tp.XS_SEQ)
    K = 64
    _, _, xs = oracle.quantize_q8_1(x, K, 1, with_xs=True)
    assert np.array_equal(xs, want)
    assert np.array_equal(tp.butterfly16(x), want)


def test_xs_butterfly_in_fused_producers(oracle):
    """The same xs through swiglu_q8 (u = the pattern's sign times 1, g = |pattern| * 32 >= 32, so silu(g) = g),
    rmsnorm_q8 / sum_norm_rows / add_norm_rows (v = 1 and eps = 0 make the scale exactly 1, so y = w) and
    gated_rmsnorm_q8 (a head of ones with eps = 0: scale 1; y = w * silu(z))."""
    x, want = tp.xs_blocks()
    g = np.abs(x) * f32(32)
    u = np.sign(x).astype(np.float32)
    _, _, xs = oracle.swiglu_q8(g, u, with_xs=True)
    assert np.array_equal(xs, want * f32(32))
    w = np.tile(x, E // x.size)
    ones = np.ones(E, np.float32)
    wx = np.tile(want, E // x.size)
    assert np.array_equal(oracle.rmsnorm_q8(ones, w, E, 1, 0.0, with_xs=True)[3], wx)
    assert np.array_equal(oracle.sum_norm_rows(ones, np.zeros(E, np.float32), w, E, 1, 0.0)[4], wx)
    assert np.array_equal(oracle.add_norm_rows(ones, np.zeros(E, np.float32), None, w, E, 1, 0.0)[4], wx)
    o = np.ones(128, np.float32)
    wg = np.sign(np.tile(x, 2)).astype(np.float32)
    zg = np.abs(np.tile(x, 2)) * f32(32)
    _, _, xsg = oracle.gated_rmsnorm_q8(o, wg, zg, 1, 0.0, with_xs=True)
    assert np.array_equal(xsg, np.tile(want, 2) * f32(32))
