"""GPU parity: every HIP entry point (through the C ABI) against the CPU oracle on the same seeded inputs.

The bar is bit-exact for every output: int8 values, fp16-rounded scales, block sums, gathered rows, the KV
cache, and also the float outputs (h, y, qn, x), which north_star would accept within 1e-5 relative (fp32)
and 2^-8 (bf16) -- the kernels reproduce the oracle's operation order, so anything but equality is a bug.
Shapes are the BASELINE.json configurations at full size (cfg1-cfg5) plus edge cases.
"""
import sys

import numpy as np
import pytest

import cfgdata as cd
from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu

E, FF, EPS = cd.E, cd.FF, cd.EPS


def say(msg):
    print(f"[gpu-parity] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def T(dev):
    import torch

    class H:
        def up(self, a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

        def empty(self, n, dtype=torch.float32):
            return torch.zeros(n, dtype=dtype, device=dev)

        def down(self, t):
            torch.cuda.synchronize()
            return t.cpu().numpy()

        def i32(self, a):
            return self.up(np.asarray(a, np.int32))

    H.torch = torch
    return H()


def q8_bufs(T, n, with_xs):
    import torch

    return T.empty(n, torch.int8), T.empty(n // 32), (T.empty(n // 16) if with_xs else None)


# ---------------------------------------------------------------- row kernels
@pytest.mark.parametrize("with_h,with_xs", [(True, True), (True, False), (False, True)])
def test_rmsnorm_q8_cfg1(q27, oracle, T, with_h, with_xs):
    say(f"rmsnorm_q8 cfg1 h={with_h} xs={with_xs}")
    x, w = cd.cfg1()
    h = T.empty(E) if with_h else None
    xq, xd, xs = q8_bufs(T, E, with_xs)
    q27.ops.rmsnorm_q8(T.up(x), T.up(w), h, xq, xd, E, 1, EPS, None, xs)
    oh, oq, od, os_ = oracle.rmsnorm_q8(x, w, E, 1, EPS, with_h=with_h, with_xs=with_xs)
    assert_bits_equal(T.down(xq), oq, "xq")
    assert_bits_equal(T.down(xd), od, "xd")
    if with_h:
        assert_bits_equal(T.down(h), oh, "h")
    if with_xs:
        assert_bits_equal(T.down(xs), os_, "xs")


@pytest.mark.parametrize("rows,seed", [(4, 2), (2048, 3), (7, 4)])
def test_rmsnorm_q8_rows(q27, oracle, T, rows, seed):
    say(f"rmsnorm_q8 rows={rows}")
    r = cd.rng(seed)
    x = cd.prefill_rows(r, rows)
    w = cd.normal(r, E, 0.1, 1.0)
    h = T.empty(rows * E)
    xq, xd, xs = q8_bufs(T, rows * E, True)
    q27.ops.rmsnorm_q8(T.up(x), T.up(w), h, xq, xd, E, rows, EPS, None, xs)
    oh, oq, od, os_ = oracle.rmsnorm_q8(x, w, E, rows, EPS, with_h=True, with_xs=True)
    for got, want, what in ((h, oh, "h"), (xq, oq, "xq"), (xd, od, "xd"), (xs, os_, "xs")):
        assert_bits_equal(T.down(got), want, what)


@pytest.mark.parametrize("rows", [4, 2048])
def test_sum_norm_q8_and_rows(q27, oracle, T, rows):
    say(f"sum_norm_q8 / sum_norm_rows / add_norm_rows rows={rows}")
    r = cd.rng(10 + rows)
    x0 = cd.prefill_rows(r, rows)
    part = cd.normal(r, rows * E)
    w = cd.normal(r, E, 0.1, 1.0)
    # decode form (h, no xs)
    x = T.up(x0)
    h = T.empty(rows * E)
    xq, xd, _ = q8_bufs(T, rows * E, False)
    q27.ops.sum_norm_q8(x, T.up(part), E, rows, None, T.up(w), EPS, h, xq, xd)
    ox, oh, oq, od = oracle.sum_norm_q8(x0, part, w, E, rows, EPS)
    for got, want, what in ((x, ox, "x"), (h, oh, "h"), (xq, oq, "xq"), (xd, od, "xd")):
        assert_bits_equal(T.down(got), want, what)
    # prefill form (xs, h null)
    x = T.up(x0)
    xq, xd, xs = q8_bufs(T, rows * E, True)
    q27.ops.sum_norm_rows(x, T.up(part), E, rows, None, T.up(w), EPS, None, xq, xd, xs)
    ox, _, oq, od, os_ = oracle.sum_norm_rows(x0, part, w, E, rows, EPS)
    for got, want, what in ((x, ox, "x"), (xq, oq, "xq"), (xd, od, "xd"), (xs, os_, "xs")):
        assert_bits_equal(T.down(got), want, what)
    # add_norm_rows with a bf16 partner partial
    recv = (cd.to_bf16_values(cd.normal(r, rows * E)).view(np.uint32) >> 16).astype(np.uint16)
    x = T.up(x0)
    h = T.empty(rows * E)
    xq, xd, xs = q8_bufs(T, rows * E, True)
    q27.ops.add_norm_rows(x, T.up(part), T.up(recv.view(np.int16)), E, rows, T.up(w), EPS, h, xq, xd, xs)
    ox, oh, oq, od, os_ = oracle.add_norm_rows(x0, part, recv, w, E, rows, EPS, with_h=True)
    for got, want, what in ((x, ox, "x"), (h, oh, "h"), (xq, oq, "xq"), (xd, od, "xd"), (xs, os_, "xs")):
        assert_bits_equal(T.down(got), want, what)


@pytest.mark.parametrize("ncols,K", [(2048, 6144), (4, 2 * E), (3, 96)])
def test_quantize_q8_1(q27, oracle, T, ncols, K):
    say(f"quantize_q8_1 {ncols}x{K}")
    r = cd.rng(20 + ncols)
    x = cd.normal(r, ncols * K, 3.0)
    x[::1001] = 0
    x[:32] = 0  # an all-zero block
    xq, xd, xs = q8_bufs(T, ncols * K, True)
    q27.ops.quantize_q8_1(T.up(x), xq, xd, K, ncols, None, xs)
    oq, od, os_ = oracle.quantize_q8_1(x, K, ncols, with_xs=True)
    for got, want, what in ((xq, oq, "xq"), (xd, od, "xd"), (xs, os_, "xs")):
        assert_bits_equal(T.down(got), want, what)


# Launches of up to 64 rows of 5120 values take the branch-free exact quotient, larger ones the reciprocal fast path
# with its IEEE fallback: reps = 1 runs the first, reps = 3 (the same blocks three times over) the second.
LAT_LIMIT = 64 * E


@pytest.mark.parametrize("reps", [1, 3])
def test_q8_rounding_near_half_integers(q27, oracle, T, reps):
    """Values whose quotient y / d lies on or within a few ulps of k + 0.5: both quotient paths must round them as the
    IEEE quotient does (roundf, ties away from zero), exactly as the oracle rounds them."""
    say(f"q8_1 rounding near half-integers reps={reps}")
    r = cd.rng(123)
    nblk = 4096
    amax = np.exp(r.uniform(-8, 8, nblk)).astype(np.float32)
    d = amax / np.float32(127)
    k = r.integers(-126, 126, (nblk, 31)).astype(np.float32)
    y = ((k + np.float32(0.5)) * d[:, None]).astype(np.float32)
    ulps = r.integers(-3, 4, (nblk, 31)).astype(np.int32)
    y = (y.view(np.int32) + ulps).view(np.float32)  # on the tie and a few ulps either side
    x = np.tile(np.concatenate([amax[:, None], y], 1).reshape(-1), reps)  # lane 0 of each block fixes amax (and so d)
    assert (x.size <= LAT_LIMIT) == (reps == 1)
    xq, xd, xs = q8_bufs(T, x.size, True)
    q27.ops.quantize_q8_1(T.up(x), xq, xd, x.size, 1, None, xs)
    oq, od, os_ = oracle.quantize_q8_1(x, x.size, 1, with_xs=True)
    for got, want, what in ((xq, oq, "xq"), (xd, od, "xd"), (xs, os_, "xs")):
        assert_bits_equal(T.down(got), want, what)


@pytest.mark.parametrize("reps", [1, 3])
def test_q8_rounding_beside_the_guard_band(q27, oracle, T, reps):
    """Quotients 4 to 64 ulps from k + 0.5 (2^-15 .. 2^-11 for |q| in [64, 128)): on both sides of the reciprocal
    path's guard band around half-integers, so values that the fast path rounds by itself are checked next to those it
    hands to the IEEE quotient."""
    say(f"q8_1 rounding beside the guard band reps={reps}")
    r = cd.rng(124)
    nblk = 4096
    amax = np.exp(r.uniform(-8, 8, nblk)).astype(np.float32)
    d = amax / np.float32(127)
    k = r.integers(-126, 126, (nblk, 31)).astype(np.float32)
    y = ((k + np.float32(0.5)) * d[:, None]).astype(np.float32)
    ulps = r.integers(4, 65, (nblk, 31)).astype(np.int32) * np.where(r.random((nblk, 31)) < 0.5, -1, 1).astype(np.int32)
    y = (y.view(np.int32) + ulps).view(np.float32)
    x = np.tile(np.concatenate([amax[:, None], y], 1).reshape(-1), reps)
    assert (x.size <= LAT_LIMIT) == (reps == 1)
    xq, xd, xs = q8_bufs(T, x.size, True)
    q27.ops.quantize_q8_1(T.up(x), xq, xd, x.size, 1, None, xs)
    oq, od, os_ = oracle.quantize_q8_1(x, x.size, 1, with_xs=True)
    for got, want, what in ((xq, oq, "xq"), (xd, od, "xd"), (xs, os_, "xs")):
        assert_bits_equal(T.down(got), want, what)


@pytest.mark.parametrize("reps", [1, 6])
def test_q8_tiny_and_huge_scales(q27, oracle, T, reps):
    """Blocks whose scale d = amax / 127 is subnormal or tiny (the reciprocal path hands them to the IEEE quotient) or
    very large, subnormal inputs, and all-zero blocks, through both quotient paths."""
    say(f"q8_1 tiny and huge scales reps={reps}")
    r = cd.rng(321)
    nblk = 2048
    e = np.concatenate([r.uniform(-149, -100, nblk // 2), r.uniform(100, 127, nblk // 2)])
    amax = np.exp2(e).astype(np.float32)
    y = (r.uniform(-1, 1, (nblk, 31)) * amax[:, None]).astype(np.float32)
    x = np.concatenate([amax[:, None], y], 1)
    x[::7] = 0  # all-zero blocks
    x = np.tile(x.reshape(-1), reps)
    assert (x.size <= LAT_LIMIT) == (reps == 1)
    xq, xd, xs = q8_bufs(T, x.size, True)
    q27.ops.quantize_q8_1(T.up(x), xq, xd, x.size, 1, None, xs)
    oq, od, os_ = oracle.quantize_q8_1(x, x.size, 1, with_xs=True)
    for got, want, what in ((xq, oq, "xq"), (xd, od, "xd"), (xs, os_, "xs")):
        assert_bits_equal(T.down(got), want, what)


@pytest.mark.parametrize("n,with_xs", [(4 * FF, False), (2048 * FF, True), (96, True)])
def test_swiglu_q8(q27, oracle, T, n, with_xs):
    say(f"swiglu_q8 n={n}")
    r = cd.rng(30 + n % 97)
    g = cd.normal(r, n, 2.0)
    u = cd.normal(r, n, 2.0)
    g[:64] = 0
    g[64:96] = np.linspace(-120, 120, 32)
    xq, xd, xs = q8_bufs(T, n, with_xs)
    q27.ops.swiglu_q8(T.up(g), T.up(u), xq, xd, n, None, xs)
    oq, od, os_ = oracle.swiglu_q8(g, u, with_xs=with_xs)
    assert_bits_equal(T.down(xq), oq, "xq")
    assert_bits_equal(T.down(xd), od, "xd")
    if with_xs:
        assert_bits_equal(T.down(xs), os_, "xs")


@pytest.mark.parametrize("heads", [4 * 48, 2048 * 48, 4099 * 48, 5])
def test_gated_rmsnorm_q8(q27, oracle, T, heads):
    say(f"gated_rmsnorm_q8 heads={heads}")
    r = cd.rng(40 + heads % 101)
    o = cd.normal(r, heads * 128)
    z = cd.normal(r, heads * 128)
    z[7::997] = 0  # silu arguments outside the fast range: the wave's values are recomputed with the general silu
    z[11::1999] = 75.0
    z[13::2999] = -80.0
    w = cd.normal(r, 128, 0.1, 1.0)
    xq, xd, xs = q8_bufs(T, heads * 128, True)
    q27.ops.gated_rmsnorm_q8(T.up(o), T.up(w), T.up(z), xq, xd, heads, EPS, None, xs)
    oq, od, os_ = oracle.gated_rmsnorm_q8(o, w, z, heads, EPS, with_xs=True)
    for got, want, what in ((xq, oq, "xq"), (xd, od, "xd"), (xs, os_, "xs")):
        assert_bits_equal(T.down(got), want, what)


# ---------------------------------------------------------------- silu over a sweep of float32 bit patterns
def test_silu_bit_pattern_sweep(q27, oracle, T):
    """silu(g) * 1 through the unfused swiglu: every 61st float32 bit pattern (about 70 million values: both
    signs, subnormals, zeros, infinities), plus the neighbours of the fast range's edges 2^-60 and 60 and of 2^-23 (the
    one argument whose quotient depends on the hardware reciprocal of 2 - 2^-23 being correctly rounded). The
    kernels compute silu with a division without range scaling for 2^-60 <= |x| <= 60 and the general one elsewhere; both
    must give the oracle's bits. NaN inputs and outputs only have to be NaN (payloads are not specified)."""
    say("silu bit-pattern sweep")
    pats = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
    edges = []
    for e in (np.float32(2.0 ** -60), np.float32(60.0), np.float32(2.0 ** -23)):
        b = int(np.array(e).view(np.uint32))
        edges += list(range(b - 64, b + 65))
    edges = np.array(edges, np.uint32)
    pats = np.concatenate([pats, edges, edges | np.uint32(0x80000000)])
    g = pats.view(np.float32)
    u = np.ones_like(g)
    y = T.empty(g.size)
    q27.ops.swiglu(T.up(g), T.up(u), y, g.size)
    got = T.down(y)
    want = oracle.swiglu(g, u)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), "silu: NaN positions differ"
    assert_bits_equal(got[~nan], want[~nan], "silu sweep")


# ---------------------------------------------------------------- unfused twins and the fused == unfused identity
def test_unfused_twins(q27, oracle, T):
    say("unfused rmsnorm / add / swiglu / gated_rmsnorm / gdn_gates / gdn_conv")
    r = cd.rng(50)
    rows = 4
    x = cd.normal(r, rows * E, 3.0)
    a = cd.normal(r, rows * E)
    w = cd.normal(r, E, 0.5)
    y = T.empty(rows * E)
    q27.ops.rmsnorm(T.up(x), T.up(w), y, E, rows, EPS)
    assert_bits_equal(T.down(y), oracle.rmsnorm(x, w, E, rows, EPS), "rmsnorm")
    q27.ops.rmsnorm(T.up(x[:4 * 640]), T.up(w[:640]), y, 640, 4, EPS)  # the 256-thread form (n < 1024)
    assert_bits_equal(T.down(y)[:4 * 640], oracle.rmsnorm(x[:4 * 640], w[:640], 640, 4, EPS), "rmsnorm n=640")
    q27.ops.add(T.up(x), T.up(a), y, rows * E)
    assert_bits_equal(T.down(y), x + a, "add")
    q27.ops.swiglu(T.up(x), T.up(a), y, rows * E)
    assert_bits_equal(T.down(y), oracle.swiglu(x, a), "swiglu")
    heads = 4 * 48
    o, z = cd.normal(r, heads * 128), cd.normal(r, heads * 128)
    w128 = cd.normal(r, 128, 0.1, 1.0)
    yg = T.empty(heads * 128)
    q27.ops.gated_rmsnorm(T.up(o), T.up(w128), T.up(z), yg, 128, heads, EPS)
    assert_bits_equal(T.down(yg), oracle.gated_rmsnorm(o, w128, z, 128, heads, EPS), "gated_rmsnorm")


def test_fused_equals_unfused_on_gpu(q27, T):
    """tools/test_fused.cu, on the GPU: fused kernels against the unfused chains, bit for bit."""
    import torch

    say("fused == unfused (test_fused)")
    r = cd.rng(7)
    Tn = 4
    x0, part, w = cd.normal(r, Tn * E, 3.0), cd.normal(r, Tn * E), cd.normal(r, E, 0.5)
    xa, xb = T.up(x0), T.up(x0)
    ha, hb = T.empty(Tn * E), T.empty(Tn * E)
    qa, da, _ = q8_bufs(T, Tn * E, False)
    qb, db, _ = q8_bufs(T, Tn * E, False)
    q27.ops.sum_norm_q8(xa, T.up(part), E, Tn, None, T.up(w), EPS, ha, qa, da)
    q27.ops.add(xb, T.up(part), xb, Tn * E)
    q27.ops.rmsnorm(xb, T.up(w), hb, E, Tn, EPS)
    q27.ops.quantize_q8_1(hb, qb, db, E, Tn)
    for a_, b_, what in ((xa, xb, "x"), (ha, hb, "h"), (qa, qb, "xq"), (da, db, "xd")):
        assert_bits_equal(T.down(a_), T.down(b_), what)
    KH, H = 8, 24
    C = 2 * KH * 128 + H * 128
    qkv, cw, st0 = cd.normal(r, Tn * C), cd.normal(r, C * 4, 0.5), cd.normal(r, 4 * C * 3)
    ab, sa, dtb = cd.normal(r, 2 * Tn * H, 2.0), cd.normal(r, H), cd.normal(r, H)
    sta, stb = T.up(st0), T.up(st0)
    ya, yb = T.empty(Tn * C), T.empty(Tn * C)
    ga, gb, ba, bb = (T.empty(Tn * H) for _ in range(4))
    plane = T.i32([0])
    abd = T.up(ab)
    q27.ops.gdn_conv_l2(T.up(qkv), T.up(cw), sta, plane, ya, C, Tn, True, 2 * KH, EPS, abd, abd[Tn * H:], T.up(sa),
                        T.up(dtb), ga, ba, H)
    q27.ops.gdn_gates(abd, abd[Tn * H:], T.up(sa), T.up(dtb), gb, bb, H, Tn)
    q27.ops.gdn_conv(T.up(qkv), T.up(cw), stb, plane, yb, C, Tn, True)
    q27.ops.l2norm_heads(yb, 128, 2 * KH, Tn, C, EPS)
    torch.cuda.synchronize()
    for a_, b_, what in ((ya, yb, "y"), (sta, stb, "state"), (ga, gb, "g"), (ba, bb, "beta")):
        assert_bits_equal(T.down(a_), T.down(b_), what)


# ---------------------------------------------------------------- Gated-DeltaNet input stage
@pytest.mark.parametrize("Tn,pin,snap", [(4, 0, True), (4, 3, False), (1, 2, True), (3, 1, True)])
def test_gdn_conv_l2_decode(q27, oracle, T, Tn, pin, snap):
    say(f"gdn_conv_l2 T={Tn} in_plane={pin} snapshots={snap}")
    r = cd.rng(60 + Tn + 10 * pin)
    C, H, KH = cd.C_CONV, cd.HV, cd.KH
    x, cw, st0 = cd.normal(r, Tn * C), cd.normal(r, C * 4, 0.5), cd.normal(r, 4 * C * 3)
    a, b, sa, dtb = cd.normal(r, Tn * H, 2.0), cd.normal(r, Tn * H, 2.0), cd.normal(r, H), cd.normal(r, H)
    st, y, g, beta = T.up(st0), T.empty(Tn * C), T.empty(Tn * H), T.empty(Tn * H)
    q27.ops.gdn_conv_l2(T.up(x), T.up(cw), st, T.i32([pin]), y, C, Tn, snap, 2 * KH, EPS, T.up(a), T.up(b), T.up(sa),
                        T.up(dtb), g, beta, H)
    oy, ost, og, ob = oracle.gdn_conv_l2(x, cw, st0, pin, C, Tn, snap, 2 * KH, EPS, a, b, sa, dtb, H)
    for got, want, what in ((y, oy, "y"), (st, ost, "planes"), (g, og, "g"), (beta, ob, "beta")):
        assert_bits_equal(T.down(got), want, what)


def conv_prefill_run(q27, T, M, pin, seed, exact, xscale=1.0):
    r = cd.rng(seed)
    C, H, KH = cd.C_CONV, cd.HV, cd.KH
    x, cw, st0 = cd.normal(r, M * C, xscale), cd.normal(r, C * 4, 0.5), cd.normal(r, 4 * C * 3, xscale)
    a, b, sa, dtb = cd.normal(r, M * H, 2.0), cd.normal(r, M * H, 2.0), cd.normal(r, H), cd.normal(r, H)
    st, y, g, beta = T.up(st0), T.empty(M * C), T.empty(M * H), T.empty(M * H)
    prev = q27.ops.gdn_prefill_exact(exact)
    try:
        q27.ops.gdn_conv_prefill(T.up(x), T.up(cw), st, T.i32([pin]), y, C, M, 2 * KH, EPS, T.up(a), T.up(b), T.up(sa),
                                 T.up(dtb), g, beta, H)
    finally:
        q27.ops.gdn_prefill_exact(prev)
    return (x, cw, st0, a, b, sa, dtb), (T.down(y), T.down(st), T.down(g), T.down(beta))


@pytest.mark.parametrize("M,pin", [(2048, 0), (4099, 1), (1, 0), (2, 1), (3, 0), (17, 1), (33, 0), (70, 1), (129, 0)])
def test_gdn_conv_prefill(q27, oracle, T, M, pin):
    """Exact mode (q27h_gdn_prefill_exact(1)): every output bit for bit."""
    say(f"gdn_conv_prefill exact M={M} in_plane={pin}")
    C, H, KH = cd.C_CONV, cd.HV, cd.KH
    (x, cw, st0, a, b, sa, dtb), got = conv_prefill_run(q27, T, M, pin, 70 + M, True)
    want = oracle.gdn_conv_prefill(x, cw, st0, pin, C, M, 2 * KH, EPS, a, b, sa, dtb, H)
    for g_, w_, what in zip(got, want, ("y", "planes", "g", "beta")):
        assert_bits_equal(g_, w_, what)


SILU_RTOL = 1e-5   # the north_star's fp32 bar, per value
SILU_TINY = 1e-30  # |y| below this: silu of arguments under about -71 (e^-x near the float32 range end)


@pytest.mark.parametrize("M,pin,xscale", [(2048, 0, 1.0), (4099, 1, 1.0), (3, 0, 1.0), (129, 1, 1.0), (2048, 1, 40.0)])
def test_gdn_conv_prefill_default_tolerance(q27, oracle, T, M, pin, xscale):
    """Default mode: y within 1e-5 relative of the checker's value, per value (the v heads, which leave the conv
    unnormed, and the normed q / k heads); planes, g and beta bit for bit. xscale 40 reaches SiLU arguments past
    +-100 (overflowing e^-x on the negative side)."""
    say(f"gdn_conv_prefill default M={M} in_plane={pin} xscale={xscale}")
    C, H, KH = cd.C_CONV, cd.HV, cd.KH
    (x, cw, st0, a, b, sa, dtb), got = conv_prefill_run(q27, T, M, pin, 170 + M, False, xscale)
    oy, ost, og, ob = oracle.gdn_conv_prefill(x, cw, st0, pin, C, M, 2 * KH, EPS, a, b, sa, dtb, H)
    y = got[0].astype(np.float64)
    w = oy.astype(np.float64)
    err = np.abs(y - w)
    big = np.abs(w) >= SILU_TINY
    rel = (err[big] / np.abs(w[big])).max()
    say(f"  max relative error {rel:.2e}; values differing from the checker's bits: "
        f"{np.count_nonzero(got[0].view(np.uint32) != oy.view(np.uint32))} of {oy.size}")
    assert rel <= SILU_RTOL
    # values under the floor stay under it, up to the relative tolerance at its edge
    off = np.flatnonzero(~big & (np.abs(y) > SILU_TINY * (1 + SILU_RTOL)))
    assert off.size == 0, f"tiny values: {off.size}, first (index, got, want): " + str(
        [(int(i), float(y[i]), float(w[i])) for i in off[:5]])
    for g_, w_, what in zip(got[1:], (ost, og, ob), ("planes", "g", "beta")):
        assert_bits_equal(g_, w_, what)


@pytest.mark.parametrize("rows,n,heads,stride", [(4099, 128, 32, cd.C_CONV), (4, 128, 32, cd.C_CONV), (3, 64, 5, 400)])
def test_l2norm_heads(q27, oracle, T, rows, n, heads, stride):
    say(f"l2norm_heads rows={rows} n={n}")
    r = cd.rng(80 + rows)
    x = cd.normal(r, rows * stride)
    xd = T.up(x)
    q27.ops.l2norm_heads(xd, n, heads, rows, stride, EPS)
    assert_bits_equal(T.down(xd), oracle.l2norm_heads(x, n, heads, rows, stride, EPS), "x")


# ---------------------------------------------------------------- attention input stage
def run_attn_pair(q27, oracle, T, Tn, pos0, n_ctx, q8, seed, rope3=None, rdelta=None):
    import torch

    r = cd.rng(seed)
    qg, k, v = cd.normal(r, Tn * cd.NQH * 512), cd.normal(r, Tn * cd.NKVH * 256), cd.normal(r, Tn * cd.NKVH * 256)
    qw, kw = cd.normal(r, 256, 0.1, 1.0), cd.normal(r, 256, 0.1, 1.0)
    nb = q27.ops.kv_cache_bytes(cd.NKVH, n_ctx, q8)
    assert nb == oracle.kv_cache_bytes(cd.NKVH, n_ctx, q8)
    kc, vc = T.empty(nb, torch.uint8), T.empty(nb, torch.uint8)
    qn = T.empty(Tn * cd.NQH * 256)
    q27.ops.attn_prep(T.up(qg), T.up(k), T.up(v), T.up(qw), T.up(kw), qn, kc, vc, T.i32([pos0]), Tn, EPS, cd.THETA_SCALE,
                      cd.NQH, cd.NKVH, n_ctx, q8, None, None, 0, None if rope3 is None else T.i32(rope3),
                      None if rdelta is None else T.i32([rdelta]))
    okc, ovc = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
    oqn = oracle.attn_prep(qg, k, v, qw, kw, okc, ovc, pos0, Tn, EPS, cd.THETA_SCALE, cd.NQH, cd.NKVH, n_ctx, q8, rope3, rdelta)
    assert_bits_equal(T.down(qn), oqn, "qn")
    assert_bits_equal(T.down(kc), okc, "kcache")
    assert_bits_equal(T.down(vc), ovc, "vcache")


@pytest.mark.parametrize("Tn,pos0,q8,rdelta", [(4, 150000, True, None), (4, 150000, False, None), (2048, 0, True, None),
                                               (2048, 131072, True, 5), (1, cd.N_CTX - 1, True, None)])
def test_attn_prep(q27, oracle, T, Tn, pos0, q8, rdelta):
    say(f"attn_prep T={Tn} pos0={pos0} q8={q8} rdelta={rdelta}")
    run_attn_pair(q27, oracle, T, Tn, pos0, cd.N_CTX, q8, 90 + Tn, rdelta=rdelta)


@pytest.mark.parametrize("Tn,pos0,q8,rdelta", [(74, 0, False, None), (75, 180224 - 40, True, None), (2048, 7, False, None),
                                               (513, 100000, True, 9)])
def test_attn_prep_token_workgroups(q27, oracle, T, Tn, pos0, q8, rdelta):
    # launches of T * 28 >= 2048 heads take one workgroup per token (angles shared through LDS): f16 and q8_0 caches,
    # rows past n_ctx, an rdelta shift and odd token counts
    say(f"attn_prep (workgroup per token) T={Tn} pos0={pos0} q8={q8} rdelta={rdelta}")
    run_attn_pair(q27, oracle, T, Tn, pos0, cd.N_CTX, q8, 700 + Tn, rdelta=rdelta)


def test_attn_prep_imrope_cfg5(q27, oracle, T):
    say("attn_prep cfg5 IMRoPE 4099 rows")
    rope3 = cd.rope3_grid()
    run_attn_pair(q27, oracle, T, 4099, 0, 8192, True, 95, rope3=rope3)


def test_attn_prep_rows_outside_cache_untouched(q27, oracle, T):
    say("attn_prep rows past n_ctx")
    run_attn_pair(q27, oracle, T, 4, 14, 16, True, 96)  # rows 16, 17 do not exist and are skipped


# ---------------------------------------------------------------- embedding gather
FMT_FN = {"iq2_s": "get_rows_iq2_s", "q4_k": "get_rows_q4_k", "q6_k": "get_rows_q6_k", "q8_0": "get_rows_q8_0"}


@pytest.mark.parametrize("kind", ["q4_k", "q6_k", "q8_0", "iq2_s"])
def test_get_rows_cfg4(q27, oracle, T, kind):
    say(f"get_rows {kind} cfg4")
    r = cd.rng(100 + len(kind))
    bb, bv = cd.BLOCK[kind]
    row_bytes = E // bv * bb
    table = cd.random_table(r, kind, cd.VOCAB, E)
    ids = cd.gather_ids()
    ids_img = ids.copy()
    ids_img[7] = -1
    ids_img[9] = -3
    img = cd.normal(r, 3 * E)
    dt = T.up(table)
    for idv, im in ((ids, None), (ids_img, img)):
        y = T.empty(idv.size * E)
        getattr(q27.ops, FMT_FN[kind])(dt, row_bytes, T.i32(idv), idv.size, y, E, None, None if im is None else T.up(im))
        want = oracle.get_rows(kind, table, row_bytes, idv, E, im)
        assert_bits_equal(T.down(y), want, f"y ({kind})")
    y = T.empty(2 * E)
    getattr(q27.ops, FMT_FN[kind])(dt, row_bytes, T.i32([-1, 5]), 2, y, E)  # no image array: zeros
    got = T.down(y)
    assert np.all(got[:E] == 0)
    assert_bits_equal(got[E:], oracle.get_rows(kind, table, row_bytes, np.array([5], np.int32), E), "row 5")


# ---------------------------------------------------------------- graph capture (decode step)
def test_decode_ops_replay_in_hip_graph(q27, oracle, T):
    """The decode ops recorded in a HIP graph give the eager result on every replay (eager work in between)."""
    import torch

    say("hip graph replay")
    r = cd.rng(111)
    Tn = 4
    x0, part, w = cd.normal(r, Tn * E), cd.normal(r, Tn * E), cd.normal(r, E, 0.1, 1.0)
    g, u = cd.normal(r, Tn * FF, 2.0), cd.normal(r, Tn * FF, 2.0)
    dx, dp, dw, dg, du = (T.up(a) for a in (x0, part, w, g, u))
    h = T.empty(Tn * E)
    xq, xd, _ = q8_bufs(T, Tn * FF, False)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        q27.ops.sum_norm_q8(dx, dp, E, Tn, None, dw, EPS, h, xq, xd)  # warm-up outside capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            q27.ops.sum_norm_q8(dx, dp, E, Tn, None, dw, EPS, h, xq[:Tn * E], xd[:Tn * E // 32])
            q27.ops.swiglu_q8(dg, du, xq, xd, Tn * FF)
    ox, oh, _, _ = oracle.sum_norm_q8(x0, part, w, E, Tn, EPS)
    oq, od, _ = oracle.swiglu_q8(g, u)
    for rep in range(3):
        dx.copy_(T.up(x0))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_bits_equal(T.down(dx), ox, f"x replay {rep}")
        assert_bits_equal(T.down(h), oh, f"h replay {rep}")
        assert_bits_equal(T.down(xq), oq, f"xq replay {rep}")
        assert_bits_equal(T.down(xd), od, f"xd replay {rep}")
        _ = (dg * 2).sum().item()  # eager work between replays
