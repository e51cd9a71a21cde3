"""GPU side of the summation-tree pins: the HIP kernels, through the C ABI, on the inputs of tests/treepins.py whose
sums depend on the order of the float32 additions, checked against the sums derived by hand.

The kernels do not use the reference's thread layout (a 256-thread workgroup holds a row, each thread four of the
reference's 1024 virtual threads; a gated or L2 head sits in part of a wave), so these tests are what shows that the
lane exchanges reproduce the reference's tree: strided per-thread partials (src/ops.cu:93-99), the xor butterflies
within and across warps (src/ops.cu:34-50), the L2 head's strided lanes (src/ops.cu:441-443), and the q8_1 block
sums (src/common.cuh:83-86). Each kernel runs at a decode size and a prefill size, where the launch shapes differ.
"""
import sys

import numpy as np
import pytest

import treepins as tp

pytestmark = pytest.mark.gpu
E = tp.N_ROW
f32 = np.float32


def say(msg):
    print(f"[gpu-trees] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def T(dev):
    import torch

    class H:
        def up(self, a, dtype=None):
            t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
            return t if dtype is None else t.to(dtype)

        def empty(self, n, dtype=torch.float32):
            return torch.zeros(n, dtype=dtype, device=dev)

        def down(self, t):
            torch.cuda.synchronize()
            return t.cpu().numpy()

    return H()


def assert_same(got, want, what):
    got, want = np.asarray(got, np.float32).ravel(), np.asarray(want, np.float32).ravel()
    bad = np.flatnonzero(got.view(np.int32) != want.view(np.int32))
    assert bad.size == 0, f"{what}: {bad.size} differ, first {bad[0]}: {got[bad[0]]!r} vs {want[bad[0]]!r}"


ROW_CASES = [("warps", tp.row_warps, tp.ROW_WARPS_SUM, tp.ROW_WARPS_SEQ),
             ("cross", tp.row_cross, tp.ROW_CROSS_SUM, tp.ROW_CROSS_SEQ),
             ("korder", tp.row_korder, tp.ROW_KORDER_SUM, tp.ROW_KORDER_REV)]


@pytest.mark.parametrize("name,make,t_good,t_bad", ROW_CASES, ids=[c[0] for c in ROW_CASES])
@pytest.mark.parametrize("rows", [2, 258])
def test_row_norm_tree_on_gpu(q27, T, name, make, t_good, t_bad, rows):
    import torch

    say(f"row engine, pattern {name}, rows={rows}")
    eps = tp.eps_separating(t_good, t_bad, E)
    v = make()
    mult = np.exp2(np.arange(rows) % 5).astype(np.float32)     # row r is the pattern times 2^(r % 5)
    x = (v[None, :] * mult[:, None]).ravel()
    w = np.ones(E, np.float32)
    want = np.concatenate([(tp.row_scale(t_good * float(m) ** 2, E, eps) * (v * m)) * w for m in mult])
    other = np.concatenate([(tp.row_scale(t_bad * float(m) ** 2, E, eps) * (v * m)) * w for m in mult])
    assert not np.array_equal(want, other)
    n = rows * E
    wd, zero = T.up(w), T.empty(n)
    y = T.empty(n)
    q27.ops.rmsnorm(T.up(x), wd, y, E, rows, eps)
    assert_same(T.down(y), want, "rmsnorm")
    for kind in ("rmsnorm_q8", "sum_norm_q8", "sum_norm_rows", "add_norm_rows"):
        h, xq, xd, xs = T.empty(n), T.empty(n, torch.int8), T.empty(n // 32), T.empty(n // 16)
        xd_ = T.up(x)
        if kind == "rmsnorm_q8":
            q27.ops.rmsnorm_q8(xd_, wd, h, xq, xd, E, rows, eps, None, xs)
        elif kind == "sum_norm_q8":
            q27.ops.sum_norm_q8(xd_, zero, E, rows, None, wd, eps, h, xq, xd)
        elif kind == "sum_norm_rows":
            q27.ops.sum_norm_rows(xd_, zero, E, rows, None, wd, eps, h, xq, xd, xs)
        else:
            q27.ops.add_norm_rows(xd_, zero, None, E, rows, wd, eps, h, xq, xd, xs)
        assert_same(T.down(h), want, kind)


def test_row_products_on_gpu(q27, oracle, T):
    """h = (scale * v) * w on integer rows (exact sums of squares), at 4 and 300 rows."""
    import torch

    r = np.random.default_rng(191)
    w = (1 + 0.1 * r.standard_normal(E)).astype(np.float32)
    for rows in (4, 300):
        say(f"row products rows={rows}")
        x = r.integers(-8, 9, rows * E).astype(np.float32)
        t = (x.astype(np.float64).reshape(rows, E) ** 2).sum(1)
        s = np.array([tp.row_scale(ti, E, 1e-6) for ti in t], np.float32)[:, None]
        left = (s * x.reshape(rows, E)) * w
        n = rows * E
        h, xq, xd = T.empty(n), T.empty(n, torch.int8), T.empty(n // 32)
        q27.ops.rmsnorm_q8(T.up(x), T.up(w), h, xq, xd, E, rows, 1e-6)
        assert_same(T.down(h), left, "rmsnorm_q8 h")


@pytest.mark.parametrize("heads", [1, 2048])
def test_gated_head_tree_on_gpu(q27, T, heads):
    import torch

    say(f"gated heads={heads}")
    cases = [(tp.head_warps(128), tp.HEAD_WARPS_SUM[128], tp.HEAD_WARPS_SEQ[128]),
             (tp.gated_cross(), tp.GATED_CROSS_SUM, tp.GATED_CROSS_SEQ)]
    for v, t_good, t_bad in cases:
        eps = tp.eps_separating(t_good, t_bad, 128)
        want1 = ((tp.row_scale(t_good, 128, eps) * v) * f32(1)) * f32(64)
        assert not np.array_equal(want1, ((tp.row_scale(t_bad, 128, eps) * v) * f32(1)) * f32(64))
        o = np.tile(v, heads)
        z = np.full(heads * 128, 64.0, np.float32)
        od, wd, zd = T.up(o), T.up(np.ones(128, np.float32)), T.up(z)
        y = T.empty(heads * 128)
        q27.ops.gated_rmsnorm(od, wd, zd, y, 128, heads, eps)
        assert_same(T.down(y), np.tile(want1, heads), "gated_rmsnorm")
        xq, xd, xs = T.empty(heads * 128, torch.int8), T.empty(heads * 4), T.empty(heads * 8)
        q27.ops.gated_rmsnorm_q8(od, wd, zd, xq, xd, heads, eps, None, xs)
        assert_same(T.down(xs), np.tile(tp.butterfly16(want1), heads), "gated_rmsnorm_q8 xs")


@pytest.mark.parametrize("heads", [1, 2048])
def test_gated_products_on_gpu(q27, T, heads):
    import torch

    say(f"gated products heads={heads}")
    r = np.random.default_rng(192 + heads)
    o = r.integers(-8, 9, heads * 128).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(128)).astype(np.float32)
    z = r.uniform(32, 64, heads * 128).astype(np.float32)
    t = (o.astype(np.float64).reshape(heads, 128) ** 2).sum(1)
    s = np.array([tp.row_scale(ti, 128, 1e-6) for ti in t], np.float32)[:, None]
    left = (((s * o.reshape(heads, 128)) * w) * z.reshape(heads, 128)).ravel()
    xq, xd, xs = T.empty(heads * 128, torch.int8), T.empty(heads * 4), T.empty(heads * 8)
    q27.ops.gated_rmsnorm_q8(T.up(o), T.up(w), T.up(z), xq, xd, heads, 1e-6, None, xs)
    assert_same(T.down(xs), tp.butterfly16(left), "gated_rmsnorm_q8 xs")


L2_CASES = [("lanes", tp.l2_lanes, tp.L2_LANES_SUM, tp.L2_LANES_SEQ),
            ("korder", tp.l2_korder, tp.L2_KORDER_SUM, tp.L2_KORDER_REV)]


def l2_expect(v, t, eps):
    return (v * tp.l2_scale(t, 128, eps)) * (f32(1) / np.sqrt(f32(128)))


@pytest.mark.parametrize("name,make,t_good,t_bad", L2_CASES, ids=[c[0] for c in L2_CASES])
def test_l2_tree_on_gpu(q27, T, name, make, t_good, t_bad):
    say(f"l2norm_heads pattern {name}")
    eps = tp.eps_separating(t_good, t_bad, 128, tp.l2_scale)
    v = make()
    want = l2_expect(v, t_good, eps)
    assert not np.array_equal(want, l2_expect(v, t_bad, eps))
    rows = 4099
    x = np.tile(np.concatenate([v, v * f32(0.5), v]), rows)
    xd = T.up(x)
    q27.ops.l2norm_heads(xd, 128, 2, rows, 384, eps)
    got = T.down(xd).reshape(rows, 3, 128)
    assert_same(got[:, 0], np.tile(want, rows), "head 0")
    assert_same(got[:, 1], np.tile(l2_expect(v * f32(0.5), t_good * 0.25, eps), rows), "head 1")
    assert_same(got[:, 2], np.tile(v, rows), "head 2 (untouched)")


@pytest.mark.parametrize("name,make,t_good,t_bad", L2_CASES, ids=[c[0] for c in L2_CASES])
@pytest.mark.parametrize("kind,M", [("conv_l2", 3), ("conv_prefill", 3), ("conv_prefill", 2048)])
def test_conv_l2_tree_on_gpu(q27, T, name, make, t_good, t_bad, kind, M):
    """Conv weights (0, 0, 0, 1) and a zero state pass the input through; 32 and 2^17 pass SiLU unchanged."""
    import torch

    say(f"{kind} pattern {name} M={M}")
    m = 32.0
    eps = tp.eps_separating(t_good, t_bad, 128, tp.l2_scale, m2=m * m)
    v = make(m)
    KH, H = 32, 48          # the model's conv layout: 2 x 16 normed key heads, then 48 value heads
    C = (KH + H) * 128
    x = np.concatenate([np.tile(v, KH), np.full(H * 128, m, np.float32)])
    x = np.tile(x, M)
    w = np.tile(np.array([0, 0, 0, 1], np.float32), C)
    planes = T.up(np.zeros(4 * C * 3, np.float32))
    in_plane = T.up(np.zeros(1, np.int32))
    y, g, beta = T.empty(M * C), T.empty(M * H), T.empty(M * H)
    a = T.up(np.zeros(M * H, np.float32))
    one = T.up(np.ones(H, np.float32))
    if kind == "conv_l2":
        q27.ops.gdn_conv_l2(T.up(x), T.up(w), planes, in_plane, y, C, M, False, KH, eps, a, a, one, one, g, beta, H)
    else:
        q27.ops.gdn_conv_prefill(T.up(x), T.up(w), planes, in_plane, y, C, M, KH, eps, a, a, one, one, g, beta, H)
    want = l2_expect(v, t_good * m * m, eps)
    assert not np.array_equal(want, l2_expect(v, t_bad * m * m, eps))
    got = T.down(y).reshape(M, C)
    assert_same(got[:, :KH * 128], np.tile(want, M * KH), "normed heads")
    assert_same(got[:, KH * 128:], np.full(M * H * 128, m, np.float32), "value heads")


@pytest.mark.parametrize("ntok", [1, 4, 64])
def test_attn_head_tree_on_gpu(q27, T, ntok):
    """attn_prep with every token at rotary position 0 (rope3 of zeros): qn = (scale * v) * w for every dim, and
    the f16 K cache rows hold it rounded."""
    import torch

    say(f"attn_prep tree ntok={ntok}")
    n = 256
    t_good, t_bad = tp.HEAD_WARPS_SUM[n], tp.HEAD_WARPS_SEQ[n]
    eps = tp.eps_separating(t_good, t_bad, n)
    v = tp.head_warps(n)
    nqh, nkvh, n_ctx = 24, 4, 128
    qg = np.zeros((ntok, nqh, 512), np.float32)
    qg[:, :, :256] = v
    k = np.tile(v, ntok * nkvh)
    w = T.up(np.ones(256, np.float32))
    nb = q27.ops.kv_cache_bytes(nkvh, n_ctx, False)
    kc, vc = T.empty(nb, torch.uint8), T.empty(nb, torch.uint8)
    qn = T.empty(ntok * nqh * 256)
    pos0 = T.up(np.array([5], np.int32))
    rope3 = T.up(np.zeros(ntok * 3, np.int32))
    q27.ops.attn_prep(T.up(qg.ravel()), T.up(k), T.up(k), w, w, qn, kc, vc, pos0, ntok, eps, float(tp.f32(0.6)), nqh,
                      nkvh, n_ctx, False, rope3=rope3)
    want = (tp.row_scale(t_good, n, eps) * v) * f32(1)
    assert not np.array_equal(want, (tp.row_scale(t_bad, n, eps) * v) * f32(1))
    assert_same(T.down(qn), np.tile(want, ntok * nqh), "qn")
    kcache = T.down(kc).view(np.float16).reshape(nkvh, n_ctx, 256)
    assert np.array_equal(kcache[:, 5:5 + ntok].reshape(-1), np.tile(want.astype(np.float16), nkvh * ntok))


@pytest.mark.parametrize("ncols", [1, 2048])
def test_xs_butterfly_on_gpu(q27, T, ncols):
    """xs of quantize_q8_1, swiglu_q8, rmsnorm_q8 / sum_norm_rows / add_norm_rows (v = 1, eps = 0: scale 1, y = w)
    and gated_rmsnorm_q8 (ones, eps = 0: y = w * silu(z)) on the hand-derived blocks."""
    import torch

    say(f"xs butterfly ncols={ncols}")
    x, want = tp.xs_blocks()
    K = E
    xx = np.tile(x, K // x.size * ncols)
    wx = np.tile(want, K // x.size * ncols)
    n = xx.size
    xq, xd, xs = T.empty(n, torch.int8), T.empty(n // 32), T.empty(n // 16)
    q27.ops.quantize_q8_1(T.up(xx), xq, xd, K, ncols, None, xs)
    assert_same(T.down(xs), wx, "quantize_q8_1")
    q27.ops.swiglu_q8(T.up(np.abs(xx) * f32(32)), T.up(np.sign(xx).astype(np.float32)), xq, xd, n, None, xs)
    assert_same(T.down(xs), wx * f32(32), "swiglu_q8")
    rows = ncols
    ones, zero, wd = T.up(np.ones(n, np.float32)), T.empty(n), T.up(np.tile(x, E // x.size))
    h = T.empty(n)
    q27.ops.rmsnorm_q8(ones, wd, None, xq, xd, E, rows, 0.0, None, xs)
    assert_same(T.down(xs), wx, "rmsnorm_q8")
    q27.ops.sum_norm_rows(T.up(np.ones(n, np.float32)), zero, E, rows, None, wd, 0.0, h, xq, xd, xs)
    assert_same(T.down(xs), wx, "sum_norm_rows")
    q27.ops.add_norm_rows(T.up(np.ones(n, np.float32)), zero, None, E, rows, wd, 0.0, None, xq, xd, xs)
    assert_same(T.down(xs), wx, "add_norm_rows")
    heads = n // 128
    q27.ops.gated_rmsnorm_q8(ones, T.up(np.sign(np.tile(x, 2)).astype(np.float32)),
                             T.up(np.abs(xx) * f32(32)), xq, xd, heads, 0.0, None, xs)
    assert_same(T.down(xs), wx * f32(32), "gated_rmsnorm_q8")
