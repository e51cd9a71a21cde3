"""Independent pins of four oracle semantics that the bit-exact GPU parity rests on (CPU only).

Each check is built so that the plausible alternative reading of the reference line fails it:

- q8_1 rounds the IEEE quotient y / d (src/common.cuh:76), not y * (1/d);
- the q8_0 KV cache rounds x * (1/d) (src/ops.cu:644-646), not x / d;
- IMRoPE takes pair j's position from rope3[t][j % 3] (src/ops.cu:616-619), not from contiguous sections;
- the L2 norm adds eps / n under the root (src/ops.cu:444), not eps.

The expected values come from numpy's correctly rounded float32 arithmetic and float64 closed forms, not from a
second copy of the oracle's code.
"""
import numpy as np

from cfgdata import near_tie_blocks, round_half_away
from conftest import assert_bits_equal

NQH, NKVH = 24, 4
EPS = 1e-6
THETA_SCALE = float(np.float32(1e7) ** np.float32(-2.0 / 64))


def test_q8_1_rounds_the_ieee_quotient(oracle):
    """xq == roundf(float32(y) / float32(d)) on 10^6 random blocks and 2*10^5 near-tie blocks."""
    r = np.random.default_rng(71)
    rand = (r.standard_normal((10 ** 6, 32)) * np.exp2(r.uniform(-30, 30, (10 ** 6, 1)))).astype(np.float32)
    ties = near_tie_blocks(72, 200000)
    x = np.concatenate([rand, ties]).ravel()
    K = 32 * 1024
    ncols = x.size // K
    x = x[:K * ncols]
    xq, xd, _ = oracle.quantize_q8_1(x, K, ncols)
    b = x.reshape(-1, 32)
    d = np.abs(b).max(1) / np.float32(127)
    quot = round_half_away(b / d[:, None])
    prod = round_half_away(b * (np.float32(1) / d)[:, None])
    # the blocks must tell the two readings apart, or this test pins nothing
    assert np.count_nonzero(quot != prod) > 1000
    assert np.array_equal(xq.reshape(-1, 32).astype(np.float64), quot)
    assert np.array_equal(xd, d.astype(np.float16).astype(np.float32))


def test_q8_1_quotient_in_fused_producers(oracle):
    """The fused producers share the rule: swiglu_q8 with u = 1 and g >= 200 (silu(g) == g exactly in float32, as
    e^-g underflows to 0) quantizes g itself."""
    g = near_tie_blocks(73, 20000, log2_amax=(10, 12), k_min=25, signed=False).ravel()
    assert g.min() >= 200
    u = np.ones_like(g)
    xq, xd, _ = oracle.swiglu_q8(g, u)
    b = g.reshape(-1, 32)
    d = np.abs(b).max(1) / np.float32(127)
    quot = round_half_away(b / d[:, None])
    assert np.count_nonzero(quot != round_half_away(b * (np.float32(1) / d)[:, None])) > 100
    assert np.array_equal(xq.reshape(-1, 32).astype(np.float64), quot)


def attn_run(oracle, qg, k, v, qw, kw, pos0, T, n_ctx, q8, rope3=None):
    nb = oracle.kv_cache_bytes(NKVH, n_ctx, q8)
    kc = np.zeros(nb, np.uint8)
    vc = np.zeros(nb, np.uint8)
    qn = oracle.attn_prep(qg, k, v, qw, kw, kc, vc, pos0, T, EPS, THETA_SCALE, NQH, NKVH, n_ctx, q8, rope3)
    return qn, kc, vc


def test_q8_0_kv_rounds_the_product_with_the_reciprocal(oracle):
    """V is written to the q8_0 cache unnormalised, so its int8 values are roundf(v * float32(1/d)) exactly."""
    T = 512
    n_ctx = T
    r = np.random.default_rng(74)
    nblk = T * NKVH * 8
    v = near_tie_blocks(75, nblk)
    perm = r.permuted(np.tile(np.arange(32), (nblk, 1)), axis=1)   # amax anywhere in the block
    v = np.take_along_axis(v, perm, 1).ravel()
    qg = r.standard_normal(T * NQH * 512).astype(np.float32)
    k = r.standard_normal(T * NKVH * 256).astype(np.float32)
    w = np.ones(256, np.float32)
    _, _, vc = attn_run(oracle, qg, k, v, w, w, 0, T, n_ctx, True)
    so = NKVH * n_ctx * 256
    got = vc[:so].view(np.int8).reshape(NKVH, n_ctx, 8, 32).astype(np.float64)
    vb = v.reshape(T, NKVH, 8, 32).transpose(1, 0, 2, 3)
    d = np.abs(vb).max(3) / np.float32(127)
    prod = round_half_away(vb * (np.float32(1) / d)[..., None])
    quot = round_half_away(vb / d[..., None])
    assert np.count_nonzero(prod != quot) > 100
    assert np.array_equal(got, prod)
    assert np.array_equal(vc[so:].view(np.float16).reshape(NKVH, n_ctx, 8), d.astype(np.float16))


def test_imrope_sections_interleave_by_j_mod_3(oracle):
    """One of t/h/w changed: exactly the pairs j with j % 3 == c rotate by the changed position."""
    T = 3
    P, P2 = 1000, 77777
    r = np.random.default_rng(76)
    qg = r.standard_normal(T * NQH * 512).astype(np.float32)
    k = r.standard_normal(T * NKVH * 256).astype(np.float32)
    v = r.standard_normal(T * NKVH * 256).astype(np.float32)
    qw = (1 + 0.1 * r.standard_normal(256)).astype(np.float32)
    kw = qw.copy()
    # position 0 leaves the normed head unrotated (cos 0 = 1, sin 0 = 0 exactly)
    q0, _, _ = attn_run(oracle, qg, k, v, qw, kw, 0, T, 8, False, rope3=np.zeros(3 * T, np.int32))
    q0 = q0.reshape(T, NQH, 256).astype(np.float64)
    base = np.full((T, 3), P, np.int32)
    qb, _, _ = attn_run(oracle, qg, k, v, qw, kw, 0, T, 8, False, rope3=base.ravel())
    qb = qb.reshape(T, NQH, 256)
    freq = oracle.rope_freqs(np.float32(THETA_SCALE))
    j = np.arange(32)
    for c in range(3):
        r3 = base.copy()
        r3[:, c] = P2                                     # token t: component c moves, the other two stay at P
        qc, _, _ = attn_run(oracle, qg, k, v, qw, kw, 0, T, 8, False, rope3=r3.ravel())
        qc = qc.reshape(T, NQH, 256)
        moved = (j % 3) == c
        cols = np.concatenate([j, j + 32])
        mcols = np.concatenate([moved, moved])
        # pairs of other sections keep the bits of the all-P run, dims >= 64 are never rotated
        assert_bits_equal(qc[:, :, cols[~mcols]], qb[:, :, cols[~mcols]], f"unmoved pairs c={c}")
        assert_bits_equal(qc[:, :, 64:], qb[:, :, 64:], "dims >= 64")
        th = (np.float32(P2) * freq[moved]).astype(np.float64)      # one float32 multiply, as the contract states
        x0, x1 = q0[:, :, j[moved]], q0[:, :, j[moved] + 32]
        want0 = x0 * np.cos(th) - x1 * np.sin(th)
        want1 = x0 * np.sin(th) + x1 * np.cos(th)
        assert np.max(np.abs(qc[:, :, j[moved]] - want0)) < 4e-6
        assert np.max(np.abs(qc[:, :, j[moved] + 32] - want1)) < 4e-6
        # and they did move (the position-P rotation differs)
        assert np.count_nonzero(qc[:, :, j[moved]] != qb[:, :, j[moved]]) > qc[:, :, j[moved]].size // 2


def test_l2norm_eps_is_divided_by_n(oracle):
    """Heads with sum(x^2) comparable to eps: y = x / sqrt(n) / sqrt(S/n + eps/n) = x / sqrt(S + eps)."""
    T, heads, C = 2, 32, 10240
    r = np.random.default_rng(77)
    x = r.standard_normal((T, C)).astype(np.float32)
    scale = np.exp2(r.uniform(-14, -8, (T, heads, 1)))                 # S from about 1e-6 to 2e-3
    xh = (x[:, :128 * heads].reshape(T, heads, 128) * scale / np.sqrt(128)).astype(np.float32)
    x[:, :128 * heads] = xh.reshape(T, -1)
    y = oracle.l2norm_heads(x.ravel(), 128, heads, T, C, EPS).reshape(T, C)
    x64 = xh.astype(np.float64)
    S = (x64 ** 2).sum(2, keepdims=True)
    want = x64 / np.sqrt(S / 128 + EPS / 128) / np.sqrt(128)
    wrong = x64 / np.sqrt(S / 128 + EPS) / np.sqrt(128)
    got = y[:, :128 * heads].reshape(T, heads, 128).astype(np.float64)
    rel = np.abs(got - want) / np.abs(want).max(2, keepdims=True)
    assert rel.max() < 1e-5
    assert (np.abs(wrong - want) / np.abs(want).max(2, keepdims=True)).max() > 0.1
