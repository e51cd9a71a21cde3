"""GPU side of the four independently pinned semantics: the HIP kernels, through the C ABI, on inputs built so the
alternative readings differ, checked against numpy's correctly rounded forms directly and against the CPU oracle.

- q8_1 rounds y / d (src/common.cuh:76): quantize_q8_1, swiglu_q8;
- the q8_0 KV cache rounds x * (1/d) (src/ops.cu:644-646): attn_prep's V rows;
- IMRoPE position of pair j is rope3[t][j % 3] (src/ops.cu:616-619): attn_prep with distinct t, h, w per token;
- the L2 norm adds eps / n (src/ops.cu:444): l2norm_heads and gdn_conv_prefill's fused form, sum(x^2) near eps.
"""
import sys

import numpy as np
import pytest

import cfgdata as cd
from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu
EPS = cd.EPS


def say(msg):
    print(f"[gpu-pins] {msg}", flush=True)
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

    return H()


@pytest.mark.parametrize("nblk", [64, 262144])
def test_q8_1_quotient_on_gpu(q27, oracle, T, nblk):
    import torch

    say(f"quantize_q8_1 near-tie blocks nblk={nblk}")
    x = cd.near_tie_blocks(200 + nblk, nblk).ravel()
    K = 32 * 64
    ncols = x.size // K
    xq, xd = T.empty(x.size, torch.int8), T.empty(x.size // 32)
    q27.ops.quantize_q8_1(T.up(x), xq, xd, K, ncols)
    got = T.down(xq).reshape(-1, 32).astype(np.float64)
    b = x.reshape(-1, 32)
    d = np.abs(b).max(1) / np.float32(127)
    quot = cd.round_half_away(b / d[:, None])
    assert np.array_equal(got, quot)
    oq, od, _ = oracle.quantize_q8_1(x, K, ncols)
    assert_bits_equal(T.down(xq), oq, "xq")
    assert_bits_equal(T.down(xd), od, "xd")


@pytest.mark.parametrize("nblk", [64, 65536])
def test_swiglu_q8_quotient_on_gpu(q27, T, nblk):
    import torch

    say(f"swiglu_q8 near-tie blocks nblk={nblk}")
    g = cd.near_tie_blocks(300 + nblk, nblk, log2_amax=(10, 12), k_min=25, signed=False).ravel()
    u = np.ones_like(g)
    xq, xd = T.empty(g.size, torch.int8), T.empty(g.size // 32)
    q27.ops.swiglu_q8(T.up(g), T.up(u), xq, xd, g.size)
    b = g.reshape(-1, 32)
    d = np.abs(b).max(1) / np.float32(127)
    assert np.array_equal(T.down(xq).reshape(-1, 32).astype(np.float64), cd.round_half_away(b / d[:, None]))


def attn(q27, oracle, T, Tn, n_ctx, qg, k, v, qw, kw, rope3=None):
    import torch

    nb = q27.ops.kv_cache_bytes(cd.NKVH, n_ctx, True)
    kc, vc = T.empty(nb, torch.uint8), T.empty(nb, torch.uint8)
    qn = T.empty(Tn * cd.NQH * 256)
    q27.ops.attn_prep(T.up(qg), T.up(k), T.up(v), T.up(qw), T.up(kw), qn, kc, vc, T.i32([0]), Tn, EPS, cd.THETA_SCALE,
                      cd.NQH, cd.NKVH, n_ctx, True, None, None, 0, None if rope3 is None else T.i32(rope3), None)
    okc, ovc = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
    oqn = oracle.attn_prep(qg, k, v, qw, kw, okc, ovc, 0, Tn, EPS, cd.THETA_SCALE, cd.NQH, cd.NKVH, n_ctx, True, rope3)
    got = T.down(qn), T.down(kc), T.down(vc)
    assert_bits_equal(got[0], oqn, "qn")
    assert_bits_equal(got[1], okc, "kcache")
    assert_bits_equal(got[2], ovc, "vcache")
    return got


@pytest.mark.parametrize("Tn", [4, 2048])
def test_q8_0_kv_product_on_gpu(q27, oracle, T, Tn):
    say(f"attn_prep q8_0 near-tie V rows T={Tn}")
    r = cd.rng(400 + Tn)
    nblk = Tn * cd.NKVH * 8
    v = cd.near_tie_blocks(401 + Tn, nblk)
    v = np.take_along_axis(v, r.permuted(np.tile(np.arange(32), (nblk, 1)), axis=1), 1).ravel()
    qg, k = cd.normal(r, Tn * cd.NQH * 512), cd.normal(r, Tn * cd.NKVH * 256)
    w = np.ones(256, np.float32)
    _, _, vc = attn(q27, oracle, T, Tn, Tn, qg, k, v, w, w)
    so = cd.NKVH * Tn * 256
    vb = v.reshape(Tn, cd.NKVH, 8, 32).transpose(1, 0, 2, 3)
    d = np.abs(vb).max(3) / np.float32(127)
    want = cd.round_half_away(vb * (np.float32(1) / d)[..., None])
    assert np.array_equal(vc[:so].view(np.int8).reshape(cd.NKVH, Tn, 8, 32).astype(np.float64), want)


def test_imrope_distinct_sections_on_gpu(q27, oracle, T):
    say("attn_prep IMRoPE with distinct t, h, w per token")
    Tn = 512
    r = cd.rng(500)
    rope3 = r.integers(0, 200000, (Tn, 3)).astype(np.int32)
    qg, k, v = cd.normal(r, Tn * cd.NQH * 512), cd.normal(r, Tn * cd.NKVH * 256), cd.normal(r, Tn * cd.NKVH * 256)
    qw, kw = cd.normal(r, 256, 0.1, 1.0), cd.normal(r, 256, 0.1, 1.0)
    qn, _, _ = attn(q27, oracle, T, Tn, Tn, qg, k, v, qw, kw, rope3.ravel())
    # float64 check of the section map: pair j turns by rope3[t][j % 3] * freq[j]
    qn = qn.reshape(Tn, cd.NQH, 256).astype(np.float64)
    q = qg.reshape(Tn, cd.NQH, 512)[:, :, :256].astype(np.float64)
    qs = q / np.sqrt((q ** 2).mean(2, keepdims=True) + EPS) * qw
    freq = oracle.rope_freqs(np.float32(cd.THETA_SCALE))
    j = np.arange(32)
    th = (rope3[:, j % 3].astype(np.float32) * freq[None, :]).astype(np.float64)[:, None, :]
    x0, x1 = qs[:, :, :32], qs[:, :, 32:64]
    assert np.max(np.abs(qn[:, :, :32] - (x0 * np.cos(th) - x1 * np.sin(th)))) < 5e-5
    assert np.max(np.abs(qn[:, :, 32:64] - (x0 * np.sin(th) + x1 * np.cos(th)))) < 5e-5


def small_heads(r, rows, heads, stride):
    x = cd.normal(r, rows * stride).reshape(rows, stride)
    scale = np.exp2(r.uniform(-14, -8, (rows, heads, 1))) / np.sqrt(128)
    x[:, :128 * heads] = (x[:, :128 * heads].reshape(rows, heads, 128) * scale).astype(np.float32).reshape(rows, -1)
    return np.ascontiguousarray(x, np.float32)


def test_l2norm_small_sums_on_gpu(q27, oracle, T):
    say("l2norm_heads with sum(x^2) near eps")
    rows, heads, C = 2048, 32, cd.C_CONV
    x = small_heads(cd.rng(600), rows, heads, C)
    xd = T.up(x.ravel())
    q27.ops.l2norm_heads(xd, 128, heads, rows, C, EPS)
    got = T.down(xd).reshape(rows, C)
    assert_bits_equal(got, oracle.l2norm_heads(x.ravel(), 128, heads, rows, C, EPS).reshape(rows, C), "x")
    x64 = x[:, :128 * heads].reshape(rows, heads, 128).astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).sum(2, keepdims=True) + EPS)
    g = got[:, :128 * heads].reshape(rows, heads, 128)
    assert (np.abs(g - want) / np.abs(want).max(2, keepdims=True)).max() < 1e-5
