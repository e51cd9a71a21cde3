"""Seeded synthetic inputs for the five BASELINE.json configurations (numpy, host side).

cfg1  RMSNorm -> q8_1 on one 5120 row, N(0,1) with 0.1% of the values x50, w ~ N(1, 0.1), eps 1e-6
cfg2  decode verify pass, T = 4: rows [4][5120]; gate/up [4][17408] ~ N(0, 2) (standard deviation 2);
      q|gate [4][24][512], k, v [4][4][256]; positions 150000..150003; q8_0 cache of 180224 rows
cfg3  prefill M = 2048: activations N(0,1) * s[c], s ~ LogNormal(0, 1) per channel, rounded to bf16 values;
      positions from 0 or 131072; q8_0 cache of 180224 rows
cfg4  embedding gather: 248320 x 5120 tables (Q4_K, Q6_K, Q8_0, IQ2_S), fp16 scales in [2^-10, 2^-4];
      2048 Zipf(1.1) ids + 4 uniform ids
cfg5  multimodal + GDN, 4099 rows = 3 text + a 64 x 64 image grid (IMRoPE positions t, h, w)
"""
from __future__ import annotations

import numpy as np

E = 5120
FF = 17408
NQH, NKVH = 24, 4
KH, HV = 16, 48
C_CONV = 2 * KH * 128 + HV * 128
EPS = 1e-6
N_CTX = 180224
VOCAB = 248320
THETA_SCALE = float(np.float32(1e7) ** np.float32(-2.0 / 64))  # powf(rope_base, -2 / rope_dims), src/model.cu:712
BLOCK = {"q4_k": (144, 256), "q6_k": (210, 256), "q8_0": (34, 32), "iq2_s": (82, 256)}
D_OFFSETS = {"q4_k": (0, 2), "q6_k": (208,), "q8_0": (0,), "iq2_s": (0,)}  # fp16 scale fields inside a block


def rng(seed):
    return np.random.default_rng(seed)


def normal(r, n, std=1.0, mean=0.0):
    return (r.standard_normal(n) * std + mean).astype(np.float32)


def to_bf16_values(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def cfg1(seed=1):
    r = rng(seed)
    x = normal(r, E)
    x[r.choice(E, 5, replace=False)] *= 50
    return x, normal(r, E, 0.1, 1.0)


def prefill_rows(r, M, n=E):
    s = np.exp(r.standard_normal(n)).astype(np.float32)
    return to_bf16_values(r.standard_normal((M, n)).astype(np.float32) * s).reshape(-1)


def zipf_ids(r, T, vocab=VOCAB, s=1.1):
    w = np.arange(1, vocab + 1, dtype=np.float64) ** -s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    ranks = np.minimum(np.searchsorted(cdf, r.random(T)), vocab - 1)
    perm = r.permutation(vocab)
    return perm[ranks].astype(np.int32)


def gather_ids(seed=4, T=2048, U=4, vocab=VOCAB):
    r = rng(seed)
    return np.concatenate([zipf_ids(r, T, vocab), r.integers(0, vocab, U).astype(np.int32)])


def random_table(r, kind, rows, n):
    """Random block bytes with every fp16 scale field set to a finite value in [2^-10, 2^-4]."""
    bb, bv = BLOCK[kind]
    nblk = rows * (n // bv)
    t = r.integers(0, 256, nblk * bb, dtype=np.uint8).reshape(nblk, bb)
    for off in D_OFFSETS[kind]:
        d = np.exp2(r.uniform(-10, -4, nblk)).astype(np.float16)
        t[:, off:off + 2] = d.view(np.uint8).reshape(nblk, 2)
    return t.reshape(-1)


def rope3_grid(text_before=3, nx=64, ny=64):
    """IMRoPE rows as tools/q27_server.cpp:353-369 builds them: text rows t = h = w = p, then the image rows
    (P, P + i / nx, P + i % nx)."""
    rows = []
    p = 0
    for _ in range(text_before):
        rows.append((p, p, p))
        p += 1
    for i in range(nx * ny):
        rows.append((p, p + i // nx, p + i % nx))
    return np.array(rows, np.int32).reshape(-1)


# ---------------------------------------------------------------- decode GEMV weights (ggml type ids)
Q2_K, Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 10, 12, 14, 16, 17, 18, 21, 22, 23, 29
QG_TYPES = [Q2_K, Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ1_M]
QG_BLOCK = {Q2_K: 84, Q4_K: 144, Q6_K: 210, IQ2_XXS: 66, IQ2_XS: 74, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ4_XS: 136,
            IQ1_M: 56}
# fp16 scale fields inside a block (IQ1_M has none: its scale is the four top nibbles of the scales words)
QG_D_OFFSETS = {Q2_K: (80, 82), Q4_K: (0, 2), Q6_K: (208,), IQ2_XXS: (0,), IQ2_XS: (0,), IQ3_XXS: (0,), IQ3_S: (0,),
                IQ2_S: (0,), IQ4_XS: (0,), IQ1_M: ()}
QG_NAMES = {Q2_K: "q2_k", Q4_K: "q4_k", Q6_K: "q6_k", IQ2_XXS: "iq2_xxs", IQ2_XS: "iq2_xs", IQ3_XXS: "iq3_xxs",
            IQ3_S: "iq3_s", IQ2_S: "iq2_s", IQ4_XS: "iq4_xs", IQ1_M: "iq1_m"}


def set_iq1m_scale(blocks, h16):
    """Write fp16 bit patterns h16 [nblk] as the IQ1_M super-block scale: nibble k of h16 is the top nibble of the
    scales word k (bytes 48 + 2 k, 49 + 2 k)."""
    for k in range(4):
        nib = ((h16.astype(np.uint32) >> (4 * k)) & 0xF).astype(np.uint8)
        blocks[:, 49 + 2 * k] = (blocks[:, 49 + 2 * k] & 0x0F) | (nib << 4)
# decode GEMV shapes of the model (N outputs x K inputs, tp = 1): wk/wv, ssm_out / wo, gate z, qkv, wq, ffn up/gate,
# ffn down
QG_SHAPES = [(1024, 5120), (5120, 6144), (6144, 5120), (10240, 5120), (12288, 5120), (17408, 5120), (5120, 17408)]


def random_weights(r, type_, N, K, d_range=(-10, -4)):
    """N rows of K/256 random blocks of a GEMV weight type, fp16 scale fields finite in 2^d_range."""
    bb = QG_BLOCK[type_]
    nblk = N * (K // 256)
    t = r.integers(0, 256, nblk * bb, dtype=np.uint8).reshape(nblk, bb)
    for off in QG_D_OFFSETS[type_]:
        d = np.exp2(r.uniform(d_range[0], d_range[1], nblk)).astype(np.float16)
        t[:, off:off + 2] = d.view(np.uint8).reshape(nblk, 2)
    if type_ == IQ1_M:
        set_iq1m_scale(t, np.exp2(r.uniform(d_range[0], d_range[1], nblk)).astype(np.float16).view(np.uint16))
    return t.reshape(-1)


def q8_activations(oracle, r, ncols, K, std=1.0):
    x = normal(r, ncols * K, std)
    xq, xd, _ = oracle.quantize_q8_1(x, K, ncols)
    return xq, xd


def gdn_inputs(r, T, H=HV, HK=KH, planes_std=0.5):
    """Inputs of the delta rule as the model feeds them: one conv-output row per token ([q | k | v], stride
    2 * HK * 128 + H * 128) with q and k of unit norm per head, g = softplus(.) * ssm_a < 0, beta in (0, 1), and
    four random state planes [4][H][128][128]."""
    stride = 2 * HK * 128 + H * 128
    x = normal(r, T * stride).reshape(T, stride)
    qk = x[:, : 2 * HK * 128].reshape(T, 2 * HK, 128)
    qk /= np.sqrt((qk.astype(np.float64) ** 2).sum(-1, keepdims=True)).astype(np.float32)
    g = (-np.abs(r.standard_normal(T * H)) * 0.5 - 0.01).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-r.standard_normal(T * H)))).astype(np.float32)
    planes = normal(r, 4 * H * 128 * 128, std=planes_std)
    return x.reshape(-1).copy(), stride, g, beta, planes


def round_half_away(r32):
    """roundf of float32 values, computed in float64 (exact for float32 inputs)."""
    r = r32.astype(np.float64)
    return np.sign(r) * np.floor(np.abs(r) + 0.5)


def near_tie_blocks(seed, nblk, log2_amax=(-20, 20), k_min=0, signed=True):
    """Blocks of 32 whose values sit within a few ulps of (k + 1/2) * d, where d = amax / 127 in float32.

    Value 0 of each block is the amax (so it fixes d); the others are k + 1/2 steps of d nudged by -3..3 ulps, which
    is where the quotient and the product with the rounded reciprocal can round differently."""
    r = np.random.default_rng(seed)
    amax = np.exp2(r.integers(*log2_amax, nblk)).astype(np.float32) * r.uniform(1, 2, nblk).astype(np.float32)
    d = amax / np.float32(127)
    k = r.integers(k_min, 126, (nblk, 31)).astype(np.float32)
    base = ((k + np.float32(0.5)) * d[:, None]).astype(np.float32)
    ulp = r.integers(-3, 4, (nblk, 31)).astype(np.int32)
    y = (base.view(np.int32) + ulp).view(np.float32)
    flip = (lambda shape: np.where(r.random(shape) < 0.5, -1, 1)) if signed else (lambda shape: np.ones(shape))
    sign = flip((nblk, 31)).astype(np.float32)
    blk = np.empty((nblk, 32), np.float32)
    blk[:, 0] = amax * flip(nblk).astype(np.float32)
    blk[:, 1:] = np.minimum(np.abs(y), amax[:, None]) * sign
    return blk
