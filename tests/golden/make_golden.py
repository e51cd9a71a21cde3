"""Writes tests/golden/known_answers.npz: inputs and expected outputs of four ops of the path whose results are fixed
without the oracle, by numpy's correctly rounded float32 arithmetic, by sums derived by hand (tests/treepins.py) and
by exact closed forms. The reference ships no golden vectors for this path, so these are the known answers; the
CPU oracle (tests/test_golden.py) and the HIP kernels (tests/test_gpu_golden.py) are both checked bit for bit
against the file.

- quantize_q8_1 (src/common.cuh:68-87): per 32 values d = amax / 127 in float32, q = roundf(y / d) with the IEEE
  quotient, xd = fp16(d), xs = the xor 8-4-2-1 butterfly sum of each 16 values; blocks: zero, one value +-A, d = 1
  with exact half-integer ties, the butterfly blocks of treepins.xs_blocks, near-tie blocks, random blocks over
  2^-30..2^30.
- rmsnorm_q8 (src/ops.cu:57-121): rows whose sum of squares depends on the summation tree (treepins row_warps,
  row_cross, row_korder), each with the eps at which the reference tree's sum and the other orders' sums give
  different scales; h = (scale * x) * w with scale = 1 / sqrtf(sum / n + eps) from the hand-derived sum; xq / xd /
  xs of h by the q8_1 rule above. w = 1 for the tree rows; a row of small integers (sum of squares exact in any
  order) with random w pins the product order.
- l2norm_heads (src/ops.cu:437-447): heads of 128 from treepins.l2_lanes / l2_korder, y = (x * scale) * post with
  scale = 1 / sqrtf(sum / 128 + eps / 128), post = 1 / sqrtf(128).
- get_rows_q8_0 (src/ops.cu:343-375 with ggml's Q8_0 block: fp16 d, 32 int8): y = fp16(d) * q, exact in float32.
- attn_prep (src/ops.cu:587-654) with every IMRoPE position 0 (rope3 all zero), so every rotary angle is 0 and the
  rotation is the identity (sin 0 = 0 and cos 0 = 1 exactly): qn = (scale * q) * q_norm per head of 256, with scale =
  1 / sqrtf(sum / 256 + eps) from the hand-derived sum of treepins.head_warps(256) (token 0) or the exact sum of
  nonzero small integers (tokens 1-3); the q8_0 K / V cache rows of (scale * k) * k_norm and of v: per 32 values d =
  amax / 127, q = roundf(y * (1 / d)), fp16(d) in the scale area after the int8 area (src/attn.cu:890-892).

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import treepins as tp  # noqa: E402
from cfgdata import near_tie_blocks, round_half_away  # noqa: E402

f32 = np.float32
E = tp.N_ROW


def q8_1(y):
    """The q8_1 rule over blocks of 32 (see the module text); returns xq, xd, xs."""
    b = np.ascontiguousarray(y, np.float32).reshape(-1, 32)
    d = (np.abs(b).max(1) / f32(127)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        quot = (b / d[:, None]).astype(np.float32)
    q = np.where(d[:, None] == 0, 0.0, round_half_away(quot)).astype(np.int8)
    with np.errstate(over="ignore"):  # d above 65504 (blocks of |y| > 8.3e6) rounds to fp16 infinity
        xd = d.astype(np.float16).astype(np.float32)
    xs = tp.butterfly16(b.reshape(-1))
    return q.reshape(-1), xd, xs


def q8_blocks():
    r = np.random.default_rng(20260)
    blocks = [np.zeros((2, 32), np.float32)]
    one = np.zeros((4, 32), np.float32)
    one[0, 0], one[1, 31], one[2, 7], one[3, 16] = 3.5, -1e-3, 6.0e4, -2.0 ** -20
    blocks.append(one)
    ties = np.zeros((4, 32), np.float32)  # amax 127 gives d = 1 exactly: the quotient is y itself
    for i in range(4):
        ties[i, 0] = 127.0 if i % 2 == 0 else -127.0
        ties[i, 1:] = (r.integers(-126, 126, 31) + 0.5).astype(np.float32)
    blocks.append(ties)
    xsb, _ = tp.xs_blocks()
    blocks.append(xsb.reshape(-1, 32))
    blocks.append(near_tie_blocks(20261, 200))
    rnd = (r.standard_normal((250, 32)) * np.exp2(r.uniform(-30, 30, (250, 1)))).astype(np.float32)
    blocks.append(rnd)
    x = np.concatenate(blocks).reshape(-1)
    pad = (-x.size) % 256  # K = 256 per column
    return np.concatenate([x, np.zeros(pad, np.float32)])


def row_cases():
    rows = []
    for make, good, bad in [(tp.row_warps, tp.ROW_WARPS_SUM, tp.ROW_WARPS_SEQ),
                            (tp.row_cross, tp.ROW_CROSS_SUM, tp.ROW_CROSS_SEQ),
                            (tp.row_korder, tp.ROW_KORDER_SUM, tp.ROW_KORDER_REV)]:
        e = tp.eps_separating(good, bad, E)
        x = make(1.0)
        w = np.ones(E, np.float32)
        h = (f32(tp.row_scale(good, E, e)) * x) * w
        rows.append((x, w, e, h))
    r = np.random.default_rng(20262)
    xi = r.integers(-8, 9, E).astype(np.float32)
    w = (r.standard_normal(E) * 0.7 + 1).astype(np.float32)
    t = float(np.sum(xi.astype(np.float64) ** 2))  # exact (an integer below 2^24), so every order gives it
    e = 1e-6
    rows.append((xi, w, e, (f32(tp.row_scale(t, E, e)) * xi) * w))
    return rows


def l2_cases():
    out = []
    post = f32(1) / np.sqrt(f32(128))
    for make, good, bad in [(tp.l2_lanes, tp.L2_LANES_SUM, tp.L2_LANES_SEQ),
                            (tp.l2_korder, tp.L2_KORDER_SUM, tp.L2_KORDER_REV)]:
        e = tp.eps_separating(good, bad, 128, tp.l2_scale)
        x = make(1.0)
        out.append((x, e, (x * f32(tp.l2_scale(good, 128, e))) * post))
    return out


def q8_0_table():
    """8 rows of 5120 values in Q8_0 blocks (34 bytes: fp16 d, 32 int8), d = 2^-k times a random mantissa."""
    r = np.random.default_rng(20263)
    rows, nblk = 8, E // 32
    d = (np.exp2(-r.integers(0, 12, (rows, nblk))) * r.uniform(0.5, 1.0, (rows, nblk))).astype(np.float16)
    q = r.integers(-128, 128, (rows, nblk, 32)).astype(np.int8)
    q[0, 0, :] = np.arange(-16, 16)  # a block that shows any lane or byte swap
    tab = np.zeros((rows, nblk, 34), np.uint8)
    tab[:, :, 0:2] = d.view(np.uint8).reshape(rows, nblk, 2)
    tab[:, :, 2:] = q.view(np.uint8)
    ids = np.array([3, 0, 7, 3, 5, 0, 6, 1], np.int32)
    y = (d.astype(np.float32)[:, :, None] * q.astype(np.float32)).reshape(rows, E)[ids]
    return tab.reshape(-1), ids, y.reshape(-1)


def q8_0_rows(y):
    """The q8_0 cache rule over blocks of 32: q = roundf(y * (1 / d)), d = amax / 127; returns int8 and fp16 bits."""
    b = np.ascontiguousarray(y, np.float32).reshape(-1, 32)
    d = (np.abs(b).max(1) / f32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, f32(1) / d, f32(0)).astype(np.float32)
    q = round_half_away((b * inv[:, None]).astype(np.float32)).astype(np.int8)
    return q.reshape(-1), d.astype(np.float16).view(np.uint16)


def attn_case():
    r = np.random.default_rng(20264)
    Tn, nqh, nkvh, n_ctx, pos0 = 4, 24, 4, 16, 7
    good, bad = tp.HEAD_WARPS_SUM[256], tp.HEAD_WARPS_SEQ[256]
    eps = tp.eps_separating(good, bad, 256)
    tree = tp.head_warps(256)

    def heads(n):
        h = r.integers(1, 9, (Tn, n, 256)) * np.where(r.random((Tn, n, 256)) < 0.5, -1, 1)
        h = h.astype(np.float32)
        h[0, :] = tree
        return h

    q, k = heads(nqh), heads(nkvh)
    v = (r.standard_normal((Tn, nkvh, 256)) * 2).astype(np.float32)
    qw = (r.standard_normal(256) * 0.1 + 1).astype(np.float32)
    kw = (r.standard_normal(256) * 0.1 + 1).astype(np.float32)
    qg = np.zeros((Tn, nqh, 512), np.float32)
    qg[:, :, :256] = q
    qg[:, :, 256:] = r.integers(-99, 100, (Tn, nqh, 256)).astype(np.float32)  # the gate half, not read

    def normed(x, w):
        sums = np.sum(x.astype(np.float64) ** 2, axis=-1)
        sums[0, :] = good  # token 0: the reference tree's sum, derived by hand
        sc = np.vectorize(lambda t: tp.row_scale(t, 256, eps))(sums).astype(np.float32)
        return (sc[..., None] * x) * w

    qn = normed(q, qw)
    kn = normed(k, kw)
    kc = np.zeros(nkvh * n_ctx * 272, np.uint8)
    vc = np.zeros(nkvh * n_ctx * 272, np.uint8)
    so = nkvh * n_ctx * 256
    for cache, src in ((kc, kn), (vc, v)):
        for t in range(Tn):
            for h in range(nkvh):
                row = h * n_ctx + pos0 + t
                qq, dd = q8_0_rows(src[t, h])
                cache[row * 256:(row + 1) * 256] = qq.view(np.uint8)
                cache[so + row * 16:so + (row + 1) * 16] = dd.view(np.uint8)
    return {"att_qg": qg.reshape(-1), "att_k": k.reshape(-1), "att_v": v.reshape(-1), "att_qw": qw, "att_kw": kw,
            "att_eps": np.float32(eps), "att_pos0": np.int32(pos0), "att_nctx": np.int32(n_ctx),
            "att_rope3": np.zeros((Tn, 3), np.int32), "att_qn": qn.reshape(-1), "att_kc": kc, "att_vc": vc}


def build():
    """Every array of the file, by name."""
    out = {}
    x = q8_blocks()
    out["q8_x"] = x
    out["q8_xq"], out["q8_xd"], out["q8_xs"] = q8_1(x)
    for i, (xr, w, e, h) in enumerate(row_cases()):
        out[f"row{i}_x"], out[f"row{i}_w"], out[f"row{i}_eps"], out[f"row{i}_h"] = xr, w, np.float32(e), h
        out[f"row{i}_xq"], out[f"row{i}_xd"], out[f"row{i}_xs"] = q8_1(h)
    for i, (xh, e, y) in enumerate(l2_cases()):
        out[f"l2{i}_x"], out[f"l2{i}_eps"], out[f"l2{i}_y"] = xh, np.float32(e), y
    out["q80_table"], out["q80_ids"], out["q80_y"] = q8_0_table()
    out.update(attn_case())
    return out


def main():
    out = build()
    path = os.path.join(HERE, "known_answers.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays")


if __name__ == "__main__":
    main()
