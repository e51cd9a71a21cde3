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


def main():
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
    path = os.path.join(HERE, "known_answers.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays")


if __name__ == "__main__":
    main()
