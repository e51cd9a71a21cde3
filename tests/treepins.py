"""Inputs that expose the summation order of every reduction on the path, with the sums derived by hand.

Every reduction of the reference adds float32 values in a fixed tree:

- a row of 5120 is held by 1024 threads, thread u adding v[u + 1024 k]^2 for k = 0..4 starting from 0
  (src/ops.cu:93-99); the per-thread partials go through the 32-lane xor butterfly 16, 8, 4, 2, 1 (warp_sum,
  src/ops.cu:34-38) and the 32 warp sums through the same butterfly again (block_sum, src/ops.cu:40-50);
- a gated head of 128 (src/ops.cu:279) and an attention head of 256 (src/ops.cu:605) are block_sums over 4 and 8 warps
  of one value per thread;
- an L2 head of 128 is one warp, lane l adding p[l + 32 k]^2 for k = 0..3 (src/ops.cu:441-443, 318-324);
- the q8_1 block sum xs adds 16 values by the xor butterfly 8, 4, 2, 1 (src/common.cuh:80-86).

The inputs below put one large value beside small ones. In float32, 2^24 + 1 is a tie that rounds back to 2^24 (the
even neighbour), while 2^24 + 2 is exact. So a small value added alone to the large one is lost, and small values
added to each other first are kept. Which of them are kept depends only on the order of the additions. That makes
the sum a function of the tree, and each sum here is worked out by hand (the derivation is beside each constant).
A sequential sum, a contiguous thread layout or another butterfly order gives a different, also hand-derivable
value; the tests check that the derived sums tell these orders apart.

Values are in units of m, a power of two (squares scale by m^2 exactly, so the rounding pattern is the same for
every m).
"""
from __future__ import annotations

import numpy as np

N_ROW = 5120
BIG = 4096.0          # BIG^2 = 2^24
P24 = float(2 ** 24)


# ------------------------------------------------------------------------------------------------ row of 5120
def row_warps(m=1.0):
    """v[i] = 4096 m for i < 1024 with i % 32 == 0, m for the other i < 1024, 0 for i >= 1024.

    Thread u holds v[u] only (its other four values are 0), so warp w's lanes hold (2^24, 1, ..., 1) m^2.
    Warp butterfly, lane 0: xor 16 adds lane 16 alone: 2^24 + 1 -> 2^24; xor 8 adds (l8 + l24) = 2 -> 2^24 + 2;
    xor 4 adds 4 -> 2^24 + 6; xor 2 adds 8 -> 2^24 + 14; xor 1 adds 16 -> 2^24 + 30 (all exact: even and < 2^25).
    All 32 warp sums are equal, so the cross-warp butterfly doubles exactly five times: 2^29 + 960.
    A sequential sum loses every one: 32 * 2^24 = 2^29."""
    v = np.zeros(N_ROW, np.float32)
    v[:1024] = m
    v[:1024:32] = BIG * m
    return v


ROW_WARPS_SUM = 2.0 ** 29 + 960.0
ROW_WARPS_SEQ = 2.0 ** 29


def row_cross(m=1.0):
    """v[0] = 4096 m, v[32 w] = m for w = 1..31, 0 elsewhere: warp sums (2^24, 1, ..., 1) m^2 (exact within each
    warp), and the cross-warp butterfly over them is the one of row_warps: 2^24 + 30. Sequential: 2^24."""
    v = np.zeros(N_ROW, np.float32)
    v[32:1024:32] = m
    v[0] = BIG * m
    return v


ROW_CROSS_SUM = P24 + 30.0
ROW_CROSS_SEQ = P24


def row_korder(m=1.0):
    """v[u + 1024 k] = m for k = 0..3 and v[u + 4096] = 4096 m, every thread u.

    Thread u adds 0 + 1 + 1 + 1 + 1 = 4, then 2^24: 2^24 + 4 (exact). 1024 equal partials double exactly ten times
    (2^(24+j) + 2^(j+2) is a multiple of the ulp 2^(j+1)): 2^34 + 4096. The large value first (k = 4 down to 0)
    loses all four ones: 2^34."""
    v = np.full(N_ROW, m, np.float32)
    v[4096:] = BIG * m
    return v


ROW_KORDER_SUM = 2.0 ** 34 + 4096.0
ROW_KORDER_REV = 2.0 ** 34


# ------------------------------------------------------------------------------------------------ heads
def head_warps(n, m=1.0):
    """A head of n = 128 or 256 values, one per thread: lane 0 of each warp 4096 m, the other lanes m.
    Each warp sums to 2^24 + 30 (row_warps); 4 or 8 equal warp sums double exactly: 4 (2^24 + 30) = 2^26 + 120,
    8 (2^24 + 30) = 2^27 + 240. Sequential: 2^26, 2^27."""
    v = np.full(n, m, np.float32)
    v[::32] = BIG * m
    return v


HEAD_WARPS_SUM = {128: 2.0 ** 26 + 120.0, 256: 2.0 ** 27 + 240.0}
HEAD_WARPS_SEQ = {128: 2.0 ** 26, 256: 2.0 ** 27}


def gated_cross(m=1.0):
    """A gated head of 128: v[0] = 4096 m, v[32] = v[64] = v[96] = m, 0 elsewhere: warp sums (2^24, 1, 1, 1) m^2.
    The cross-warp butterfly over 4 live lanes adds (w0 + w2) + (w1 + w3) = (2^24 + 1 -> 2^24) + 2 = 2^24 + 2.
    Sequential ((w0 + w1) + w2) + w3 loses each one: 2^24."""
    v = np.zeros(128, np.float32)
    v[[32, 64, 96]] = m
    v[0] = BIG * m
    return v


GATED_CROSS_SUM = P24 + 2.0
GATED_CROSS_SEQ = P24


def l2_lanes(m=1.0):
    """An L2 head of 128 held by one warp: p[0] = 4096 m, p[1..31] = m, p[32..127] = 0, so lane l holds p[l]^2 and
    the warp butterfly gives 2^24 + 30 (row_warps); sequential 2^24. A contiguous layout (lane l holding
    p[4l..4l+3]) would give lane 0 2^24 + 1 + 1 + 1 -> 2^24 and lanes 1..7 four each."""
    v = np.zeros(128, np.float32)
    v[:32] = m
    v[0] = BIG * m
    return v


L2_LANES_SUM = P24 + 30.0
L2_LANES_SEQ = P24


def l2_korder(m=1.0):
    """p[l] = p[l + 32] = p[l + 64] = m, p[l + 96] = 4096 m for every lane l: lane sums 0 + 1 + 1 + 1 = 3, then
    3 + 2^24 is a tie between 2^24 + 2 and 2^24 + 4 and goes to the even mantissa, 2^24 + 4. 32 equal lanes double
    exactly: 2^29 + 128. The large value first: 2^24 + 1 + 1 + 1 -> 2^24 per lane, 2^29."""
    v = np.full(128, m, np.float32)
    v[96:] = BIG * m
    return v


L2_KORDER_SUM = 2.0 ** 29 + 128.0
L2_KORDER_REV = 2.0 ** 29


# ------------------------------------------------------------------------------------------------ q8_1 xs
def xs_blocks():
    """32-value blocks (two xs sums each) and their xor 8, 4, 2, 1 butterfly sums, lane 0's value.

    Block A, half 0: (2^24, 1 x 7, -2^24, 1 x 7). xor 8: a0 + a8 = 0; xor 4 adds a4 + a12 = 2; xor 2 adds
      (a2 + a10) + (a6 + a14) = 4 -> 6; xor 1 adds the 8 odd lanes = 8 -> 14. Sequential: 2^24 + 1 ... stays 2^24,
      then -2^24 -> 0, then 7 ones: 7.
    Block A, half 1: (1, 2^24, 1 x 7, -2^24, 1 x 6) (2^24 at 1, -2^24 at 9). xor 8: a0 + a8 = 2; xor 4: + 2 -> 4;
      xor 2: + 4 -> 8; xor 1 adds ((a1 + a9) + (a5 + a13)) + ((a3 + a11) + (a7 + a15)) = (0 + 2) + 4 = 6 -> 14.
      Sequential: 1 + 2^24 -> 2^24, the next seven ones lost, -2^24 -> 0, six ones: 6.
    Block B, half 0: (2^24, 1 x 15). xor 8 adds a8 alone: 2^24 + 1 -> 2^24; then + 2, + 4, + 8: 2^24 + 14.
      Sequential: 2^24.
    Block B, half 1: all 1: 16 in every order (a control).
    """
    a0 = np.ones(16, np.float32)
    a0[0], a0[8] = P24, -P24
    a1 = np.ones(16, np.float32)
    a1[1], a1[9] = P24, -P24
    b0 = np.ones(16, np.float32)
    b0[0] = P24
    b1 = np.ones(16, np.float32)
    return np.concatenate([a0, a1, b0, b1]), np.array([14.0, 14.0, P24 + 14.0, 16.0], np.float32)


XS_SEQ = np.array([7.0, 6.0, P24, 16.0], np.float32)


# ------------------------------------------------------------------------------------------------ scales
def f32(x):
    return np.float32(x)


def row_scale(t, n, eps):
    """1 / sqrtf(t / n + eps) in float32 (each operation correctly rounded, as in the contract)."""
    return f32(1.0) / np.sqrt(f32(t) / f32(n) + f32(eps))


def l2_scale(t, n, eps):
    """1 / sqrtf(t / n + eps / n) (src/ops.cu:444)."""
    return f32(1.0) / np.sqrt(f32(t) / f32(n) + f32(eps) / f32(n))


def eps_separating(t_good, t_bad, n, scale=row_scale, m2=1.0):
    """The first eps of 1e-6, then k 2^-10 (k = 1..4096) times m^2 / n, at which the two sums give different float32
    scales (a one-ulp difference in t does not always survive the square root; eps moves where the root falls)."""
    for e in [1e-6] + [k * 2.0 ** -10 * m2 for k in range(1, 4097)]:
        if scale(t_good * m2, n, e) != scale(t_bad * m2, n, e):
            return float(f32(e))
    raise AssertionError("no eps separates the two sums")


def butterfly16(y):
    """The xor 8, 4, 2, 1 butterfly over each 16 consecutive values of y, lane 0's result (src/common.cuh:83-86):
    after step o, lane l holds a[l] + a[l ^ o]. Checked against the hand-derived sums of xs_blocks."""
    a = np.ascontiguousarray(y, np.float32).reshape(-1, 16).copy()
    for o in (8, 4, 2, 1):
        a = a + a[:, np.arange(16) ^ o]
    return a[:, 0].copy()
