"""Pins of the oracle's scalar math against independent references (CPU only).

exp/log are compared with the C library in ulps, sin/cos with mpmath (correctly rounded to float), the fp16 and
bf16 conversions exhaustively with numpy. These routines replace the reference's fast-math expf/logf/sinf/cosf
(src/ops.cu:52-54, 621-622) on both the CPU and the GPU side.
"""
import math

import numpy as np
import pytest


def ulp_dist(a, b):
    ia = np.array([a], np.float32).view(np.int32)[0].astype(np.int64)
    ib = np.array([b], np.float32).view(np.int32)[0].astype(np.int64)
    if ia < 0:
        ia = -(ia & 0x7FFFFFFF)
    if ib < 0:
        ib = -(ib & 0x7FFFFFFF)
    return abs(int(ia) - int(ib))


def test_expf_ulp(oracle):
    rng = np.random.default_rng(11)
    xs = np.concatenate([rng.uniform(-103, 88.7, 40000), rng.normal(0, 3, 20000),
                         [0.0, -0.0, 1.0, -1.0, 88.7, -87.3, 1e-8, -1e-8, 20.0, -20.0]]).astype(np.float32)
    worst = 0
    for x in xs:
        ref = np.float32(math.exp(float(x)))
        got = oracle.expf(float(x))
        worst = max(worst, ulp_dist(got, ref))
    assert worst <= 2, worst
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(89.0) == math.inf
    assert oracle.expf(-104.0) == 0.0
    assert math.isnan(oracle.expf(float("nan")))
    # subnormal results keep one rounding: compare with the exactly rounded value
    for x in (-90.0, -95.5, -100.25, -103.0):
        assert ulp_dist(oracle.expf(x), np.float32(math.exp(x))) <= 2


def test_logf_ulp(oracle):
    rng = np.random.default_rng(12)
    ys = np.concatenate([np.exp(rng.uniform(-85, 88, 40000)), rng.uniform(1.0, 5e8, 20000),
                         [1.0, 2.0, 0.5, 1.4142135, 1e-40, 3e-45, 3.4e38]]).astype(np.float32)
    worst = 0
    for y in ys:
        if y <= 0:
            continue
        worst = max(worst, ulp_dist(oracle.logf(float(y)), np.float32(math.log(float(y)))))
    assert worst <= 2, worst
    assert oracle.logf(1.0) == 0.0
    assert oracle.logf(0.0) == -math.inf
    assert math.isnan(oracle.logf(-1.0))


def test_sincos_correctly_rounded(oracle):
    mpmath = pytest.importorskip("mpmath")
    mpmath.mp.prec = 120
    rng = np.random.default_rng(13)
    # RoPE angles: p * theta_scale^j for positions up to 262144 (src/model.h:27) plus small angles
    th = np.concatenate([rng.uniform(-3e5, 3e5, 3000), rng.uniform(-8, 8, 2000),
                         [0.0, 1e-30, math.pi / 2, math.pi, 150000.0, 131072.0]]).astype(np.float32)
    worst = 0
    for t in th:
        s, c = oracle.sincos(float(t))
        rs = np.float32(float(mpmath.sin(mpmath.mpf(float(t)))))
        rc = np.float32(float(mpmath.cos(mpmath.mpf(float(t)))))
        worst = max(worst, ulp_dist(s, rs), ulp_dist(c, rc))
    assert worst <= 1, worst
    assert oracle.sincos(0.0) == (0.0, 1.0)


def test_silu_special_values(oracle):
    assert oracle.silu(0.0) == 0.0
    assert oracle.silu(100.0) == 100.0            # 1 + e^-100 rounds to 1
    assert oracle.silu(-200.0) == 0.0             # e^200 -> inf, -200 / inf = -0
    assert abs(oracle.silu(1.0) - 1.0 / (1.0 + math.exp(-1.0))) < 1e-7


def test_f2h_exhaustive_against_numpy(oracle):
    L = oracle.lib()
    # every fp16 code decodes like numpy and re-encodes to itself (NaNs excluded: payload not part of the contract)
    for h in range(65536):
        f = np.array([h], np.uint16).view(np.float16)[0]
        if np.isnan(f):
            continue
        got = L.q27o_h2f(h)
        assert np.float32(got) == np.float32(f) or (got == 0 and f == 0), h
        assert L.q27o_f2h(got) == h, h
    # rounding of random floats (normal and subnormal fp16 range, ties) matches numpy's RNE
    rng = np.random.default_rng(14)
    xs = np.concatenate([rng.normal(0, 1, 20000), rng.uniform(-7e-5, 7e-5, 20000), rng.uniform(-70000, 70000, 5000),
                         [2049.0, 2051.0, 65520.0, 65519.0, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -24 * 1.5]]).astype(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.q27o_f2h(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)


def test_bf16_round_to_nearest_even(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(15)
    xs = rng.normal(0, 10, 20000).astype(np.float32)
    u = xs.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    got = np.array([L.q27o_f2bf(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)
    # ties: 1 + 2^-8 is halfway between bf16 1.0 and 1.0078125 -> even (1.0); 1 + 3*2^-8 -> 1.015625
    assert L.q27o_bf2f(L.q27o_f2bf(1.0 + 2 ** -8)) == 1.0
    assert L.q27o_bf2f(L.q27o_f2bf(1.0 + 3 * 2 ** -8)) == 1.015625


def test_rope_freqs(oracle):
    ts = np.float32(1e7) ** np.float32(-2.0 / 64)
    f = oracle.rope_freqs(float(ts))
    assert f[0] == 1.0
    want = np.array([float(ts) ** j for j in range(32)])
    assert np.max(np.abs(f / want - 1)) < 1e-6
