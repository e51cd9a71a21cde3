"""Pins of the CPU oracle's decode GEMV (oracle/q27_oracle_qgemv.c) without the GPU.

- Exact integer cases: every fp16 scale = 1 and every activation scale = 1, so each sub-block contribution and
  every partial sum is an integer below 2^24 and the float result must equal the integer dot product of the
  dequantized weights (numpy dequantizers written here from the ggml block formats) with the int8 activations.
  A wrong nibble, scale, sign, grid index or offset changes that integer.
- Random blocks at the model's shapes: the oracle against a float64 dequantize-then-dot (Q4_K / Q6_K rows from the
  oracle's already pinned get_rows, IQ4_XS / IQ3_S from the numpy dequantizers), within a bound of a few float32
  roundings per term.
- The waves-per-tile rule (part of the summation order) is the same function in the oracle and the library.
"""
import os
import re

import numpy as np
import pytest

import cfgdata as cd

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "qwen27-engine_amd", "csrc")


def _inc_values(name):
    text = open(os.path.join(CSRC, name)).read()
    text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//"))
    return [int(v, 0) for v in re.findall(r"-?0x[0-9a-fA-F]+|-?\d+", text.replace("u,", ","))]


IQ3S_GRID = np.array(_inc_values("iq3s_grid.inc"), np.uint32)
IQ4NL = np.array(_inc_values("iq4nl_values.inc"), np.int64)


def _f16(lo, hi):
    return (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8)).view(np.float16).astype(np.float64)


def dequant_int(type_, raw, N, K):
    """(integer weights [N][K] (int64) before the fp16 super-block scales, d [N][K/256], dmin-term [N][K])
    such that weight = d * wi - dmin_term (dmin_term = 0 except Q4_K)."""
    bb = cd.QG_BLOCK[type_]
    nb = K // 256
    B = raw.reshape(N * nb, bb).astype(np.int64)
    wi = np.zeros((N * nb, 256), np.int64)
    mterm = np.zeros((N * nb, 256), np.float64)
    if type_ == cd.Q4_K:
        d, dmin = _f16(B[:, 0], B[:, 1]), _f16(B[:, 2], B[:, 3])
        sc = B[:, 4:16]
        for s in range(8):
            if s < 4:
                scv, mv = sc[:, s] & 63, sc[:, s + 4] & 63
            else:
                scv = (sc[:, s + 4] & 0xF) | ((sc[:, s - 4] >> 6) << 4)
                mv = (sc[:, s + 4] >> 4) | ((sc[:, s] >> 6) << 4)
            q = (B[:, 16 + 32 * (s // 2):16 + 32 * (s // 2) + 32] >> (4 * (s & 1))) & 0xF
            wi[:, 32 * s:32 * s + 32] = q * scv[:, None]
            mterm[:, 32 * s:32 * s + 32] = (dmin * mv)[:, None]
    elif type_ == cd.Q6_K:
        d = _f16(B[:, 208], B[:, 209])
        scales = B[:, 192:208].astype(np.int8).astype(np.int64)
        for n in range(2):
            for l in range(32):
                ql0, ql1, qh = B[:, 64 * n + l], B[:, 64 * n + l + 32], B[:, 128 + 32 * n + l]
                qs = [(ql0 & 0xF) | ((qh & 3) << 4), (ql1 & 0xF) | (((qh >> 2) & 3) << 4),
                      (ql0 >> 4) | (((qh >> 4) & 3) << 4), (ql1 >> 4) | (((qh >> 6) & 3) << 4)]
                for j in range(4):
                    wi[:, 128 * n + 32 * j + l] = (qs[j] - 32) * scales[:, 8 * n + l // 16 + 2 * j]
    elif type_ == cd.IQ4_XS:
        d = _f16(B[:, 0], B[:, 1])
        sh = B[:, 2] | (B[:, 3] << 8)
        for s in range(8):
            ls = (((B[:, 4 + s // 2] >> (4 * (s & 1))) & 0xF) | (((sh >> (2 * s)) & 3) << 4)) - 32
            qs = B[:, 8 + 16 * s:8 + 16 * s + 16]
            wi[:, 32 * s:32 * s + 16] = IQ4NL[qs & 0xF] * ls[:, None]
            wi[:, 32 * s + 16:32 * s + 32] = IQ4NL[qs >> 4] * ls[:, None]
    elif type_ == cd.IQ3_S:
        d = _f16(B[:, 0], B[:, 1])
        for s in range(8):
            mul = 1 + 2 * ((B[:, 106 + s // 2] >> (4 * (s & 1))) & 0xF)
            qh = B[:, 66 + s]
            for k in range(8):
                idx = B[:, 2 + 8 * s + k] | ((qh << (8 - k)) & 256)
                g = IQ3S_GRID[idx].astype(np.int64)
                for j in range(4):
                    mag = (g >> (8 * j)) & 0xFF
                    neg = (B[:, 74 + 4 * s + k // 2] >> (j + 4 * (k & 1))) & 1
                    wi[:, 32 * s + 4 * k + j] = np.where(neg == 1, -mag, mag) * mul
    return wi.reshape(N, K), d.reshape(N, nb), mterm.reshape(N, K)


def _ones_scales(raw, type_):
    one = np.array([1.0], np.float16).view(np.uint8)
    B = raw.reshape(-1, cd.QG_BLOCK[type_])
    for off in cd.QG_D_OFFSETS[type_]:
        B[:, off], B[:, off + 1] = one[0], one[1]
    return B.reshape(-1)


@pytest.mark.parametrize("type_", [cd.Q4_K, cd.Q6_K, cd.IQ4_XS, cd.IQ3_S])
@pytest.mark.parametrize("ncols", [1, 3, 4])
def test_qgemv_exact_integer_cases(oracle, type_, ncols):
    r = cd.rng(100 + type_ + ncols)
    N, K = 64, 1024
    raw = _ones_scales(cd.random_weights(r, type_, N, K), type_)
    xq = r.integers(-8, 9, ncols * K).astype(np.int8)  # small activations keep every partial sum below 2^24
    xd = np.ones(ncols * K // 32, np.float32)
    y = oracle.qgemv(type_, raw, N, K, xq, xd, ncols)
    wi, d, mterm = dequant_int(type_, raw, N, K)
    assert np.all(d == 1.0)
    if type_ == cd.Q4_K:  # dmin = 1: weight = sc q - m with integer m
        wi = wi - mterm.astype(np.int64)
    want = wi @ xq.reshape(ncols, K).astype(np.int64).T  # [N][ncols]
    assert np.abs(want).max() < 2 ** 24
    np.testing.assert_array_equal(y, want.T.astype(np.float32))


@pytest.mark.parametrize("type_", [cd.Q4_K, cd.Q6_K, cd.IQ4_XS, cd.IQ3_S])
@pytest.mark.parametrize("shape", [(1024, 5120), (6144, 1024), (12288, 512)])
def test_qgemv_matches_float64_dequant(oracle, type_, shape):
    N, K = shape
    ncols = 4
    r = cd.rng(200 + type_ + N)
    raw = cd.random_weights(r, type_, N, K)
    xq, xd = cd.q8_activations(oracle, r, ncols, K)
    y = oracle.qgemv(type_, raw, N, K, xq, xd, ncols).astype(np.float64)
    if type_ in (cd.Q4_K, cd.Q6_K):
        kind = cd.QG_NAMES[type_]
        W = oracle.get_rows(kind, raw, (K // 256) * cd.QG_BLOCK[type_], np.arange(N, dtype=np.int32), K)
        W = W.reshape(N, K).astype(np.float64)
    else:
        wi, d, _ = dequant_int(type_, raw, N, K)
        W = wi * np.repeat(d, 256, axis=1)
    x = xq.reshape(ncols, K).astype(np.float64) * np.repeat(xd.reshape(ncols, K // 32).astype(np.float64), 32, axis=1)
    want = (W @ x.T).T
    mag = (np.abs(W) @ np.abs(x).T).T
    # each sub-block term carries a few float32 roundings (relative 2^-22 at most), the 8 W ... sums one more each
    assert np.all(np.abs(y - want) <= 4e-6 * mag + 1e-30), np.max(np.abs(y - want) / (mag + 1e-30))


def test_qgemv_waves_rule_matches_library(oracle, q27):
    lib = q27.lib()
    for N in [8, 1024, 5120, 248320]:
        for K in [256, 1024, 2048, 2304, 4096, 5120, 6144, 8192, 10240, 17408, 32768, 40960]:
            assert lib.q27h_qgemv_waves(N, K) == oracle.qgemv_waves(N, K), (N, K)
    assert [oracle.qgemv_waves(8, K) for K in (256, 2048, 2304, 5120, 8192, 17408, 40960)] == [1, 1, 2, 3, 4, 4, 4]


def test_qgemv_rejects_bad_shapes(oracle):
    with pytest.raises(ValueError):
        oracle.qgemv(cd.Q4_K, np.zeros(144 * 4, np.uint8), 4, 256, np.zeros(256, np.int8), np.zeros(8, np.float32), 1)
