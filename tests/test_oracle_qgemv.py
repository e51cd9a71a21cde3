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
IQ2XXS_GRID = np.array(_inc_values("iq2xxs_grid.inc"), np.uint64)
IQ2XS_GRID = np.array(_inc_values("iq2xs_grid.inc"), np.uint64)
IQ2S_GRID = np.array(_inc_values("iq2s_grid.inc"), np.uint64)
IQ3XXS_GRID = np.array(_inc_values("iq3xxs_grid.inc"), np.uint32)
IQ1S_GRID = np.array(_inc_values("iq1s_grid.inc"), np.uint32)
# the reference's integer scale rules with truncating divisions (one unit per 32-weight sub-block at most)
TRUNCATING = {cd.IQ2_XXS, cd.IQ2_XS, cd.IQ2_S, cd.IQ3_XXS}


def _ksigns(v7):
    v7 = v7.astype(np.int64)
    par = np.zeros_like(v7)
    for b in range(7):
        par ^= (v7 >> b) & 1
    return v7 | (par << 7)


def _grid8(grid, idx, signs):
    """[nblk][8] signed magnitudes of 64-bit grid entries idx with sign byte `signs`."""
    g = grid[idx].astype(np.uint64)
    out = np.zeros(idx.shape + (8,), np.int64)
    for j in range(8):
        mag = ((g >> np.uint64(8 * j)) & np.uint64(0xFF)).astype(np.int64)
        out[..., j] = np.where((signs >> j) & 1, -mag, mag)
    return out


def _f16(lo, hi):
    return (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8)).view(np.float16).astype(np.float64)


def dequant_int(type_, raw, N, K):
    """(weights before the fp16 super-block scale [N][K] (float64, exact: integers or multiples of 1/8), d [N][K/256],
    dmin-term [N][K]) such that weight = d * wi - dmin_term (dmin_term = 0 except Q4_K / Q2_K)."""
    bb = cd.QG_BLOCK[type_]
    nb = K // 256
    B = raw.reshape(N * nb, bb).astype(np.int64)
    wi = np.zeros((N * nb, 256), np.float64)
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
    elif type_ == cd.Q2_K:
        d, dmin = _f16(B[:, 80], B[:, 81]), _f16(B[:, 82], B[:, 83])
        for n in range(2):
            for j in range(4):
                for h in range(2):
                    sc = B[:, 8 * n + 2 * j + h]
                    base = 128 * n + 32 * j + 16 * h
                    q = (B[:, 16 + 32 * n + 16 * h:16 + 32 * n + 16 * h + 16] >> (2 * j)) & 3
                    wi[:, base:base + 16] = q * (sc & 0xF)[:, None]
                    mterm[:, base:base + 16] = (dmin * (sc >> 4))[:, None]
    elif type_ == cd.IQ2_XXS:
        d = _f16(B[:, 0], B[:, 1])
        for s in range(8):
            aux = B[:, 6 + 8 * s] | (B[:, 7 + 8 * s] << 8) | (B[:, 8 + 8 * s] << 16) | (B[:, 9 + 8 * s] << 24)
            db = (0.5 + (aux >> 28)) * 0.25
            for p in range(4):
                w8 = _grid8(IQ2XXS_GRID, B[:, 2 + 8 * s + p], _ksigns((aux >> (7 * p)) & 0x7F))
                wi[:, 32 * s + 8 * p:32 * s + 8 * p + 8] = w8 * db[:, None]
    elif type_ in (cd.IQ2_XS, cd.IQ2_S):
        d = _f16(B[:, 0], B[:, 1])
        for s in range(8):
            sc = B[:, (66 if type_ == cd.IQ2_XS else 74) + s]
            for p in range(4):
                if type_ == cd.IQ2_XS:
                    q16 = B[:, 2 + 8 * s + 2 * p] | (B[:, 3 + 8 * s + 2 * p] << 8)
                    w8 = _grid8(IQ2XS_GRID, q16 & 0x1FF, _ksigns(q16 >> 9))
                else:
                    gi = B[:, 2 + 4 * s + p] | ((B[:, 66 + s] << (8 - 2 * p)) & 0x300)
                    w8 = _grid8(IQ2S_GRID, gi, B[:, 34 + 4 * s + p])
                db = (0.5 + ((sc & 0xF) if p < 2 else (sc >> 4))) * 0.25
                wi[:, 32 * s + 8 * p:32 * s + 8 * p + 8] = w8 * db[:, None]
    elif type_ == cd.IQ3_XXS:
        d = _f16(B[:, 0], B[:, 1])
        for s in range(8):
            a = 66 + 4 * s
            aux = B[:, a] | (B[:, a + 1] << 8) | (B[:, a + 2] << 16) | (B[:, a + 3] << 24)
            db = (0.5 + (aux >> 28)) * 0.5
            for p in range(4):
                g = (IQ3XXS_GRID[B[:, 2 + 8 * s + 2 * p]].astype(np.uint64) |
                     (IQ3XXS_GRID[B[:, 3 + 8 * s + 2 * p]].astype(np.uint64) << np.uint64(32)))
                sg = _ksigns((aux >> (7 * p)) & 0x7F)
                for j in range(8):
                    mag = ((g >> np.uint64(8 * j)) & np.uint64(0xFF)).astype(np.int64)
                    wi[:, 32 * s + 8 * p + j] = np.where((sg >> j) & 1, -mag, mag) * db
    elif type_ == cd.IQ1_M:
        s16 = [B[:, 48 + 2 * k] | (B[:, 49 + 2 * k] << 8) for k in range(4)]
        dh = (s16[0] >> 12) | ((s16[1] >> 8) & 0xF0) | ((s16[2] >> 4) & 0xF00) | (s16[3] & 0xF000)
        d = dh.astype(np.uint16).view(np.float16).astype(np.float64)
        for s in range(8):
            qh16 = B[:, 32 + 2 * s] | (B[:, 33 + 2 * s] << 8)
            sc6 = (s16[s // 2] >> (6 * (s % 2))) & 63
            for p in range(4):
                qhl = (qh16 >> (4 * p)) & 0xF
                grid = IQ1S_GRID[B[:, 4 * s + p] | ((qhl & 7) << 8)].astype(np.int64)
                delta = np.where(qhl & 8, -1.125, -0.875)
                scale = 2 * ((sc6 >> (3 * (p // 2))) & 7) + 1
                for j in range(8):
                    g = (grid >> (8 * j)) & 0xF if j < 4 else (grid >> (8 * (j - 4) + 4)) & 0xF
                    wi[:, 32 * s + 8 * p + j] = (g + delta) * scale
    return wi.reshape(N, K), d.reshape(N, nb), mterm.reshape(N, K)


def _ones_scales(raw, type_):
    one = np.array([1.0], np.float16).view(np.uint8)
    B = raw.reshape(-1, cd.QG_BLOCK[type_])
    for off in cd.QG_D_OFFSETS[type_]:
        B[:, off], B[:, off + 1] = one[0], one[1]
    if type_ == cd.IQ1_M:
        cd.set_iq1m_scale(B, np.full(B.shape[0], 0x3C00, np.uint16))
    return B.reshape(-1)


@pytest.mark.parametrize("type_", cd.QG_TYPES)
@pytest.mark.parametrize("ncols", [1, 3, 4])
def test_qgemv_exact_integer_cases(oracle, type_, ncols):
    """All fp16 scales 1 and activation scales 1: the exact value is a multiple of 1/8 below 2^20, so the float
    result must equal it, except for the reference's truncating integer scale rules (IQ2 / IQ3_XXS types), where it
    is an integer within 1.25 units per sub-block of it."""
    r = cd.rng(100 + type_ + ncols)
    N, K = 64, 1024
    raw = _ones_scales(cd.random_weights(r, type_, N, K), type_)
    xq = r.integers(-8, 9, ncols * K).astype(np.int8)  # small activations keep every partial sum below 2^24
    xd = np.ones(ncols * K // 32, np.float32)
    y = oracle.qgemv(type_, raw, N, K, xq, xd, ncols)
    wi, d, mterm = dequant_int(type_, raw, N, K)
    assert np.all(d == 1.0)
    want = ((wi - mterm) @ xq.reshape(ncols, K).astype(np.float64).T).T  # [ncols][N], exact in float64
    assert np.abs(want).max() < 2 ** 20
    if type_ in TRUNCATING:
        assert np.all(y == np.round(y))
        assert np.all(np.abs(y - want) <= 1.25 * (K // 32)), np.abs(y - want).max()
        assert np.abs(y - want).max() > 0  # the truncation is really there (a float rule would match exactly)
    else:
        np.testing.assert_array_equal(y, want.astype(np.float32))


@pytest.mark.parametrize("type_", cd.QG_TYPES)
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
        wi, d, mterm = dequant_int(type_, raw, N, K)
        W = wi * np.repeat(d, 256, axis=1) - mterm
    xs = np.repeat(xd.reshape(ncols, K // 32).astype(np.float64), 32, axis=1)
    x = xq.reshape(ncols, K).astype(np.float64) * xs
    want = (W @ x.T).T
    mag = (np.abs(W) @ np.abs(x).T).T
    # each sub-block term carries a few float32 roundings (relative 2^-22 at most), the 8 W ... sums one more each;
    # the truncating types lose at most 1.25 d * dy per sub-block (a halving and a final division, both truncated)
    bound = 4e-6 * mag + 1e-30
    if type_ in TRUNCATING:
        dd = np.repeat(d, 8, axis=1)  # [N][K/32]
        bound = bound + 1.25 * (dd @ np.abs(xd.reshape(ncols, K // 32).astype(np.float64)).T).T
    assert np.all(np.abs(y - want) <= bound), np.max(np.abs(y - want) / bound)


def test_qgemv_waves_rule_matches_library(oracle, q27):
    lib = q27.lib()
    for type_ in cd.QG_BLOCK:
        for nc in (1, 2, 3, 4):
            for K in [256, 1024, 2048, 2304, 4096, 5120, 6144, 8192, 10240, 17408, 32768, 33024, 40960]:
                assert lib.q27h_qgemv_waves(type_, K, nc) == oracle.qgemv_waves(type_, K, nc), (type_, K, nc)
    Ks = (256, 2048, 2304, 5120, 8192, 17408, 32768, 33024, 40960)
    wide, narrow = [1, 1, 2, 3, 4, 9, 16, 4, 4], [1, 1, 2, 3, 4, 4, 4, 4, 4]
    assert [oracle.qgemv_waves(cd.Q4_K, K, 1) for K in Ks] == wide
    assert [oracle.qgemv_waves(cd.IQ3_S, K, 1) for K in Ks] == wide
    assert [oracle.qgemv_waves(cd.Q4_K, K, 2) for K in Ks] == wide
    assert [oracle.qgemv_waves(cd.IQ3_S, K, 2) for K in Ks] == narrow
    assert [oracle.qgemv_waves(cd.Q4_K, K, 4) for K in Ks] == narrow


def test_qgemv_rejects_bad_shapes(oracle):
    with pytest.raises(ValueError):
        oracle.qgemv(cd.Q4_K, np.zeros(144 * 4, np.uint8), 4, 256, np.zeros(256, np.int8), np.zeros(8, np.float32), 1)
