"""Pins of the oracle's Gated-DeltaNet recurrence (q27o_gdn_step, CPU only).

The reference ships no vectors for gdn_step (src/ops.cu:449-572); the oracle is pinned by a float64 numpy
recurrence of the delta rule (catches a dropped term, a swapped q / k, a wrong head mapping or a transposed
state), exact one-hot cases (k = e_j, q = e_m make every sum a single term, so the float32 result is known to the
bit and a wrong row / column index fails), the decay-only identities (beta = 0 and g = 0), the reference's plane
semantics (snapshots, flip) and the decode == prefill identity (one token at a time gives the same bits as the
whole sequence in one flip call, as the per-token update does not depend on how tokens are batched).
"""
import numpy as np
import pytest

import cfgdata as cd


def f64_recurrence(x, stride, g, beta, S0, H, HK, T, scale):
    """Delta rule in float64: S [H][col][i]; returns o [T][H][128] and the state after every token."""
    S = S0.astype(np.float64).reshape(H, 128, 128).copy()
    x = x.astype(np.float64).reshape(T, stride)
    kh = np.arange(H) % HK
    outs, states = [], []
    for t in range(T):
        q = x[t, : HK * 128].reshape(HK, 128)[kh]
        k = x[t, HK * 128: 2 * HK * 128].reshape(HK, 128)[kh]
        v = x[t, 2 * HK * 128: 2 * HK * 128 + H * 128].reshape(H, 128)
        gv = np.exp(g.astype(np.float64).reshape(T, H)[t])[:, None]
        bv = beta.astype(np.float64).reshape(T, H)[t][:, None]
        kv = np.einsum("hci,hi->hc", S, k)
        delta = (v - gv * kv) * bv
        S = gv[:, :, None] * S + delta[:, :, None] * k[:, None, :]
        outs.append(np.einsum("hci,hi->hc", S, q) * scale)
        states.append(S.copy())
    return np.stack(outs), states


def run(oracle, x, stride, g, beta, planes, in_plane, H, HK, T, snapshots, flip, scale=1.0 / np.sqrt(128.0)):
    return oracle.gdn_step(x, x[HK * 128:], x[2 * HK * 128:], stride, g, beta, planes, in_plane, H, HK, T,
                           np.float32(scale), snapshots, flip)


@pytest.mark.parametrize("in_plane", [0, 2, 3])
def test_decode_snapshots_float64_bound(oracle, in_plane):
    H, HK, T = 6, 2, 4
    r = cd.rng(10 + in_plane)
    x, stride, g, beta, planes = cd.gdn_inputs(r, T, H, HK)
    scale = 1.0 / np.sqrt(128.0)
    o, P = run(oracle, x, stride, g, beta, planes, in_plane, H, HK, T, True, False)
    S0 = planes.reshape(4, -1)[in_plane]
    o64, st64 = f64_recurrence(x, stride, g, beta, S0, H, HK, T, scale)
    o = o.reshape(T, H, 128)
    assert np.abs(o - o64).max() <= 1e-5 * np.abs(o64).max()
    P = P.reshape(4, H, 128, 128)
    for t in range(T):
        assert np.abs(P[t] - st64[t]).max() <= 1e-5 * np.abs(st64[t]).max(), f"snapshot plane {t}"


def test_prefill_float64_bound(oracle):
    H, HK, T = 4, 2, 200
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(20), T, H, HK)
    o, P = run(oracle, x, stride, g, beta, planes, 1, H, HK, T, False, True)
    o64, st64 = f64_recurrence(x, stride, g, beta, planes.reshape(4, -1)[1], H, HK, T, 1.0 / np.sqrt(128.0))
    o = o.reshape(T, H, 128)
    for t in range(T):
        assert np.abs(o[t] - o64[t]).max() <= 1e-5 * np.abs(o64[t]).max() + 1e-7, f"token {t}"
    P = P.reshape(4, H, 128, 128)
    assert np.abs(P[0] - st64[-1]).max() <= 1e-5 * np.abs(st64[-1]).max()
    assert np.array_equal(P[1:], planes.reshape(4, H, 128, 128)[1:])  # only the other plane of {0, 1} is written


def test_one_hot_exact(oracle):
    """k = e_j and q = e_m per head: kv = S[j][col], only row j changes, o = S'[m][col] * scale, all in float32."""
    H, HK, T = 4, 2, 3
    r = cd.rng(30)
    x, stride, g, beta, planes = cd.gdn_inputs(r, T, H, HK)
    xs = x.reshape(T, stride)
    js, ms = {}, {}
    for t in range(T):
        for kh in range(HK):
            j, m = int(r.integers(128)), int(r.integers(128))
            js[t, kh], ms[t, kh] = j, m
            xs[t, kh * 128:(kh + 1) * 128] = 0
            xs[t, kh * 128 + m] = 1
            xs[t, (HK + kh) * 128:(HK + kh + 1) * 128] = 0
            xs[t, (HK + kh) * 128 + j] = 1
    scale = np.float32(0.125)
    o, P = oracle.gdn_step(x, x[HK * 128:], x[2 * HK * 128:], stride, g, beta, planes, 3, H, HK, T, scale, True, False)
    S = planes.reshape(4, H, 128, 128)[3].copy()
    o = o.reshape(T, H, 128)
    for t in range(T):
        for h in range(H):
            j, m = js[t, h % HK], ms[t, h % HK]
            gv = np.float32(oracle.expf(float(g[t * H + h])))
            bv = beta[t * H + h]
            v = xs[t, 2 * HK * 128 + h * 128: 2 * HK * 128 + (h + 1) * 128]
            kv = S[h, :, j].copy()
            delta = (v - gv * kv) * bv
            S[h] = gv * S[h]
            S[h, :, j] += delta
            assert np.array_equal(o[t, h], S[h, :, m] * scale), (t, h)
        if t < T - 1:
            assert np.array_equal(P.reshape(4, H, 128, 128)[t], S), f"snapshot {t}"
    assert np.array_equal(P.reshape(4, H, 128, 128)[T - 1], S)


def test_decay_only(oracle):
    """beta = 0: S <- e^g S exactly; g = 0 as well: the state is unchanged and o = S^T q * scale."""
    H, HK, T = 2, 1, 2
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(40), T, H, HK)
    beta[:] = 0
    _, P = run(oracle, x, stride, g, beta, planes, 0, H, HK, T, True, False)
    S = planes.reshape(4, -1)[0]
    for t in range(T):
        S = np.float32([oracle.expf(float(g[t * H + h])) for h in range(H)]).repeat(128 * 128) * S
        assert np.array_equal(P.reshape(4, -1)[t], S)
    g[:] = 0
    o, P = run(oracle, x, stride, g, beta, planes, 0, H, HK, T, False, False)
    assert np.array_equal(P.reshape(4, -1)[T - 1], planes.reshape(4, -1)[0])
    o64, _ = f64_recurrence(x, stride, g, beta, planes.reshape(4, -1)[0], H, HK, T, 1.0 / np.sqrt(128.0))
    assert np.abs(o.reshape(T, H, 128) - o64).max() <= 1e-6 * np.abs(o64).max()


def test_plane_semantics_without_snapshots(oracle):
    H, HK, T = 2, 1, 3
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(50), T, H, HK)
    _, Ps = run(oracle, x, stride, g, beta, planes, 1, H, HK, T, True, False)
    _, Pn = run(oracle, x, stride, g, beta, planes, 1, H, HK, T, False, False)
    Ps, Pn, P0 = (a.reshape(4, -1) for a in (Ps, Pn, planes))
    assert np.array_equal(Pn[T - 1], Ps[T - 1])        # same final state, plane T - 1
    assert np.array_equal(Pn[0], P0[0]) and np.array_equal(Pn[1], P0[1]) and np.array_equal(Pn[3], P0[3])


def test_prefill_equals_chained_decode(oracle):
    H, HK, M = 3, 1, 37
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(60), M, H, HK)
    o_pf, P_pf = run(oracle, x, stride, g, beta, planes, 1, H, HK, M, False, True)
    P = planes.copy()
    P.reshape(4, -1)[0] = P.reshape(4, -1)[1]
    outs = []
    for t in range(M):  # decode T = 1, in plane 0, result to plane T - 1 = 0
        xt = x.reshape(M, stride)[t].copy()
        o, P = run(oracle, xt, stride, g.reshape(M, H)[t].copy(), beta.reshape(M, H)[t].copy(), P, 0, H, HK, 1, False,
                   False)
        outs.append(o)
    assert np.array_equal(o_pf, np.concatenate(outs))
    assert np.array_equal(P_pf.reshape(4, -1)[0], P.reshape(4, -1)[0])


def test_rejects_bad_shapes(oracle):
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(70), 5, 2, 1)
    with pytest.raises(ValueError):
        run(oracle, x, stride, g, beta, planes, 0, 2, 1, 5, True, False)   # T > 4 without flip: 4 planes only
    o, P = run(oracle, x, stride, g, beta, planes, 0, 2, 1, 0, False, True)
    assert o.size == 0 and np.array_equal(P, planes)
