"""Host-side bounds of the device's tolerance SiLUs (csrc/q27h_device.h): `silu_lean`, the default SiLU of
gdn_conv_prefill, and `silu_tol`, its refined form (rounding term of the exp2 argument, one Newton step; build switch
Q27H_SILU_LEAN=0). The same sequence of float32 operations in numpy, with the hardware exp2 and reciprocal modelled as
the correctly rounded value moved by -1, 0 or +1 ulp, against silu in float64. The north_star's fp32 bar is 1e-5
relative; silu_lean stays within 4.1e-6 and silu_tol within 4e-7 on [-87, 87] (beyond -87, e^-|x| leaves the normal
float32 range and the exact silu is below 1e-36)."""
import numpy as np
import pytest

f32 = np.float32
L2E_HI, L2E_LO, LN2 = f32(1.44269502), f32(1.925963e-8), f32(0.693147181)


def ulp_move(a, k):
    """a moved by k ulps (k in {-1, 0, 1}) in float32."""
    a = np.ascontiguousarray(a, np.float32)
    return (a.view(np.int32) + np.int32(k) * np.where(a >= 0, 1, -1).astype(np.int32)).view(np.float32) if k else a


def silu_tol(x, exp_ulp, rcp_ulp):
    ax = np.abs(x)
    t = (ax * -L2E_HI).astype(np.float32)
    # fma(ax, -L2E_HI, -t): the exact product minus t, rounded once (float64 holds the product exactly)
    lo = (ax.astype(np.float64) * np.float64(-L2E_HI) - t.astype(np.float64)).astype(np.float32)
    lo = (lo + (ax * -L2E_LO).astype(np.float32)).astype(np.float32)
    e = ulp_move(np.exp2(t.astype(np.float64)).astype(np.float32), exp_ulp)
    e = (e.astype(np.float64) * np.float64((lo * LN2).astype(np.float32)) + e.astype(np.float64)).astype(np.float32)
    d = (f32(1) + e).astype(np.float32)
    r = ulp_move((1.0 / d.astype(np.float64)).astype(np.float32), rcp_ulp)
    nr = (-(d.astype(np.float64)) * r.astype(np.float64) + 1.0).astype(np.float32)         # fma(-d, r, 1)
    r = (nr.astype(np.float64) * r.astype(np.float64) + r.astype(np.float64)).astype(np.float32)  # fma(nr, r, r)
    num = np.where(x < 0, (e * r).astype(np.float32), r)
    return (x * num).astype(np.float32)


def silu_lean(x, exp_ulp, rcp_ulp):
    t = (np.abs(x) * -L2E_HI).astype(np.float32)
    e = ulp_move(np.exp2(t.astype(np.float64)).astype(np.float32), exp_ulp)
    d = (f32(1) + e).astype(np.float32)
    r = ulp_move((1.0 / d.astype(np.float64)).astype(np.float32), rcp_ulp)
    num = np.where(x < 0, (e * r).astype(np.float32), r)
    return (x * num).astype(np.float32)


def _inputs():
    r = np.random.default_rng(5)
    return np.concatenate([np.linspace(-87, 87, 400001, dtype=np.float32), (r.standard_normal(200000) * 4).astype(np.float32),
                           np.float32([0.0, -0.0, 1e-30, -1e-30, 2.0 ** -60, 60.0, -60.0])])


@pytest.mark.parametrize("fn,bound", [(silu_tol, 4e-7), (silu_lean, 4.1e-6)], ids=["silu_tol", "silu_lean"])
@pytest.mark.parametrize("exp_ulp", [-1, 0, 1])
@pytest.mark.parametrize("rcp_ulp", [-1, 0, 1])
def test_silu_tol_relative_error(fn, bound, exp_ulp, rcp_ulp):
    x = _inputs()
    want = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    got = fn(x, exp_ulp, rcp_ulp).astype(np.float64)
    nz = want != 0
    rel = np.abs(got[nz] - want[nz]) / np.abs(want[nz])
    assert rel.max() < bound, rel.max()
    assert np.all(got[~nz] == 0)


def test_silu_lean_error_grows_with_the_argument():
    """The lean form's error is the exp2 argument's rounding (up to |x| 2^-24 relative in e): small for small |x|,
    largest near -87, which is what the bound above covers."""
    x = _inputs()
    want = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    got = silu_lean(x, 0, 0).astype(np.float64)
    small = (np.abs(x) <= 4) & (want != 0)
    rel = np.abs(got[small] - want[small]) / np.abs(want[small])
    assert rel.max() < 5e-7, rel.max()
