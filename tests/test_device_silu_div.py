"""Host check of the device's silu quotient (`div_silu` in csrc/q27h_device.h: the IEEE division's steps with one
residual correction) against the IEEE quotient x / (1 + e^-x) over silu's fast range 2^-60 <= |x| <= 60, with the
hardware reciprocal modelled as the correctly rounded value moved by -1, 0 or +1 ulp, and the two-correction IEEE
sequence beside it. Both forms give x / d for every x, except x = 2^-23 (d = 2 - 2^-23) when the reciprocal is one ulp
off, where both are off by one ulp. Every float of the range is checked (3.3e9 cases, about 15 s on 8 cores);
Q27_SILU_DIV_STRIDE=n takes every n-th float instead (every float of [2^-26, 2^-20] is always included)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_silu_division_one_correction(tmp_path):
    exe = tmp_path / "silu_div_check"
    r = subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), os.path.join(HERE, "silu_div_check.c"),
                        "-lpthread", "-lm"], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail(r.stderr)
    stride = os.environ.get("Q27_SILU_DIV_STRIDE", "1")
    out = subprocess.run([str(exe), stride, "8"], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr
    res = {}
    for line in out.stdout.strip().splitlines():
        form, k, n, x = line.split()
        res[(form, int(k))] = (int(n), float.fromhex(x))
    for form in ("one", "two"):
        assert res[(form, 0)][0] == 0, f"{form}: mismatches with the correctly rounded reciprocal: {res[(form, 0)]}"
        for k in (-1, 1):
            n, x = res[(form, k)]
            # the only exception: x = 2^-23
            assert n == 1 and x == 2.0 ** -23, f"{form}, reciprocal {k:+d} ulp: {n} mismatches, first x = {x}"
