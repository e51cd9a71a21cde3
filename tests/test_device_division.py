"""Host-side proof of the device's correctly rounded amax / 127 (the q8_1 / q8_0 scale): the fma-corrected
reciprocal product is checked against the IEEE quotient for all 2^31 non-negative finite float32 values."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_div127_exhaustive(tmp_path):
    exe = tmp_path / "div127_check"
    # -ffp-contract=off keeps a * inv a separate rounding; fmaf is the correctly rounded fused multiply-add
    r = subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), os.path.join(HERE, "div127_check.c"),
                        "-lpthread", "-lm"], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail(r.stderr)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0
    assert int(out.stdout.strip()) == 0, f"{out.stdout.strip()} mismatches of the fma-corrected amax / 127"
