"""The MuonLP kernels' quotient m / sc (lp.hip, lp_codes8): Markstein's method from one
correctly rounded reciprocal equals the IEEE division on its fast-path range. Compiled from
tests/markstein_check.c with gcc; checked against C's own division on every |m| <= sc for
the scale with an all-ones mantissa just below 1.0 and on random pairs (the program takes
more scales: `markstein_check <pairs> 8` covers eight, 1.3e10 quotients)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_matches_ieee_division(tmp_path):
    exe = tmp_path / "markstein_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", str(exe),
                    os.path.join(HERE, "markstein_check.c"), "-lm"], check=True)
    out = subprocess.run([str(exe), "2000000", "1"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 mismatches" in out.stdout
