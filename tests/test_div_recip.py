"""The Int8Absmax dequantisation divides through a per-row reciprocal with two corrections
(div_by_recip, mmf_device.hpp). Its C restatement, compiled here with gcc, must give the
correctly rounded quotient of every integer numerator |a| <= 2^21 for 16 divisors (the
scales' range and random normals). The GPU parity tests compare the kernels' outputs with
the oracle's division."""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not found")
def test_div_by_recip_matches_division():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "div_recip_check")
        subprocess.run(["gcc", "-O2", "-o", exe, os.path.join(HERE, "div_recip_check.c"), "-lm"], check=True)
        r = subprocess.run([exe, "16"], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stdout + r.stderr
        assert "mismatches 0" in r.stdout
