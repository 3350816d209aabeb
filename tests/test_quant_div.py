"""quant_div (cuda_inf_amd/csrc/common.h), the commit's x / scale with the
reciprocal taken once, against IEEE division over its whole input domain:
every fp16 x and the scale amax / 448 + 1e-12 of every fp16 amax (finite
and infinite), NaN inputs, and two planted mistakes that the sweep must
catch.  The sweep is tests/quant_div_check.c, compiled with gcc so that each
operation is one IEEE operation as on the GPU (2.0e9 pairs per sweep, a few
seconds on 8 threads)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_quant_div_equals_ieee_division(tmp_path):
    exe = str(tmp_path / "quant_div_check")
    cmd = ["gcc", "-O2", "-mfma", "-ffp-contract=off", "-fopenmp",
           os.path.join(HERE, "quant_div_check.c"), "-o", exe, "-lm"]
    subprocess.run(cmd, check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "finite amax x finite x: 0 mismatches" in r.stdout
