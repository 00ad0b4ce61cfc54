"""The gating kernels divide by 6 with a reciprocal product and one fma
correction instead of an IEEE division (pom_amd/csrc/common.h, hsig).  This
CPU test runs the exhaustive check that the two agree on every fp32 value the
hardsigmoid can divide (tests/native/hsig_div6_check.c), so the kernels'
hardsigmoid equals torch's relu6(z + 3) / 6 bit for bit."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fma_corrected_division_by_six_is_exact(tmp_path):
    exe = str(tmp_path / "div6")
    src = os.path.join(HERE, "native", "hsig_div6_check.c")
    subprocess.run(["gcc", "-O2", "-march=native", "-o", exe, src, "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout
    assert "0 mismatches" in r.stdout
