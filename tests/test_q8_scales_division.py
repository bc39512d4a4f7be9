"""The Q8_1 block scales in Markstein's division form (the GPU's q8_scales:
d = a / 127 with the constant RN(1/127), inv = 127 / a from a reciprocal
within 1 ulp and the remainder-corrected quotient) equal the IEEE quotients:
d for every positive float, inv for every significand with either float next
to 1 / a and over the exponents where the steps scale exactly.  Planted
mistakes (either remainder correction left out) must be caught."""
import os
import shutil
import subprocess

import pytest

SRC = os.path.join(os.path.dirname(__file__), "cpp", "q8_scales_check.c")


def _run(tmp_path, extra=()):
    exe = tmp_path / "q8_scales_check"
    # -march=native: hardware fma (the check's fmaf must be the fused, once-rounded operation,
    # which libm's software fmaf also is, only slower)
    subprocess.run(["gcc", "-O2", "-march=native", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
                    *extra, "-o", str(exe), SRC, "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600).stdout
    return {k: int(v) for k, v in (line.split() for line in out.splitlines())}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_q8_scales_equal_ieee_quotients(tmp_path):
    r = _run(tmp_path)
    assert r == {"d_bad": 0, "inv_bad": 0, "inv_exp_bad": 0}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
@pytest.mark.parametrize("plant,key", [(1, "inv_bad"), (2, "d_bad")])
def test_q8_scales_check_catches_planted_mistakes(tmp_path, plant, key):
    assert _run(tmp_path, [f"-DPLANT={plant}"])[key] > 0
