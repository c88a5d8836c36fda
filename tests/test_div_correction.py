"""The reference-format quantizer on the GPU divides each fp16 value by its
row's scale with one reciprocal per row and Markstein's FMA correction per
element instead of an IEEE division per element.  This test compiles
tests/native/div_correction_check.c with gcc and checks, over every finite
fp16 numerator and every positive finite fp16 scale (2.0e9 pairs), that the
corrected quotient equals the IEEE quotient bit for bit."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_markstein_correction_equals_ieee_division(tmp_path):
    exe = tmp_path / "div_correction_check"
    src = os.path.join(HERE, "native", "div_correction_check.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", src, "-o", str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip() == "pairs 2015299584 mismatches 0"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_reciprocal_newton_step_is_correctly_rounded(tmp_path):
    """The per-row reciprocal RN(1 / s) the correction above needs comes from
    the hardware reciprocal (within one ulp) and one FMA Newton step:
    tests/native/rcp_newton_check.c checks every positive finite fp16 s with
    each starting value within one ulp."""
    exe = tmp_path / "rcp_newton_check"
    src = os.path.join(HERE, "native", "rcp_newton_check.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", src, "-o", str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip() == "cases 95229 mismatches 0"
