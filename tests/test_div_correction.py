"""Exhaustive CPU proofs for the divisions of the reference-format quantizer
on the GPU, which uses one reciprocal per token row instead of an IEEE
division per element.  The stored scale's quotient takes Markstein's FMA
correction (tests/native/div_correction_check.c: equal to the IEEE quotient
bit for bit over every finite fp16 numerator and positive finite fp16 scale,
2.0e9 pairs); the reciprocal comes from the hardware estimate and a Newton
step (tests/native/rcp_newton_check.c); the per-element quotients, which
only feed round(), take one multiply (tests/native/quotient_rint_check.c)."""

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


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_quotient_by_reciprocal_rounds_to_the_same_integer(tmp_path):
    """The quantizer's per-element quotients only feed round(): the kernel
    multiplies by the row's correctly rounded reciprocal instead of dividing.
    tests/native/quotient_rint_check.c checks, over every finite fp16
    numerator and every positive finite fp16 scale, that
    rint(RN16(RN32(x * RN32(1 / s)))) -- and the same with the product
    rounded to fp16 once -- equals the reference's rint(RN16(RN32(x / s)))."""
    exe = tmp_path / "quotient_rint_check"
    src = os.path.join(HERE, "native", "quotient_rint_check.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", src, "-o", str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip() == "pairs 2015299584 mismatches 0 0"
