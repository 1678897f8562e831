"""The quantizer's fp16-input normalisation divides by the row's norm with one reciprocal per row and
an FMA correction per element; tests/fp16_div_check.c checks, for every fp16 numerator and every
positive fp16 denominator, that this gives the IEEE fp32 quotient bit for bit."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is needed to build the exhaustive checker")
def test_fp16_division_by_reciprocal_and_fma_is_exact(tmp_path):
    exe = str(tmp_path / "fp16_div_check")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", os.path.join(HERE, "fp16_div_check.c"), "-lm",
                    "-o", exe], check=True)
    out = subprocess.run([exe, "1"], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout
    assert "checked 2015299584 pairs" in out.stdout  # every finite fp16 a x every positive finite fp16 d
