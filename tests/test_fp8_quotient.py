"""The fp8 append's codes (F8E4M3::from_f32 of x / scale, src/fp8.rs:54-91)
are computed on the GPU from a Markstein-corrected reciprocal product instead
of a division per element (air.rs_amd/csrc/kernels/codecs.hpp fp8_code).
tests/fp8_quotient_check.c compares the two on 2e7 random and boundary cases
(random fractions of random absmax values, subnormal elements, quotients at
the smallest subnormal and at the encoder's half-up mantissa boundaries,
every code range, groups holding an infinity, and quotients exactly at the
zero rounding boundary 2^-150); built with gcc here, on the CPU, whose f32
arithmetic and fma round as the GPU's do.  Skipping the correction step makes
codes at the mantissa boundaries differ.  The exact division the GPU keeps
for quotients that come out subnormal or zero guards the sign of a quotient
at the zero boundary, and groups holding an infinity divide."""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fp8_codes_product_equals_division():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "fp8_quotient_check")
        subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-o", exe,
                        os.path.join(HERE, "fp8_quotient_check.c"), "-lm"], check=True)
        out = subprocess.run([exe, "20000000"], capture_output=True, text=True, timeout=300)
        print(out.stdout)
        assert out.returncode == 0, out.stdout
        assert "0 differ" in out.stdout
