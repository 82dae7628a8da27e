"""The append and gather kernels divide by launch constants (head_dim / 8,
the kv head count) with the invariant-divisor method of
air.rs_amd/csrc/kernels/fastdiv.hpp instead of an integer division per use.
tests/fastdiv_check.cpp includes that header unchanged, builds with g++ here
and compares it with the division operator on ~1.3e9 cases: every divisor
up to 300 over dense, top-of-range, multiple-boundary and random numerators,
and random divisors up to 2^32 - 1.  (Dropping the shift of n - t, or the
+ 1 of the multiplier, fails it.)"""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "air.rs_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_fast_div_equals_division():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "fastdiv_check")
        subprocess.run(["g++", "-O2", "-std=c++17", "-I", CSRC, "-o", exe, os.path.join(HERE, "fastdiv_check.cpp")],
                       check=True)
        out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
        print(out.stdout)
        assert out.returncode == 0, out.stdout
        assert " 0 differ" in out.stdout
