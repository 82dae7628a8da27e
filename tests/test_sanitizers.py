"""The host-side C++ (allocator, sequence manager, swap manager: the C ABI's
host half) and the C oracle under AddressSanitizer + UndefinedBehaviorSanitizer.

Both are rebuilt with -fsanitize=address,undefined (g++ / gcc, no GPU code:
`make -C air.rs_amd asan`, `make -C oracle asan`), and the CPU suites that
drive them -- the reference's allocator and swap tests with the random
differential test, the oracle's codec / attention / kv_compress tests and
the c1 digests -- run in a child Python with libasan preloaded and the
sanitized libraries selected (AIRKV_HOST_LIB, AIRKV_ORACLE_LIB).  Any
sanitizer report ends the child with a non-zero status (UBSan does not
recover).  CPU only."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SUITES = ["tests/test_host_allocator.py", "tests/test_oracle_attention.py", "tests/test_oracle_codecs.py",
          "tests/test_oracle_kv_compress.py", "tests/test_golden_c1.py", "tests/test_wire_frames.py"]


def _libasan():
    try:
        p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                           check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return None
    return p if os.path.isabs(p) and os.path.exists(p) else None


def test_host_code_and_oracle_under_asan_ubsan():
    libasan = _libasan()
    if libasan is None:
        pytest.skip("gcc's libasan is not installed")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "air.rs_amd"), "asan"], check=True)
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": libasan,
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:exitcode=86",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1:exitcode=87",
        "AIRKV_HOST_LIB": os.path.join(ROOT, "air.rs_amd", "airkv", "libairkv_host_asan.so"),
        "AIRKV_ORACLE_LIB": os.path.join(ROOT, "oracle", "libairkv_oracle_asan.so"),
    })
    # -s: a sanitizer report goes to stderr, which pytest's capture would drop
    # when the child exits from inside the report
    r = subprocess.run([sys.executable, "-m", "pytest", *SUITES, "-q", "-s", "-x", "-p", "no:cacheprovider",
                        "-m", "not gpu"], cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert " passed" in r.stdout, tail
