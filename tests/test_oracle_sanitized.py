"""The CPU oracle's own tests, run against its AddressSanitizer + UndefinedBehaviorSanitizer build.

``oracle/Makefile`` builds ``oracle_asan.so`` from the same ``sdpa_oracle.c`` with
``-fsanitize=address,undefined`` (host code only: the oracle is plain C).  A child pytest loads it
(``DC_ORACLE_LIB``) with the ASan runtime preloaded, as a sanitized shared library inside an
uninstrumented interpreter needs, and runs the oracle, math-path and generator tests; any
out-of-bounds access, use after free or undefined behaviour aborts the child, and the test fails
with its report.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")


def _runtime(name):
    r = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if r.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


def test_oracle_tests_under_asan_and_ubsan():
    libasan = _runtime("libasan.so")
    if libasan is None:
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    subprocess.run(["make", "-s", "-C", ORACLE, "oracle_asan.so"], check=True)
    env = dict(os.environ)
    env["DC_ORACLE_LIB"] = os.path.join(ORACLE, "oracle_asan.so")
    env["LD_PRELOAD"] = " ".join(x for x in (libasan, os.environ.get("LD_PRELOAD", "")) if x)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
           "tests/test_oracle.py", "tests/test_oracle_math.py", "tests/test_generator_cpu.py"]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    report = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, report
    assert "passed" in r.stdout and "error" not in r.stdout.lower().split("passed")[-1], report
