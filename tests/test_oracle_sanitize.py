"""CPU only: the oracle under AddressSanitizer and UndefinedBehaviorSanitizer.

`make -C oracle sanitize` builds oracle/_build/san_check from the oracle's C
sources and a driver (oracle/san_check.c) that runs every entry point once on
small ragged inputs held in buffers of their exact sizes; any out-of-bounds
access, leak or undefined operation aborts it with a sanitizer report.
"""
import os
import shutil
import subprocess

import pytest

ORACLE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_oracle_runs_clean_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-C", ORACLE, "sanitize"], check=True)
    # verify_asan_link_order=0: the sanitizer runtime need not be the first library loaded
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([os.path.join(ORACLE, "_build", "san_check")], capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ran clean" in r.stdout and "runtime error" not in r.stderr, r.stderr
