"""The oracle's CPU tests with the C restatement built under AddressSanitizer
and UndefinedBehaviorSanitizer (`make -C oracle asan`): an out-of-bounds
access, use after free or undefined operation in oracle.c fails the run."""
import os
import subprocess
import sys

import pytest

from conftest import ROOT

SUITES = ["tests/test_oracle_golden.py", "tests/test_oracle_math.py", "tests/test_kvcache_convert.py"]


def test_oracle_suites_clean_under_asan_ubsan():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    rt = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(rt) or not os.path.exists(rt):
        pytest.skip("gcc ASan runtime not installed")
    env = dict(os.environ, LD_PRELOAD=rt, ORACLE_LIB=os.path.join(ROOT, "oracle", "_build", "liboracle_asan.so"),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               OMP_NUM_THREADS="4")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", *SUITES],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert "passed" in r.stdout
