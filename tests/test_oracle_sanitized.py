"""The oracle's own tests, run once more against its AddressSanitizer +
UndefinedBehaviorSanitizer build (host code only: the oracle is a CPU
library).  Out-of-bounds accesses, use after free, signed overflow, invalid
shifts and misaligned loads in any oracle function those tests reach fail
the run.  (ThreadSanitizer is not used: the OpenMP runtime in this image is
not instrumented, so its reports would be about libgomp, not the oracle.)"""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_TESTS = ["test_oracle_golden.py", "test_oracle_math.py", "test_oracle_projection.py",
                "test_oracle_binning.py", "test_oracle_render.py", "test_oracle_statistics.py",
                "test_oracle_tile_modes.py", "test_oracle_error_bounds.py"]


def _runtime(name):
    out = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return out if os.path.isabs(out) and os.path.exists(out) else None


def test_oracle_tests_pass_under_asan_and_ubsan():
    asan = _runtime("libasan.so")
    if asan is None:
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "sanitized"], check=True, stdout=subprocess.DEVNULL)
    lib = os.path.join(ROOT, "oracle", "liboracle_gs3d_san.so")
    preload = " ".join(p for p in (asan, os.environ.get("LD_PRELOAD", "")) if p)
    env = dict(os.environ, LD_PRELOAD=preload, ORACLE_LIBRARY=lib,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=86",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1:exitcode=87")
    check = subprocess.run([sys.executable, "-c", "import oracle; oracle.lib(); print(oracle._LIB_PATH)"], cwd=ROOT,
                           env=env, capture_output=True, text=True)
    assert check.returncode == 0, check.stderr[-2000:]
    assert check.stdout.strip() == lib
    tests = [os.path.join(ROOT, "tests", t) for t in ORACLE_TESTS if os.path.exists(os.path.join(ROOT, "tests", t))]
    run = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
                          *tests], cwd=ROOT, env=env, capture_output=True, text=True)
    assert run.returncode == 0, (run.stdout[-3000:], run.stderr[-3000:])
