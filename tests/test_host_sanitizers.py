"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only, no GPU).

`tests/asan/Makefile` builds two check programs with every host-side `-fsanitize=` applied:
- `oracle_checks`: the oracle's C restatement (`oracle/selection.c`) on exact-size heap buffers over
  its edge cases (partial blocks, k at and above the frame size, signed zeros, inf, NaN, ties,
  probe chunking, every key-set mode and rejected parameters);
- `host_checks`: the C-ABI library's host code (its sources, device code compiled but never
  launched), driving every entry's argument validation, size queries, error messages and fault
  injection: paths that end before any HIP call.
A sanitizer finding aborts the program with a report; the test fails on it or on any failed check.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN_DIR = os.path.join(ROOT, "tests", "asan")


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    if not (shutil.which("gcc") and os.path.exists("/opt/rocm/bin/hipcc") and os.path.exists(ASAN_DIR)):
        pytest.skip("gcc, hipcc or tests/asan missing")
    out = tmp_path_factory.mktemp("asan")
    r = subprocess.run(["make", "-j8", "-C", ASAN_DIR, f"O={out}"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return out


def _run(path):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    env.pop("SAF3R_FAULT_INJECT", None)
    return subprocess.run([str(path)], capture_output=True, text=True, timeout=300, env=env)


def test_oracle_c_under_sanitizers(built):
    r = _run(built / "oracle_checks")
    assert r.returncode == 0 and "oracle checks passed" in r.stdout, r.stdout + r.stderr
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr


def test_library_host_validation_under_sanitizers(built):
    r = _run(built / "host_checks")
    assert r.returncode == 0 and "host checks passed" in r.stdout, r.stdout + r.stderr
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
