"""Host AddressSanitizer + UndefinedBehaviorSanitizer pass over the CPU oracle and over
libsxq's host code (tests/sanitize/): both are built with the sanitizers (the library's
device code as usual, its host side instrumented) and driven over their CPU paths -- the
oracle through every function on random and edge-case inputs, the C-ABI through every
argument check, error text and the thread-local error string under 8 threads.  Any
out-of-bounds access, use after free, undefined shift or overflow aborts the driver."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")


def _make(target):
    if shutil.which("make") is None:
        pytest.skip("make is not installed")
    r = subprocess.run(["make", "-s", "-j8", "-C", HERE, os.path.join(HERE, "_build", target)],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    return os.path.join(HERE, "_build", target)


def _run(exe):
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=ENV)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr


def test_oracle_under_address_and_ub_sanitizers():
    _run(_make("oracle_san"))


def test_library_host_code_under_address_and_ub_sanitizers():
    if not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc is not installed")
    _run(_make("abi_san"))
