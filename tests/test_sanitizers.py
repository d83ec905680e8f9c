"""AddressSanitizer + UndefinedBehaviorSanitizer runs of the host code (CPU
only): the oracle driven through every exit and filter, and the C ABI
layer's validation, workspace sizing and PRNG (llz_api.cpp built with the
sanitizers on the host side).  Builds with tests/sanitize/Makefile."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")


@pytest.fixture(scope="module")
def built():
    if shutil.which("gcc") is None or shutil.which("g++") is None:
        pytest.skip("no host compiler")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "llama.zig_amd")], check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    subprocess.run(["make", "-s", "-C", SAN], check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    return SAN


def _run(path, leaks: bool):
    env = dict(os.environ, ASAN_OPTIONS=f"detect_leaks={1 if leaks else 0}:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([path], env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    return r.stdout


def test_oracle_under_sanitizers(built):
    assert "ok" in _run(os.path.join(built, "build", "oracle_san"), leaks=True)


def test_host_abi_under_sanitizers(built):
    # the HIP runtime itself is not instrumented: leak reports stay off
    assert "ok" in _run(os.path.join(built, "build", "host_san"), leaks=False)
