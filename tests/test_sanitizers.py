"""Host-side AddressSanitizer + UndefinedBehaviorSanitizer runs (CPU only).

`neo-theano_amd/build.py --sanitize` builds the C oracle and the C++ host layer
(allocator, storage, serialization, Module API; the C++ tests link the oracle)
with -fsanitize=address,undefined into neo-theano_amd/_build/sanitize/.  These
tests build that when it is missing or older than its sources, then run
  * the C++ host-layer tests' CPU cases, leak checks on, and
  * the Python oracle and golden tests against the sanitized oracle, with gcc's
    libasan preloaded into the interpreter (leak checks off: CPython itself
    keeps allocations until exit),
and fail on any sanitizer report.  No device code is instrumented."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "neo-theano_amd")
SAN = os.path.join(PKG, "_build", "sanitize")
EXE = os.path.join(SAN, "test_theano_quantize")
OLIB = os.path.join(SAN, "libtq_oracle.so")
SOURCES = [os.path.join(ROOT, "oracle", "tq_oracle.c"), os.path.join(ROOT, "oracle", "tq_oracle.h"),
           os.path.join(ROOT, "tests", "cpp", "test_theano_quantize.cpp")] + \
          [os.path.join(PKG, "host", f) for f in os.listdir(os.path.join(PKG, "host"))]
REPORTS = ("ERROR: AddressSanitizer", "ERROR: LeakSanitizer", "runtime error:")


@pytest.fixture(scope="module")
def sanitized():
    newest = max(os.path.getmtime(p) for p in SOURCES)
    if not all(os.path.exists(p) and os.path.getmtime(p) >= newest for p in (EXE, OLIB)):
        r = subprocess.run([sys.executable, os.path.join(PKG, "build.py"), "--sanitize"], stdout=subprocess.PIPE,
                           stderr=subprocess.STDOUT, text=True, timeout=900)
        assert r.returncode == 0, r.stdout[-4000:]
    return EXE, OLIB


def _check(r):
    out = r.stdout
    bad = [line for line in out.splitlines() if any(s in line for s in REPORTS)]
    assert r.returncode == 0 and not bad, out[-6000:]
    return out


def test_cpp_host_layer_under_asan_ubsan(sanitized):
    exe, _ = sanitized
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", TQ_GOLDEN_DIR=os.path.join(ROOT, "tests", "golden"))
    r = subprocess.run([exe, "--cpu"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600,
                       env=env)
    out = _check(r)
    assert "26 of 26 tests passed" in out


def test_oracle_under_asan_ubsan(sanitized):
    _, olib = sanitized
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], stdout=subprocess.PIPE, text=True).stdout.strip()
    if not os.path.isabs(asan):
        pytest.fail("gcc's libasan.so was not found")
    pre = os.environ.get("LD_PRELOAD", "")
    env = dict(os.environ, LD_PRELOAD=asan + (" " + pre if pre else ""), TQ_ORACLE_LIB=olib,
               ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                        os.path.join(ROOT, "tests", "test_oracle.py"), os.path.join(ROOT, "tests", "test_golden.py")],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=900, env=env, cwd=ROOT)
    out = _check(r)
    assert " passed" in out and "failed" not in out
