"""Runs the C++ host-layer tests (tests/cpp/test_theano_quantize, built by
__graft_entry__.build()): the host-only cases on the CPU, all cases on the GPU."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_theano_quantize")


def run(*args, timeout=300):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    r = subprocess.run([BIN, *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    return r.stdout


def test_cpp_host_layer_cpu_cases():
    out = run("--cpu")
    assert "26 of 26 tests passed" in out


@pytest.mark.gpu
def test_cpp_host_layer_all_cases():
    out = run()
    assert " tests passed" in out and "FAILED" not in out
