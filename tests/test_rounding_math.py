"""The f32 arithmetic of the quantize coders, checked on the CPU.

The device coders replace f64 division by f32 steps: a candidate biased 2^-12
below the half-way points plus one exact-residual correction for the integer
codes (`rhaz_div`, `code_i8_row`; reference rounding: quantize.rs:8-19, round
half away from zero of the f64 quotient), and x * (1/s) with one fma correction
for the FP8 quotient (`FmtFp8::Row::quot`, against IEEE x / s).  tests/cpp/
rounding_check.c restates those expressions for the host and compares them with
the exact results over random rows, constructed ties +-3 ulp, f16-subnormal INT4
scales, specials, and a stride through every f32 of [0, 449 s] for 12 FP8
scales.  The GPU tests check the kernels themselves against the oracle.
"""
import os
import shutil
import subprocess

import pytest

SRC = os.path.join(os.path.dirname(__file__), "cpp", "rounding_check.c")
CLANG = "/opt/rocm/llvm/bin/clang"  # _Float16 on the host (the INT4 f16 scales)


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    if not os.path.exists(CLANG):
        pytest.skip("ROCm clang not found")
    out = str(tmp_path_factory.mktemp("rounding") / "rounding_check")
    subprocess.run([CLANG, "-O2", "-ffp-contract=off", "-fno-fast-math", SRC, "-o", out, "-lm"], check=True)
    return out


def test_coders_match_exact_rounding(exe):
    r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
    assert " 0 differ" in r.stdout


def test_smaller_bias_is_caught(exe):
    # the check has the power to see a bias too small for the product's rounding error
    r = subprocess.run([exe, "0x1p-20"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert r.returncode != 0, r.stdout
