import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "neo-theano_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libtq.so")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def tq():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import theano_quantize

    theano_quantize._abi.lib()
    return theano_quantize


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda", 0)


def assert_close(got, ref, rtol=1e-3, atol=1e-4, what=""):
    """|got - ref| <= atol + rtol * |ref| elementwise."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    if bad.any():
        i = np.unravel_index(np.argmax(err - (atol + rtol * np.abs(ref))), ref.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {ref.size} outside tolerance; worst at {i}: "
            f"got {got[i]!r} ref {ref[i]!r}")


def ieee_equal(a, b):
    """Bitwise-equal except that +0 == -0 and NaN == NaN (IEEE == plus NaN)."""
    a = np.asarray(a)
    b = np.asarray(b)
    return bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))
