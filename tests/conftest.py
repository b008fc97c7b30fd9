"""Shared fixtures.

CPU tests (``-m "not gpu"``) check the oracle against the reference's golden
vectors and closed forms, the host-side code, and that libqr_hip.so loads and
exports its C ABI.  GPU tests (``-m gpu``) run the HIP kernels through the C ABI
and compare them with the oracle; they never skip for lack of the native
library -- a missing build or device is an error.
"""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "quantr-in-c_amd"), os.path.join(REPO, "oracle"),
          os.path.join(REPO, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and runs HIP kernels")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def golden():
    def load(name):
        return np.load(os.path.join(REPO, "tests", "golden", name), allow_pickle=False)
    return load


@pytest.fixture(scope="session")
def dev():
    import quantr_amd
    d = quantr_amd.Device(0)
    yield d
    d.close()


def bits(a):
    """float32 array -> uint32 bit patterns (for bit-exact comparisons)."""
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits_equal(got, want, what=""):
    g, w = bits(got), bits(want)
    if g.shape != w.shape:
        raise AssertionError("%s: shape %s vs %s" % (what, g.shape, w.shape))
    bad = np.flatnonzero(g.ravel() != w.ravel())
    if bad.size:
        i = bad[0]
        raise AssertionError("%s: %d of %d values differ; first at %d: got %r want %r" % (
            what, bad.size, g.size, i, np.ravel(got)[i], np.ravel(want)[i]))
