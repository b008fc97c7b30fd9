"""The library's scalar numerics (quantr-in-c_amd/csrc/qr_common.h, the same
source the gfx950 kernels compile) built for the host and checked against the C
library and the oracle: expf on all 2^32 inputs, the fp16 helpers on all codes."""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import REPO

LIB = os.path.join(REPO, "tests", "native", "libexpf_check.so")


@pytest.fixture(scope="module")
def hostlib():
    if not os.path.exists(LIB):
        pytest.fail("tests/native/libexpf_check.so missing: run __graft_entry__.build()")
    L = C.CDLL(LIB)
    L.qrh_expf_mismatches.restype = C.c_longlong
    L.qrh_expf_mismatches.argtypes = [C.c_uint32, C.c_uint64, C.c_uint32, C.POINTER(C.c_uint32)]
    L.qrh_h2f_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
    L.qrh_f2h_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
    return L


def test_expf_all_inputs_match_libm(hostlib):
    """Every float bit pattern (NaNs skipped): the restated expf returns the
    host libm's bits -- the function the reference calls."""
    first = C.c_uint32()
    bad = hostlib.qrh_expf_mismatches(0, 1 << 32, 1, C.byref(first))
    assert bad == 0, "first mismatch at 0x%08x" % first.value


def test_fp16_helpers_all_codes(hostlib, oracle):
    codes = np.arange(65536, dtype=np.uint16)
    got = np.empty(65536, np.float32)
    hostlib.qrh_h2f_batch(codes.ctypes.data, got.ctypes.data, 65536)
    assert (got.view(np.uint32) == oracle.h2f_bits(codes)).all()
    rng = np.random.default_rng(9)
    f = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    h = np.empty(f.size, np.uint16)
    hostlib.qrh_f2h_batch(f.ctypes.data, h.ctypes.data, f.size)
    want_h = np.array([oracle.f2h(v) for v in f[:20000]], np.uint16)
    assert (h[:20000] == want_h).all()
