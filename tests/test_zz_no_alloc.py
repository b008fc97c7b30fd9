"""qr_moe_forward_noalloc (include/qr_hip.h) against qr_moe_forward.

The allocation-free entry point has no reference counterpart; its results
must equal the allocating entry point's bit for bit (which the other GPU tests
pin to the oracle), on consecutive calls that share the fixed per-GPU scratch
array, the second call with fewer tokens than the first.
"""
import ctypes as C

import numpy as np
import pytest

import inputs as I
import quantr_amd as Q
from conftest import assert_bits_equal
from oracle import ORDER_AVX2, ORDER_SEQ
from quantr_amd import synth

pytestmark = pytest.mark.gpu


def _layer(dev, dim, hidden, E, K, ut, dt, seed):
    ue, de = I.BLOCK[ut][0], I.BLOCK[dt][0]
    arrs = [I.activations(seed, E, dim, std=0.05),
            I.blocks(seed + 1, ut, E * hidden * (dim // ue)),
            I.blocks(seed + 2, ut, E * hidden * (dim // ue)),
            I.blocks(seed + 3, dt, E * dim * (hidden // de))]
    bufs = [dev.upload(a) for a in arrs]
    L = Q.MoeLayer(dim, hidden, E, K, *[b.ptr for b in bufs], ut, ut, dt)
    return L, bufs


def _run(dev, fn, L, x, xb, order):
    T, dim = x.shape
    K = L.n_used
    xd, xbd = dev.upload(x), dev.upload(xb)
    idx, w = dev.alloc(T * K * 4), dev.alloc(T * K * 4)
    rc = fn(dev.ctx, C.byref(L), C.c_void_p(xd.ptr), C.c_void_p(xbd.ptr), T, order,
            C.c_void_p(idx.ptr), C.c_void_p(w.ptr))
    assert rc == 0, dev.last_error()
    dev.sync()
    return (dev.download(xd, (T, dim), np.float32), dev.download(idx, (T, K), np.int32),
            dev.download(w, (T, K), np.float32))


@pytest.mark.parametrize("order", [ORDER_SEQ, ORDER_AVX2])
def test_noalloc_matches_forward_qwen3(dev, order):
    """The Qwen3-30B-A3B-shaped layer (gate/up Q4_K, down Q6_K) at T = 64
    (grouped MFMA products), then T = 16 and T = 1 on the same scratch."""
    lib = dev.lib
    dim, hidden, E, K = 2048, 768, 128, 8
    router, u, _ = synth.zipf_router(7700, E, dim)
    bufs = [dev.upload(router),
            dev.upload(synth.weights(7701, E * hidden, dim, Q.TYPE_Q4_K)),
            dev.upload(synth.weights(7702, E * hidden, dim, Q.TYPE_Q4_K)),
            dev.upload(synth.weights(7703, E * dim, hidden, Q.TYPE_Q6_K))]
    L = Q.MoeLayer(dim, hidden, E, K, *[b.ptr for b in bufs], Q.TYPE_Q4_K, Q.TYPE_Q4_K,
                   Q.TYPE_Q6_K)
    for T in (64, 16, 1):
        xb = synth.zipf_tokens(7710 + T, T, dim, u)
        x = synth.normal(7720 + T, (T, dim))
        want = _run(dev, lib.qr_moe_forward, L, x, xb, order)
        got = _run(dev, lib.qr_moe_forward_noalloc, L, x, xb, order)
        assert (got[1] == want[1]).all(), "routing indices T=%d" % T
        assert_bits_equal(got[2], want[2], "routing weights T=%d" % T)
        assert_bits_equal(got[0], want[0], "layer output T=%d" % T)


def test_noalloc_matches_forward_small_layer(dev):
    """A small layer with Q8_0 down experts in the AVX2 build's order (the
    grouped GEMV kernels), T = 40 then T = 3."""
    lib = dev.lib
    L, bufs = _layer(dev, 512, 256, 16, 4, Q.TYPE_Q4_K, Q.TYPE_Q8_0, 7800)
    for T in (40, 3):
        x = I.activations(7810 + T, T, 512)
        xb = I.activations(7820 + T, T, 512)
        want = _run(dev, lib.qr_moe_forward, L, x, xb, ORDER_AVX2)
        got = _run(dev, lib.qr_moe_forward_noalloc, L, x, xb, ORDER_AVX2)
        assert (got[1] == want[1]).all()
        assert_bits_equal(got[0], want[0], "layer output T=%d" % T)


def test_noalloc_rejects_beyond_fixed_scratch(dev):
    """A token count whose scratch exceeds the fixed array is refused before
    anything runs (QR_ERR_INVALID with a message)."""
    lib = dev.lib
    L, bufs = _layer(dev, 512, 256, 16, 4, Q.TYPE_Q4_K, Q.TYPE_Q6_K, 7900)
    T = 4096  # about 31 MB of scratch at this shape
    x, xb = dev.alloc(T * 512 * 4), dev.alloc(T * 512 * 4)
    rc = lib.qr_moe_forward_noalloc(dev.ctx, C.byref(L), C.c_void_p(x.ptr), C.c_void_p(xb.ptr),
                                    T, ORDER_SEQ, None, None)
    assert rc == -1
    assert "fixed" in dev.last_error()
