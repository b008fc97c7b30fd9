"""CPU checks of the native library: it loads, exports every function the
public headers declare, and reports a missing device as an error rather than
falling back to anything."""
import ctypes as C
import os

import numpy as np

import quantr_amd as Q


def test_library_built_and_loads():
    assert os.path.exists(Q.LIB_PATH), "run __graft_entry__.build()"
    lib = Q.load()
    assert b"gfx950" in lib.qr_version()


def test_exports_every_declared_symbol():
    lib = C.CDLL(Q.LIB_PATH)
    names = Q.declared_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_exports_nothing_else():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", Q.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    declared = set(Q.declared_symbols())
    assert exported <= declared | {"_init", "_fini"}, sorted(exported - declared)


def test_row_bytes_matches_reference_table():
    """src/quant.c:477-484 / src/model.c:20-30."""
    lib = Q.load()
    for d in (2048, 5632, 768, 1408, 300, 31):
        assert lib.qr_row_bytes(Q.TYPE_Q8_0, d) == (d // 32) * 34
        assert lib.qr_row_bytes(Q.TYPE_Q4_K, d) == (d // 256) * 144
        assert lib.qr_row_bytes(Q.TYPE_Q5_K, d) == (d // 256) * 176
        assert lib.qr_row_bytes(Q.TYPE_Q6_K, d) == (d // 256) * 210
        assert lib.qr_row_bytes(Q.TYPE_F32, d) == d * 4
    assert lib.qr_row_bytes(99, 2048) == 0


def test_argument_errors_without_device():
    """Null context and bad arguments fail with a status and a message; no
    kernel is launched."""
    lib = Q.load()
    assert lib.qr_gemv(None, Q.TYPE_Q4_K, None, None, None, 1, 256, 1) == -1
    assert b"null ctx" in lib.qr_last_error()
    ctx = C.c_void_p()
    rc = lib.qr_ctx_create(0, C.byref(ctx))
    if rc == 0:  # a GPU is present: exercise argument checks on a real context
        try:
            assert lib.qr_gemv(ctx, 99, None, None, None, 1, 256, 1) == -1
            assert lib.qr_gemv(ctx, Q.TYPE_Q4_K, None, None, None, 1, 256, 5) == -4
        finally:
            lib.qr_ctx_destroy(ctx)
    else:
        assert rc == -5, rc  # QR_ERR_NODEV
        assert ctx.value is None


def test_dropin_without_device_zero_fills():
    """With no usable GPU the drop-in follows the reference's failure
    convention: zero output and a message (src/quant.c:470-473)."""
    lib = Q.load()
    n_dev = C.c_int(0)
    lib.qr_device_count(C.byref(n_dev))
    if n_dev.value > 0:
        return
    out = np.full(8, 3.0, np.float32)
    x = np.ones(256, np.float32)
    w = np.zeros(8 * 144, np.uint8)
    lib.qr_matmul_q_fused(out.ctypes.data_as(C.c_void_p), x.ctypes.data_as(C.c_void_p),
                          w.ctypes.data_as(C.c_void_p), Q.TYPE_Q4_K, 8, 256, 1)
    assert (out == 0).all()
    assert lib.qr_gpu_available() == 0
