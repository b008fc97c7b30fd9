"""GPU parity of the quantized GEMV path against the oracle, through the C ABI.

Every comparison is bit-exact: int32 unit sums, activation block sums, fp32
outputs (the reference's sequential term order), the device Q8_0 quantizer,
expf, softmax and the fp32 router GEMV in each reference order.
"""
import ctypes as C

import numpy as np
import pytest

import inputs as I
import quantr_amd as Q
from conftest import assert_bits_equal, bits
from oracle import ORDER_AVX2, ORDER_AVX512, ORDER_SEQ
from quantr_amd import synth

pytestmark = pytest.mark.gpu

TYPES = (Q.TYPE_Q8_0, Q.TYPE_Q4_K, Q.TYPE_Q5_K, Q.TYPE_Q6_K)


def _run_gemv(dev, qtype, W, X, n, d, nt, with_acc=True):
    """Upload W [n][rb] and X [nt][d]; return (y [nt][n], acc [nt][n][units], accb)."""
    units = (d // 32) if qtype == Q.TYPE_Q8_0 else (d // 256) * 8
    wb = dev.upload(W)
    xb = dev.upload(np.ascontiguousarray(X, np.float32))
    yb = dev.alloc(nt * n * 4)
    acc = dev.alloc(max(nt * n * units, 1) * 4) if with_acc else None
    accb = dev.alloc(max(nt * units, 1) * 4) if with_acc else None
    dev.gemv(qtype, wb.ptr, xb.ptr, yb.ptr, n, d, nt, acc_ptr=acc.ptr if acc else None,
             accb_ptr=accb.ptr if accb else None)
    y = dev.download(yb, (nt, n), np.float32)
    if not with_acc:
        return y, None, None
    return (y, dev.download(acc, (nt, n, units), np.int32),
            dev.download(accb, (nt, units), np.int32))


def _check_gemv(dev, oracle, qtype, W, X, n, d, nt, check_acc=True):
    y, acc, accb = _run_gemv(dev, qtype, W, X, n, d, nt, with_acc=check_acc)
    want = oracle.matmul_q_fused(X, W, qtype, n, d, threads=16)
    assert_bits_equal(y, want.reshape(nt, n), "gemv type %d %dx%d nt=%d" % (qtype, n, d, nt))
    if check_acc:
        for t in range(nt):
            xq = oracle.quantize_q8_0(X[t])
            for r in range(n):
                isum, bsum = oracle.row_accum(qtype, W[r], xq, d)
                assert (acc[t, r] == isum).all(), "int sums row %d tok %d" % (r, t)
            assert (accb[t] == bsum).all(), "activation block sums tok %d" % t


@pytest.mark.parametrize("nt", [1, 4])
@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n,d", [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632)])
def test_gemv_tinyllama_shapes(dev, oracle, qtype, n, d, nt):
    """TinyLlama-1.1B layer shapes, weights N(0, 0.02) quantized, x N(0, 1), at
    batch 1 and the speculative-verify width 4 (2048 x 5632 at 4 tokens takes
    the block engine's register-staged activation path for Q4_K / Q5_K)."""
    W = synth.weights(1000 + n + d + qtype, n, d, qtype)
    X = synth.normal(7 + nt, (nt, d))
    _check_gemv(dev, oracle, qtype, W, X, n, d, nt, check_acc=(n * d <= 2048 * 2048))


@pytest.mark.parametrize("order", [ORDER_AVX2, ORDER_AVX512])
@pytest.mark.parametrize("n,d,nt", [(n, d, nt) for (n, d) in ((2048, 2048), (256, 2048),
                                                            (2048, 5632), (37, 1408))
                                    for nt in (1, 2, 4, 8) if not (d > 2048 and nt == 8)])
def test_gemv_q8_0_build_orders(dev, oracle, order, nt, n, d):
    """Q8_0 in the dot order of the -mavx2 -mfma build (8 lane accumulators,
    multiply then add, src/quant.c:245-277) and of an -mavx512f build (the
    lanes updated by fused multiply-adds): fp32 outputs and int32 unit sums
    bit-exact with the oracle, whose lane orders the reference builds pin
    (test_oracle_golden.py); one token on the streaming engine, more on the
    general kernel."""
    W = synth.weights(2000 + n + d + order, n, d, Q.TYPE_Q8_0)
    X = synth.normal(2100 + nt, (nt, d))
    units = d // 32
    wb, xb, yb = dev.upload(W), dev.upload(X), dev.alloc(nt * n * 4)
    acc, accb = dev.alloc(nt * n * units * 4), dev.alloc(nt * units * 4)
    dev.gemv(Q.TYPE_Q8_0, wb.ptr, xb.ptr, yb.ptr, n, d, nt, acc_ptr=acc.ptr, accb_ptr=accb.ptr,
             order=order)
    y = dev.download(yb, (nt, n), np.float32)
    want = oracle.matmul_q_fused(X, W, Q.TYPE_Q8_0, n, d, threads=16, order=order)
    assert_bits_equal(y, want.reshape(nt, n), "Q8_0 order %d %dx%d nt=%d" % (order, n, d, nt))
    seq = oracle.matmul_q_fused(X, W, Q.TYPE_Q8_0, n, d, threads=16, order=ORDER_SEQ)
    assert (bits(want) != bits(seq)).any(), "the orders must differ on these inputs"
    got_acc = dev.download(acc, (nt, n, units), np.int32)
    for t in range(nt):
        xq = oracle.quantize_q8_0(X[t])
        for r in range(0, n, max(1, n // 64)):
            isum, _ = oracle.row_accum(Q.TYPE_Q8_0, W[r], xq, d)
            assert (got_acc[t, r] == isum).all(), "int sums row %d tok %d" % (r, t)


@pytest.mark.parametrize("d", [2048, 768])
def test_gemv_q8_0_orders_vs_reference_builds(dev, golden, d):
    """The Q8_0 GEMV in each build's order against the dots the compiled
    reference builds wrote (tests/golden/dots.npz): -std=c99, -mavx2 -mfma and
    -mavx512f."""
    g = golden("dots.npz")
    X = I.activations(300 + d, 4, d)
    W = I.dot_set(200 + Q.TYPE_Q8_0 + d, Q.TYPE_Q8_0, 15, d)
    n = W.shape[0]
    wb, xb, yb = dev.upload(W), dev.upload(X), dev.alloc(4 * n * 4)
    for order, key in ((ORDER_SEQ, "c99"), (ORDER_AVX2, "avx2"), (ORDER_AVX512, "avx512")):
        dev.gemv(Q.TYPE_Q8_0, wb.ptr, xb.ptr, yb.ptr, n, d, 4, order=order)
        got = dev.download(yb, (4, n), np.float32).T
        assert_bits_equal(got, g["dot_%s_8_%d" % (key, d)], "Q8_0 GEMV vs %s build" % key)


@pytest.mark.parametrize("qtype", (Q.TYPE_Q4_K, Q.TYPE_Q5_K, Q.TYPE_Q6_K))
def test_gemv_lm_head_32000(dev, oracle, qtype):
    """The 32000 x 2048 lm_head of the K-quant sweep, batch 1 and 4."""
    W = synth.weights(77 + qtype, 32000, 2048, qtype)
    for nt in (1, 4):
        X = synth.normal(8 + nt, (nt, 2048))
        _check_gemv(dev, oracle, qtype, W, X, 32000, 2048, nt, check_acc=False)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("nt", [1, 2, 3, 4, 8])
def test_gemv_batch_widths(dev, oracle, qtype, nt):
    """Token counts 1..8 (speculative-verify width 4): int sums per token."""
    W = synth.weights(31 + qtype, 384, 2048, qtype)
    X = synth.normal(32 + nt, (nt, 2048))
    _check_gemv(dev, oracle, qtype, W, X, 384, 2048, nt)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("d", [2048, 768])
def test_gemv_random_blocks(dev, oracle, qtype, d):
    """Random block bytes (every nibble / fifth-bit / scale pattern) plus a row
    of edge-case blocks: zero, subnormal, largest and negative half scales."""
    W = I.dot_set(900 + qtype + d, qtype, 63, d)
    X = I.activations(901, 4, d)
    _check_gemv(dev, oracle, qtype, W, X, W.shape[0], d, 4)


@pytest.mark.parametrize("qtype,d", [(Q.TYPE_Q4_K, 1408), (Q.TYPE_Q6_K, 1408), (Q.TYPE_Q5_K, 300),
                                     (Q.TYPE_Q8_0, 1408), (Q.TYPE_Q8_0, 48), (Q.TYPE_Q4_K, 128),
                                     (Q.TYPE_Q8_0, 16)])
def test_gemv_ragged_widths(dev, oracle, qtype, d):
    """Widths that are not whole blocks: the reference keeps only whole blocks
    (src/quant.c:292, 467, 477-484) and a row shorter than one block is 0."""
    elems, bb = I.BLOCK[qtype]
    nb = d // elems
    n = 37
    W = I.blocks(5 + d, qtype, max(n * nb, 1))[: n * nb * bb].reshape(n, nb * bb)
    X = I.activations(6, 1, d)
    y, _, _ = _run_gemv(dev, qtype, W, X, n, d, 1, with_acc=False)
    want = oracle.matmul_q_fused(X, W, qtype, n, d)
    assert_bits_equal(y, want, "ragged d=%d" % d)


def test_gemv_f32_rows(dev, oracle):
    """matmul_q_fused's F32 rows (src/quant.c:448-464): sequential order."""
    W = I.activations(3, 129, 2048, std=0.02)
    X = I.activations(4, 2, 2048)
    wb, xb, yb = dev.upload(W), dev.upload(X), dev.alloc(2 * 129 * 4)
    dev.gemv(Q.TYPE_F32, wb.ptr, xb.ptr, yb.ptr, 129, 2048, 2)
    got = dev.download(yb, (2, 129), np.float32)
    want = np.stack([oracle.matmul_f32(x, W, 129, 2048, ORDER_SEQ) for x in X])
    assert_bits_equal(got, want, "F32 rows")


def test_gemv_null_weights_zero(dev):
    """NULL weights give zeros (src/quant.c:443-446)."""
    xb, yb = dev.upload(np.ones((1, 256), np.float32)), dev.upload(np.full(64, 7.0, np.float32))
    dev.gemv(Q.TYPE_Q4_K, None, xb.ptr, yb.ptr, 64, 256, 1)
    assert (dev.download(yb, 64, np.float32) == 0).all()


def test_quantize_q8_0_device(dev, oracle):
    """quantize_row_q8_0 (src/quant.c:143-158) on the device, edge rows and
    N(0, 1) rows."""
    rows = np.concatenate([I.q8_edge_rows().reshape(-1), I.activations(12, 8, 4096).reshape(-1)])
    xb = dev.upload(rows)
    yb = dev.alloc(rows.size // 32 * 34)
    dev.quantize_q8_0(xb.ptr, yb.ptr, rows.size)
    got = dev.download(yb, rows.size // 32 * 34, np.uint8)
    assert (got == oracle.quantize_q8_0(rows)).all()


@pytest.mark.parametrize("E,d", [(128, 2048), (60, 2048), (16, 2051)])
@pytest.mark.parametrize("order", [ORDER_SEQ, ORDER_AVX2, ORDER_AVX512])
def test_router_matmul(dev, oracle, E, d, order):
    """Router logits in each reference order (src/kernels.c:18-73)."""
    W = I.activations(40 + E, E, d, std=0.02)
    X = I.activations(41 + E, 16, d)
    wb, xb, yb = dev.upload(W), dev.upload(X), dev.alloc(16 * E * 4)
    dev.matmul_f32(order, wb.ptr, xb.ptr, yb.ptr, E, d, 16)
    got = dev.download(yb, (16, E), np.float32)
    want = np.stack([oracle.matmul_f32(x, W, E, d, order) for x in X])
    assert_bits_equal(got, want, "router order %d" % order)


def test_softmax_device(dev, oracle):
    """softmax_ref rows with glibc-exact expf, including ties and -inf gaps."""
    rows = [I.activations(50, 1, 128)[0] * 4, np.zeros(60, np.float32),
            np.array([1.0, 2.0, 3.0, 4.0], np.float32), I.activations(51, 1, 2048)[0] * 30]
    for r in rows:
        xb = dev.upload(r)
        dev.softmax(xb.ptr, 1, r.size)
        assert_bits_equal(dev.download(xb, r.size, np.float32), oracle.softmax(r), "softmax")


def test_expf_device_vs_libm(dev, oracle):
    """The device expf restatement against the host C library, on a stride
    through all float bit patterns plus the special values."""
    pats = np.arange(0, 2 ** 32, 251, dtype=np.uint64).astype(np.uint32)
    x = pats.view(np.float32)
    x = np.concatenate([x[~np.isnan(x)], np.array([0.0, -0.0, np.inf, -np.inf, 88.72, -103.97,
                                                   -87.3, 1e-30, -1e-30], np.float32)])
    xb, yb = dev.upload(x), dev.alloc(x.size * 4)
    dev.test_expf(xb.ptr, yb.ptr, x.size)
    assert_bits_equal(dev.download(yb, x.size, np.float32), oracle.expf(x), "expf")


# ---- drop-in host-pointer entry points (include/qr_dropin.h) ----------------
def _fp(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.mark.parametrize("qtype", TYPES + (Q.TYPE_F32,))
def test_dropin_matmul_q_fused(oracle, qtype):
    lib = Q.load()
    assert lib.qr_gpu_available() != 0
    n, d = 500, 2048
    W = (I.activations(60, n, d, std=0.02) if qtype == Q.TYPE_F32
         else synth.weights(61 + qtype, n, d, qtype))
    x = I.activations(62, 1, d)[0]
    out = np.zeros(n, np.float32)
    # The registry keys on the host address, valid while the weights live (the
    # reference's mmap lives until free_transformer): drop the copies of
    # earlier tests, whose freed arrays may share W's address.
    lib.qr_dropin_release_weights()
    try:
        # qr_dropin_init selects the reference build whose arithmetic to match
        for order in (ORDER_SEQ, ORDER_AVX2, ORDER_AVX512):
            assert lib.qr_dropin_init(0, order) == 0
            want = oracle.matmul_q_fused(x, W, qtype, n, d, order=order)
            for _ in range(2):  # second call reuses the registered device copy
                lib.qr_matmul_q_fused(_fp(out), _fp(x), _fp(W), qtype, n, d, 8)
                assert_bits_equal(out, want, "drop-in order %d" % order)
        lib.qr_matmul_q_fused(_fp(out), _fp(x), None, qtype, n, d, 8)
        assert (out == 0).all()
    finally:
        lib.qr_dropin_init(0, ORDER_AVX2)
        lib.qr_dropin_release_weights()


def test_dropin_quantize_and_ops(oracle):
    lib = Q.load()
    lib.qr_dropin_release_weights()
    x = I.activations(70, 1, 4096)[0]
    y = np.zeros(4096 // 32 * 34, np.uint8)
    lib.qr_quantize_row_q8_0(_fp(x), _fp(y), 4096)
    assert (y == oracle.quantize_q8_0(x)).all()
    W = I.activations(71, 128, 2048, std=0.02)
    xb = I.activations(72, 1, 2048)[0]
    out = np.zeros(128, np.float32)
    assert lib.qr_dropin_init(0, ORDER_AVX2) == 0
    lib.qr_ops_matmul(_fp(out), _fp(xb), _fp(W), 128, 2048, 1)
    assert_bits_equal(out, oracle.matmul_f32(xb, W, 128, 2048, ORDER_AVX2), "ops matmul")
    p = out.copy()
    lib.qr_ops_softmax(_fp(p), 128)
    assert_bits_equal(p, oracle.softmax(out), "ops softmax")


@pytest.mark.parametrize("qtype,n", [(Q.TYPE_Q4_K, 32000), (Q.TYPE_Q6_K, 4096), (Q.TYPE_Q8_0, 4096)])
def test_gemv_graph_replays(dev, qtype, n):
    """The GEMV captured into a HIP graph (as bench.py times it): four replays,
    each after an eager clear of the output and a synchronization, every one
    bit-exact with the eager launch (block engine for Q4_K, streaming engine
    for Q6_K / Q8_0)."""
    d = 2048
    W = I.blocks(9100 + qtype, qtype, n * (d // I.BLOCK[qtype][0]))
    X = I.activations(9200 + qtype, 1, d)
    wb, xb, yb = dev.upload(W), dev.upload(X), dev.alloc(n * 4)
    dev.gemv(qtype, wb.ptr, xb.ptr, yb.ptr, n, d, 1)
    want = dev.download(yb, (n,), np.float32)
    g = dev.capture(lambda: dev.gemv(qtype, wb.ptr, xb.ptr, yb.ptr, n, d, 1))
    try:
        for r in range(4):
            dev.write(yb, np.full(n, np.nan, np.float32))
            dev.sync()
            dev.graph_launch(g)
            dev.sync()
            assert_bits_equal(dev.download(yb, (n,), np.float32), want, "replay %d" % r)
    finally:
        dev.graph_destroy(g)


# ---- graph-capture contract (include/qr_hip.h) -----------------------------
def _capture_raw(dev, fn):
    """Begin capture, run fn (its exception is returned), end capture and
    destroy the graph."""
    lib = dev.lib
    assert lib.qr_capture_begin(dev.ctx) == 0
    err = None
    try:
        fn()
    except Q.QrError as e:
        err = e
    g = C.c_void_p()
    assert lib.qr_capture_end(dev.ctx, C.byref(g)) == 0, dev.last_error()
    lib.qr_graph_destroy(g)
    return err


def test_capture_refuses_allocation_and_sync(dev):
    """Calls that would allocate or synchronize refuse while capturing; the
    capture itself stays usable."""
    err = _capture_raw(dev, lambda: dev.alloc(1024))
    assert err is not None and "captured" in str(err)
    buf = dev.alloc(64)
    err = _capture_raw(dev, lambda: dev.download(buf, 16, np.float32))
    assert err is not None and "captured" in str(err)


def test_capture_null_weights_zero_fill(dev):
    """qr_gemv with NULL weights writes zeros by a kernel, so the captured
    graph zeroes y on every replay (no memset node)."""
    n, d = 300, 256
    xb = dev.upload(np.ones((2, d), np.float32))
    yb = dev.alloc(2 * n * 4)
    g = dev.capture(lambda: dev.gemv(Q.TYPE_Q4_K, None, xb.ptr, yb.ptr, n, d, 2))
    try:
        for r in range(3):
            dev.write(yb, np.full(2 * n, 5.0, np.float32))
            dev.sync()
            dev.graph_launch(g)
            dev.sync()
            assert (dev.download(yb, 2 * n, np.float32) == 0).all(), "replay %d" % r
    finally:
        dev.graph_destroy(g)


def test_capture_memset_is_a_kernel(dev):
    """qr_memset under capture records a fill kernel; replays refill."""
    buf = dev.alloc(1000)
    g = dev.capture(lambda: dev.memset(buf, 0x5A, 1000))
    try:
        for r in range(3):
            dev.write(buf, np.zeros(1000, np.uint8))
            dev.sync()
            dev.graph_launch(g)
            dev.sync()
            assert (dev.download(buf, 1000, np.uint8) == 0x5A).all()
    finally:
        dev.graph_destroy(g)


# ---- weight registry keying -------------------------------------------------
def test_registry_reuploads_changed_contents(dev):
    """An entry is reused only while the host bytes at both ends still match:
    the same address holding other weights is uploaded again."""
    lib = dev.lib
    W = np.ascontiguousarray(synth.weights(4400, 64, 256, Q.TYPE_Q4_K))
    p1 = C.c_void_p()
    assert lib.qr_weights_upload(dev.ctx, _fp(W), W.nbytes, C.byref(p1)) == 0
    p2 = C.c_void_p()
    assert lib.qr_weights_upload(dev.ctx, _fp(W), W.nbytes, C.byref(p2)) == 0
    assert p1.value == p2.value  # unchanged: reused
    W[-1, -1] ^= 0xFF  # change the last byte in place
    assert lib.qr_weights_upload(dev.ctx, _fp(W), W.nbytes, C.byref(p2)) == 0
    got = dev.download(p2.value, W.shape, np.uint8)
    assert (got == W).all()
    lib.qr_weights_release(dev.ctx, _fp(W))


def test_registry_parts_regather(dev):
    """A gathered tensor remembers its parts: the same key with other parts
    gathers again instead of returning the first gather."""
    lib = dev.lib
    parts_a = [np.full(256, i, np.uint8) for i in range(4)]
    parts_b = [np.full(256, 10 + i, np.uint8) for i in range(4)]
    key = np.zeros(1, np.uint8)
    for parts in (parts_a, parts_b):
        arr = (C.c_void_p * 4)(*[p.ctypes.data for p in parts])
        out = C.c_void_p()
        assert lib.qr_weights_upload_parts(dev.ctx, _fp(key), arr, 256, 4, C.byref(out)) == 0
        got = dev.download(out.value, 1024, np.uint8)
        assert (got == np.concatenate(parts)).all()
    lib.qr_weights_release(dev.ctx, _fp(key))


@pytest.mark.parametrize("layout", ["rows", "tiled"])
@pytest.mark.parametrize("T", [1, 2, 4, 5, 16, 37])
@pytest.mark.parametrize("qtype", TYPES)
def test_gemv_rows_mfma(dev, oracle, qtype, T, layout):
    """qr_gemv_rows (T tokens on int8 MFMA, the prefill projections' kernel):
    every token's output bit-exact with matmul_q_fused, at 1..37 tokens, on
    the TinyLlama 5632 x 2048 shape (Q6_K / Q8_0 tiles take the GEMV, so
    their tiled layout is refused here)."""
    n, d = 5632, 2048
    W = synth.weights(2000 + qtype, n, d, qtype)
    X = synth.normal(60 + T, (T, d))
    ty = qtype
    wb = dev.upload(W)
    if layout == "tiled":
        if qtype not in (Q.TYPE_Q4_K, Q.TYPE_Q5_K):
            xb, yb = dev.upload(X), dev.alloc(4 * n * T)
            with pytest.raises(Q.QrError, match="qr_gemv_rows"):
                dev.gemv_rows(qtype | Q.TILED, wb.ptr, xb.ptr, yb.ptr, n, d, T)
            return
        tb = dev.alloc(W.nbytes)
        dev.tile(qtype, wb.ptr, tb.ptr, n, d)
        wb, ty = tb, qtype | Q.TILED
    xb, yb = dev.upload(X), dev.alloc(4 * n * T)
    print("gemv_rows type %d T %d %s" % (qtype, T, layout), flush=True)
    dev.gemv_rows(ty, wb.ptr, xb.ptr, yb.ptr, n, d, T)
    got = dev.download(yb, (T, n), np.float32)
    want = oracle.matmul_q_fused(X, W, qtype, n, d, threads=16).reshape(T, n)
    assert_bits_equal(got, want, "gemv_rows type %d T=%d %s" % (qtype, T, layout))


def test_gemv_rows_lm_head_and_refusals(dev, oracle):
    """The 32000 x 2048 Q6_K lm_head at 4 tokens with strided rows; Q8_0 in a
    lane order and ggml layouts are refused."""
    n, d, T = 32000, 2048, 4
    W = synth.weights(77, n, d, Q.TYPE_Q6_K)
    X = synth.normal(78, (T, d + 64))
    wb, xb, yb = dev.upload(W), dev.upload(X), dev.alloc(4 * (n + 8) * T)
    dev.gemv_rows(Q.TYPE_Q6_K, wb.ptr, xb.ptr, yb.ptr, n, d, T, xstride=d + 64, ystride=n + 8)
    got = dev.download(yb, (T, n + 8), np.float32)[:, :n]
    want = oracle.matmul_q_fused(np.ascontiguousarray(X[:, :d]), W, Q.TYPE_Q6_K, n, d,
                                 threads=16).reshape(T, n)
    assert_bits_equal(got, want, "gemv_rows lm_head")
    W8 = synth.weights(79, 256, d, Q.TYPE_Q8_0)
    w8 = dev.upload(W8)
    with pytest.raises(Q.QrError, match="lane order"):
        dev.gemv_rows(Q.TYPE_Q8_0, w8.ptr, xb.ptr, yb.ptr, 256, d, T, xstride=d + 64,
                      order=ORDER_AVX2)
    with pytest.raises(Q.QrError, match="qr_gemv_rows"):
        dev.gemv_rows(Q.TYPE_Q4_K | Q.GGML, wb.ptr, xb.ptr, yb.ptr, 256, d, T, xstride=d + 64)
