"""GPU parity of the tiled Q4_K / Q5_K / Q6_K / Q8_0 layouts (qr_weights_tile)
and their GEMV.

The tiled layout is this library's own permutation of the reference's
row-major super-blocks (no reference counterpart): a tile of 64 / nb rows
stores the k-th 16-byte chunk of each of its super-blocks together.  Checked
here:

- qr_weights_tile against the layout written out in numpy below, and
  qr_weights_untile as its exact inverse, including a short last tile;
- the GEMV over tiled weights against the oracle's matmul_q_fused
  (src/quant.c:441-523) bit for bit: the 32000 x 2048 lm_head, the TinyLlama
  layer shapes, ragged row counts, one block per row (64-row tiles) and 64
  blocks per row (one-row tiles), random block bytes with edge-case scales,
  every batch width;
- the refusals (no integer sums, no other types, d not whole super-blocks).
"""
import numpy as np
import pytest

import inputs as I
import quantr_amd as Q
from conftest import assert_bits_equal
from quantr_amd import synth

pytestmark = pytest.mark.gpu

KTYPES = (Q.TYPE_Q4_K, Q.TYPE_Q5_K)


def tiled_numpy(W, qtype, n, d):
    """The tiled layout of W ([n][nb * BB] bytes), restated from its
    definition: tile t of RB = 64 // nb rows at t * RB * nb * BB, chunk k of
    lane l (row l // nb, block l % nb of the tile) at + 16 * (k * L + l),
    L the tile's lanes."""
    bb = I.BLOCK[qtype][1]
    nb, nch = d // 256, bb // 16
    rb = 64 // nb
    blocks = W.reshape(n * nb, nch, 16)
    out = np.zeros(n * nb * bb, np.uint8)
    for t in range((n + rb - 1) // rb):
        rows = min(rb, n - t * rb)
        lanes = rows * nb
        tile = blocks[t * rb * nb: t * rb * nb + lanes]  # [lanes][nch][16]
        base = t * rb * nb * bb
        out[base: base + lanes * bb] = tile.transpose(1, 0, 2).reshape(-1)
    return out.reshape(n, nb * bb)


def run_tiled(dev, qtype, W, X, n, d, nt):
    wb, tb = dev.upload(W), dev.alloc(W.nbytes)
    dev.tile(qtype, wb.ptr, tb.ptr, n, d)
    xb = dev.upload(np.ascontiguousarray(X, np.float32))
    yb = dev.alloc(nt * n * 4)
    dev.gemv(qtype | Q.TILED, tb.ptr, xb.ptr, yb.ptr, n, d, nt)
    return dev.download(yb, (nt, n), np.float32)


@pytest.mark.parametrize("qtype", KTYPES)
@pytest.mark.parametrize("n,d", [(64, 2048), (1001, 2048), (77, 256), (5, 16384), (45, 5632)])
def test_tile_layout_and_inverse(dev, qtype, n, d):
    bb = I.BLOCK[qtype][1]
    W = I.blocks(400 + n + d + qtype, qtype, n * (d // 256)).reshape(n, (d // 256) * bb)
    wb, tb, ub = dev.upload(W), dev.alloc(W.nbytes), dev.alloc(W.nbytes)
    dev.tile(qtype, wb.ptr, tb.ptr, n, d)
    dev.tile(qtype, tb.ptr, ub.ptr, n, d, reverse=True)
    got = dev.download(tb, W.shape, np.uint8)
    assert np.array_equal(got, tiled_numpy(W, qtype, n, d))
    assert np.array_equal(dev.download(ub, W.shape, np.uint8), W)


@pytest.mark.parametrize("qtype", KTYPES)
def test_gemv_tiled_lm_head_32000(dev, oracle, qtype):
    """The 32000 x 2048 lm_head of the K-quant sweep at 1, 2, 3 and 4 tokens."""
    W = synth.weights(77 + qtype, 32000, 2048, qtype)
    for nt in (1, 2, 3, 4):
        X = synth.normal(8 + nt, (nt, 2048))
        print("tiled lm_head type %d nt %d" % (qtype, nt), flush=True)
        y = run_tiled(dev, qtype, W, X, 32000, 2048, nt)
        want = oracle.matmul_q_fused(X, W, qtype, 32000, 2048, threads=16).reshape(nt, 32000)
        assert_bits_equal(y, want, "tiled type %d nt=%d" % (qtype, nt))


@pytest.mark.parametrize("nt", [1, 4, 8])
@pytest.mark.parametrize("qtype", KTYPES)
@pytest.mark.parametrize("n,d", [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632),
                                 (1001, 2048), (333, 256), (40, 16384), (7, 4096)])
def test_gemv_tiled_shapes(dev, oracle, qtype, n, d, nt):
    """TinyLlama layer shapes (2048 x 5632: 22 blocks per row, 2-row tiles of
    44 lanes), a short last tile, 64-row tiles (d = 256), 1-row tiles
    (d = 16384), few tiles; batch 1, the verify width 4, and 8 (two launches)."""
    W = synth.weights(3000 + n + d + qtype, n, d, qtype)
    X = synth.normal(3100 + nt, (nt, d))
    print("tiled type %d %dx%d nt %d" % (qtype, n, d, nt), flush=True)
    y = run_tiled(dev, qtype, W, X, n, d, nt)
    want = oracle.matmul_q_fused(X, W, qtype, n, d, threads=16).reshape(nt, n)
    assert_bits_equal(y, want, "tiled type %d %dx%d nt=%d" % (qtype, n, d, nt))


@pytest.mark.parametrize("qtype", KTYPES)
@pytest.mark.parametrize("d", [2048, 768])
def test_gemv_tiled_random_blocks(dev, oracle, qtype, d):
    """Random block bytes plus a row of edge-case blocks (zero, subnormal,
    largest and negative half scales), 2 and 3 tokens."""
    W = I.dot_set(900 + qtype + d, qtype, 63, d)
    for nt in (2, 3):
        X = I.activations(901 + nt, nt, d)
        y = run_tiled(dev, qtype, W, X, W.shape[0], d, nt)
        want = oracle.matmul_q_fused(X, W, qtype, W.shape[0], d).reshape(nt, -1)
        assert_bits_equal(y, want, "tiled random type %d d=%d nt=%d" % (qtype, d, nt))


def test_gemv_tiled_refusals(dev):
    W = synth.weights(5, 64, 2048, Q.TYPE_Q4_K)
    wb, xb, yb = dev.upload(W), dev.alloc(2048 * 4), dev.alloc(64 * 4)
    acc, accb = dev.alloc(64 * 64 * 4), dev.alloc(64 * 4)
    with pytest.raises(Q.QrError, match="integer sums"):
        dev.gemv(Q.TYPE_Q4_K | Q.TILED, wb.ptr, xb.ptr, yb.ptr, 64, 2048, 1, acc_ptr=acc.ptr,
                 accb_ptr=accb.ptr)
    with pytest.raises(Q.QrError, match="tiled layout"):
        dev.gemv(Q.TYPE_F32 | Q.TILED, wb.ptr, xb.ptr, yb.ptr, 64, 2048, 1)
    with pytest.raises(Q.QrError, match="tiled"):
        dev.gemv(Q.TYPE_Q4_K | Q.TILED, wb.ptr, xb.ptr, yb.ptr, 64, 1408, 1)
    with pytest.raises(Q.QrError, match="tiled"):  # Q6_K tiles: n (d / 256) a multiple of 8
        dev.gemv(Q.TYPE_Q6_K | Q.TILED, wb.ptr, xb.ptr, yb.ptr, 15, 768, 1)
    with pytest.raises(Q.QrError, match="order"):  # Q8_0 tiles: the sequential order only
        dev.gemv(Q.TYPE_Q8_0 | Q.TILED, wb.ptr, xb.ptr, yb.ptr, 64, 2048, 1, order=Q.ORDER_AVX2)
    with pytest.raises(Q.QrError, match="no tiled layout"):
        dev.tile(Q.TYPE_F32, wb.ptr, yb.ptr, 64, 2048)
    with pytest.raises(Q.QrError, match="multiple of 8"):
        dev.tile(Q.TYPE_Q6_K, wb.ptr, yb.ptr, 15, 768)
    with pytest.raises(Q.QrError, match="overlap"):
        dev.tile(Q.TYPE_Q4_K, wb.ptr, wb.ptr, 64, 2048)


# ---- Q6_K and Q8_0 (qr_tiled_sq.h) -------------------------------------------
SQTYPES = (Q.TYPE_Q6_K, Q.TYPE_Q8_0)


def sq_weights(seed, qtype, n, d):
    if qtype == Q.TYPE_Q8_0:
        return I.blocks(seed, qtype, n * (d // 32)).reshape(n, (d // 32) * 34)
    return I.blocks(seed, qtype, n * (d // 256)).reshape(n, (d // 256) * 210)


@pytest.mark.parametrize("qtype,n,d", [(Q.TYPE_Q6_K, 64, 2048), (Q.TYPE_Q6_K, 1001, 2048),
                                       (Q.TYPE_Q6_K, 9, 4096), (Q.TYPE_Q6_K, 3, 16384),
                                       (Q.TYPE_Q6_K, 2048, 5632), (Q.TYPE_Q6_K, 40, 768),
                                       (Q.TYPE_Q6_K, 336, 256), (Q.TYPE_Q6_K, 12, 5632),
                                       (Q.TYPE_Q8_0, 64, 2048), (Q.TYPE_Q8_0, 1001, 2048),
                                       (Q.TYPE_Q8_0, 77, 256), (Q.TYPE_Q8_0, 45, 5632),
                                       (Q.TYPE_Q8_0, 7, 768)])
def test_tile_layout_sq_and_inverse(dev, qtype, n, d):
    """qr_weights_tile of Q6_K / Q8_0 against the layout written out from its
    definition (inputs.tile_sq), and the reverse permutation back."""
    W = sq_weights(600 + n + d + qtype, qtype, n, d)
    wb, tb, ub = dev.upload(W), dev.alloc(W.nbytes), dev.alloc(W.nbytes)
    dev.tile(qtype, wb.ptr, tb.ptr, n, d)
    dev.tile(qtype, tb.ptr, ub.ptr, n, d, reverse=True)
    got = dev.download(tb, W.nbytes, np.uint8)
    assert np.array_equal(got, I.tile_sq(W, qtype, n, d))
    assert np.array_equal(dev.download(ub, W.shape, np.uint8), W)


@pytest.mark.parametrize("nt", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("qtype,n,d", [(Q.TYPE_Q6_K, 32000, 2048), (Q.TYPE_Q6_K, 2048, 2048),
                                       (Q.TYPE_Q6_K, 256, 2048), (Q.TYPE_Q6_K, 5632, 2048),
                                       (Q.TYPE_Q6_K, 512, 2048), (Q.TYPE_Q6_K, 1001, 2048),
                                       (Q.TYPE_Q6_K, 13, 4096), (Q.TYPE_Q6_K, 7, 16384),
                                       (Q.TYPE_Q6_K, 2048, 5632), (Q.TYPE_Q6_K, 12, 5632),
                                       (Q.TYPE_Q6_K, 40, 768), (Q.TYPE_Q6_K, 336, 256),
                                       (Q.TYPE_Q6_K, 4, 1536),
                                       (Q.TYPE_Q8_0, 32000, 2048), (Q.TYPE_Q8_0, 2048, 2048),
                                       (Q.TYPE_Q8_0, 256, 2048), (Q.TYPE_Q8_0, 5632, 2048),
                                       (Q.TYPE_Q8_0, 2048, 5632), (Q.TYPE_Q8_0, 1001, 2048),
                                       (Q.TYPE_Q8_0, 333, 256), (Q.TYPE_Q8_0, 5, 768),
                                       (Q.TYPE_Q8_0, 40, 16384)])
def test_gemv_tiled_sq_shapes(dev, oracle, qtype, n, d, nt):
    """The Q6_K / Q8_0 tiled GEMV against the oracle's matmul_q_fused
    (src/quant.c:441-523; Q8_0 in the -std=c99 build's order) bit for bit:
    the sweep's shapes and lm_head, wv (512 rows), short last tiles, 64-row
    and 1-row tiles, every batch width; Q6_K tiles whose d fields start
    inside a 16-byte unit (22, 3, 1 and 6 super-blocks per row)."""
    W = synth.weights(3300 + n + d + qtype, n, d, qtype)
    X = synth.normal(3400 + nt, (nt, d))
    print("tiled sq type %d %dx%d nt %d" % (qtype, n, d, nt), flush=True)
    y = run_tiled(dev, qtype, W, X, n, d, nt)
    want = oracle.matmul_q_fused(X, W, qtype, n, d, threads=16).reshape(nt, n)
    assert_bits_equal(y, want, "tiled type %d %dx%d nt=%d" % (qtype, n, d, nt))


@pytest.mark.parametrize("qtype,d", [(Q.TYPE_Q6_K, 2048), (Q.TYPE_Q8_0, 2048),
                                     (Q.TYPE_Q8_0, 768)])
def test_gemv_tiled_sq_random_blocks(dev, oracle, qtype, d):
    """Random block bytes plus a row of edge-case blocks (zero, subnormal,
    largest and negative half scales; Q6_K's int8 scales over their whole
    range), 1 and 3 tokens."""
    W = I.dot_set(950 + qtype + d, qtype, 63, d)
    for nt in (1, 3):
        X = I.activations(951 + nt, nt, d)
        y = run_tiled(dev, qtype, W, X, W.shape[0], d, nt)
        want = oracle.matmul_q_fused(X, W, qtype, W.shape[0], d).reshape(nt, -1)
        assert_bits_equal(y, want, "tiled random type %d d=%d nt=%d" % (qtype, d, nt))


def test_gemv_tiled_sq_lm_head_151936(dev, oracle):
    """The Qwen3-30B-A3B lm_head: 151936 x 2048 Q6_K, 1 token."""
    n, d = 151936, 2048
    W = np.tile(synth.weights(3500, 4096, d, Q.TYPE_Q6_K), (n // 4096 + 1, 1))[:n].copy()
    X = synth.normal(3501, (1, d))
    y = run_tiled(dev, Q.TYPE_Q6_K, W, X, n, d, 1)
    want = oracle.matmul_q_fused(X, W, Q.TYPE_Q6_K, n, d, threads=16).reshape(1, n)
    assert_bits_equal(y, want, "tiled Q6_K lm_head")
