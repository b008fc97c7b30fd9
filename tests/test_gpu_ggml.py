"""GPU parity of the llama.cpp / ggml K-quant path (QR_GGML) with the oracle's
restatement (oracle/qr_oracle_ggml.c, pinned by closed forms in
tests/test_oracle_ggml.py; ggml itself is not in the container), bit for bit:

- qr_quantize_q8_k against quantize_row_q8_K (zero blocks, ties, negative
  extremes, large and tiny magnitudes);
- qr_dequantize of Q4_K / Q5_K / Q6_K blocks with edge-case scales;
- the GEMV against ggml_vec_dot_q*_K_q8_K at the TinyLlama layer shapes, the
  32000 x 2048 lm_head, ragged row counts, 1 and 64 blocks per row, 1 to 8
  tokens.
"""
import numpy as np
import pytest

import ggml_blocks as GB
import quantr_amd as Q
from conftest import assert_bits_equal
from quantr_amd import synth

pytestmark = pytest.mark.gpu

KT = (GB.Q4_K, GB.Q5_K, GB.Q6_K)


def test_quantize_q8_k_device(dev, oracle):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(256 * 10) * 3).astype(np.float32)
    x[256:512] = 0.0
    x[512 + 5] = -77.0
    x[768:1024] = 0.5
    x[1024:1280] *= np.float32(1e-30)
    x[1280:1536] *= np.float32(1e30)
    x[1536 + 200] = 1e38
    xb, yb = dev.upload(x), dev.alloc(292 * 10)
    dev.quantize_q8_k(xb.ptr, yb.ptr, x.size)
    got = dev.download(yb, 292 * 10, np.uint8)
    assert np.array_equal(got, oracle.quantize_q8_K(x))


@pytest.mark.parametrize("qtype", KT)
def test_dequantize_ggml(dev, oracle, qtype):
    blob, _ = GB.make_blocks(40 + qtype, qtype, 16, edge=True)
    n = 4 * 256
    sb, ob = dev.upload(blob), dev.alloc(16 * 256 * 4)
    dev.dequantize(qtype | Q.GGML, sb.ptr, 4, n, ob.ptr)
    got = dev.download(ob, 16 * 256, np.float32)
    assert_bits_equal(got, oracle.ggml_dequantize(blob, qtype, 16 * 256), "ggml dequantize")


def run(dev, qtype, W, X, n, d, nt):
    wb, xb = dev.upload(W), dev.upload(np.ascontiguousarray(X, np.float32))
    yb = dev.alloc(nt * n * 4)
    dev.gemv(qtype | Q.GGML, wb.ptr, xb.ptr, yb.ptr, n, d, nt)
    return dev.download(yb, (nt, n), np.float32)


@pytest.mark.parametrize("nt", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("qtype", KT)
@pytest.mark.parametrize("n,d", [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632),
                                 (1001, 2048), (77, 256), (5, 16384), (300, 4096), (64, 3072),
                                 (40, 1024), (13, 512)])
def test_gemv_ggml_shapes(dev, oracle, qtype, n, d, nt):
    """Every start-up: one token's activation loaded into registers (d up to
    2048: one group of 8 per thread, some threads idle below 2048; up to 4096:
    two), staged in LDS, or quantized first (d = 5632, 16384, several
    tokens)."""
    W = GB.random_rows(50 + n + d + qtype, qtype, n, d)
    X = synth.normal(60 + nt, (nt, d))
    print("ggml gemv type %d %dx%d nt %d" % (qtype, n, d, nt), flush=True)
    y = run(dev, qtype, W, X, n, d, nt)
    assert_bits_equal(y, oracle.ggml_matmul(X, W, qtype, n, d), "ggml %d %dx%d nt=%d" % (qtype, n, d, nt))


@pytest.mark.parametrize("nt", [1, 4])
@pytest.mark.parametrize("qtype", KT)
def test_gemv_ggml_lm_head(dev, oracle, qtype, nt):
    """The 32000 x 2048 lm_head at 1 token and at 4 (the width the benchmark
    reports)."""
    W = GB.random_rows(70 + qtype, qtype, 32000, 2048)
    X = synth.normal(71 + nt, (nt, 2048))
    y = run(dev, qtype, W, X, 32000, 2048, nt)
    assert_bits_equal(y, oracle.ggml_matmul(X, W, qtype, 32000, 2048), "ggml lm_head nt=%d" % nt)


@pytest.mark.parametrize("qtype", KT)
def test_gemv_ggml_edge_blocks(dev, oracle, qtype):
    """Blocks with zero, subnormal, largest and negative half scales, against
    activations with a zero block and extreme magnitudes."""
    blob, _ = GB.make_blocks(80 + qtype, qtype, 8 * 4, edge=True)
    W = blob.reshape(8, 4 * GB.BLOCK[qtype])
    X = synth.normal(81, (3, 1024))
    X[1, 256:512] = 0.0
    X[2] *= np.float32(1e3)
    y = run(dev, qtype, W, X, 8, 1024, 3)
    assert_bits_equal(y, oracle.ggml_matmul(X, W, qtype, 8, 1024), "ggml edge")


def test_gemv_ggml_refusals(dev):
    W = GB.random_rows(1, GB.Q4_K, 8, 512)
    wb, xb, yb = dev.upload(W), dev.alloc(512 * 4), dev.alloc(8 * 4)
    with pytest.raises(Q.QrError, match="ggml"):
        dev.gemv(Q.TYPE_Q8_0 | Q.GGML, wb.ptr, xb.ptr, yb.ptr, 8, 512, 1)
    with pytest.raises(Q.QrError, match="ggml"):
        dev.gemv(Q.TYPE_Q4_K | Q.GGML | Q.TILED, wb.ptr, xb.ptr, yb.ptr, 8, 512, 1)
    with pytest.raises(Q.QrError, match="integer sums"):
        acc = dev.alloc(8 * 16 * 4)
        dev.gemv(Q.TYPE_Q4_K | Q.GGML, wb.ptr, xb.ptr, yb.ptr, 8, 512, 1, acc_ptr=acc.ptr,
                 accb_ptr=acc.ptr)
