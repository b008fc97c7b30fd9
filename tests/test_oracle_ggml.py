"""Pins of the oracle's llama.cpp / ggml K-quant restatement (qr_oracle_ggml.c).

ggml itself is not in the container and the reference (bharqav/quantr-in-c)
has its own K-quant layouts, so these functions are pinned by closed forms
only (no golden vectors from ggml: "parity unpinned" against ggml itself):

- the half conversion against numpy's IEEE binary16 on all 65,536 codes;
- the 12-byte scale/min packing round trip (packer written from the layout,
  tests/ggml_blocks.py, separately from the oracle's get_scale_min_k4);
- dequantize_row of blocks built from chosen fields against those fields
  ((d sc) q - (dmin m) in float32, Q6_K (d sc)(q - 32));
- quantize_row_q8_K: the largest-magnitude element maps to -127, every
  element is within half a step, bsums are the 16-element sums, an all-zero
  block has d = 0;
- the dots' integer parts (the 8 lane sums and the bsums-by-mins sum) against
  brute force over the fields, and the float dot against a float64
  dequantize-then-dot.
"""
import numpy as np
import pytest

import ggml_blocks as GB


@pytest.fixture(scope="module")
def o():
    from oracle import Oracle
    return Oracle()


def test_h2f_all_codes(o):
    codes = np.arange(65536, dtype=np.uint16)
    got = o.ggml_h2f_bits(codes)
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan], want[~nan].view(np.uint32))
    assert np.isnan(got.view(np.float32)[nan]).all()


def test_scale_min_round_trip(o):
    rng = np.random.default_rng(3)
    for _ in range(200):
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        gs, gm = o.ggml_scale_min(GB.pack_scales12(sc, mn))
        assert np.array_equal(gs, sc) and np.array_equal(gm, mn)


@pytest.mark.parametrize("qtype", [GB.Q4_K, GB.Q5_K, GB.Q6_K])
def test_dequantize_against_fields(o, qtype):
    blob, f = GB.make_blocks(10 + qtype, qtype, 12, edge=True)
    got = o.ggml_dequantize(blob, qtype, 12 * 256)
    want = GB.dequant_expected(qtype, f)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _q8k_fields(q):
    d = np.frombuffer(q[0:4].tobytes(), np.float32)[0]
    qs = q[4:260].view(np.int8).astype(np.int64)
    bs = np.frombuffer(q[260:292].tobytes(), np.int16).astype(np.int64)
    return d, qs, bs


def test_quantize_q8_K_properties(o):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(256 * 6).astype(np.float32) * np.float32(3.0)
    x[256:512] = 0.0                 # an all-zero block
    x[512 + 17] = np.float32(-50.0)  # a negative extreme
    x[768:1024] = np.float32(0.25)   # ties everywhere: the first one sets the sign
    q = o.quantize_q8_K(x)
    for b in range(6):
        d, qs, bs = _q8k_fields(q[292 * b: 292 * (b + 1)])
        xb = x[256 * b: 256 * (b + 1)].astype(np.float64)
        assert np.array_equal(bs, qs.reshape(16, 16).sum(axis=1))
        if not np.any(xb):
            assert d == 0 and not qs.any()
            continue
        imax = int(np.argmax(np.abs(xb)))  # the first of the largest magnitudes
        assert qs[imax] == -127
        assert np.sign(d) == -np.sign(xb[imax])
        assert qs.max() <= 127 and qs.min() >= -128
        err = np.abs(xb - float(d) * qs)
        assert (err <= abs(float(d)) * 0.5 * (1 + 1e-5) + 1e-12).all()


@pytest.mark.parametrize("qtype", [GB.Q4_K, GB.Q5_K, GB.Q6_K])
def test_dot_integer_parts_and_closed_form(o, qtype):
    nb = 6
    blob, f = GB.make_blocks(20 + qtype, qtype, nb)
    rng = np.random.default_rng(30 + qtype)
    x = rng.standard_normal(256 * nb).astype(np.float32)
    q = o.quantize_q8_K(x)
    B = GB.BLOCK[qtype]
    for i in range(nb):
        yb = q[292 * i: 292 * (i + 1)]
        _, qs, bs = _q8k_fields(yb)
        aux, sumi = o.ggml_block_ints(qtype, blob[B * i: B * (i + 1)], yb)
        want_aux, want_sumi = GB.ints_expected(qtype, f, i, qs, bs)
        assert np.array_equal(aux.astype(np.int64), want_aux)
        assert sumi == want_sumi
    got = o.ggml_vec_dot(qtype, blob, q, 256 * nb)
    w = o.ggml_dequantize(blob, qtype, 256 * nb).astype(np.float64)
    xq = np.concatenate([(lambda d, qs, bs: float(d) * qs)(*_q8k_fields(q[292 * i: 292 * (i + 1)]))
                         for i in range(nb)])
    want = float(np.dot(w, xq))
    scale = float(np.abs(w * xq).sum())
    assert abs(got - want) <= 1e-5 * scale + 1e-30
