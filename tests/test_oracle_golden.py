"""The oracle (oracle/qr_oracle.c) against the reference's own outputs.

The fixtures in tests/golden/ were written by tests/golden/gen_golden.py from
the reference's sources compiled as they are (the Makefile's -std=c99
flavour, the CI's -mavx2 -mfma flavour and an -mavx512f flavour).  Every comparison is bit-exact.
"""
import numpy as np
import pytest

import inputs as I
from conftest import assert_bits_equal, bits
from oracle import KV_F16, KV_F32, ORDER_AVX2, ORDER_AVX512, ORDER_SEQ

TYPES = (I.TYPE_Q8_0, I.TYPE_Q4_K, I.TYPE_Q5_K, I.TYPE_Q6_K)


def test_fp16_decode_all_codes(oracle, golden):
    """include/quant.h:53-66 on all 65536 codes, subnormals included."""
    g = golden("fp16.npz")
    h2f = oracle.h2f_bits(np.arange(65536))
    assert I.digest(h2f) == str(g["h2f_sha"])
    assert (h2f[g["h2f_sample_codes"]] == g["h2f_sample"]).all()


def test_fp16_encode(oracle, golden):
    """include/quant.h:68-77: truncation, flush to zero, saturation to inf."""
    g = golden("fp16.npz")
    got = np.array([oracle.f2h(f) for f in g["f2h_in"]], np.uint16)
    assert (got == g["f2h_out"]).all()


def test_quantize_q8_0_edge_rows(oracle, golden):
    """src/quant.c:143-158 on zero, flushed, saturated and tie-rounding rows."""
    g = golden("q8_quant.npz")
    assert (g["edge_in"].view(np.uint32) == I.q8_edge_rows().view(np.uint32)).all()
    for row, want in zip(g["edge_in"], g["edge_out"]):
        assert (oracle.quantize_q8_0(row) == want).all()


def test_quantize_q8_0_random(oracle, golden):
    g = golden("q8_quant.npz")
    x = I.activations(11, 16, 2048)
    assert I.digest(x) == str(g["rand_sha"])
    for row, want in zip(x, g["rand_out"]):
        assert (oracle.quantize_q8_0(row) == want).all()


@pytest.mark.parametrize("qtype", TYPES)
def test_dequantize(oracle, golden, qtype):
    """src/quant.c:160-240 on random and edge-case blocks."""
    g = golden("dequant.npz")
    elems, bb = I.BLOCK[qtype]
    blob = np.concatenate([I.blocks(100 + qtype, qtype, 16), I.special_blocks(qtype)])
    assert I.digest(blob) == str(g["in_sha_%d" % qtype])
    got = oracle.dequantize(blob, qtype, (blob.size // bb) * elems)
    assert (bits(got) == g["out_%d" % qtype]).all()


@pytest.mark.parametrize("d", [2048, 768])
@pytest.mark.parametrize("qtype", TYPES)
def test_vec_dot(oracle, golden, qtype, d):
    """The fused dots in both reference builds.  Q4_K is pinned to the
    reference's Q5_K dot on the same blocks with a zero fifth-bit plane (its
    own Q4_K dot is defective, src/quant.c:302-309)."""
    g = golden("dots.npz")
    x = I.activations(300 + d, 4, d)
    assert I.digest(x) == str(g["x_sha_%d" % d])
    W = I.dot_set(200 + qtype + d, qtype, 15, d)
    assert I.digest(W) == str(g["w_sha_%d_%d" % (qtype, d)])
    xq = [oracle.quantize_q8_0(row) for row in x]
    seq = np.array([[oracle.vec_dot(qtype, W[i], xq[j], d, ORDER_SEQ) for j in range(4)]
                    for i in range(W.shape[0])], np.float32)
    assert_bits_equal(seq, g["dot_c99_%d_%d" % (qtype, d)], "SEQ vs -std=c99 build")
    avx = np.array([[oracle.vec_dot(qtype, W[i], xq[j], d, ORDER_AVX2) for j in range(4)]
                    for i in range(W.shape[0])], np.float32)
    assert_bits_equal(avx, g["dot_avx2_%d_%d" % (qtype, d)], "AVX2 vs -mavx2 -mfma build")
    if qtype == I.TYPE_Q8_0:
        # the -mavx512f build updates the 8 lanes with fused multiply-adds
        v5 = np.array([[oracle.vec_dot(qtype, W[i], xq[j], d, ORDER_AVX512) for j in range(4)]
                       for i in range(W.shape[0])], np.float32)
        assert_bits_equal(v5, g["dot_avx512_%d_%d" % (qtype, d)], "AVX512 vs -mavx512f build")
        assert (bits(v5) != bits(avx)).any() and (bits(avx) != bits(seq)).any()
    mm = np.stack([oracle.matmul_q_fused(x[j], W, qtype, W.shape[0], d, threads=4)
                   for j in range(4)], axis=1)
    assert_bits_equal(mm, g["mm_c99_%d_%d" % (qtype, d)], "matmul_q_fused")


@pytest.mark.parametrize("E,d", [(128, 2048), (60, 2048), (16, 2051)])
def test_router_matmul_orders(oracle, golden, E, d):
    """matmul_ref, matmul_omp (AVX2 build) and matmul_omp (AVX-512 build),
    src/kernels.c:18-73, including the tails of a d that is not a multiple of
    8 or 16; and softmax_ref (src/kernels.c:191-207)."""
    g = golden("router.npz")
    seed = {(128, 2048): 400, (60, 2048): 410, (16, 2051): 420}[(E, d)]
    W = I.activations(seed, E, d, std=0.02)
    X = I.activations(seed + 1, 4, d)
    assert I.digest(W, X) == str(g["sha_%d_%d" % (E, d)])
    for order, key in ((ORDER_SEQ, "ref"), (ORDER_AVX2, "avx2"), (ORDER_AVX512, "avx512")):
        if "%s_%d_%d" % (key, E, d) not in g:
            continue
        got = np.stack([oracle.matmul_f32(x, W, E, d, order) for x in X])
        assert_bits_equal(got, g["%s_%d_%d" % (key, E, d)], key)
    sm = np.stack([oracle.softmax(l) for l in g["ref_%d_%d" % (E, d)]])
    assert_bits_equal(sm, g["softmax_%d_%d" % (E, d)], "softmax")


def _layer(oracle, keep, m):
    return oracle.make_layer(keep, m["dim"], m["hidden"], m["E"], m["K"], m["router"], m["up"],
                             m["up_type"], m["gate"], m["up_type"], m["down"], m["down_type"])


@pytest.mark.parametrize("name", sorted(I.MOE_CASES))
@pytest.mark.parametrize("build", ["c99", "avx2", "avx512"])
def test_moe_block(oracle, golden, name, build):
    """The reference's MoE block (src/runtime.c:202-269) run through its own
    forward_runtime: routing, SwiGLU experts, slot-order combine, residual."""
    g = golden("moe.npz")
    m = I.moe_inputs(name)
    assert I.digest(m["up"], m["gate"], m["down"], m["router"], m["x"]) == str(g["sha_" + name])
    keep = []
    L = _layer(oracle, keep, m)
    xb = g["xb_%s_%s" % (name, build)]
    order = {"c99": ORDER_SEQ, "avx2": ORDER_AVX2, "avx512": ORDER_AVX512}[build]
    xo, idx, w = oracle.moe_forward(m["x"], xb, L, order=order, dot_order=order, threads=4)
    assert_bits_equal(xo, g["xo_%s_%s" % (name, build)], "MoE block %s/%s" % (name, build))
    assert (idx >= 0).all() and (idx < m["E"]).all()


@pytest.mark.parametrize("name", sorted(I.DECODE_CASES))
@pytest.mark.parametrize("build", ["c99", "avx2", "avx512"])
@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_decode_step(oracle, golden, name, build, kv):
    """The oracle's decode step (oracle/qr_oracle_decode.c) against the
    reference's own forward_runtime (src/runtime.c:94-288) on a two-layer MoE
    model, token by token from position 0 (head_dim = dim / n_heads), with
    the fp32 KV cache and with the fp16 one (kv_cache_type 1: truncating
    stores, fp16_to_fp32 reads, src/runtime.c:74-92): embedding
    dequantization, RMSNorm, Q/K/V, RoPE, the attention over the growing
    cache, Wo and the residual, the MoE block, the final norm and the lm_head
    -- logits and residual bit-exact."""
    g = golden("decode.npz")
    m = I.decode_model(name)
    assert I.decode_digest(m) == str(g["sha_" + name])
    tag = "" if kv == "f32" else "16"
    key = "logits%s_%s_%s" % (tag, name, build)
    if key not in g:
        pytest.skip("fixture written without an -mavx512f build")
    order = {"c99": ORDER_SEQ, "avx2": ORDER_AVX2, "avx512": ORDER_AVX512}[build]
    lg, xs = oracle.forward_seq(m, m["tokens"], order, KV_F16 if kv == "f16" else KV_F32)
    assert_bits_equal(lg, g[key], "logits %s/%s/%s" % (name, build, kv))
    assert_bits_equal(xs, g["x%s_%s_%s" % (tag, name, build)], "residual %s/%s/%s" % (
        name, build, kv))


def test_rope_table_matches_rope(oracle):
    """The per-position cos / sin table (what the device decoder reads) gives
    the same rotation as apply_rope's per-call powf / cosf / sinf: rotating with
    the table in the reference's operation order reproduces qro_rope bit for
    bit (q of 8 heads of 64, k of 2 kv heads, positions 0, 1, 4095)."""
    qlen, hd, kvh, base = 512, 64, 2, 1e6
    q0 = I.activations(77, 1, qlen)[0]
    k0 = I.activations(78, 1, kvh * hd)[0]
    for pos in (0, 1, 4095):
        q, k = oracle.rope(q0, k0, hd, kvh, pos, base)
        cs = oracle.rope_table(qlen, hd, pos, base)
        c, s = cs[0::2], cs[1::2]
        a, b = q0[0::2], q0[1::2]
        qt = np.empty_like(q0)
        qt[0::2] = (a * c - b * s).astype(np.float32)
        qt[1::2] = (a * s + b * c).astype(np.float32)
        # numpy float32 ops round once each, in the same order as the C code
        assert_bits_equal(q, qt, "q at pos %d" % pos)
        ka, kb = k0[0::2], k0[1::2]
        kt = k0.copy()
        kt[0::2] = ka * c[: kvh * hd // 2] - kb * s[: kvh * hd // 2]
        kt[1::2] = ka * s[: kvh * hd // 2] + kb * c[: kvh * hd // 2]
        assert_bits_equal(k[: kvh * hd], kt, "k at pos %d" % pos)
