"""GPU parity of the decode step and the prefill of a dense model at
TinyLlama-1.1B's layer shapes (the FFN branch of forward_runtime,
src/runtime.c:270-284): dim 2048, 32 heads of 64 over 4 kv heads, FFN 5632,
vocab 32000, Q8_0 weights (and a Q4_K / Q6_K FFN).  head_dim is
dim / n_heads, the shape the reference itself runs; the oracle that checks
it is pinned to the reference's own forward_runtime on the dense decode cases
of tests/golden/decode.npz (fp32 and fp16 caches, every build).  Two layers
stand for the 22.
"""
import numpy as np
import pytest

import inputs as I
import quantr_amd as Q
from conftest import assert_bits_equal
from oracle import ORDER_AVX2, ORDER_SEQ

pytestmark = pytest.mark.gpu


def make_decoder(dev, m, kv_type, order, page=0, flags=0):
    model, layers, keep = Q.upload_decode_model(dev, m)
    d = Q.Decoder(dev, model, layers, kv_type=kv_type, order=order, page=page, flags=flags)
    d._keep = keep
    return d


@pytest.mark.parametrize("ffn", ["q8_0", "q4k_q6k"])
@pytest.mark.parametrize("kv_type", [Q.KV_F32, Q.KV_F16])
@pytest.mark.parametrize("order,graph", [(ORDER_SEQ, 0), (ORDER_AVX2, Q.DEC_GRAPH)],
                         ids=["seq_eager", "avx2_graph"])
def test_tinyllama_decode(dev, oracle, order, graph, kv_type, ffn):
    """Five decode steps from position 0: logits and residual bit-exact with
    the oracle."""
    ut = Q.TYPE_Q8_0 if ffn == "q8_0" else Q.TYPE_Q4_K
    m = I.tinyllama_model(ffn_type=ut)
    if ffn != "q8_0":
        for l, lw in enumerate(m["layers"]):
            lw["down"] = I._rows(9990 + l, Q.TYPE_Q6_K, m["dim"], m["hidden"]).reshape(-1)
        m["down_type"] = Q.TYPE_Q6_K
    toks = [1, 31999, 450, 450, 7]
    print("tinyllama decode order %d graph %d kv %d ffn %s" % (order, graph, kv_type, ffn),
          flush=True)
    d = make_decoder(dev, m, kv_type, order, flags=graph)
    lg_d, x_d = dev.alloc(4 * m["vocab"]), dev.alloc(4 * m["dim"])
    lg = np.zeros((len(toks), m["vocab"]), np.float32)
    xs = np.zeros((len(toks), m["dim"]), np.float32)
    for i, t in enumerate(toks):
        d.forward(t, i, lg_d.ptr, x_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
        xs[i] = dev.download(x_d, m["dim"], np.float32)
    d.close()
    wl, wx = oracle.forward_seq(m, toks, order, kv_type)
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")


@pytest.mark.parametrize("ffn", ["q8_0", "q4k_q6k"])
def test_tinyllama_prefill(dev, oracle, ffn):
    """40 prompt tokens in chunks of 16 (the projections and the FFN as T-row
    products): every position's logits and the last residual bit-exact with
    the oracle."""
    ut = Q.TYPE_Q8_0 if ffn == "q8_0" else Q.TYPE_Q4_K
    m = I.tinyllama_model(ffn_type=ut)
    if ffn != "q8_0":
        for l, lw in enumerate(m["layers"]):
            lw["down"] = I._rows(9990 + l, Q.TYPE_Q6_K, m["dim"], m["hidden"]).reshape(-1)
        m["down_type"] = Q.TYPE_Q6_K
    toks = np.random.default_rng(3).integers(0, m["vocab"], size=40).astype(np.int32)
    print("tinyllama prefill ffn %s" % ffn, flush=True)
    d = make_decoder(dev, m, Q.KV_F32, ORDER_SEQ)
    n = len(toks)
    lg_d, x_d = dev.alloc(4 * m["vocab"] * n), dev.alloc(4 * m["dim"])
    d.prefill(toks, 0, lg_d.ptr, x_d.ptr, chunk=16, all_logits=True)
    lg = dev.download(lg_d, (n, m["vocab"]), np.float32)
    x = dev.download(x_d, m["dim"], np.float32)
    d.close()
    wl, wx = oracle.forward_seq(m, [int(t) for t in toks], ORDER_SEQ, Q.KV_F32)
    assert_bits_equal(x, wx[-1], "prefill residual")
    assert_bits_equal(lg, wl, "prefill logits")


def test_tinyllama_gguf_tiled_q6k_head(dev, oracle):
    """The dense model as a GGUF file with a Q6_K lm_head: qr_gguf_load stores
    the lm_head in the tiled layout (rows of 2048), and the decoder reads it
    with the tiled Q6_K GEMV; four decode steps bit-exact with the oracle."""
    import gguf_writer as G
    m = I.tinyllama_model(n_layers=1, seq_len=64)
    m["wcls"] = I._rows(9950, Q.TYPE_Q6_K, m["vocab"], m["dim"])
    m["wcls_type"] = Q.TYPE_Q6_K
    gf = Q.Gguf(G.decode_model_gguf(m, arch="llama")[0])
    gm = gf.load(dev, m["seq_len"])
    assert gm.model.wcls_type == Q.TYPE_Q6_K | Q.TILED
    d = gm.decoder(kv_type=Q.KV_F32, order=ORDER_SEQ, flags=Q.DEC_GRAPH)
    toks = [2, 31000, 17, 17]
    lg_d = dev.alloc(4 * m["vocab"])
    lg = np.zeros((len(toks), m["vocab"]), np.float32)
    for i, t in enumerate(toks):
        d.forward(t, i, lg_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
    d.close()
    gm.close()
    gf.close()
    wl, _ = oracle.forward_seq(m, toks, ORDER_SEQ, Q.KV_F32)
    assert_bits_equal(lg, wl, "logits")
