"""GPU parity of models whose K-quant tensors are in llama.cpp's block layouts
(QR_GGML: a checkpoint quantized by llama.cpp, read with ggml's Q8_K dots)
with the oracle, bit for bit.  The oracle's ggml arithmetic is pinned by
closed forms (tests/test_oracle_ggml.py); its decode step and MoE block are
the ones the reference's own forward_runtime pins, with the ggml dot in place
of the fused one.

- A dense model at TinyLlama-1.1B's layer shapes in llama.cpp's Q4_K_M type
  mix (Q4_K embedding, wq / wk / wo and FFN up / gate; Q6_K wv, ffn_down and
  lm_head): decode steps (eager and graph, fp32 and Q8_0 caches) and a
  chunked prefill.
- The same model as a GGUF file loaded with QR_GGUF_GGML_KQUANTS: every
  K-quant type carries QR_GGML, none is tiled, and the decoder's logits are
  the oracle's.
- A MoE layer at Qwen3-30B-A3B's shapes (128 experts, top-8, dim 2048, ffn
  768) with ggml experts through qr_moe_forward at T = 1, 5 and 64, and a
  two-layer MoE decoder (decode and prefill).

The weights are random block bytes with small fp16 scales: every byte
pattern is a valid block of these layouts.
"""
import numpy as np
import pytest

import inputs as I
import quantr_amd as Q
from conftest import assert_bits_equal
from oracle import ORDER_AVX2, ORDER_SEQ, Oracle

pytestmark = pytest.mark.gpu

KQ = (Q.TYPE_Q4_K, Q.TYPE_Q5_K, Q.TYPE_Q6_K)


def as_ggml(t):
    return t | Q.GGML if t in KQ else t


def ggml_model(m):
    """m with every K-quant type read in llama.cpp's layouts."""
    g = dict(m)
    g["wtype"] = [as_ggml(t) for t in m["wtype"]]
    for k in ("tok_type", "wcls_type", "up_type", "down_type"):
        g[k] = as_ggml(m[k])
    return g


def q4km_dense(n_layers=2, seq_len=64):
    """TinyLlama-1.1B's shapes in the Q4_K_M mix, plain K-quant types."""
    m = I.tinyllama_model(n_layers=n_layers, seq_len=seq_len, ffn_type=Q.TYPE_Q4_K)
    dim, H, KVH, hd, hidden, vocab = (m["dim"], m["n_heads"], m["n_kv_heads"], m["head_dim"],
                                      m["hidden"], m["vocab"])
    m["wtype"] = [Q.TYPE_Q4_K, Q.TYPE_Q4_K, Q.TYPE_Q6_K, Q.TYPE_Q4_K]
    m["tok_type"], m["wcls_type"], m["down_type"] = Q.TYPE_Q4_K, Q.TYPE_Q6_K, Q.TYPE_Q6_K
    m["tok_embd"] = I._rows(9700, Q.TYPE_Q4_K, vocab, dim)
    m["wcls"] = I._rows(9701, Q.TYPE_Q6_K, vocab, dim)
    for l, lw in enumerate(m["layers"]):
        s = 9710 + 20 * l
        lw["wq"] = I._rows(s, Q.TYPE_Q4_K, H * hd, dim)
        lw["wk"] = I._rows(s + 1, Q.TYPE_Q4_K, KVH * hd, dim)
        lw["wv"] = I._rows(s + 2, Q.TYPE_Q6_K, KVH * hd, dim)
        lw["wo"] = I._rows(s + 3, Q.TYPE_Q4_K, dim, H * hd)
        lw["down"] = I._rows(s + 4, Q.TYPE_Q6_K, dim, hidden).reshape(-1)
    return m


def make_decoder(dev, m, kv_type, order, page=0, flags=0):
    model, layers, keep = Q.upload_decode_model(dev, m)
    d = Q.Decoder(dev, model, layers, kv_type=kv_type, order=order, page=page, flags=flags)
    d._keep = keep
    return d


def decode(dev, d, m, toks):
    lg_d, x_d = dev.alloc(4 * m["vocab"]), dev.alloc(4 * m["dim"])
    lg = np.zeros((len(toks), m["vocab"]), np.float32)
    xs = np.zeros((len(toks), m["dim"]), np.float32)
    for i, t in enumerate(toks):
        d.forward(int(t), i, lg_d.ptr, x_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
        xs[i] = dev.download(x_d, m["dim"], np.float32)
    return lg, xs


@pytest.fixture(scope="module")
def dense_m():
    return ggml_model(q4km_dense())


@pytest.mark.parametrize("kv_type", [Q.KV_F32, Q.KV_Q8_0])
@pytest.mark.parametrize("order,graph", [(ORDER_SEQ, 0), (ORDER_AVX2, Q.DEC_GRAPH)],
                         ids=["seq_eager", "avx2_graph"])
def test_ggml_dense_decode(dev, oracle, dense_m, order, graph, kv_type):
    """Four decode steps from position 0: logits and residual bit-exact."""
    m = dense_m
    toks = [1, 31999, 450, 450]
    print("ggml dense decode order %d graph %d kv %d" % (order, graph, kv_type), flush=True)
    d = make_decoder(dev, m, kv_type, order, flags=graph)
    lg, xs = decode(dev, d, m, toks)
    d.close()
    wl, wx = oracle.forward_seq(m, toks, order, kv_type)
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")


def test_ggml_dense_prefill(dev, oracle, dense_m):
    """20 prompt tokens in chunks of 8 (the projections as 4-row ggml GEMVs):
    every position's logits and the last residual bit-exact."""
    m = dense_m
    toks = np.random.default_rng(5).integers(0, m["vocab"], size=20).astype(np.int32)
    print("ggml dense prefill", flush=True)
    d = make_decoder(dev, m, Q.KV_F32, ORDER_SEQ)
    n = len(toks)
    lg_d, x_d = dev.alloc(4 * m["vocab"] * n), dev.alloc(4 * m["dim"])
    d.prefill(toks, 0, lg_d.ptr, x_d.ptr, chunk=8, all_logits=True)
    lg = dev.download(lg_d, (n, m["vocab"]), np.float32)
    x = dev.download(x_d, m["dim"], np.float32)
    d.close()
    wl, wx = oracle.forward_seq(m, [int(t) for t in toks], ORDER_SEQ, Q.KV_F32)
    assert_bits_equal(x, wx[-1], "prefill residual")
    assert_bits_equal(lg, wl, "prefill logits")


def test_ggml_dense_gguf(dev, oracle):
    """The Q4_K_M dense model as a llama GGUF file, loaded with
    QR_GGUF_GGML_KQUANTS: K-quant types carry QR_GGML and are not tiled,
    Q8_0 keeps its type; three decode steps bit-exact with the oracle run on
    the ggml types."""
    import gguf_writer as G
    m = q4km_dense(n_layers=1)
    # one Q8_0 matrix, which keeps its own type under the flag
    m["wtype"][1] = Q.TYPE_Q8_0
    m["layers"][0]["wk"] = I._rows(9790, Q.TYPE_Q8_0, m["n_kv_heads"] * m["head_dim"], m["dim"])
    gf = Q.Gguf(G.decode_model_gguf(m, arch="llama")[0])
    gm = gf.load(dev, m["seq_len"], ggml_kquants=True)
    mo, L0 = gm.model, gm.layers[0]
    assert mo.tok_type == Q.TYPE_Q4_K | Q.GGML and mo.wcls_type == Q.TYPE_Q6_K | Q.GGML
    assert [L0.wq_type, L0.wk_type, L0.wv_type, L0.wo_type] == [
        Q.TYPE_Q4_K | Q.GGML, Q.TYPE_Q8_0, Q.TYPE_Q6_K | Q.GGML, Q.TYPE_Q4_K | Q.GGML]
    assert L0.moe.up_type == Q.TYPE_Q4_K | Q.GGML and L0.moe.down_type == Q.TYPE_Q6_K | Q.GGML
    print("ggml dense gguf", flush=True)
    d = gm.decoder(kv_type=Q.KV_F32, order=ORDER_SEQ, flags=Q.DEC_GRAPH)
    toks = [2, 31000, 17]
    lg, xs = decode(dev, d, m, toks)
    d.close()
    gm.close()
    gf.close()
    wl, wx = oracle.forward_seq(ggml_model(m), toks, ORDER_SEQ, Q.KV_F32)
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")


def test_ggml_gguf_load_rejects_unknown_flags(dev):
    import gguf_writer as G
    m = q4km_dense(n_layers=1, seq_len=16)
    gf = Q.Gguf(G.decode_model_gguf(m, arch="llama")[0])
    with pytest.raises(Q.QrError, match="unknown flags"):
        Q.GgufModel(dev, gf, m["seq_len"], flags=2)
    gf.close()


# ---- MoE ---------------------------------------------------------------------
@pytest.fixture(scope="module")
def qwen3_layer(dev):
    """One MoE layer at Qwen3-30B-A3B's shapes, ggml experts (Q4_K up / gate,
    Q6_K down), uploaded once."""
    dim, hidden, E, K = 2048, 768, 128, 8
    s = 9850
    router = I.activations(s, E, dim, std=0.05)
    up = I.blocks(s + 1, Q.TYPE_Q4_K, E * hidden * (dim // 256))
    gate = I.blocks(s + 2, Q.TYPE_Q4_K, E * hidden * (dim // 256))
    down = I.blocks(s + 3, Q.TYPE_Q6_K, E * dim * (hidden // 256))
    bufs = [dev.upload(router), dev.upload(up), dev.upload(gate), dev.upload(down)]
    ut, dt = Q.TYPE_Q4_K | Q.GGML, Q.TYPE_Q6_K | Q.GGML
    L = Q.MoeLayer(dim, hidden, E, K, *[b.ptr for b in bufs], ut, ut, dt)
    host = dict(dim=dim, hidden=hidden, E=E, K=K, router=router, up=up, gate=gate, down=down,
                ut=ut, dt=dt)
    return L, host, bufs


@pytest.mark.parametrize("T", [1, 5, 64])
def test_ggml_moe_layer(dev, oracle, qwen3_layer, T):
    """qr_moe_forward over T tokens: routing and layer output bit-exact."""
    L, h, _ = qwen3_layer
    rng = np.random.default_rng(40 + T)
    x = rng.standard_normal((T, h["dim"])).astype(np.float32)
    xb = rng.standard_normal((T, h["dim"])).astype(np.float32)
    print("ggml moe layer T=%d" % T, flush=True)
    xd, xbd = dev.upload(x), dev.upload(xb)
    idx, w = dev.alloc(T * h["K"] * 4), dev.alloc(T * h["K"] * 4)
    dev.moe_forward(L, xd.ptr, xbd.ptr, T, ORDER_SEQ, idx.ptr, w.ptr)
    got = dev.download(xd, (T, h["dim"]), np.float32)
    gi = dev.download(idx, (T, h["K"]), np.int32)
    gw = dev.download(w, (T, h["K"]), np.float32)
    keep = []
    ol = Oracle.make_layer(keep, h["dim"], h["hidden"], h["E"], h["K"], h["router"], h["up"],
                           h["ut"], h["gate"], h["ut"], h["down"], h["dt"])
    want, wi, ww = oracle.moe_forward(x, xb, ol, order=ORDER_SEQ, dot_order=ORDER_SEQ, threads=16)
    assert (gi == wi).all(), "routing indices differ"
    assert_bits_equal(gw, ww, "routing weights")
    assert_bits_equal(got, want, "layer output")


def test_ggml_moe_rejects_mixed_layouts(dev, qwen3_layer):
    """ggml experts need all three matrices in llama.cpp's layouts."""
    L0, h, _ = qwen3_layer
    L = Q.MoeLayer(h["dim"], h["hidden"], h["E"], h["K"], L0.router, L0.up, L0.gate, L0.down,
                   h["ut"], h["ut"], Q.TYPE_Q6_K)
    xd, xbd = dev.alloc(4 * h["dim"]), dev.alloc(4 * h["dim"])
    with pytest.raises(Q.QrError, match="ggml experts"):
        dev.moe_forward(L, xd.ptr, xbd.ptr, 1, ORDER_SEQ)


@pytest.fixture(scope="module")
def moe_m():
    return ggml_model(I.qwen3_small_model(seq_len=64))


@pytest.mark.parametrize("order,graph", [(ORDER_SEQ, Q.DEC_GRAPH), (ORDER_AVX2, 0)],
                         ids=["seq_graph", "avx2_eager"])
def test_ggml_moe_decode(dev, oracle, moe_m, order, graph):
    """A two-layer MoE decoder (Qwen3-shaped heads, 8 experts top-2) in the
    ggml layouts: four decode steps bit-exact."""
    m = moe_m
    toks = [3, 319, 3, 100]
    print("ggml moe decode order %d graph %d" % (order, graph), flush=True)
    d = make_decoder(dev, m, Q.KV_Q8_0, order, flags=graph)
    lg, xs = decode(dev, d, m, toks)
    d.close()
    wl, wx = oracle.forward_seq(m, toks, order, Q.KV_Q8_0)
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")


def test_ggml_moe_prefill(dev, oracle, moe_m):
    """18 prompt tokens in chunks of 8 (MoE at T = 8 and 2 through the pair
    GEMVs): every position's logits and the last residual bit-exact."""
    m = moe_m
    toks = np.random.default_rng(6).integers(0, m["vocab"], size=18).astype(np.int32)
    print("ggml moe prefill", flush=True)
    d = make_decoder(dev, m, Q.KV_F32, ORDER_SEQ)
    n = len(toks)
    lg_d, x_d = dev.alloc(4 * m["vocab"] * n), dev.alloc(4 * m["dim"])
    d.prefill(toks, 0, lg_d.ptr, x_d.ptr, chunk=8, all_logits=True)
    lg = dev.download(lg_d, (n, m["vocab"]), np.float32)
    x = dev.download(x_d, m["dim"], np.float32)
    d.close()
    wl, wx = oracle.forward_seq(m, [int(t) for t in toks], ORDER_SEQ, Q.KV_F32)
    assert_bits_equal(x, wx[-1], "prefill residual")
    assert_bits_equal(lg, wl, "prefill logits")
