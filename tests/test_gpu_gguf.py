"""GPU parity of a model read from a GGUF file (load_gguf_transformer,
src/model.c:253-449, feeding forward_runtime, src/runtime.c:94-288) through
qr_gguf_open / qr_gguf_parse, qr_gguf_load and qr_decoder_*.

- The two-layer MoE models of tests/golden/decode.npz written as GGUF (one
  3-D tensor per expert kind, or per-expert tensors; 32- and 64-byte
  alignment; from memory and from an mmap'd file): the decoder's logits and
  residual are the reference's own, bit-exact, for every build.
- A Qwen3-like head shape (attention.key_length 128, q_dim != dim) over a
  Q8_0 cache, its Q4_K / Q5_K projections stored tiled by the loader:
  identical to the same weights handed over as plain row-major pointers.
- A load owns its device copy: the file may be closed, and freeing one of
  two loads leaves the other working.
"""
import numpy as np
import pytest

import gguf_writer as G
import inputs as I
import quantr_amd as Q
from conftest import assert_bits_equal
from oracle import ORDER_AVX2, ORDER_AVX512, ORDER_SEQ

pytestmark = pytest.mark.gpu

BUILDS = {"c99": ORDER_SEQ, "avx2": ORDER_AVX2, "avx512": ORDER_AVX512}


def run_tokens(dev, d, m, tokens, pos0=0):
    lg_d, x_d = dev.alloc(4 * m["vocab"]), dev.alloc(4 * m["dim"])
    lg = np.zeros((len(tokens), m["vocab"]), np.float32)
    xs = np.zeros((len(tokens), m["dim"]), np.float32)
    for i, t in enumerate(tokens):
        d.forward(int(t), pos0 + i, lg_d.ptr, x_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
        xs[i] = dev.download(x_d, m["dim"], np.float32)
    return lg, xs


@pytest.mark.parametrize("layout", ["slab", "split", "align64", "file"])
@pytest.mark.parametrize("build", list(BUILDS))
@pytest.mark.parametrize("name", list(I.DECODE_CASES))
def test_gguf_decoder_matches_reference_logits(dev, golden, tmp_path, name, build, layout):
    g = golden("decode.npz")
    m = I.decode_model(name)
    assert I.decode_digest(m) == str(g["sha_" + name])
    key = "logits_%s_%s" % (name, build)
    if key not in g:
        pytest.skip("fixture written without an -mavx512f build")
    data = G.decode_model_gguf(m, split_experts=layout == "split",
                               alignment=64 if layout == "align64" else 32)[0]
    if layout == "file":
        p = tmp_path / ("%s.gguf" % name)
        p.write_bytes(data)
        gf = Q.Gguf(str(p))
    else:
        gf = Q.Gguf(data)
    print("gguf case %s build %s layout %s" % (name, build, layout), flush=True)
    gm = gf.load(dev, m["seq_len"])
    assert gm.model.n_layers == m["n_layers"] and gm.model.vocab == m["vocab"]
    d = gm.decoder(kv_type=Q.KV_F32, order=BUILDS[build], flags=Q.DEC_GRAPH)
    lg, xs = run_tokens(dev, d, m, m["tokens"])
    d.close()
    gm.close()
    gf.close()
    assert_bits_equal(xs, g["x_%s_%s" % (name, build)], "residual %s/%s" % (name, build))
    assert_bits_equal(lg, g[key], "logits %s/%s" % (name, build))


@pytest.mark.parametrize("split", [False, True], ids=["slab", "split"])
def test_gguf_head128_matches_pointer_model(dev, split):
    """attention.key_length 128 with 8 heads over dim 512 (q_dim 1024), GQA
    4:1, Q8_0 cache in pages of 64: the GGUF-loaded decoder and one built
    from the same arrays as plain pointers produce the same bits."""
    m = I.qwen3_small_model(n_layers=2, seq_len=256)
    gf = Q.Gguf(G.decode_model_gguf(m, head_dim_key=True, split_experts=split)[0])
    print("gguf head128 split %d" % split, flush=True)
    gm = gf.load(dev, m["seq_len"])
    assert gm.model.head_dim == 128 and gm.model.n_heads == 8
    # the Q4_K / Q5_K projections are stored tiled (wq Q4_K, wo Q5_K here)
    wt = m["wtype"]
    for l in range(2):
        y = gm.layers[l]
        for got, want in ((y.wq_type, wt[0]), (y.wk_type, wt[1]), (y.wv_type, wt[2]),
                          (y.wo_type, wt[3])):
            tiled = want in (Q.TYPE_Q4_K, Q.TYPE_Q5_K)
            assert got == (want | Q.TILED if tiled else want)
    toks = [3, 250, 17, 99, 4]
    d = gm.decoder(kv_type=Q.KV_Q8_0, order=ORDER_AVX2, page=64)
    lg, xs = run_tokens(dev, d, m, toks)
    d.close()
    model, layers, keep = Q.upload_decode_model(dev, m)
    d2 = Q.Decoder(dev, model, layers, kv_type=Q.KV_Q8_0, order=ORDER_AVX2, page=64)
    lg2, xs2 = run_tokens(dev, d2, m, toks)
    d2.close()
    del keep
    gm.close()
    gf.close()
    assert np.isfinite(lg).all()
    assert_bits_equal(xs, xs2, "residual")
    assert_bits_equal(lg, lg2, "logits")


def test_gguf_loads_are_independent(dev, golden):
    """The loaded model owns its device copy: the file may be closed after
    loading, and freeing one of two loads leaves the other's decoder giving
    the reference's logits."""
    g = golden("decode.npz")
    m = I.decode_model("b")
    gf = Q.Gguf(G.decode_model_gguf(m, split_experts=True)[0])
    a = gf.load(dev, m["seq_len"])
    b = gf.load(dev, m["seq_len"])
    gf.close()
    assert a.model.tok_embd != b.model.tok_embd
    a.close()
    d = b.decoder(kv_type=Q.KV_F32, order=ORDER_SEQ)
    lg, xs = run_tokens(dev, d, m, m["tokens"])
    d.close()
    b.close()
    assert_bits_equal(lg, g["logits_b_c99"], "logits b/c99")


def test_gguf_tied_output(dev):
    """No output.weight: the logits come from token_embd (src/model.c:323-330),
    the same bits as a pointer model whose wcls is the embedding."""
    m = I.decode_model("a")
    mt = dict(m)
    mt["wcls"], mt["wcls_type"] = m["tok_embd"], m["tok_type"]

    def drop_output(ts):
        return [t for t in ts if t[0] != "output.weight"]
    gf = Q.Gguf(G.decode_model_gguf(mt, mutate=drop_output)[0])
    gm = gf.load(dev, m["seq_len"])
    assert gm.model.wcls == gm.model.tok_embd
    d = gm.decoder(kv_type=Q.KV_F32, order=ORDER_SEQ)
    lg, xs = run_tokens(dev, d, m, m["tokens"])
    d.close()
    gm.close()
    model, layers, keep = Q.upload_decode_model(dev, mt)
    d2 = Q.Decoder(dev, model, layers, kv_type=Q.KV_F32, order=ORDER_SEQ)
    lg2, xs2 = run_tokens(dev, d2, m, m["tokens"])
    d2.close()
    del keep
    assert_bits_equal(xs, xs2, "residual")
    assert_bits_equal(lg, lg2, "logits")
