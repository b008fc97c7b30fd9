"""GPU parity of the batched prompt prefill / speculative verify
(qr_decoder_prefill; prefill_runtime, src/runtime.c:294-304, and the verify
loop of src/speculative.c:107-140 both call forward_runtime once per token).

- The two decode.npz models: the whole token sequence in one call (and in
  chunks of 3 and of 1) gives the reference's own logits for every position
  and its last residual, bit for bit, in every build.
- A prefill followed by single-token steps continues exactly as the
  sequential decode does.
- A Qwen3-like head shape (GQA 4:1 and 8:1) over a Q8_0 or fp32 cache in
  permuted pages: 300 prompt tokens in chunks of 128 (the MFMA row products,
  three chunks) give the oracle's logits at every position, its last residual
  and its cache rows, bit for bit; also with the projections stored tiled
  (GGUF load).
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


def make_decoder(dev, m, kv_type, order, page=0, flags=0):
    model, layers, keep = Q.upload_decode_model(dev, m)
    d = Q.Decoder(dev, model, layers, kv_type=kv_type, order=order, page=page, flags=flags)
    d._keep = keep
    return d


def sequential(dev, d, m, tokens, pos0=0):
    lg_d, x_d = dev.alloc(4 * m["vocab"]), dev.alloc(4 * m["dim"])
    lg = np.zeros((len(tokens), m["vocab"]), np.float32)
    for i, t in enumerate(tokens):
        d.forward(int(t), pos0 + i, lg_d.ptr, x_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
    return lg, dev.download(x_d, m["dim"], np.float32)


def prefill(dev, d, m, tokens, pos0=0, chunk=0):
    n = len(tokens)
    lg_d, x_d = dev.alloc(4 * m["vocab"] * n), dev.alloc(4 * m["dim"])
    d.prefill(tokens, pos0, lg_d.ptr, x_d.ptr, chunk=chunk, all_logits=True)
    return (dev.download(lg_d, (n, m["vocab"]), np.float32),
            dev.download(x_d, m["dim"], np.float32))


@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("chunk", [0, 3, 1])
@pytest.mark.parametrize("build", list(BUILDS))
@pytest.mark.parametrize("name", list(I.DECODE_CASES))
def test_prefill_matches_reference_logits(dev, golden, name, build, chunk, kv):
    g = golden("decode.npz")
    m = I.decode_model(name)
    tag = "" if kv == "f32" else "16"
    key = "logits%s_%s_%s" % (tag, name, build)
    if key not in g:
        pytest.skip("fixture written without an -mavx512f build")
    print("prefill case %s build %s chunk %d kv %s" % (name, build, chunk, kv), flush=True)
    d = make_decoder(dev, m, Q.KV_F16 if kv == "f16" else Q.KV_F32, BUILDS[build])
    lg, x = prefill(dev, d, m, m["tokens"], chunk=chunk)
    d.close()
    assert_bits_equal(lg, g[key], "prefill logits %s/%s" % (name, build))
    assert_bits_equal(x, g["x%s_%s_%s" % (tag, name, build)][-1], "prefill residual")


@pytest.mark.parametrize("name", list(I.DECODE_CASES))
def test_prefill_then_decode(dev, golden, name):
    """The first tokens by prefill (last logits only), the rest one step at a
    time: the reference's logits at every following position."""
    g = golden("decode.npz")
    m = I.decode_model(name)
    toks = m["tokens"]
    k = len(toks) - 2
    d = make_decoder(dev, m, Q.KV_F32, ORDER_AVX2, flags=Q.DEC_GRAPH)
    lg_d = dev.alloc(4 * m["vocab"])
    d.prefill(toks[:k], 0, lg_d.ptr)
    first = dev.download(lg_d, m["vocab"], np.float32)
    rest, _ = sequential(dev, d, m, toks[k:], pos0=k)
    d.close()
    want = g["logits_%s_avx2" % name]
    assert_bits_equal(first, want[k - 1], "last prefill logits")
    assert_bits_equal(rest, want[k:], "decode after prefill")


def _kv_rows(dev, d, L, positions, rs):
    out = []
    for l in range(L):
        for t in positions:
            kr, vr = d.kv_rows(l, t)
            out.append(dev.download(kr, rs, np.uint8))
            out.append(dev.download(vr, rs, np.uint8))
    return np.stack(out)


def oracle_prompt(oracle, m, toks, kv_type, order):
    """The oracle over the whole prompt from an empty cache: every position's
    logits, the residuals and the cache it wrote ([L][seq_len][row bytes])."""
    rs = oracle.kv_row_bytes(kv_type, m["n_kv_heads"] * m["head_dim"])
    kc = np.zeros((m["n_layers"], m["seq_len"], rs), np.uint8)
    vc = np.zeros_like(kc)
    lg, xs = oracle.forward_cached(m, kc.reshape(-1), vc.reshape(-1), [int(t) for t in toks], 0,
                                   order, kv_type)
    return lg, xs, kc, vc


def _oracle_rows(kc, vc, L, positions):
    out = []
    for l in range(L):
        for t in positions:
            out.append(kc[l, t])
            out.append(vc[l, t])
    return np.stack(out)


@pytest.mark.parametrize("source,page", [("pointers", 64), ("gguf_tiled", 64), ("pointers", 16)])
def test_prefill_head128_chunks(dev, oracle, source, page):
    """300 prompt tokens of a head_dim-128 model (q_dim 1024 != dim 512, GQA
    4:1) over a Q8_0 cache in permuted pages of 64 (16: pages smaller than
    the attention values' 32-position groups), prefilled in chunks of 128
    (the projections as MFMA row products), against the oracle: every
    token's logits, the last residual and the cache rows."""
    m = I.qwen3_small_model(n_layers=2, seq_len=320)
    rng = np.random.default_rng(9)
    toks = rng.integers(0, m["vocab"], size=300).astype(np.int32)
    order = ORDER_AVX2
    want_lg, want_xs, kc, vc = oracle_prompt(oracle, m, toks, Q.KV_Q8_0, order)
    probe = [0, 63, 64, 127, 128, 200, 299]
    want_kv = _oracle_rows(kc, vc, m["n_layers"], probe)
    rs = kc.shape[2]
    if source == "gguf_tiled":
        gf = Q.Gguf(G.decode_model_gguf(m, head_dim_key=True)[0])
        gm = gf.load(dev, m["seq_len"])
        assert gm.layers[0].wq_type == Q.TYPE_Q4_K | Q.TILED
        d = gm.decoder(kv_type=Q.KV_Q8_0, order=order, page=page)
    else:
        d = make_decoder(dev, m, Q.KV_Q8_0, order, page=page)
    ppl, _ = d.pages()
    d.set_pages(np.stack([rng.permutation(ppl) for _ in range(m["n_layers"])]).astype(np.int32))
    print("prefill head128 %s page %d" % (source, page), flush=True)
    lg, x = prefill(dev, d, m, toks, chunk=128)
    kv = _kv_rows(dev, d, m["n_layers"], probe, rs)
    d.close()
    assert_bits_equal(lg, want_lg, "prefill logits")
    assert_bits_equal(x, want_xs[-1], "prefill residual")
    assert np.array_equal(kv, want_kv)


@pytest.mark.parametrize("kv_type,page", [(Q.KV_Q8_0, 64), (Q.KV_F32, 16), (Q.KV_F16, 32)],
                         ids=["q8_0_pages64", "f32_pages16", "f16_pages32"])
def test_prefill_gqa8_chunks(dev, oracle, kv_type, page):
    """GQA 8:1 at head_dim 128, the shape whose prefill attention values run
    the query heads of a kv head in one workgroup (V staged once for the
    eight): 300 prompt tokens in chunks of 128 against the oracle, every
    token's logits, the last residual and the cache rows bit for bit."""
    m = I.qwen3_small_model(n_layers=2, seq_len=320, n_kv_heads=1)
    rng = np.random.default_rng(19)
    toks = rng.integers(0, m["vocab"], size=300).astype(np.int32)
    want_lg, want_xs, kc, vc = oracle_prompt(oracle, m, toks, kv_type, ORDER_AVX2)
    probe = [0, 127, 128, 255, 256, 299]
    d = make_decoder(dev, m, kv_type, ORDER_AVX2, page=page)
    print("prefill gqa8 chunks kv %d page %d" % (kv_type, page), flush=True)
    lg, x = prefill(dev, d, m, toks, chunk=128)
    kv = _kv_rows(dev, d, m["n_layers"], probe, kc.shape[2])
    d.close()
    assert_bits_equal(lg, want_lg, "prefill logits")
    assert_bits_equal(x, want_xs[-1], "prefill residual")
    assert np.array_equal(kv, _oracle_rows(kc, vc, m["n_layers"], probe))


def test_prefill_gqa8_lds_boundary(dev, oracle):
    """GQA 8:1 at head_dim 128 in pages of 256 near 4096 positions, where the
    per-kv-head values kernel's LDS (eight score rows of the chunk's extent
    plus the value tiles and page table) reaches the CU's 160 KiB: a chunk
    ending at extent 4088 still fits it, one ending at 4092 runs the per-head
    kernel instead.  The prefix is prefilled on the device; the oracle then
    runs the two chunks' tokens over that cache: every logit bit-exact."""
    m = I.qwen3_small_model(n_layers=1, seq_len=4096, n_kv_heads=1)
    rng = np.random.default_rng(41)
    toks = rng.integers(0, m["vocab"], size=4092).astype(np.int32)
    d = make_decoder(dev, m, Q.KV_Q8_0, ORDER_SEQ, page=256)
    print("prefill gqa8 lds boundary", flush=True)
    d.prefill(toks[:4080], 0, chunk=512)
    rs = oracle.kv_row_bytes(Q.KV_Q8_0, m["n_kv_heads"] * m["head_dim"])
    kc = np.zeros((1, m["seq_len"], rs), np.uint8)
    vc = np.zeros_like(kc)
    for t in range(4080):
        kr, vr = d.kv_rows(0, t)
        kc[0, t] = dev.download(kr, rs, np.uint8)
        vc[0, t] = dev.download(vr, rs, np.uint8)
    lg1, _ = prefill(dev, d, m, toks[4080:4088], pos0=4080, chunk=8)   # extent 4088
    lg2, x2 = prefill(dev, d, m, toks[4088:4092], pos0=4088, chunk=4)  # extent 4092
    d.close()
    want_lg, want_xs = oracle.forward_cached(m, kc.reshape(-1), vc.reshape(-1),
                                             [int(t) for t in toks[4080:]], 4080, ORDER_SEQ,
                                             Q.KV_Q8_0)
    assert_bits_equal(lg1, want_lg[:8], "logits, chunk ending at extent 4088")
    assert_bits_equal(lg2, want_lg[8:], "logits, chunk ending at extent 4092")
    assert_bits_equal(x2, want_xs[-1], "last residual")


def test_prefill_matches_sequential_decode(dev):
    """Prefill in chunks of 128 against the same decoder's own single steps
    (a consistency check beside the oracle comparisons above)."""
    m = I.qwen3_small_model(n_layers=2, seq_len=320)
    toks = np.random.default_rng(29).integers(0, m["vocab"], size=200).astype(np.int32)
    ref = make_decoder(dev, m, Q.KV_Q8_0, ORDER_AVX2, page=64, flags=Q.DEC_GRAPH)
    want_lg, want_x = sequential(dev, ref, m, toks)
    ref.close()
    d = make_decoder(dev, m, Q.KV_Q8_0, ORDER_AVX2, page=64)
    lg, x = prefill(dev, d, m, toks, chunk=128)
    d.close()
    assert_bits_equal(lg, want_lg, "prefill logits")
    assert_bits_equal(x, want_x, "prefill residual")


@pytest.mark.parametrize("chunk", [0, 256, 1024])
def test_prefill_large_chunks(dev, chunk):
    """The default chunk (0: QR_PREFILL_CHUNK) and chunks up to the maximum
    against the same decoder's single steps: a 300-token prompt in one chunk
    (0, 1024) or two (256)."""
    m = I.qwen3_small_model(n_layers=2, seq_len=320)
    toks = np.random.default_rng(31).integers(0, m["vocab"], size=300).astype(np.int32)
    print("prefill chunk %d" % chunk, flush=True)
    ref = make_decoder(dev, m, Q.KV_Q8_0, ORDER_AVX2, page=64, flags=Q.DEC_GRAPH)
    want_lg, want_x = sequential(dev, ref, m, toks)
    ref.close()
    d = make_decoder(dev, m, Q.KV_Q8_0, ORDER_AVX2, page=64)
    lg, x = prefill(dev, d, m, toks, chunk=chunk)
    d.close()
    assert_bits_equal(lg, want_lg, "prefill logits, chunk %d" % chunk)
    assert_bits_equal(x, want_x, "prefill residual, chunk %d" % chunk)


def test_prefill_bad_args(dev):
    m = I.decode_model("a")
    d = make_decoder(dev, m, Q.KV_F32, ORDER_SEQ)
    lg = dev.alloc(4 * m["vocab"])
    with pytest.raises(Q.QrError, match="positions"):
        d.prefill([1, 2, 3], m["seq_len"] - 2, lg.ptr)
    with pytest.raises(Q.QrError, match="token"):
        d.prefill([1, m["vocab"]], 0, lg.ptr)
    with pytest.raises(Q.QrError, match="chunk"):
        d.prefill([1, 2], 0, lg.ptr, chunk=100000)
    d.prefill([], 0, lg.ptr)  # nothing to do
    d.close()
