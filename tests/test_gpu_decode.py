"""GPU parity of the single-token decode step (forward_runtime,
src/runtime.c:94-288) and its ops, through the C ABI.

- The decoder against the reference's own logits (tests/golden/decode.npz,
  written by the compiled reference's forward_runtime): two-layer MoE models,
  token by token from position 0, fp32 KV cache, every build -- bit-exact.
- The decoder at a Qwen3-30B-A3B-like head shape the reference cannot express
  (head_dim 128 with q_dim != dim, GQA 4:1) over a prefilled Q8_0 cache with
  a permuted page table, against the oracle's restatement -- bit-exact.
- The ops alone (dequantize, rmsnorm, attention) against the oracle.
"""
import numpy as np
import pytest

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


def run_tokens(dev, d, m, tokens, pos0=0):
    lg_d, x_d = dev.alloc(4 * m["vocab"]), dev.alloc(4 * m["dim"])
    lg = np.zeros((len(tokens), m["vocab"]), np.float32)
    xs = np.zeros((len(tokens), m["dim"]), np.float32)
    for i, t in enumerate(tokens):
        d.forward(int(t), pos0 + i, lg_d.ptr, x_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
        xs[i] = dev.download(x_d, m["dim"], np.float32)
    return lg, xs


@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("graph", [0, Q.DEC_GRAPH], ids=["eager", "graph"])
@pytest.mark.parametrize("build", list(BUILDS))
@pytest.mark.parametrize("name", list(I.DECODE_CASES))
def test_decoder_matches_reference_logits(dev, golden, name, build, graph, kv):
    """The reference's own logits and residuals, with its fp32 KV cache and
    with its fp16 one (kv_cache_type 1, src/runtime.c:74-92)."""
    g = golden("decode.npz")
    m = I.decode_model(name)
    assert I.decode_digest(m) == str(g["sha_" + name])
    tag = "" if kv == "f32" else "16"
    key = "logits%s_%s_%s" % (tag, name, build)
    if key not in g:
        pytest.skip("fixture written without an -mavx512f build")
    print("decode case %s build %s graph %d kv %s" % (name, build, graph, kv), flush=True)
    d = make_decoder(dev, m, Q.KV_F16 if kv == "f16" else Q.KV_F32, BUILDS[build], flags=graph)
    lg, xs = run_tokens(dev, d, m, m["tokens"])
    d.close()
    assert_bits_equal(xs, g["x%s_%s_%s" % (tag, name, build)], "residual %s/%s" % (name, build))
    assert_bits_equal(lg, g[key], "logits %s/%s" % (name, build))


def prefilled(oracle, m, npre, seed, kv_type=Q.KV_Q8_0):
    """Seeded N(0, 1) K / V values for positions 0 .. npre-1 of every layer
    and the oracle's contiguous cache holding them."""
    L, kvd = m["n_layers"], m["n_kv_heads"] * m["head_dim"]
    rng = np.random.default_rng(seed)
    kv = rng.standard_normal((L, 2, npre, kvd)).astype(np.float32)
    rs = oracle.kv_row_bytes(kv_type, kvd)
    kc = np.zeros((L, m["seq_len"], rs), np.uint8)
    vc = np.zeros_like(kc)
    for l in range(L):
        kc[l, :npre] = oracle.kv_rows(kv[l, 0], kv_type)
        vc[l, :npre] = oracle.kv_rows(kv[l, 1], kv_type)
    return kv, kc, vc


@pytest.mark.parametrize("graph", [0, Q.DEC_GRAPH], ids=["eager", "graph"])
@pytest.mark.parametrize("order,kvh,kv_type", [(ORDER_SEQ, 2, Q.KV_Q8_0), (ORDER_AVX2, 2, Q.KV_Q8_0),
                                               (ORDER_AVX2, 1, Q.KV_Q8_0),
                                               (ORDER_AVX2, 1, Q.KV_F16)],
                         ids=["seq_gqa4", "avx2_gqa4", "avx2_gqa8", "avx2_gqa8_f16"])
def test_decoder_q8_cache_head128(dev, oracle, order, kvh, kv_type, graph):
    """Qwen3-like heads (head_dim 128, q_dim 1024 != dim 512, 8 heads over 2
    kv heads, or over 1: GQA 8:1, the Qwen3-30B-A3B ratio) over a Q8_0 (or
    fp16) cache prefilled to 517 positions through a permuted page table
    (pages of 64), then three decode steps at 517..519: logits, residual and
    the cache rows the steps wrote, bit-exact with the oracle."""
    m = I.qwen3_small_model(n_layers=2, seq_len=640, n_kv_heads=kvh)
    npre = 517
    kv, kc, vc = prefilled(oracle, m, npre, seed=41, kv_type=kv_type)
    print("decode head128 order %d kv heads %d kv %d graph %d" % (order, kvh, kv_type, graph),
          flush=True)
    d = make_decoder(dev, m, kv_type, order, page=64, flags=graph)
    ppl, page = d.pages()
    assert (ppl, page) == (10, 64)
    rng = np.random.default_rng(5)
    d.set_pages(np.stack([rng.permutation(ppl) for _ in range(m["n_layers"])]).astype(np.int32))
    for l in range(m["n_layers"]):
        kb, vb = dev.upload(kv[l, 0]), dev.upload(kv[l, 1])
        d.kv_write(l, 0, npre, kb.ptr, vb.ptr)
    rs = kc.shape[2]
    # the prefill's rows are the oracle's quantize_row_q8_0 rows
    for l, t in ((0, 0), (1, 63), (1, 64), (0, npre - 1)):
        kr, vr = d.kv_rows(l, t)
        assert np.array_equal(dev.download(kr, rs, np.uint8), kc[l, t])
        assert np.array_equal(dev.download(vr, rs, np.uint8), vc[l, t])
    toks = [11, 319, 200]
    lg, xs = run_tokens(dev, d, m, toks, pos0=npre)
    wl, wx = oracle.forward_cached(m, kc.reshape(-1), vc.reshape(-1), toks, npre, order, kv_type)
    for l in range(m["n_layers"]):
        for t in range(npre, npre + len(toks)):
            kr, vr = d.kv_rows(l, t)
            assert np.array_equal(dev.download(kr, rs, np.uint8), kc[l, t]), (l, t)
            assert np.array_equal(dev.download(vr, rs, np.uint8), vc[l, t]), (l, t)
    d.close()
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")


@pytest.mark.parametrize("tiled", [False, True], ids=["rows", "tiled"])
def test_decoder_stacked_qk(dev, oracle, tiled):
    """wq and wk of one type stored back to back (the decoder then runs them
    as one GEMV of q_dim + kv_dim rows), row-major and in the tiled layout:
    three decode steps over a Q8_0 cache, bit-exact with the oracle."""
    m = I.qwen3_small_model(n_layers=2, seq_len=640)
    H, KVH, hd, dim = m["n_heads"], m["n_kv_heads"], m["head_dim"], m["dim"]
    wt = list(m["wtype"])
    wt[1] = Q.TYPE_Q4_K
    m["wtype"] = wt
    keep = []
    for l, lw in enumerate(m["layers"]):
        lw["wk"] = I._rows(9700 + l, Q.TYPE_Q4_K, KVH * hd, dim)
    npre = 130
    kv, kc, vc = prefilled(oracle, m, npre, seed=43)
    mdev = dict(m)
    mdev["layers"] = [dict(lw) for lw in m["layers"]]
    for lw in mdev["layers"]:
        qb, kb = lw["wq"].reshape(-1), lw["wk"].reshape(-1)
        both = dev.upload(np.concatenate([qb, kb]))
        keep.append(both)
        if tiled:
            t = dev.alloc(qb.nbytes + kb.nbytes)
            keep.append(t)
            dev.tile(Q.TYPE_Q4_K, both.ptr, t.ptr, H * hd + KVH * hd, dim)
            dev.sync()
            both = t
        lw["wq"], lw["wk"] = both.ptr, both.ptr + qb.nbytes
    if tiled:
        mdev["wtype"] = [wt[0] | Q.TILED, wt[1] | Q.TILED, wt[2], wt[3]]
    print("decode stacked qk tiled %d" % tiled, flush=True)
    d = make_decoder(dev, mdev, Q.KV_Q8_0, ORDER_AVX2, page=64)
    for l in range(m["n_layers"]):
        kb, vb = dev.upload(kv[l, 0]), dev.upload(kv[l, 1])
        d.kv_write(l, 0, npre, kb.ptr, vb.ptr)
    toks = [5, 300, 77]
    lg, xs = run_tokens(dev, d, mdev, toks, pos0=npre)
    d.close()
    wl, wx = oracle.forward_cached(m, kc.reshape(-1), vc.reshape(-1), toks, npre, ORDER_AVX2,
                                   Q.KV_Q8_0)
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")


@pytest.mark.parametrize("qtype", [Q.TYPE_F32, Q.TYPE_Q8_0, Q.TYPE_Q4_K, Q.TYPE_Q5_K,
                                   Q.TYPE_Q6_K])
def test_dequantize(dev, oracle, qtype):
    """dequantize_row (src/quant.c:160-240) of 7 rows of 512: bit-exact."""
    rows, n = 7, 512
    src = I._rows(60 + qtype, qtype, rows, n)
    out = dev.alloc(rows * n * 4)
    sb = dev.upload(src)
    dev.dequantize(qtype, sb.ptr, rows, n, out.ptr)
    got = dev.download(out, (rows, n), np.float32)
    want = np.stack([oracle.dequantize(np.ascontiguousarray(src[r]).view(np.uint8), qtype, n)
                     for r in range(rows)])
    assert_bits_equal(got, want, "dequantize type %d" % qtype)


@pytest.mark.parametrize("n", [64, 2048, 5120, 8192])
def test_rmsnorm(dev, oracle, n):
    """rmsnorm_ref (src/kernels.c:170-180), alone and after the residual add:
    bit-exact."""
    x = I.activations(70, 1, n)[0]
    a = I.activations(71, 1, n, std=0.5)[0]
    w = (1.0 + I.activations(72, 1, n, std=0.1)[0]).astype(np.float32)
    xd, ad, wd, od = dev.upload(x), dev.upload(a), dev.upload(w), dev.alloc(4 * n)
    dev.rmsnorm(od.ptr, xd.ptr, wd.ptr, n)
    assert_bits_equal(dev.download(od, n, np.float32), oracle.rmsnorm(x, w), "rmsnorm")
    dev.rmsnorm(od.ptr, xd.ptr, wd.ptr, n, add_ptr=ad.ptr)
    xs = (x + a).astype(np.float32)
    assert_bits_equal(dev.download(xd, n, np.float32), xs, "residual")
    assert_bits_equal(dev.download(od, n, np.float32), oracle.rmsnorm(xs, w), "rmsnorm(x + a)")


@pytest.mark.parametrize("kv_type", [Q.KV_F32, Q.KV_F16, Q.KV_Q8_0])
@pytest.mark.parametrize("npos,H,KVH,hd", [(1, 4, 4, 64), (130, 8, 2, 128), (4097, 32, 4, 128),
                                           (300, 4, 1, 512)])
def test_attention(dev, oracle, kv_type, npos, H, KVH, hd):
    """The attention of src/runtime.c:136-193 over a paged cache (pages of 128
    in reversed order): weights and outputs bit-exact with the oracle,
    including the Qwen3-30B-A3B shape (32 heads over 4, head_dim 128) at 4097
    positions and head_dim 512 (the reference's kh_buf bound)."""
    kvd = KVH * hd
    rng = np.random.default_rng(npos + hd)
    q = rng.standard_normal(H * hd).astype(np.float32)
    kv = rng.standard_normal((2, npos, kvd)).astype(np.float32)
    kc, vc = oracle.kv_rows(kv[0], kv_type), oracle.kv_rows(kv[1], kv_type)
    print("attention npos %d H %d KVH %d hd %d kv %d" % (npos, H, KVH, hd, kv_type), flush=True)
    page = 128
    npages = (npos + page - 1) // page
    ptab = np.arange(npages, dtype=np.int32)[::-1].copy()
    rs = kc.shape[1]
    kp = np.zeros((npages * page, rs), np.uint8)
    vp = np.zeros_like(kp)
    for t in range(npos):
        slot = ptab[t // page] * page + t % page
        kp[slot], vp[slot] = kc[t], vc[t]
    qd, kd, vd, pd = dev.upload(q), dev.upload(kp), dev.upload(vp), dev.upload(ptab)
    att, out = dev.alloc(4 * H * npos), dev.alloc(4 * H * hd)
    dev.attention(qd.ptr, kd.ptr, vd.ptr, pd.ptr, page, kv_type, npos, H, KVH, hd, att.ptr,
                  out.ptr)
    wo, wa = oracle.attention(q, kc, vc, kv_type, npos - 1, H, KVH, hd)
    assert_bits_equal(dev.download(att, (H, npos), np.float32), wa, "weights")
    assert_bits_equal(dev.download(out, H * hd, np.float32), wo, "output")


def test_decoder_rejects_bad_arguments(dev):
    m = I.qwen3_small_model(n_layers=1, seq_len=64)
    model, layers, keep = Q.upload_decode_model(dev, m)
    with pytest.raises(Q.QrError, match="head_dim"):
        model.head_dim = 100
        Q.Decoder(dev, model, layers)
    model.head_dim = 128
    d = Q.Decoder(dev, model, layers, page=16)
    lg = dev.alloc(4 * m["vocab"])
    with pytest.raises(Q.QrError, match="pos"):
        d.forward(1, 64, lg.ptr)
    with pytest.raises(Q.QrError, match="token"):
        d.forward(m["vocab"], 0, lg.ptr)
    with pytest.raises(Q.QrError, match="permutation"):
        d.set_pages(np.zeros((1, 4), np.int32))
    d.close()


@pytest.mark.parametrize("qk_type", [Q.TYPE_Q4_K, Q.TYPE_Q5_K], ids=["qk_q4k", "qk_q5k"])
@pytest.mark.parametrize("wv_tiled", [False, True], ids=["wv_rows", "wv_tiled"])
@pytest.mark.parametrize("order", [ORDER_SEQ, ORDER_AVX2], ids=["c99", "avx2"])
def test_decode_stacked_qk_q8_v(dev, oracle, order, wv_tiled, qk_type):
    """wq and wk back to back in the tiled Q4_K / Q5_K layout and a Q8_0 wv: in the
    C99 build the attention norm, q / k and v run in one launch (the v matrix
    tiled by the caller, or a tiled copy the decoder makes); in the AVX2
    build v keeps its own GEMV (the tiled Q8_0 dot is the C99 order, so a
    tiled Q8_0 v is refused there).  Four decode steps from position 0,
    graph-replayed, bit-exact with the oracle."""
    m = I.qwen3_small_model(n_layers=2, seq_len=64)
    H, KVH, hd, dim = m["n_heads"], m["n_kv_heads"], m["head_dim"], m["dim"]
    qd, kvd = H * hd, KVH * hd
    m["wtype"] = [qk_type, qk_type, Q.TYPE_Q8_0, Q.TYPE_Q5_K]
    for l, lw in enumerate(m["layers"]):
        lw["wq"] = I._rows(9590 + l, qk_type, qd, dim)
        lw["wk"] = I._rows(9600 + l, qk_type, kvd, dim)
        lw["wv"] = I._rows(9610 + l, Q.TYPE_Q8_0, kvd, dim)
    mdev = dict(m)
    mdev["layers"] = [dict(lw) for lw in m["layers"]]
    keep = []
    for lw in mdev["layers"]:
        qk = np.concatenate([lw["wq"].reshape(-1), lw["wk"].reshape(-1)])
        src = dev.upload(qk)
        both = dev.alloc(qk.nbytes)
        dev.tile(qk_type, src.ptr, both.ptr, qd + kvd, dim)
        keep += [src, both]
        lw["wq"], lw["wk"] = both.ptr, both.ptr + lw["wq"].nbytes
        if wv_tiled:
            vs = dev.upload(lw["wv"])
            vt = dev.alloc(lw["wv"].nbytes)
            dev.tile(Q.TYPE_Q8_0, vs.ptr, vt.ptr, kvd, dim)
            keep += [vs, vt]
            lw["wv"] = vt.ptr
    dev.sync()
    mdev["wtype"] = [qk_type | Q.TILED, qk_type | Q.TILED,
                     Q.TYPE_Q8_0 | (Q.TILED if wv_tiled else 0), Q.TYPE_Q5_K]
    model, layers, k2 = Q.upload_decode_model(dev, mdev)
    print("stacked qk, Q8_0 v (tiled %d) order %d" % (wv_tiled, order), flush=True)
    if wv_tiled and order != ORDER_SEQ:  # tiled Q8_0 holds only the C99 dot order
        with pytest.raises(Q.QrError, match="tiled type 8"):
            Q.Decoder(dev, model, layers, kv_type=Q.KV_Q8_0, order=order, page=16)
        return
    d = Q.Decoder(dev, model, layers, kv_type=Q.KV_Q8_0, order=order, page=16,
                  flags=Q.DEC_GRAPH)
    toks = [5, 300, 5, 17]
    lg_d, x_d = dev.alloc(4 * m["vocab"]), dev.alloc(4 * m["dim"])
    lg = np.zeros((len(toks), m["vocab"]), np.float32)
    xs = np.zeros((len(toks), m["dim"]), np.float32)
    for i, t in enumerate(toks):
        d.forward(t, i, lg_d.ptr, x_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
        xs[i] = dev.download(x_d, m["dim"], np.float32)
    d.close()
    del k2, keep
    wl, wx = oracle.forward_seq(m, toks, order, Q.KV_Q8_0)
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")


@pytest.mark.parametrize("order,graph", [(ORDER_SEQ, Q.DEC_GRAPH), (ORDER_AVX2, 0)],
                         ids=["c99_graph", "avx2_eager"])
def test_decode_shared_expert(dev, oracle, order, graph):
    """A MoE decoder whose layers also have a shared expert with a sigmoid gate
    (Qwen1.5-MoE's layer form): the router's launch forms the FFN norm and the
    shared gate logit beside the router logits, the shared gate / up rows run
    in the gate / up launch and its down on the GEMV.  Four decode steps
    bit-exact with the oracle."""
    m = I.qwen3_small_model(n_layers=2, seq_len=64)
    dim, sh = m["dim"], 512
    for l, lw in enumerate(m["layers"]):
        s = 9660 + 10 * l
        lw["shared"] = dict(hidden=sh, gate_inp=I.activations(s, 1, dim, std=0.05)[0],
                            up=I._rows(s + 1, Q.TYPE_Q4_K, sh, dim).reshape(-1),
                            gate=I._rows(s + 2, Q.TYPE_Q4_K, sh, dim).reshape(-1),
                            down=I._rows(s + 3, Q.TYPE_Q6_K, dim, sh).reshape(-1),
                            up_type=Q.TYPE_Q4_K, down_type=Q.TYPE_Q6_K)
    toks = [5, 300, 5, 17]
    print("decode shared expert order %d graph %d" % (order, graph), flush=True)
    model, layers, keep = Q.upload_decode_model(dev, m)
    d = Q.Decoder(dev, model, layers, kv_type=Q.KV_Q8_0, order=order, page=16, flags=graph)
    lg_d, x_d = dev.alloc(4 * m["vocab"]), dev.alloc(4 * m["dim"])
    lg = np.zeros((len(toks), m["vocab"]), np.float32)
    xs = np.zeros((len(toks), m["dim"]), np.float32)
    for i, t in enumerate(toks):
        d.forward(t, i, lg_d.ptr, x_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
        xs[i] = dev.download(x_d, m["dim"], np.float32)
    d.close()
    del keep
    wl, wx = oracle.forward_seq(m, toks, order, Q.KV_Q8_0)
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")
