"""GPU parity of the decode step and of a prefill at the full Qwen3-30B-A3B
shape (forward_runtime, src/runtime.c:94-288): dim 2048, 32 query heads over
4 kv heads of 128, 128 experts top-8 with ffn 768 (gate / up Q4_K, down
Q6_K), the 151936-row Q6_K lm_head, a Q8_0 KV cache in permuted pages of
256 -- the weights laid out as the benchmark lays them (wq and wk back to
back, wq / wk / wo in the tiled layout, wv Q6_K row-major).

Two distinct layers (about 400 MB of expert weights each) stand for the 48:
every layer runs the same kernels, and the oracle's cost grows with each.

- Three decode steps at positions 4096..4098 over a cache prefilled to 4096
  positions, eager and graph-replayed: logits, residual and the cache rows
  the steps wrote, bit-exact with the oracle.
- 160 prompt tokens at positions 3930..4089 in chunks of 128: the first
  chunk ends at 4058, where the prefill's attention values run the GQA
  kernel (the eight query heads of a kv head in one workgroup); the second
  ends at 4090, past that kernel's LDS limit (4088 at this shape), where
  they run per query head.  Every position's logits, the last residual and
  the written cache rows, bit-exact with the oracle.
"""
import numpy as np
import pytest

import inputs as I
import quantr_amd as Q
from conftest import assert_bits_equal
from oracle import ORDER_AVX2

pytestmark = pytest.mark.gpu

PAGE = 256
NPRE = 4096


@pytest.fixture(scope="module")
def full(dev, oracle):
    print("qwen3 full shape: building 2 layers", flush=True)
    m = I.qwen3_full_model(n_layers=2)
    H, KVH, hd, dim = m["n_heads"], m["n_kv_heads"], m["head_dim"], m["dim"]
    qd, kvd = H * hd, KVH * hd
    keep = []
    mdev = dict(m)
    mdev["layers"] = [dict(lw) for lw in m["layers"]]
    for lw in mdev["layers"]:
        # [wq | wk] tiled as one matrix of qd + kvd rows (the same bytes as tiling
        # each: 8-row tiles never straddle the two), then wv and wo
        qk = np.concatenate([lw["wq"].reshape(-1), lw["wk"].reshape(-1)])
        src = dev.upload(qk)
        both = dev.alloc(qk.nbytes)
        dev.tile(Q.TYPE_Q4_K, src.ptr, both.ptr, qd + kvd, dim)
        wo_src = dev.upload(lw["wo"])
        wo = dev.alloc(lw["wo"].nbytes)
        dev.tile(Q.TYPE_Q4_K, wo_src.ptr, wo.ptr, dim, qd)
        dev.sync()
        src.free()
        wo_src.free()
        keep += [both, wo]
        lw["wq"], lw["wk"], lw["wo"] = both.ptr, both.ptr + lw["wq"].nbytes, wo.ptr
    mdev["wtype"] = [Q.TYPE_Q4_K | Q.TILED, Q.TYPE_Q4_K | Q.TILED, Q.TYPE_Q6_K,
                     Q.TYPE_Q4_K | Q.TILED]
    model, layers, k2 = Q.upload_decode_model(dev, mdev)
    keep += k2
    L = m["n_layers"]
    rng = np.random.default_rng(77)
    kv = rng.standard_normal((L, 2, NPRE, kvd)).astype(np.float32)
    rs = oracle.kv_row_bytes(Q.KV_Q8_0, kvd)
    kc = np.zeros((L, m["seq_len"], rs), np.uint8)
    vc = np.zeros_like(kc)
    for l in range(L):
        kc[l, :NPRE] = oracle.kv_rows(kv[l, 0], Q.KV_Q8_0)
        vc[l, :NPRE] = oracle.kv_rows(kv[l, 1], Q.KV_Q8_0)
    npages = m["seq_len"] // PAGE
    table = np.stack([rng.permutation(npages) for _ in range(L)]).astype(np.int32)
    yield dict(m=m, model=model, layers=layers, kv=kv, kc=kc, vc=vc, rs=rs, table=table,
               memo={})
    for b in keep:
        if isinstance(b, Q.DevBuf):
            b.free()


def decoder(dev, f, npre, flags=0):
    m = f["m"]
    d = Q.Decoder(dev, f["model"], f["layers"], kv_type=Q.KV_Q8_0, order=ORDER_AVX2, page=PAGE,
                  flags=flags)
    ppl, page = d.pages()
    assert (ppl, page) == (m["seq_len"] // PAGE, PAGE)
    d.set_pages(f["table"])
    for l in range(m["n_layers"]):
        kb, vb = dev.upload(f["kv"][l, 0, :npre]), dev.upload(f["kv"][l, 1, :npre])
        d.kv_write(l, 0, npre, kb.ptr, vb.ptr)
        dev.sync()
        kb.free()
        vb.free()
    return d


def oracle_run(oracle, f, npre, toks):
    """The oracle from a cache holding positions 0 .. npre - 1 (memoised)."""
    key = (npre, tuple(toks))
    if key not in f["memo"]:
        kc, vc = f["kc"].copy(), f["vc"].copy()
        kc[:, npre:] = 0
        vc[:, npre:] = 0
        lg, xs = oracle.forward_cached(f["m"], kc.reshape(-1), vc.reshape(-1), list(toks), npre,
                                       ORDER_AVX2, Q.KV_Q8_0)
        f["memo"][key] = (lg, xs, kc, vc)
    return f["memo"][key]


def check_rows(dev, d, f, kc, vc, positions):
    for l in range(f["m"]["n_layers"]):
        for t in positions:
            kr, vr = d.kv_rows(l, t)
            assert np.array_equal(dev.download(kr, f["rs"], np.uint8), kc[l, t]), ("K", l, t)
            assert np.array_equal(dev.download(vr, f["rs"], np.uint8), vc[l, t]), ("V", l, t)


@pytest.mark.parametrize("graph", [0, Q.DEC_GRAPH], ids=["eager", "graph"])
def test_decode_qwen3_full(dev, oracle, full, graph):
    f, m = full, full["m"]
    toks = [11, 151935, 70000]
    print("qwen3 full decode graph %d" % graph, flush=True)
    d = decoder(dev, f, NPRE, flags=graph)
    # the prefilled rows are the oracle's quantize_row_q8_0 rows
    check_rows(dev, d, f, f["kc"], f["vc"], [0, 255, 256, 4095])
    lg_d, x_d = dev.alloc(4 * m["vocab"]), dev.alloc(4 * m["dim"])
    lg = np.zeros((len(toks), m["vocab"]), np.float32)
    xs = np.zeros((len(toks), m["dim"]), np.float32)
    for i, t in enumerate(toks):
        d.forward(t, NPRE + i, lg_d.ptr, x_d.ptr)
        lg[i] = dev.download(lg_d, m["vocab"], np.float32)
        xs[i] = dev.download(x_d, m["dim"], np.float32)
    print("qwen3 full decode: oracle", flush=True)
    wl, wx, kc, vc = oracle_run(oracle, f, NPRE, toks)
    check_rows(dev, d, f, kc, vc, range(NPRE, NPRE + len(toks)))
    d.close()
    assert_bits_equal(xs, wx, "residual")
    assert_bits_equal(lg, wl, "logits")


def test_prefill_qwen3_full(dev, oracle, full):
    f, m = full, full["m"]
    p0, n = 3930, 160
    toks = np.random.default_rng(23).integers(0, m["vocab"], size=n).astype(np.int32)
    print("qwen3 full prefill %d tokens at %d, chunks of 128" % (n, p0), flush=True)
    d = decoder(dev, f, p0)
    lg_d, x_d = dev.alloc(4 * m["vocab"] * n), dev.alloc(4 * m["dim"])
    d.prefill(toks, p0, lg_d.ptr, x_d.ptr, chunk=128, all_logits=True)
    lg = dev.download(lg_d, (n, m["vocab"]), np.float32)
    x = dev.download(x_d, m["dim"], np.float32)
    lg_d.free()
    print("qwen3 full prefill: oracle", flush=True)
    wl, wx, kc, vc = oracle_run(oracle, f, p0, toks)
    check_rows(dev, d, f, kc, vc, [p0, p0 + 127, p0 + 128, p0 + n - 1])
    d.close()
    assert_bits_equal(x, wx[-1], "prefill residual")
    assert_bits_equal(lg, wl, "prefill logits")
