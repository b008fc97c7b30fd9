"""Closed-form and brute-force pins for the oracle parts the reference's golden
vectors do not reach directly: the corrected Q4_K dot, the integer unit sums,
top-k tie breaking, dispatch, and the shared expert (no reference
counterpart).  Also the synthetic-data quantizers used by tests and bench."""
import numpy as np
import pytest

import inputs as I
from conftest import assert_bits_equal
from oracle import ORDER_SEQ
from quantr_amd import synth


def test_q4k_dot_equals_fp64_dequant_dot(oracle):
    """Corrected Q4_K dot = dequantize_row(type 12) . dequantize(x_q8) up to
    fp32 rounding (the intended value; the reference's own dot is off by ~1e10)."""
    W = synth.weights(11, 64, 2048, synth.TYPE_Q4_K)
    x = synth.normal(12, (2048,))
    xq = oracle.quantize_q8_0(x)
    xd = oracle.dequantize(xq, 8, 2048).astype(np.float64)
    for r in range(64):
        wd = oracle.dequantize(W[r], 12, 2048).astype(np.float64)
        exact = float(wd @ xd)
        scale = float(np.abs(wd * xd).sum())
        assert abs(oracle.vec_dot(12, W[r], xq, 2048) - exact) <= 2e-6 * scale + 1e-30


@pytest.mark.parametrize("qtype", [8, 12, 13, 14])
def test_unit_sums_rebuild_golden_dot(oracle, golden, qtype):
    """The int32 unit sums (qro_row_accum) turned into fp32 terms in the
    reference's order and added sequentially give the reference's dot bits:
    a wrong sum anywhere would change the result."""
    g = golden("dots.npz")
    d = 2048
    x = I.activations(300 + d, 4, d)
    W = I.dot_set(200 + qtype + d, qtype, 15, d)
    f32 = np.float32
    for j in range(4):
        xq = oracle.quantize_q8_0(x[j])
        bd = [oracle.h2f(int(xq[u * 34]) | (int(xq[u * 34 + 1]) << 8)) for u in range(d // 32)]
        for i in range(W.shape[0]):
            isum, bsum = oracle.row_accum(qtype, W[i], xq, d)
            row = W[i]
            s = f32(0.0)
            for u in range(isum.size):
                if qtype == 8:
                    da = oracle.h2f(int(row[u * 34]) | (int(row[u * 34 + 1]) << 8))
                    t = f32(f32(f32(isum[u]) * f32(da)) * f32(bd[u]))
                elif qtype == 14:
                    blk = row[(u // 8) * 210:(u // 8 + 1) * 210]
                    dd = oracle.h2f(int(blk[208]) | (int(blk[209]) << 8))
                    sc = f32(f32(np.int8(blk[192 + u % 8])) * f32(dd))
                    t = f32(f32(sc * f32(isum[u])) * f32(bd[u]))
                else:
                    bb = 144 if qtype == 12 else 176
                    blk = row[(u // 8) * bb:(u // 8 + 1) * bb]
                    dd = oracle.h2f(int(blk[0]) | (int(blk[1]) << 8))
                    dm = oracle.h2f(int(blk[2]) | (int(blk[3]) << 8))
                    sb = int(blk[4 + u % 8])
                    sc = f32(f32(sb & 63) * f32(dd))
                    m = f32(f32(sb >> 6) * f32(dm))
                    t = f32(f32(f32(sc * f32(isum[u])) - f32(m * f32(bsum[u]))) * f32(bd[u]))
                s = f32(s + t)
            assert s.view(np.uint32) == g["dot_c99_%d_%d" % (qtype, d)][i, j].view(np.uint32)


def test_unit_sums_brute_force_tiny(oracle):
    """One super-block: integer sums against an element-by-element decode of
    the bytes (nibble e%2 of byte e/2, fifth bit e%8 of byte e/8, Q6_K pair
    e%4 of byte e/4) and a one-hot activation that reads each element alone."""
    rng = np.random.default_rng(3)
    for qtype, bb in ((12, 144), (13, 176), (14, 210)):
        blk = rng.integers(0, 256, bb, dtype=np.uint8)
        for e in rng.choice(256, 24, replace=False):
            x = np.zeros(256, np.float32)
            x[e] = 127.0  # quantizes to exactly 127 in its block, 0 elsewhere
            xq = oracle.quantize_q8_0(x)
            isum, bsum = oracle.row_accum(qtype, blk, xq, 256)
            if qtype == 12:
                q = (blk[16 + e // 2] >> (4 * (e % 2))) & 15
            elif qtype == 13:
                q = ((blk[48 + e // 2] >> (4 * (e % 2))) & 15) | (((blk[16 + e // 8] >> (e % 8)) & 1) << 4)
            else:
                q = (((blk[e // 2] >> (4 * (e % 2))) & 15) | (((blk[128 + e // 4] >> (2 * (e % 4))) & 3) << 4)) - 32
            assert isum[e // 32] == int(q) * 127 and bsum[e // 32] == 127
            assert (np.delete(isum, e // 32) == 0).all()


def test_topk_brute_force_ties(oracle):
    """K argmax passes with strict '>' = sort by (probability desc, index asc)."""
    rng = np.random.default_rng(4)
    for trial in range(200):
        E, K = int(rng.integers(2, 12)), 0
        K = int(rng.integers(1, E + 1))
        W = np.zeros((E, 4), np.float32)
        levels = rng.integers(0, 3, E).astype(np.float32)  # many exact ties
        W[:, 0] = levels
        x = np.array([1.0, 0, 0, 0], np.float32)
        _, p, idx, w = oracle.route(x, W, E, K, ORDER_SEQ)
        order = np.lexsort((np.arange(E), -p))[:K]
        assert (idx == order).all()
        ws = np.float32(0)
        for v in p[order]:
            ws = np.float32(ws + v)
        assert_bits_equal(w, (p[order] / ws).astype(np.float32), "renorm")


def test_dispatch_invariants(oracle):
    rng = np.random.default_rng(5)
    for T, K, E in ((1, 8, 128), (512, 8, 128), (33, 3, 7)):
        idx = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        counts, offsets, perm, inv = oracle.dispatch(idx, E)
        flat = idx.ravel()
        assert (counts == np.bincount(flat, minlength=E)).all()
        assert offsets[0] == 0 and (np.diff(offsets) == counts).all()
        assert sorted(perm.tolist()) == list(range(T * K)) and (perm[inv] == np.arange(T * K)).all()
        for e in range(E):
            seg = perm[offsets[e]:offsets[e + 1]]
            assert (flat[seg] == e).all() and (np.diff(seg) > 0).all()


def test_shared_expert_closed_form(oracle):
    """sigmoid(g . xb) * down(silu(up . xb) * (gate . xb)), composed from the
    pinned GEMV and expf in the written order (no reference counterpart)."""
    dim, H = 512, 768
    xb = synth.normal(20, (dim,))
    sh = dict(hidden=H, gate_inp=synth.normal(21, (dim,), 0.02),
              up=synth.weights(22, H, dim, 12), gate=synth.weights(23, H, dim, 12),
              down=synth.weights(24, dim, H, 14), up_type=12, down_type=14)
    keep = []
    L = oracle.make_layer(keep, dim, H, 2, 1, np.zeros((2, dim), np.float32), sh["up"], 12,
                          sh["gate"], 12, sh["down"], 14, shared=dict(sh, gate_type=12))
    L.sh_gate_type = 12
    got = oracle.shared_expert(xb, L)
    f32 = np.float32
    u = oracle.matmul_q_fused(xb, sh["up"], 12, H, dim)
    g = oracle.matmul_q_fused(xb, sh["gate"], 12, H, dim)
    e = oracle.expf(-u)
    hb = ((u / (f32(1) + e)).astype(f32) * g).astype(f32)
    y = oracle.matmul_q_fused(hb, sh["down"], 14, dim, H)
    s = f32(0)
    for j in range(dim):
        s = f32(s + f32(sh["gate_inp"][j] * xb[j]))
    sg = f32(f32(1) / f32(f32(1) + oracle.expf(np.array([-s], f32))[0]))
    assert_bits_equal(got, (sg * y).astype(f32), "shared expert")


@pytest.mark.parametrize("qtype,tol", [(8, 0.006), (12, 0.08), (13, 0.04), (14, 0.03)])
def test_synth_quantizers(oracle, qtype, tol):
    """The synthetic-weight quantizers write valid reference-layout blocks
    whose dequantized values track N(0, 0.02) weights."""
    w = synth.normal(30, (16, 2048), 0.02)
    q = synth.quantize(w, qtype)
    deq = np.stack([oracle.dequantize(q[i], qtype, 2048) for i in range(16)])
    assert np.abs(deq - w).max() <= tol * np.abs(w).max()
    if qtype == 8:  # the reference routine itself
        assert (q == np.stack([oracle.quantize_q8_0(r) for r in w])).all()


@pytest.mark.parametrize("kv_type", [0, 2])
def test_attention_closed_form(oracle, kv_type):
    """qro_attention at a shape the reference cannot express (head_dim 128,
    8 query heads over 2 kv heads, 37 positions) against softmax(q K^T /
    sqrt(hd)) V in float64 over the cache's own values (the Q8_0 rows read
    back as qs * d): a wrong kv-head mapping, scale or transposition fails."""
    H, KVH, hd, npos = 8, 2, 128, 37
    rng = np.random.default_rng(31)
    q = rng.standard_normal(H * hd).astype(np.float32)
    kv = rng.standard_normal((2, npos, KVH * hd)).astype(np.float32)
    kc, vc = oracle.kv_rows(kv[0], kv_type), oracle.kv_rows(kv[1], kv_type)
    if kv_type == 2:
        kf = np.stack([oracle.dequantize(r, 8, KVH * hd) for r in kc]).astype(np.float64)
        vf = np.stack([oracle.dequantize(r, 8, KVH * hd) for r in vc]).astype(np.float64)
    else:
        kf, vf = kv[0].astype(np.float64), kv[1].astype(np.float64)
    out, att = oracle.attention(q, kc, vc, kv_type, npos - 1, H, KVH, hd)
    for h in range(H):
        g = h // (H // KVH)
        s = kf[:, g * hd:(g + 1) * hd] @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        np.testing.assert_allclose(att[h], p, rtol=2e-5, atol=1e-7)
        o = p @ vf[:, g * hd:(g + 1) * hd]
        np.testing.assert_allclose(out[h * hd:(h + 1) * hd], o, rtol=1e-4, atol=2e-6)


def test_rope_closed_form(oracle):
    """apply_rope's rotation (src/runtime.c:19-41) in float64: pair i of q
    (over the whole q vector) and of k (only below kv_dim) turns by
    pos * base^(-i / head_dim); position 0 is the identity."""
    qlen, hd, kvh, base = 1024, 128, 2, 1e6
    rng = np.random.default_rng(32)
    q0 = rng.standard_normal(qlen).astype(np.float32)
    k0 = rng.standard_normal(kvh * hd).astype(np.float32)
    q, k = oracle.rope(q0, k0, hd, kvh, 0, base)
    assert np.array_equal(q, q0) and np.array_equal(k[: kvh * hd], k0)
    for pos in (1, 77, 4095):
        q, k = oracle.rope(q0, k0, hd, kvh, pos, base)
        i = np.arange(0, qlen, 2, dtype=np.float64)
        th = pos * base ** (-i / hd)
        c, s = np.cos(th), np.sin(th)
        a, b = q0[0::2].astype(np.float64), q0[1::2].astype(np.float64)
        # float32 theta carries a relative error of a few ulp of pos * freq
        tol = 4e-7 * pos * np.abs(np.hypot(a, b)) + 1e-6
        assert np.all(np.abs(q[0::2] - (a * c - b * s)) <= tol)
        assert np.all(np.abs(q[1::2] - (a * s + b * c)) <= tol)
        n = kvh * hd // 2
        ka, kb = k0[0::2].astype(np.float64), k0[1::2].astype(np.float64)
        assert np.all(np.abs(k[: kvh * hd][0::2] - (ka * c[:n] - kb * s[:n])) <= tol[:n] + 1e-6)
        assert np.all(k[kvh * hd:] == 0)


def test_forward_cached_from_empty_equals_forward_seq(oracle):
    """The cached-forward helper over an empty cache is forward_seq (the path
    the golden logits pin), at the head_dim-128 shape."""
    import inputs as I
    m = I.qwen3_small_model(n_layers=1, seq_len=16)
    toks = [5, 300, 17]
    lg, xs = oracle.forward_seq(m, toks, 0, kv_type=2)
    rs = oracle.kv_row_bytes(2, m["n_kv_heads"] * m["head_dim"])
    kc = np.zeros(m["n_layers"] * m["seq_len"] * rs, np.uint8)
    vc = np.zeros_like(kc)
    lg2, xs2 = oracle.forward_cached(m, kc, vc, toks, 0, 0, 2)
    assert np.array_equal(lg.view(np.uint32), lg2.view(np.uint32))
    assert np.array_equal(xs.view(np.uint32), xs2.view(np.uint32))
