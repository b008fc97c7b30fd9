"""GPU parity of the MoE layer against the oracle, through the C ABI.

Bit-exact: router top-k indices and weights, dispatch permutation, and the
layer output (the oracle's per-token block, src/runtime.c:202-269, which the
CPU suite pins to the reference's own forward_runtime).  The order argument
names the reference build: the router's accumulation order and the Q8_0 dot
order; the oracle is asked for the same build.
"""
import ctypes as C

import numpy as np
import pytest

import inputs as I
import quantr_amd as Q
from conftest import assert_bits_equal
from oracle import ORDER_AVX2, ORDER_AVX512, ORDER_SEQ, Oracle
from quantr_amd import synth

pytestmark = pytest.mark.gpu


class DevLayer:
    """A MoE layer uploaded to the device, plus the host copies for the oracle."""

    def __init__(self, dev, dim, hidden, E, K, router, up, gate, down, ut, dt, shared=None):
        self.h = dict(dim=dim, hidden=hidden, E=E, K=K, router=router, up=up, gate=gate,
                      down=down, ut=ut, dt=dt, shared=shared)
        self.bufs = [dev.upload(router), dev.upload(up), dev.upload(gate), dev.upload(down)]
        L = Q.MoeLayer(dim, hidden, E, K, *[b.ptr for b in self.bufs], ut, ut, dt)
        if shared is not None:
            sb = [dev.upload(shared["gate_inp"]), dev.upload(shared["up"]),
                  dev.upload(shared["gate"]), dev.upload(shared["down"])]
            self.bufs += sb
            L.sh_hidden = shared["hidden"]
            L.sh_gate_inp, L.sh_up, L.sh_gate, L.sh_down = [b.ptr for b in sb]
            L.sh_up_type = L.sh_gate_type = shared["up_type"]
            L.sh_down_type = shared["down_type"]
        self.L = L

    def oracle_layer(self, keep):
        h = self.h
        return Oracle.make_layer(keep, h["dim"], h["hidden"], h["E"], h["K"], h["router"], h["up"],
                                 h["ut"], h["gate"], h["ut"], h["down"], h["dt"],
                                 shared=h["shared"])


def run_moe(dev, layer, x, xb, order):
    T, dim = x.shape
    K = layer.L.n_used
    xd, xbd = dev.upload(x), dev.upload(xb)
    idx, w = dev.alloc(T * K * 4), dev.alloc(T * K * 4)
    dev.moe_forward(layer.L, xd.ptr, xbd.ptr, T, order, idx.ptr, w.ptr)
    return (dev.download(xd, (T, dim), np.float32), dev.download(idx, (T, K), np.int32),
            dev.download(w, (T, K), np.float32))


def check_moe(dev, oracle, layer, x, xb, order, what):
    """The layer in the reference build `order` (router and Q8_0 dot orders)."""
    got, gi, gw = run_moe(dev, layer, x, xb, order)
    keep = []
    want, wi, ww = oracle.moe_forward(x, xb, layer.oracle_layer(keep), order=order,
                                      dot_order=order, threads=16)
    assert (gi == wi).all(), "%s: routing indices differ" % what
    assert_bits_equal(gw, ww, what + " routing weights")
    assert_bits_equal(got, want, what + " layer output")


def random_layer(dev, name):
    m = I.moe_inputs(name)
    return DevLayer(dev, m["dim"], m["hidden"], m["E"], m["K"], m["router"], m["up"], m["gate"],
                    m["down"], m["up_type"], m["down_type"]), m


@pytest.mark.parametrize("name", sorted(I.MOE_CASES))
@pytest.mark.parametrize("order", [ORDER_SEQ, ORDER_AVX2])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_moe_golden_shapes(dev, oracle, name, order, T):
    """The golden MoE cases (random block bytes) at several token counts."""
    layer, m = random_layer(dev, name)
    x = I.activations(800 + T, T, m["dim"])
    xb = I.activations(801 + T, T, m["dim"])
    check_moe(dev, oracle, layer, x, xb, order, "case %s T=%d" % (name, T))


@pytest.mark.parametrize("name", sorted(I.MOE_CASES))
def test_moe_matches_reference_fixture(dev, golden, name):
    """End to end against the reference's own forward_runtime output
    (tests/golden/moe.npz) of each build: -std=c99, -mavx2 -mfma and
    -mavx512f, with Q4_K / Q6_K, Q8_0 / Q8_0 (lane-order Q8_0 dots in the
    vector builds) and Q5_K / Q6_K experts."""
    g = golden("moe.npz")
    layer, m = random_layer(dev, name)
    for build, order in (("c99", ORDER_SEQ), ("avx2", ORDER_AVX2), ("avx512", ORDER_AVX512)):
        xb = g["xb_%s_%s" % (name, build)]
        got, _, _ = run_moe(dev, layer, m["x"], xb, order)
        assert_bits_equal(got, g["xo_%s_%s" % (name, build)], "reference %s/%s" % (name, build))


_QWEN3 = {}


def qwen3_layer(dev):
    """Qwen3-30B-A3B-shaped layer: 2048 wide, 128 experts top-8, ffn 768,
    gate/up Q4_K, down Q6_K, N(0, 0.02) weights, Zipf(1.1) router skew."""
    if "layer" not in _QWEN3:
        dim, hidden, E, K = 2048, 768, 128, 8
        router, u, _ = synth.zipf_router(3000, E, dim)
        up = synth.weights(3001, E * hidden, dim, Q.TYPE_Q4_K)
        gate = synth.weights(3002, E * hidden, dim, Q.TYPE_Q4_K)
        down = synth.weights(3003, E * dim, hidden, Q.TYPE_Q6_K)
        _QWEN3["layer"] = DevLayer(dev, dim, hidden, E, K, router, up, gate, down, Q.TYPE_Q4_K,
                                   Q.TYPE_Q6_K)
        _QWEN3["u"] = u
    return _QWEN3["layer"], _QWEN3["u"]


@pytest.mark.parametrize("T", [1, 16, 64])
@pytest.mark.parametrize("order", [ORDER_SEQ, ORDER_AVX2])
def test_moe_qwen3_shape(dev, oracle, T, order):
    layer, u = qwen3_layer(dev)
    xb = synth.zipf_tokens(3100 + T, T, 2048, u)
    x = synth.normal(3200 + T, (T, 2048))
    check_moe(dev, oracle, layer, x, xb, order, "qwen3 T=%d" % T)


@pytest.mark.parametrize("path", [Q.MOE_PATH_GEMV, Q.MOE_PATH_MFMA], ids=["gemv", "mfma"])
@pytest.mark.parametrize("T", [2, 5, 16, 64])
def test_moe_qwen3_forced_path(dev, oracle, T, path):
    """Either expert product at any token count (qr_ctx_set_moe_path): the
    grouped GEMV at counts where the default takes the MFMA products and the
    reverse; bit-exact either way."""
    layer, u = qwen3_layer(dev)
    xb = synth.zipf_tokens(3300 + T, T, 2048, u)
    x = synth.normal(3400 + T, (T, 2048))
    dev.set_moe_path(path)
    try:
        check_moe(dev, oracle, layer, x, xb, ORDER_AVX2, "qwen3 T=%d path %d" % (T, path))
    finally:
        dev.set_moe_path(Q.MOE_PATH_AUTO)


def test_moe_qwen3_t512_routing_and_output(dev, oracle):
    """T = 512: routing and dispatch bit-exact; output bit-exact on every token."""
    layer, u = qwen3_layer(dev)
    T = 512
    xb = synth.zipf_tokens(3512, T, 2048, u)
    x = synth.normal(3513, (T, 2048))
    check_moe(dev, oracle, layer, x, xb, ORDER_AVX2, "qwen3 T=512")


def test_moe_qwen15_shared_expert(dev, oracle):
    """Qwen1.5-MoE-A2.7B shape: 60 experts top-4, ffn 1408 (gate/up Q4_K; the
    1408-wide down projection stored Q8_0, since 1408 is not a whole number of
    256-blocks), shared expert ffn 5632 Q4_K with a sigmoid gate."""
    dim, hidden, E, K, SH = 2048, 1408, 60, 4, 5632
    router = synth.normal(4000, (E, dim), 0.02)
    up = synth.weights(4001, E * hidden, dim, Q.TYPE_Q4_K)
    gate = synth.weights(4002, E * hidden, dim, Q.TYPE_Q4_K)
    down = synth.weights(4003, E * dim, hidden, Q.TYPE_Q8_0)
    shared = dict(hidden=SH, gate_inp=synth.normal(4004, (dim,), 0.02),
                  up=synth.weights(4005, SH, dim, Q.TYPE_Q4_K),
                  gate=synth.weights(4006, SH, dim, Q.TYPE_Q4_K),
                  down=synth.weights(4007, dim, SH, Q.TYPE_Q4_K),
                  up_type=Q.TYPE_Q4_K, down_type=Q.TYPE_Q4_K)
    layer = DevLayer(dev, dim, hidden, E, K, router, up, gate, down, Q.TYPE_Q4_K, Q.TYPE_Q8_0,
                     shared=shared)
    # T <= 4: the shared expert on the GEMV engines; T > 4: on the MFMA products
    for T, order in ((1, ORDER_SEQ), (3, ORDER_SEQ), (5, ORDER_AVX2), (8, ORDER_SEQ),
                     (64, ORDER_SEQ), (1, ORDER_AVX2), (64, ORDER_AVX2)):
        xb = synth.normal(4100 + T, (T, dim))
        x = synth.normal(4200 + T, (T, dim))
        check_moe(dev, oracle, layer, x, xb, order, "qwen1.5 T=%d order %d" % (T, order))


@pytest.mark.parametrize("order", [ORDER_SEQ, ORDER_AVX2])
def test_route_topk_probs(dev, oracle, order):
    """Router logits, softmax probabilities, top-8 indices and renormalised
    weights for 64 tokens, with exact ties planted in the router rows."""
    E, K, dim, T = 128, 8, 2048, 64
    W = I.activations(5000, E, dim, std=0.02)
    W[7] = W[3]  # identical experts tie on every token: lowest index must win
    W[100] = W[3]
    X = I.activations(5001, T, dim)
    wb, xb = dev.upload(W), dev.upload(X)
    L = Q.MoeLayer(dim, 768, E, K, wb.ptr, None, None, None, 0, 0, 0)
    pb, ib, wtb = dev.alloc(T * E * 4), dev.alloc(T * K * 4), dev.alloc(T * K * 4)
    dev.moe_route(L, xb.ptr, T, order, pb.ptr, ib.ptr, wtb.ptr)
    probs = dev.download(pb, (T, E), np.float32)
    idx = dev.download(ib, (T, K), np.int32)
    wts = dev.download(wtb, (T, K), np.float32)
    for t in range(T):
        _, p, i, w = oracle.route(X[t], W, E, K, order)
        assert_bits_equal(probs[t], p, "probs t=%d" % t)
        assert (idx[t] == i).all(), "indices t=%d" % t
        assert_bits_equal(wts[t], w, "weights t=%d" % t)


@pytest.mark.parametrize("dim,E,K,T,order", [
    (1056, 60, 4, 37, ORDER_AVX512),   # a 32-element last K chunk (1056 = 4 x 256 + 32)
    (1056, 60, 4, 37, ORDER_AVX2),
    (288, 256, 16, 20, ORDER_SEQ),     # largest E and K
    (544, 5, 3, 3, ORDER_AVX2),        # E below one wave, few tokens
    (2048, 128, 8, 100, ORDER_AVX512), # the 16-token x 16-row tiles, ragged token tile
    (1056, 128, 8, 70, ORDER_SEQ),     # sequential order, ragged tiles
    (2048, 128, 8, 16, ORDER_AVX512),  # one router row per workgroup: 16 tokens x 16 lanes
    (1056, 60, 4, 9, ORDER_AVX512),    # ... rows of 4224 bytes (a partial last KiB)
    (2048, 128, 8, 18, ORDER_AVX2),    # ... the most tokens whose rows fit 160 KiB
    (2048, 128, 8, 19, ORDER_AVX2),    # one token more: the tiled kernel
])
def test_route_shapes(dev, oracle, dim, E, K, T, order):
    """Tiled router logits + workgroup rank routing at widths with a partial
    last K chunk, ragged token and expert counts, in every accumulation
    order, against the oracle's per-token router (probabilities, indices,
    weights bit-exact).  (The C ABI takes widths in multiples of 32, so the
    reference's per-lane tails of matmul_omp do not arise here.)"""
    W = I.activations(5100 + dim + E, E, dim, std=0.02)
    W[E // 2] = W[0]  # a planted tie
    X = I.activations(5200 + T, T, dim)
    wb, xb = dev.upload(W), dev.upload(X)
    L = Q.MoeLayer(dim, 768, E, K, wb.ptr, None, None, None, 0, 0, 0)
    pb, ib, wtb = dev.alloc(T * E * 4), dev.alloc(T * K * 4), dev.alloc(T * K * 4)
    dev.moe_route(L, xb.ptr, T, order, pb.ptr, ib.ptr, wtb.ptr)
    probs = dev.download(pb, (T, E), np.float32)
    idx = dev.download(ib, (T, K), np.int32)
    wts = dev.download(wtb, (T, K), np.float32)
    for t in range(T):
        _, p, i, w = oracle.route(X[t], W, E, K, order)
        assert_bits_equal(probs[t], p, "probs t=%d" % t)
        assert (idx[t] == i).all(), "indices t=%d" % t
        assert_bits_equal(wts[t], w, "weights t=%d" % t)


@pytest.mark.parametrize("T,K,E", [(512, 8, 128), (64, 4, 60), (1, 8, 128), (7, 3, 5),
                                   (300, 16, 256)])
def test_dispatch(dev, oracle, T, K, E):
    """Histogram, exclusive scan and stable permute against the oracle's
    counting sort; plus the invariants (bijection, grouping, order)."""
    rng = np.random.default_rng(T * 1000 + E)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    idx = np.stack([rng.choice(E, size=K, replace=False, p=p / p.sum()) for _ in range(T)])
    idx = idx.astype(np.int32)
    ib = dev.upload(idx)
    cb, ob, pb, vb = dev.alloc(E * 4), dev.alloc((E + 1) * 4), dev.alloc(T * K * 4), dev.alloc(T * K * 4)
    dev.moe_dispatch(ib.ptr, T, K, E, cb.ptr, ob.ptr, pb.ptr, vb.ptr)
    counts = dev.download(cb, E, np.int32)
    offsets = dev.download(ob, E + 1, np.int32)
    perm = dev.download(pb, T * K, np.int32)
    inv = dev.download(vb, T * K, np.int32)
    c, o, pm, iv = oracle.dispatch(idx, E)
    assert (counts == c).all() and (offsets == o).all() and (perm == pm).all() and (inv == iv).all()
    assert counts.sum() == T * K and sorted(perm.tolist()) == list(range(T * K))
    assert (perm[inv] == np.arange(T * K)).all()
    flat = idx.ravel()
    for e in range(E):
        seg = perm[offsets[e]:offsets[e + 1]]
        assert (flat[seg] == e).all() and (np.diff(seg) > 0).all()


@pytest.mark.parametrize("T,K,E", [(600, 8, 128), (5, 3, 7)])
def test_dispatch_invalid_indices(dev, T, K, E):
    """Indices outside 0 .. E-1 (-1, E, large) are left out: inv = -1, not
    counted, not in perm; the valid pairs keep the stable expert order, which
    a brute-force stable sort fixes."""
    rng = np.random.default_rng(T + E)
    idx = rng.integers(0, E, size=(T, K)).astype(np.int32)
    bad = rng.random((T, K)) < 0.05
    idx[bad] = rng.choice(np.array([-1, E, E + 1000, -77], np.int32), size=int(bad.sum()))
    ib = dev.upload(idx)
    cb, ob, pb, vb = dev.alloc(E * 4), dev.alloc((E + 1) * 4), dev.alloc(T * K * 4), dev.alloc(T * K * 4)
    dev.moe_dispatch(ib.ptr, T, K, E, cb.ptr, ob.ptr, pb.ptr, vb.ptr)
    flat = idx.ravel()
    valid = (flat >= 0) & (flat < E)
    nv = int(valid.sum())
    counts = dev.download(cb, E, np.int32)
    offsets = dev.download(ob, E + 1, np.int32)
    perm = dev.download(pb, T * K, np.int32)[:nv]
    inv = dev.download(vb, T * K, np.int32)
    want_counts = np.bincount(flat[valid], minlength=E)
    assert (counts == want_counts).all()
    assert (offsets == np.concatenate([[0], np.cumsum(want_counts)])).all()
    order = sorted(np.nonzero(valid)[0].tolist(), key=lambda q: (flat[q], q))  # stable by expert
    assert perm.tolist() == order
    want_inv = np.full(T * K, -1, np.int64)
    want_inv[np.array(order, np.int64)] = np.arange(nv)
    assert (inv == want_inv).all()


def test_dropin_moe_block(dev, oracle):
    """qr_moe_block: the MoE block with the reference's host pointers (per
    expert pointer arrays as TransformerWeights holds them)."""
    lib = Q.load()
    m = I.moe_inputs("a")
    dim, hidden, E, K = m["dim"], m["hidden"], m["E"], m["K"]
    su = m["up"].size // E
    sd = m["down"].size // E
    base_u, base_g, base_d = (a.ctypes.data for a in (m["up"], m["gate"], m["down"]))
    up_p = (C.c_void_p * E)(*[base_u + e * su for e in range(E)])
    gate_p = (C.c_void_p * E)(*[base_g + e * su for e in range(E)])
    # a non-contiguous copy of the down experts: exercises the gather upload
    down_parts = [np.array(m["down"][e * sd:(e + 1) * sd]) for e in range(E)]
    down_p = (C.c_void_p * E)(*[a.ctypes.data for a in down_parts[::-1]][::-1])
    assert lib.qr_dropin_init(0, ORDER_SEQ) == 0
    x0 = I.activations(990, 1, dim)[0]
    xb = I.activations(991, 1, dim)[0]
    x = x0.copy()
    rc = lib.qr_moe_block(x.ctypes.data_as(C.c_void_p), xb.ctypes.data_as(C.c_void_p),
                          m["router"].ctypes.data_as(C.c_void_p), up_p, gate_p, down_p,
                          m["up_type"], m["up_type"], m["down_type"], dim, hidden, E, K, 8)
    assert rc == 0
    keep = []
    L = Oracle.make_layer(keep, dim, hidden, E, K, m["router"], m["up"], m["up_type"], m["gate"],
                          m["up_type"], m["down"], m["down_type"])
    want, _, _ = oracle.moe_forward(x0[None, :], xb[None, :], L, order=ORDER_SEQ)
    assert_bits_equal(x, want[0], "drop-in MoE block")
    lib.qr_dropin_release_weights()


@pytest.mark.parametrize("order", [ORDER_SEQ, ORDER_AVX2, ORDER_AVX512])
@pytest.mark.parametrize("ut,dt", [(Q.TYPE_Q4_K, Q.TYPE_Q4_K), (Q.TYPE_Q5_K, Q.TYPE_Q5_K),
                                   (Q.TYPE_Q4_K, Q.TYPE_Q8_0), (Q.TYPE_Q8_0, Q.TYPE_Q6_K)])
@pytest.mark.parametrize("T", [1, 5, 48])
def test_moe_type_pairs(dev, oracle, ut, dt, T, order):
    """Every expert weight-type pair through the one-token, grouped-GEMV and
    grouped-MFMA paths (T = 1, 5, 48 with 20 experts top-6: 0.3, 1.5 and 14
    pairs per expert), random block bytes; E = 20 is not a multiple of the
    router rows a workgroup stages."""
    dim, hidden, E, K = 512, 256, 20, 6
    ue, de = I.BLOCK[ut][0], I.BLOCK[dt][0]
    seed = 7000 + 100 * ut + dt
    up = I.blocks(seed, ut, E * hidden * (dim // ue))
    gate = I.blocks(seed + 1, ut, E * hidden * (dim // ue))
    down = I.blocks(seed + 2, dt, E * dim * (hidden // de))
    router = I.activations(seed + 3, E, dim, std=0.05)
    layer = DevLayer(dev, dim, hidden, E, K, router, up, gate, down, ut, dt)
    x = I.activations(seed + 4 + T, T, dim)
    xb = I.activations(seed + 5 + T, T, dim)
    check_moe(dev, oracle, layer, x, xb, order, "types %d/%d T=%d order %d" % (ut, dt, T, order))


@pytest.mark.parametrize("T", [24, 70])
def test_moe_ragged_hidden(dev, oracle, T):
    """The many-token MFMA path with an expert width that leaves the last
    64-row gate/up tile half full (hidden = 288 = 9 blocks of 32) and a Q8_0
    down product whose last K stage holds one block; T = 24 uses 16-pair work
    items, T = 70 32-pair ones (all three item forms)."""
    dim, hidden, E, K = 512, 288, 16, 4
    ut, dt = Q.TYPE_Q4_K, Q.TYPE_Q8_0
    ue, de = I.BLOCK[ut][0], I.BLOCK[dt][0]
    seed = 7900 + T
    up = I.blocks(seed, ut, E * hidden * (dim // ue))
    gate = I.blocks(seed + 1, ut, E * hidden * (dim // ue))
    down = I.blocks(seed + 2, dt, E * dim * (hidden // de))
    router = I.activations(seed + 3, E, dim, std=0.05)
    layer = DevLayer(dev, dim, hidden, E, K, router, up, gate, down, ut, dt)
    x = I.activations(seed + 4, T, dim)
    xb = I.activations(seed + 5, T, dim)
    check_moe(dev, oracle, layer, x, xb, ORDER_AVX2, "hidden 288 T=%d" % T)


@pytest.mark.parametrize("dt", [Q.TYPE_Q4_K, Q.TYPE_Q5_K, Q.TYPE_Q6_K, Q.TYPE_Q8_0])
@pytest.mark.parametrize("dim,hidden", [(1024, 288), (2048, 512)])
def test_moe_t1_down_types(dev, oracle, dt, dim, hidden):
    """One token at model widths (gate/up tiles of 8 and 4 rows per wave) for
    every down type; hidden 288 leaves a K-quant down product with one
    super-block per row (the last 32 elements dropped, as the reference
    does)."""
    E, K = 24, 6
    ut = Q.TYPE_Q4_K
    ue, de = I.BLOCK[ut][0], I.BLOCK[dt][0]
    seed = 8100 + 10 * dt + dim // 1024
    up = I.blocks(seed, ut, E * hidden * (dim // ue))
    gate = I.blocks(seed + 1, ut, E * hidden * (dim // ue))
    down = I.blocks(seed + 2, dt, E * dim * (hidden // de))
    router = I.activations(seed + 3, E, dim, std=0.05)
    layer = DevLayer(dev, dim, hidden, E, K, router, up, gate, down, ut, dt)
    x = I.activations(seed + 4, 1, dim)
    xb = I.activations(seed + 5, 1, dim)
    check_moe(dev, oracle, layer, x, xb, ORDER_AVX2, "t1 %d/%d down %d" % (dim, hidden, dt))


@pytest.mark.parametrize("T", [1, 16, 64])
def test_moe_graph_replays(dev, oracle, T):
    """The MoE layer captured into a HIP graph (as bench.py times it) at the
    one-token, skinny/16-pair and 32-pair sizes: three replays, each after an
    eager reset of the residual x and a synchronization, every one bit-exact
    with the eager layer (itself checked against the oracle)."""
    layer, m = random_layer(dev, "a")
    x = I.activations(9300 + T, T, m["dim"])
    xb = I.activations(9301 + T, T, m["dim"])
    want, _, _ = run_moe(dev, layer, x, xb, ORDER_AVX2)
    keep = []
    ref, _, _ = oracle.moe_forward(x, xb, layer.oracle_layer(keep), order=ORDER_AVX2,
                                   dot_order=ORDER_SEQ, threads=16)
    assert_bits_equal(want, ref, "eager layer T=%d" % T)
    xd, xbd = dev.upload(x), dev.upload(xb)
    g = dev.capture(lambda: dev.moe_forward(layer.L, xd.ptr, xbd.ptr, T, ORDER_AVX2))
    try:
        for r in range(3):
            dev.write(xd, x)
            dev.sync()
            dev.graph_launch(g)
            dev.sync()
            assert_bits_equal(dev.download(xd, (T, m["dim"]), np.float32), want,
                              "replay %d T=%d" % (r, T))
    finally:
        dev.graph_destroy(g)


def test_capture_moe_growth_refused(oracle):
    """On a fresh context, a captured qr_moe_forward that needs scratch
    refuses (it would allocate); after one eager call of the same size the
    capture succeeds, and scratch grown later keeps the earlier graph valid."""
    d = Q.Device(0)
    try:
        layer, m = random_layer(d, "a")
        T = 16
        x = I.activations(9600, T, m["dim"])
        xb = I.activations(9601, T, m["dim"])
        xd, xbd = d.upload(x), d.upload(xb)
        lib = d.lib
        assert lib.qr_capture_begin(d.ctx) == 0
        rc = lib.qr_moe_forward(d.ctx, C.byref(layer.L), xd.ptr, xbd.ptr, T, ORDER_AVX2, None, None)
        msg = d.last_error()
        g = C.c_void_p()
        assert lib.qr_capture_end(d.ctx, C.byref(g)) == 0
        lib.qr_graph_destroy(g)
        assert rc == -1 and "outside graph capture" in msg
        want, _, _ = run_moe(d, layer, x, xb, ORDER_AVX2)  # eager: allocates the scratch
        d.write(xd, x)
        g = d.capture(lambda: d.moe_forward(layer.L, xd.ptr, xbd.ptr, T, ORDER_AVX2))
        try:
            run_moe(d, layer, I.activations(9602, 64, m["dim"]), I.activations(9603, 64, m["dim"]),
                    ORDER_AVX2)  # grows the scratch; the graph's buffer is kept
            for r in range(2):
                d.write(xd, x)
                d.sync()
                d.graph_launch(g)
                d.sync()
                assert_bits_equal(d.download(xd, (T, m["dim"]), np.float32), want, "replay %d" % r)
        finally:
            d.graph_destroy(g)
    finally:
        d.close()
