"""Deterministic inputs for the golden fixtures (numpy PCG64 streams).

The fixtures in this directory store the reference's outputs together with a
SHA-256 of the inputs they were computed from; the tests rebuild the inputs
with these functions and check the digest before comparing, so a change here
shows up as a digest mismatch rather than as a silent parity failure.

Weight blocks are random bytes with their fp16 scale fields overwritten by
moderate normal halves: every byte pattern is a valid block under the
reference's decoding (src/quant.c:160-240), so random bytes exercise all
nibble, fifth-bit and sub-scale combinations.
"""
import hashlib

import numpy as np

TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 8, 12, 13, 14
BLOCK = {TYPE_Q8_0: (32, 34), TYPE_Q4_K: (256, 144), TYPE_Q5_K: (256, 176), TYPE_Q6_K: (256, 210)}


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def _halves(rng, n, lo, hi):
    return rng.uniform(lo, hi, size=n).astype(np.float16).view(np.uint16)


def blocks(seed, qtype, nblocks, scale_lo=2e-4, scale_hi=1e-3):
    """nblocks random blocks of qtype (uint8 [nblocks * block_bytes])."""
    rng = np.random.default_rng(seed)
    bb = BLOCK[qtype][1]
    b = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    if qtype == TYPE_Q8_0:
        b[:, 0:2] = _halves(rng, nblocks, 5e-4, 2e-3).view(np.uint8).reshape(nblocks, 2)
    elif qtype in (TYPE_Q4_K, TYPE_Q5_K):
        b[:, 0:2] = _halves(rng, nblocks, scale_lo, scale_hi).view(np.uint8).reshape(nblocks, 2)
        b[:, 2:4] = _halves(rng, nblocks, scale_lo, scale_hi).view(np.uint8).reshape(nblocks, 2)
    else:
        b[:, 208:210] = _halves(rng, nblocks, scale_lo, scale_hi).view(np.uint8).reshape(nblocks, 2)
    return b.reshape(-1)


def special_blocks(qtype):
    """Blocks with edge-case scales: zero, half subnormals (decoded by the
    reference as mant * 2^-136), the largest half, and saturated fields."""
    bb = BLOCK[qtype][1]
    codes = [0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x8400, 0xBC00]
    out = []
    rng = np.random.default_rng(1234 + qtype)
    for c in codes:
        b = rng.integers(0, 256, size=bb, dtype=np.uint8)
        if qtype == TYPE_Q8_0:
            b[0:2] = np.array([c], np.uint16).view(np.uint8)
        elif qtype in (TYPE_Q4_K, TYPE_Q5_K):
            b[0:2] = np.array([c], np.uint16).view(np.uint8)
            b[2:4] = np.array([c ^ 0x8000], np.uint16).view(np.uint8)
        else:
            b[208:210] = np.array([c], np.uint16).view(np.uint8)
        out.append(b)
    b = np.full(bb, 0xFF, np.uint8)  # every nibble 15, every scale 63 / min 3
    if qtype == TYPE_Q8_0:
        b[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    elif qtype in (TYPE_Q4_K, TYPE_Q5_K):
        b[0:4] = np.array([0x3C00, 0x3800], np.uint16).view(np.uint8)
    else:
        b[208:210] = np.array([0x3C00], np.uint16).view(np.uint8)
    out.append(b)
    return np.concatenate(out)


def q4k_to_q5k(blob):
    """Q4_K bytes -> Q5_K bytes with a zero fifth-bit plane (same decoded values)."""
    src = np.ascontiguousarray(blob, np.uint8).reshape(-1, 144)
    out = np.zeros((src.shape[0], 176), np.uint8)
    out[:, 0:16] = src[:, 0:16]
    out[:, 48:176] = src[:, 16:144]
    return out.reshape(-1)


def activations(seed, rows, d, std=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, d)) * std).astype(np.float32)


def dot_set(seed, qtype, nrows, d):
    """nrows random rows of d elements plus one row made of special_blocks."""
    elems, bb = BLOCK[qtype]
    nb = d // elems
    main = blocks(seed, qtype, nrows * nb).reshape(nrows, nb * bb)
    spec = np.resize(special_blocks(qtype), nb * bb).reshape(1, nb * bb)
    return np.concatenate([main, spec]).astype(np.uint8)


# MoE golden cases: dim, hidden, E, K, T, up/gate type, down type.  Case "a"
# stores Q4_K experts; the reference is run on their zero-fifth-bit Q5_K form.
MOE_CASES = {
    "a": (512, 256, 16, 4, 6, TYPE_Q4_K, TYPE_Q6_K),
    "b": (512, 256, 8, 2, 4, TYPE_Q8_0, TYPE_Q8_0),
    "c": (256, 256, 64, 8, 8, TYPE_Q5_K, TYPE_Q6_K),
}


def moe_inputs(name):
    dim, hidden, E, K, T, ut, dt = MOE_CASES[name]
    seed = 500 + 10 * (ord(name) - ord("a"))
    ue = BLOCK[ut][0]
    de = BLOCK[dt][0]
    return dict(dim=dim, hidden=hidden, E=E, K=K, T=T, up_type=ut, down_type=dt,
                up=blocks(seed, ut, E * hidden * (dim // ue)),
                gate=blocks(seed + 1, ut, E * hidden * (dim // ue)),
                down=blocks(seed + 2, dt, E * dim * (hidden // de)),
                router=activations(seed + 3, E, dim, std=0.05),
                x=activations(seed + 4, T, dim))


def q8_edge_rows():
    """Rows of 64 floats (two Q8_0 blocks each) hitting quantize_row_q8_0's
    edge cases."""
    rows = []
    rows.append(np.zeros(64, np.float32))                               # amax 0 -> d 0, id 0
    rows.append(np.full(64, 0.75, np.float32))                          # all equal
    rows.append(np.linspace(-1e-30, 1e-30, 64).astype(np.float32))      # d flushes to 0 in fp16
    rows.append(np.linspace(-1e30, 1e30, 64).astype(np.float32))        # d saturates to inf
    r = np.arange(64, dtype=np.float32) - 31.5                          # ties at .5 after scaling
    r[0] = 127.0
    r[32] = -127.0
    rows.append(r.astype(np.float32))
    rows.append(((np.arange(64) - 16) * 0.125).astype(np.float32))      # tests/tests.c:59-61 ramp
    rows.append(np.float32(2.0) ** np.arange(-60, 4).astype(np.float32))
    rng = np.random.default_rng(77)
    rows.append((rng.standard_normal(64) * 1e-5).astype(np.float32))    # amax near fp16 min normal * 127
    return np.stack(rows).astype(np.float32)


# ---- the single-token decode step ------------------------------------------
# Small MoE models run through the reference's own forward_runtime
# (gen_golden.py) and through the decoders under test.  head_dim is
# dim / n_heads, which is what the reference can express (src/runtime.c:102);
# expert up / gate are Q5_K (the reference's Q4_K dot is defective).
# (dim, n_heads, n_kv_heads, layers, E, K, hidden, vocab, wq/wk/wv/wo types,
#  token-embedding type, lm_head type, tokens)
TYPE_F32 = 0
DECODE_CASES = {
    "a": (256, 4, 2, 2, 8, 2, 256, 300, (TYPE_Q8_0, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0), TYPE_Q8_0,
          TYPE_Q6_K, [3, 17, 101, 42, 250, 7, 7, 199]),
    "b": (512, 8, 2, 2, 16, 4, 256, 200, (TYPE_Q6_K, TYPE_F32, TYPE_Q8_0, TYPE_Q5_K), TYPE_Q6_K,
          TYPE_Q8_0, [0, 199, 55, 55, 120]),
    # dense models (no experts: the FFN of src/runtime.c:270-284), "c" with
    # Q8_0 FFN weights as TinyLlama's GGUF stores them
    "c": (256, 4, 2, 2, 0, 0, 512, 300, (TYPE_Q8_0, TYPE_Q6_K, TYPE_Q5_K, TYPE_Q8_0), TYPE_Q6_K,
          TYPE_Q8_0, [5, 299, 17, 17, 120, 3]),
    "d": (512, 8, 4, 2, 0, 0, 768, 256, (TYPE_Q5_K, TYPE_F32, TYPE_Q8_0, TYPE_Q6_K), TYPE_Q8_0,
          TYPE_Q6_K, [1, 2, 255, 128, 64]),
}
# FFN weight types (up and gate, down) where they differ from the MoE cases'
# Q5_K / Q6_K
DECODE_FFN_TYPES = {"c": (TYPE_Q8_0, TYPE_Q8_0)}


def _rows(seed, qtype, rows, cols):
    if qtype == TYPE_F32:
        return activations(seed, rows, cols, std=0.05)
    elems, bb = BLOCK[qtype]
    return blocks(seed, qtype, rows * (cols // elems)).reshape(rows, (cols // elems) * bb)


def decode_model(name):
    """The seeded weights of decode case `name` (numpy, host order)."""
    dim, H, KVH, L, E, K, hidden, vocab, wt, tt, ct, tokens = DECODE_CASES[name]
    hd = dim // H
    seed = 9000 + 100 * (ord(name) - ord("a"))
    ut, dt = DECODE_FFN_TYPES.get(name, (TYPE_Q5_K, TYPE_Q6_K))
    m = dict(dim=dim, n_heads=H, n_kv_heads=KVH, head_dim=hd, n_layers=L, E=E, K=K,
             hidden=hidden, vocab=vocab, seq_len=max(16, len(tokens)), rope_base=1e6,
             wtype=list(wt), tok_type=tt, wcls_type=ct, tokens=list(tokens),
             up_type=ut, down_type=dt)
    ne = max(E, 1)  # a dense model (E = 0) has one up / gate / down per layer
    m["tok_embd"] = _rows(seed, tt, vocab, dim)
    m["wcls"] = _rows(seed + 1, ct, vocab, dim)
    m["rms_final"] = (1.0 + activations(seed + 2, 1, dim, std=0.1)[0]).astype(np.float32)
    layers = []
    for l in range(L):
        s = seed + 10 + 20 * l
        lay = dict(
            rms_att=(1.0 + activations(s, 1, dim, std=0.1)[0]).astype(np.float32),
            rms_ffn=(1.0 + activations(s + 1, 1, dim, std=0.1)[0]).astype(np.float32),
            wq=_rows(s + 2, wt[0], H * hd, dim), wk=_rows(s + 3, wt[1], KVH * hd, dim),
            wv=_rows(s + 4, wt[2], KVH * hd, dim), wo=_rows(s + 5, wt[3], dim, H * hd),
            router=activations(s + 6, E, dim, std=0.05),
            up=blocks(s + 7, ut, ne * hidden * (dim // BLOCK[ut][0])),
            gate=blocks(s + 8, ut, ne * hidden * (dim // BLOCK[ut][0])),
            down=blocks(s + 9, dt, ne * dim * (hidden // BLOCK[dt][0])))
        layers.append(lay)
    m["layers"] = layers
    return m


def decode_digest(m):
    arrs = [m["tok_embd"], m["wcls"], m["rms_final"]]
    for lay in m["layers"]:
        arrs += [lay[k] for k in ("rms_att", "rms_ffn", "wq", "wk", "wv", "wo", "router", "up",
                                  "gate", "down")]
    return digest(*arrs)


def qwen3_small_model(seed=9500, n_layers=2, seq_len=640, n_kv_heads=2):
    """A Qwen3-30B-A3B-shaped decoder at reduced width: head_dim 128 with
    q_dim (8 x 128) != dim (512), GQA 4:1 (8:1 with n_kv_heads=1), 8 experts
    top-2, gate/up Q4_K, down Q6_K, mixed attention types, Q4_K embeddings and
    a Q6_K lm_head.  The reference cannot run it (head_dim = dim / n_heads
    there); the oracle's restatement can."""
    dim, H, KVH, hd, E, K, hidden, vocab = 512, 8, n_kv_heads, 128, 8, 2, 256, 320
    wt = (TYPE_Q4_K, TYPE_Q8_0, TYPE_Q6_K, TYPE_Q5_K)
    m = dict(dim=dim, n_heads=H, n_kv_heads=KVH, head_dim=hd, n_layers=n_layers, E=E, K=K,
             hidden=hidden, vocab=vocab, seq_len=seq_len, rope_base=1e6, wtype=list(wt),
             tok_type=TYPE_Q4_K, wcls_type=TYPE_Q6_K, up_type=TYPE_Q4_K, down_type=TYPE_Q6_K)
    m["tok_embd"] = _rows(seed, TYPE_Q4_K, vocab, dim)
    m["wcls"] = _rows(seed + 1, TYPE_Q6_K, vocab, dim)
    m["rms_final"] = (1.0 + activations(seed + 2, 1, dim, std=0.1)[0]).astype(np.float32)
    layers = []
    for l in range(n_layers):
        s = seed + 10 + 20 * l
        layers.append(dict(
            rms_att=(1.0 + activations(s, 1, dim, std=0.1)[0]).astype(np.float32),
            rms_ffn=(1.0 + activations(s + 1, 1, dim, std=0.1)[0]).astype(np.float32),
            wq=_rows(s + 2, wt[0], H * hd, dim), wk=_rows(s + 3, wt[1], KVH * hd, dim),
            wv=_rows(s + 4, wt[2], KVH * hd, dim), wo=_rows(s + 5, wt[3], dim, H * hd),
            router=activations(s + 6, E, dim, std=0.05),
            up=blocks(s + 7, TYPE_Q4_K, E * hidden * (dim // 256)),
            gate=blocks(s + 8, TYPE_Q4_K, E * hidden * (dim // 256)),
            down=blocks(s + 9, TYPE_Q6_K, E * dim * (hidden // 256))))
    m["layers"] = layers
    return m


def qwen3_full_model(seed=9800, n_layers=2, seq_len=4352):
    """The Qwen3-30B-A3B decode step at its full width: dim 2048, 32 query
    heads over 4 kv heads of 128 (q_dim 4096), 128 experts top-8 with ffn 768
    (gate / up Q4_K, down Q6_K), wq / wk / wo Q4_K and wv Q6_K, a Q4_K
    embedding and a Q6_K lm_head of 151936 rows.  n_layers distinct layers
    (about 400 MB of expert weights each)."""
    dim, H, KVH, hd, E, K, hidden, vocab = 2048, 32, 4, 128, 128, 8, 768, 151936
    wt = (TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q4_K)
    m = dict(dim=dim, n_heads=H, n_kv_heads=KVH, head_dim=hd, n_layers=n_layers, E=E, K=K,
             hidden=hidden, vocab=vocab, seq_len=seq_len, rope_base=1e6, wtype=list(wt),
             tok_type=TYPE_Q4_K, wcls_type=TYPE_Q6_K, up_type=TYPE_Q4_K, down_type=TYPE_Q6_K)
    m["tok_embd"] = _rows(seed, TYPE_Q4_K, vocab, dim)
    m["wcls"] = _rows(seed + 1, TYPE_Q6_K, vocab, dim)
    m["rms_final"] = (1.0 + activations(seed + 2, 1, dim, std=0.1)[0]).astype(np.float32)
    layers = []
    for l in range(n_layers):
        s = seed + 10 + 20 * l
        layers.append(dict(
            rms_att=(1.0 + activations(s, 1, dim, std=0.1)[0]).astype(np.float32),
            rms_ffn=(1.0 + activations(s + 1, 1, dim, std=0.1)[0]).astype(np.float32),
            wq=_rows(s + 2, wt[0], H * hd, dim), wk=_rows(s + 3, wt[1], KVH * hd, dim),
            wv=_rows(s + 4, wt[2], KVH * hd, dim), wo=_rows(s + 5, wt[3], dim, H * hd),
            router=activations(s + 6, E, dim, std=0.05),
            up=blocks(s + 7, TYPE_Q4_K, E * hidden * (dim // 256)),
            gate=blocks(s + 8, TYPE_Q4_K, E * hidden * (dim // 256)),
            down=blocks(s + 9, TYPE_Q6_K, E * dim * (hidden // 256))))
    m["layers"] = layers
    return m


def tinyllama_model(seed=9900, n_layers=2, seq_len=256, ffn_type=TYPE_Q8_0):
    """TinyLlama-1.1B's layer shapes (dense: no experts): dim 2048, 32 heads
    of 64 over 4 kv heads, FFN 5632, vocab 32000, every matrix Q8_0 (as its
    Q8_0 GGUF stores them; ffn_type sets the FFN's type).  head_dim is
    dim / n_heads, so the reference itself can run it."""
    dim, H, KVH, hidden, vocab = 2048, 32, 4, 5632, 32000
    hd = dim // H
    wt = (TYPE_Q8_0, TYPE_Q8_0, TYPE_Q8_0, TYPE_Q8_0)
    m = dict(dim=dim, n_heads=H, n_kv_heads=KVH, head_dim=hd, n_layers=n_layers, E=0, K=0,
             hidden=hidden, vocab=vocab, seq_len=seq_len, rope_base=10000.0, wtype=list(wt),
             tok_type=TYPE_Q8_0, wcls_type=TYPE_Q8_0, up_type=ffn_type, down_type=ffn_type)
    m["tok_embd"] = _rows(seed, TYPE_Q8_0, vocab, dim)
    m["wcls"] = _rows(seed + 1, TYPE_Q8_0, vocab, dim)
    m["rms_final"] = (1.0 + activations(seed + 2, 1, dim, std=0.1)[0]).astype(np.float32)
    layers = []
    for l in range(n_layers):
        s = seed + 10 + 20 * l
        layers.append(dict(
            rms_att=(1.0 + activations(s, 1, dim, std=0.1)[0]).astype(np.float32),
            rms_ffn=(1.0 + activations(s + 1, 1, dim, std=0.1)[0]).astype(np.float32),
            wq=_rows(s + 2, wt[0], H * hd, dim), wk=_rows(s + 3, wt[1], KVH * hd, dim),
            wv=_rows(s + 4, wt[2], KVH * hd, dim), wo=_rows(s + 5, wt[3], dim, H * hd),
            router=np.zeros((0, dim), np.float32),
            up=_rows(s + 7, ffn_type, hidden, dim).reshape(-1),
            gate=_rows(s + 8, ffn_type, hidden, dim).reshape(-1),
            down=_rows(s + 9, ffn_type, dim, hidden).reshape(-1)))
    m["layers"] = layers
    return m


# ---- the tiled layouts of Q6_K and Q8_0 (qr_weights_tile) -------------------
Q6_CHUNK_MAP = (12, 8, 0, 1, 9, 2, 3, 10, 4, 5, 11, 6, 7)


def tile_sq(blob, qtype, n, d):
    """Row-major Q6_K / Q8_0 rows [n][row bytes] -> the tiled layout, written
    from its definition: 256 elements per lane (a Q6_K super-block, or 8
    Q8_0 blocks), RB = 64 / (d / 256) rows per tile, chunk k of lane l at
    16 (k L + l) of the tile; Q6_K chunks in the order Q6_CHUNK_MAP, and the
    d fields (2 bytes) of every super-block after all the tiles, in row-major
    order; Q8_0 chunk 0 = the 8 scales, chunk 1 + 2 j + h = bytes
    16 h .. 16 h + 15 of block j's values."""
    nb = d // 256
    bb = 210 if qtype == TYPE_Q6_K else 272
    src = np.ascontiguousarray(blob, np.uint8).reshape(n * nb, bb)
    if qtype == TYPE_Q6_K:
        chunks = [src[:, 16 * c:16 * c + 16] for c in Q6_CHUNK_MAP]
        tail = src[:, 208:210]
    else:
        blk = src.reshape(n * nb, 8, 34)
        chunks = [blk[:, :, 0:2].reshape(n * nb, 16)]
        for j in range(8):
            for h in range(2):
                chunks.append(blk[:, j, 2 + 16 * h:18 + 16 * h])
        tail = None
    RB = 64 // nb
    out = []
    for t0 in range(0, n, RB):
        rows = min(RB, n - t0)
        lanes = slice(t0 * nb, (t0 + rows) * nb)
        for c in chunks:
            out.append(np.ascontiguousarray(c[lanes]).reshape(-1))
    if tail is not None:
        out.append(np.ascontiguousarray(tail).reshape(-1))
    return np.concatenate(out)
