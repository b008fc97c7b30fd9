"""llama.cpp / ggml K-quant blocks built from their integer fields (test data).

Packs chosen scales, mins and quants into the ggml block layouts
(ggml-common.h: block_q4_K 144 B, block_q5_K 176 B, block_q6_K 210 B) the way
ggml's quantizers store them -- written from the layout, separately from the
oracle's unpacking -- and keeps the fields, so that tests can check the
oracle's dequantization and integer dot parts against values computed here
directly.
"""
import numpy as np

Q4_K, Q5_K, Q6_K = 12, 13, 14
BLOCK = {Q4_K: 144, Q5_K: 176, Q6_K: 210}


def pack_scales12(sc, mn):
    """8 six-bit scales and mins -> the 12 scale bytes of Q4_K / Q5_K."""
    s = np.zeros(12, np.uint8)
    for j in range(8):
        ls, lm = int(sc[j]), int(mn[j])
        if j < 4:
            s[j] = ls
            s[j + 4] = lm
        else:
            s[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            s[j - 4] |= (ls >> 4) << 6
            s[j] |= (lm >> 4) << 6
    return s


def _f16(rng, lo, hi, n):
    return (rng.uniform(lo, hi, n) * rng.choice([-1.0, 1.0], n)).astype(np.float16)


def make_blocks(seed, qtype, nblocks, edge=False):
    """Random blocks of qtype.  Returns (bytes [nblocks * B], fields) where
    fields holds d, dmin (fp16 codes), sc, mn ([nb][8] or [nb][16] for Q6_K's
    signed scales) and q ([nb][256], element order: Q4_K 0..15, Q5_K 0..31,
    Q6_K 0..63 before its -32).  edge: the first blocks get zero, subnormal
    and largest scales."""
    rng = np.random.default_rng(seed)
    B = BLOCK[qtype]
    out = np.zeros((nblocks, B), np.uint8)
    d = _f16(rng, 1e-4, 2e-2, nblocks)
    dmin = _f16(rng, 1e-4, 2e-2, nblocks)
    if edge and nblocks >= 4:
        d[0], dmin[0] = np.float16(0.0), np.float16(0.0)
        d[1], dmin[1] = np.float16(6e-8), np.float16(-6e-8)  # subnormals
        d[2], dmin[2] = np.float16(65504.0), np.float16(-65504.0)
        d[3] = np.float16(-1.0)
    if qtype == Q6_K:
        sc = rng.integers(-128, 128, (nblocks, 16))
        mn = np.zeros((nblocks, 16), np.int64)
        q = rng.integers(0, 64, (nblocks, 256))
    else:
        sc = rng.integers(0, 64, (nblocks, 8))
        mn = rng.integers(0, 64, (nblocks, 8))
        q = rng.integers(0, 16 if qtype == Q4_K else 32, (nblocks, 256))
    for i in range(nblocks):
        b = out[i]
        if qtype in (Q4_K, Q5_K):
            b[0:2] = np.frombuffer(d[i:i + 1].tobytes(), np.uint8)
            b[2:4] = np.frombuffer(dmin[i:i + 1].tobytes(), np.uint8)
            b[4:16] = pack_scales12(sc[i], mn[i])
            qs = b[16:144] if qtype == Q4_K else b[48:176]
            for g in range(4):  # 64-element groups: low nibbles, then high nibbles
                lo = q[i, 64 * g: 64 * g + 32]
                hi = q[i, 64 * g + 32: 64 * g + 64]
                qs[32 * g: 32 * g + 32] = (lo & 0xF) | ((hi & 0xF) << 4)
                if qtype == Q5_K:  # fifth bits: bit 2g (low half), 2g + 1 (high half)
                    qh = b[16:48]
                    qh[:] |= ((lo >> 4) & 1).astype(np.uint8) << (2 * g)
                    qh[:] |= ((hi >> 4) & 1).astype(np.uint8) << (2 * g + 1)
        else:
            ql, qh = b[0:128], b[128:192]
            for n in range(2):  # 128-element halves
                e = q[i, 128 * n: 128 * n + 128]
                for l in range(32):
                    q1, q2, q3, q4 = e[l], e[l + 32], e[l + 64], e[l + 96]
                    ql[64 * n + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
                    ql[64 * n + l + 32] = (q2 & 0xF) | ((q4 & 0xF) << 4)
                    qh[32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
            b[192:208] = sc[i].astype(np.int8).view(np.uint8)
            b[208:210] = np.frombuffer(d[i:i + 1].tobytes(), np.uint8)
    return out.reshape(-1), dict(d=d, dmin=dmin, sc=sc, mn=mn, q=q)


def dequant_expected(qtype, f):
    """The dequantized values from the fields, in float32 with one rounding per
    operation: Q4_K / Q5_K (d * sc) * q - (dmin * m); Q6_K (d * sc) * (q - 32)."""
    nb = f["q"].shape[0]
    out = np.zeros((nb, 256), np.float32)
    d = f["d"].astype(np.float32)
    for i in range(nb):
        for e in range(256):
            if qtype == Q6_K:
                j = e // 16
                out[i, e] = np.float32(d[i] * np.float32(f["sc"][i, j])) * np.float32(f["q"][i, e] - 32)
            else:
                j = e // 32
                d1 = np.float32(d[i] * np.float32(f["sc"][i, j]))
                m1 = np.float32(np.float32(f["dmin"][i]) * np.float32(f["mn"][i, j]))
                out[i, e] = np.float32(d1 * np.float32(f["q"][i, e])) - m1
    return out.reshape(-1)


def ints_expected(qtype, f, i, q8, bsums):
    """aux32[8] and sumi of block i against Q8_K quants q8 [256] / bsums [16]."""
    q = f["q"][i].astype(np.int64)
    a = q - 32 if qtype == Q6_K else q
    aux = np.zeros(8, np.int64)
    per = 16 if qtype == Q6_K else 32
    for e in range(256):
        aux[e % 8] += int(f["sc"][i, e // per]) * int(q8[e]) * int(a[e])
    sumi = 0
    if qtype != Q6_K:
        for j in range(16):
            sumi += int(bsums[j]) * int(f["mn"][i, j // 2])
    return aux, sumi


def random_rows(seed, qtype, n, d):
    """n rows of d / 256 random blocks (any bytes are a valid block) with
    finite half scales in [1e-4, 2e-2] of either sign (d and dmin; Q6_K's d)."""
    rng = np.random.default_rng(seed)
    B = BLOCK[qtype]
    nb = n * (d // 256)
    w = rng.integers(0, 256, (nb, B), dtype=np.uint8)
    d16 = _f16(rng, 1e-4, 2e-2, nb).view(np.uint8).reshape(nb, 2)
    if qtype == Q6_K:
        w[:, 208:210] = d16
    else:
        w[:, 0:2] = d16
        w[:, 2:4] = _f16(rng, 1e-4, 2e-2, nb).view(np.uint8).reshape(nb, 2)
    return w.reshape(n, (d // 256) * B)
