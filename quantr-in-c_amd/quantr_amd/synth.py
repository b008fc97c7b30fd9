"""Synthetic inputs in quantr-in-c's block formats (numpy, host side).

Block layouts follow the reference byte for byte:
  Q8_0  34 B  {u16 d; i8 qs[32]}                         include/quant.h:28-33
  Q4_K 144 B  {u16 d, dmin; u8 scales[12]; u8 qs[128]}   include/quant.h:35-42
  Q5_K 176 B  {u16 d, dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]}  include/quant.h:44-50
  Q6_K 210 B  {u8 ql[128]; u8 qh[64]; i8 scales[16]; u16 d}        src/quant.c:220-226
with the reference's element mapping (src/quant.c:180-238): sub-block j uses
scales[j] (6-bit scale, 2-bit min for Q4_K/Q5_K; int8 scale for Q6_K), element
e = 32j + l takes nibble (l & 1) of byte e/2, Q5_K's fifth bit is bit e%8 of
qh[e/8], Q6_K's high pair is bits 2(e%4) of qh[e/4].

The reference ships a Q8_0 quantizer (src/quant.c:143-158, restated here for
weights) but no K-quant quantizer; the K-quant quantizers below are this
project's own (min/max per 32-element sub-block, fp16 super-scales chosen so
that the truncating fp16 conversion of include/quant.h:68-77 cannot push a
sub-scale out of its field).
"""
import numpy as np

TYPE_F32, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 0, 8, 12, 13, 14
BLOCK_BYTES = {TYPE_Q8_0: 34, TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210}
BLOCK_ELEMS = {TYPE_Q8_0: 32, TYPE_Q4_K: 256, TYPE_Q5_K: 256, TYPE_Q6_K: 256}
TYPE_NAMES = {TYPE_F32: "F32", TYPE_Q8_0: "Q8_0", TYPE_Q4_K: "Q4_K", TYPE_Q5_K: "Q5_K",
              TYPE_Q6_K: "Q6_K"}


def row_bytes(qtype, d):
    """Bytes per row; whole blocks only (src/quant.c:477-484)."""
    if qtype == TYPE_F32:
        return 4 * d
    return (d // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]


def f2h(x):
    """Truncating fp32 -> fp16 bits (include/quant.h:68-77), vectorised."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    sign = ((u >> 16) & 0x8000).astype(np.uint16)
    e = ((u >> 23) & 0xFF).astype(np.int32) - 127 + 15
    mant = ((u >> 13) & 0x3FF).astype(np.uint16)
    out = sign | (np.clip(e, 0, 31).astype(np.uint16) << 10) | mant
    out = np.where(e <= 0, sign, out)
    out = np.where(e >= 31, sign | 0x7C00, out)
    return out.astype(np.uint16)


def h2f(h):
    """fp16 bits -> fp32 (include/quant.h:53-66), vectorised."""
    h = np.asarray(h, np.uint16).astype(np.uint32)
    w = (h & 0x7FFF) << 13
    e = (h >> 10) & 0x1F
    w = np.where(e == 0x1F, w | 0x7F800000, np.where(e != 0, w + 0x38000000, w))
    w = w | ((h & 0x8000) << 16)
    return w.astype(np.uint32).view(np.float32)


def normal(seed, shape, std=1.0):
    """Seeded N(0, std) float32 (numpy PCG64)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def quantize_q8_0(x):
    """quantize_row_q8_0 over the last axis (src/quant.c:143-158): amax/127,
    reciprocal, round half to even, truncating fp16 scale.  Returns uint8
    [..., (d/32)*34]."""
    x = np.ascontiguousarray(x, np.float32)
    lead, d = x.shape[:-1], x.shape[-1]
    nb = d // 32
    xb = x[..., : nb * 32].reshape(-1, nb, 32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        amax = np.abs(xb).max(axis=-1)
        dd = (amax / np.float32(127.0)).astype(np.float32)
        idv = np.where(dd != 0, np.float32(1.0) / dd, np.float32(0.0)).astype(np.float32)
        q = np.rint(xb * idv[..., None]).astype(np.int64).astype(np.int8)
    out = np.empty(xb.shape[:2] + (34,), np.uint8)
    out[..., 0:2] = f2h(dd).view(np.uint8).reshape(dd.shape + (2,))
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(lead + (nb * 34,))


def _blocks(x):
    x = np.ascontiguousarray(x, np.float32)
    lead, d = x.shape[:-1], x.shape[-1]
    if d % 256:
        raise ValueError("K-quant rows need a multiple of 256 elements, got %d" % d)
    return lead, d // 256, x.reshape(-1, 8, 32)


def _fp16_up(v):
    """An fp16 code whose decode is >= v and is a normal half: the reference's
    truncating conversion flushes anything below 2^-14 to zero, so super-scales
    are kept at or above it (the integer sub-scales then shrink instead)."""
    v = np.asarray(v, np.float32) * np.float32(1.0 + 2.0 ** -9)
    return f2h(np.maximum(v, np.float32(2.0 ** -14)))


def _pack_nibbles(q):
    # q: [B, 256] in 0..15 -> [B, 128]; byte e/2 holds element e in nibble e%2
    return (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)


def _q45k(x, bits):
    lead, nb, xs = _blocks(x)
    B = xs.shape[0]
    sb = xs
    lo = np.minimum(sb.min(axis=-1), 0.0).astype(np.float32)
    hi = np.maximum(sb.max(axis=-1), 0.0).astype(np.float32)
    levels = np.float32(15 if bits == 4 else 31)
    dmin_raw = (-lo).max(axis=-1) / np.float32(3.0)
    dmin_h = _fp16_up(dmin_raw)
    dmin = h2f(dmin_h)
    with np.errstate(divide="ignore", invalid="ignore"):
        m2 = np.where(dmin[:, None] > 0, np.ceil(-lo / dmin[:, None]), 0).clip(0, 3).astype(np.int32)
        m = (m2.astype(np.float32) * dmin[:, None]).astype(np.float32)
        sc = ((hi + m) / levels).astype(np.float32)
        d_h = _fp16_up(sc.max(axis=-1) / np.float32(63.0))
        dd = h2f(d_h)
        s6 = np.where(dd[:, None] > 0, np.rint(sc / dd[:, None]), 0).clip(0, 63).astype(np.int32)
        s6 = np.where((s6 == 0) & (sc > 0), 1, s6)
        step = (s6.astype(np.float32) * dd[:, None]).astype(np.float32)
        q = np.where(step[..., None] > 0, np.rint((sb + m[..., None]) / step[..., None]), 0)
    q = q.clip(0, levels).astype(np.int32).reshape(B, 256)
    nbytes = 144 if bits == 4 else 176
    out = np.zeros((B, nbytes), np.uint8)
    out[:, 0:2] = d_h.view(np.uint8).reshape(B, 2)
    out[:, 2:4] = dmin_h.view(np.uint8).reshape(B, 2)
    out[:, 4:12] = (s6 | (m2 << 6)).astype(np.uint8)
    if bits == 4:
        out[:, 16:144] = _pack_nibbles(q & 0xF)
    else:
        hb = ((q >> 4) & 1).astype(np.uint8).reshape(B, 32, 8)
        out[:, 16:48] = (hb << np.arange(8, dtype=np.uint8)).sum(axis=-1).astype(np.uint8)
        out[:, 48:176] = _pack_nibbles(q & 0xF)
    return out.reshape(lead + (nb * nbytes,))


def quantize_q4_k(x):
    """fp32 rows (multiple of 256) -> Q4_K bytes in the reference layout."""
    return _q45k(x, 4)


def quantize_q5_k(x):
    """fp32 rows (multiple of 256) -> Q5_K bytes in the reference layout."""
    return _q45k(x, 5)


def quantize_q6_k(x):
    """fp32 rows (multiple of 256) -> Q6_K bytes (210 B blocks, reference layout)."""
    lead, nb, xs = _blocks(x)
    B = xs.shape[0]
    sb = xs
    amax = np.abs(sb).max(axis=-1).astype(np.float32)
    sc = (amax / np.float32(31.0)).astype(np.float32)
    d_h = _fp16_up(sc.max(axis=-1) / np.float32(127.0))
    dd = h2f(d_h)
    with np.errstate(divide="ignore", invalid="ignore"):
        s8 = np.where(dd[:, None] > 0, np.rint(sc / dd[:, None]), 0).clip(0, 127).astype(np.int32)
        s8 = np.where((s8 == 0) & (sc > 0), 1, s8)
        step = (s8.astype(np.float32) * dd[:, None]).astype(np.float32)
        q = np.where(step[..., None] > 0, np.rint(sb / step[..., None]), 0)
    q = (q.clip(-32, 31) + 32).astype(np.int32).reshape(B, 256)
    out = np.zeros((B, 210), np.uint8)
    out[:, 0:128] = _pack_nibbles(q & 0xF)
    hi = ((q >> 4) & 3).astype(np.uint8).reshape(B, 64, 4)
    out[:, 128:192] = (hi << (2 * np.arange(4, dtype=np.uint8))).sum(axis=-1).astype(np.uint8)
    out[:, 192:200] = s8.astype(np.int8).view(np.uint8)
    out[:, 208:210] = d_h.view(np.uint8).reshape(B, 2)
    return out.reshape(lead + (nb * 210,))


def quantize(x, qtype):
    """fp32 [..., d] -> block bytes [..., row_bytes(qtype, d)] (F32 returns raw bytes)."""
    if qtype == TYPE_F32:
        return np.ascontiguousarray(x, np.float32).view(np.uint8)
    return {TYPE_Q8_0: quantize_q8_0, TYPE_Q4_K: quantize_q4_k, TYPE_Q5_K: quantize_q5_k,
            TYPE_Q6_K: quantize_q6_k}[qtype](x)


def weights(seed, n, d, qtype, std=0.02, chunk_rows=1024, threads=None):
    """Seeded N(0, std) [n, d] weights quantized to qtype.

    Row chunk c draws from its own stream (seed, c), so the bytes do not
    depend on how many threads build them."""
    import concurrent.futures as cf
    import os
    out = np.empty((n, row_bytes(qtype, d)), np.uint8)
    starts = list(range(0, n, chunk_rows))

    def build(ci):
        r0 = starts[ci]
        r1 = min(n, r0 + chunk_rows)
        rng = np.random.default_rng([seed, ci])
        w = rng.standard_normal(size=(r1 - r0, d), dtype=np.float32) * np.float32(std)
        out[r0:r1] = quantize(w.astype(np.float32), qtype)

    nthr = threads or min(16, os.cpu_count() or 1)
    if nthr <= 1 or len(starts) == 1:
        for ci in range(len(starts)):
            build(ci)
    else:
        with cf.ThreadPoolExecutor(nthr) as ex:
            list(ex.map(build, range(len(starts))))
    return out


def q4k_to_q5k(blob):
    """Q4_K rows -> Q5_K rows with a zero fifth-bit plane.  Under the reference
    semantics both decode to the same values, so the reference's (sound) Q5_K
    dot computes the exact value its (defective) Q4_K dot was meant to."""
    b = np.ascontiguousarray(blob, np.uint8)
    lead = b.shape[:-1]
    nb = b.shape[-1] // 144
    src = b.reshape(-1, 144)
    out = np.zeros((src.shape[0], 176), np.uint8)
    out[:, 0:16] = src[:, 0:16]
    out[:, 48:176] = src[:, 16:144]
    return out.reshape(lead + (nb * 176,))


def zipf_router(seed, E, dim, s=1.1, std=0.02, c=8.0):
    """Router weights whose logits carry a Zipf(s) expert-popularity bias.

    The bias b_e = ln p_e is folded into the data: W[e] = G_e + (b_e / c) u and
    token inputs are z_t + c u, with u a unit vector and G_e, z_t orthogonal to
    it, so W[e] . x_t = G_e . z_t + b_e and the router stays a plain
    softmax(W x).  Returns (W [E, dim] fp32, u [dim] fp64, popularity order)."""
    rng = np.random.default_rng(seed)
    G = rng.standard_normal((E, dim)) * std
    u = rng.standard_normal(dim)
    u /= np.linalg.norm(u)
    G -= np.outer(G @ u, u)
    ranks = rng.permutation(E)
    p = 1.0 / np.power(np.arange(1, E + 1, dtype=np.float64), s)
    p /= p.sum()
    b = np.log(p)[ranks]
    W = G + np.outer(b / c, u)
    return W.astype(np.float32), u, ranks


def zipf_tokens(seed, T, dim, u, c=8.0):
    """Token activations z_t + c u with z_t ~ N(0, 1) orthogonal to u."""
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((T, dim))
    z -= np.outer(z @ u, u)
    return (z + c * u[None, :]).astype(np.float32)
