#!/usr/bin/env python3
"""Benchmark of the quantized GEMV + MoE hot path on one MI355X.

Headline (one JSON line on stdout): Q4_K decode GEMV weight GB/s on the
32000 x 2048 lm_head shape of the K-quant sweep, batch 1, as a fraction of the
8 TB/s HBM peak.  A step is one GEMV launch (activation quantization fused in)
over one of 16 distinct weight copies (592 MB in total, more than the 256 MB
Infinity Cache), with the activation already resident in HBM.  The K timed
steps are replayed from a HIP graph between two synchronizations and timed
with HIP events on the launch stream.  Beside it: a plain read of the same
bytes (the rate a single kernel streaming them once reaches).

Extra keys of the same line:
  gemv_sweep   Q8_0 at the TinyLlama-1.1B layer shapes (1 token), and Q4_K /
               Q5_K / Q6_K at those shapes plus 32000 x 2048, 1 and 4 tokens;
               each shape rotates over distinct matrices filling > 590 MB;
  moe_qwen3    the Qwen3-30B-A3B-shaped MoE layer (2048 wide, 128 experts
               top-8, ffn 768, gate/up Q4_K, down Q6_K, Zipf(1.1) expert skew)
               in tokens/s at T = 1, 16 and 512, rotating over 48 layer copies
               (router included) like a 48-layer decode;
               (`paths`: the layer at T = 2 ... 64 with each expert product forced, the
               grouped GEMV against the int8 MFMA products: the crossover the default
               path choice follows);
  moe_qwen15   the Qwen1.5-MoE-A2.7B-shaped layer (60 experts top-4, ffn 1408,
               shared expert ffn 5632 with a sigmoid gate) at T = 1 and 64;
  gemv_ggml    the llama.cpp-layout Q4_K / Q5_K / Q6_K GEMV (Q8_K activations,
               ggml's dot order) on 32000 x 2048 at 1 and 4 tokens;
  decode_qwen3 the whole single-token decode step of a Qwen3-30B-A3B-shaped
               model (48 layers, 32 query / 4 kv heads of 128, the MoE layer
               above, 151936-row Q6_K lm_head) over a Q8_0 paged KV cache
               prefilled to 4096 positions, replayed as one HIP graph per
               token, in tokens/s with its algorithmic bytes; and the batched
               prefill of a 512-token prompt (qr_decoder_prefill, chunks of
               128) in tokens/s;
  cpu_baseline the reference's own matmul_q_fused and MoE block (oracle/_ref,
               its sources compiled with the CI flags) on this host's cores at
               1, 8 and all available threads: 3 warm-ups, then the median.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-moe] [--no-cpu] [--no-sweep]
                    [--no-decode] [--decode-steps N]
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "quantr-in-c_amd"))

import quantr_amd as Q  # noqa: E402
from quantr_amd import synth  # noqa: E402

HBM_PEAK_GBPS = 8000.0
# fp32 VALU lane operations per second without packed instructions: 256 CUs x 4 SIMDs x 16
# lanes x 2.4 GHz (the published 157.3 TFLOP/s counts packed FMAs as 4 flops per lane)
VALU_PEAK_OPS = 256 * 64 * 2.4e9
# fp32 operations per (output row, token, 32-element unit) that the reference's dot rounds
# one by one: (sc * isum - m * bsum) * bd added on (Q4_K / Q5_K), sc * isum * bd added on
# (Q6_K), isum * (da * db) added on (Q8_0), each after the int -> float conversion
TERM_OPS = {Q.TYPE_Q4_K: 6, Q.TYPE_Q5_K: 6, Q.TYPE_Q6_K: 4, Q.TYPE_Q8_0: 4}
METRIC = "Q4_K GEMV weight GB/s (% HBM peak); MoE layer tokens/s at 30B-A3B shape"
TNAME = {Q.TYPE_Q8_0: "Q8_0", Q.TYPE_Q4_K: "Q4_K", Q.TYPE_Q5_K: "Q5_K", Q.TYPE_Q6_K: "Q6_K"}
TINYLLAMA = [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_cpus():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# A buffer larger than the 256 MB Infinity Cache and the L2s together, read
# (untimed) before every timed replay: a replay's first launches then find
# none of the weights the previous replay's last launches left cached, however
# the replay's length relates to the number of rotating copies.
FLUSH_BYTES = 1 << 30
_flush = {}


def flush_caches(dev):
    if "buf" not in _flush:
        _flush["buf"], _flush["sink"] = dev.alloc(FLUSH_BYTES), dev.alloc(16)
        dev.memset(_flush["buf"], 0, FLUSH_BYTES)
    dev.read_kernel(_flush["buf"].ptr, FLUSH_BYTES, _flush["sink"].ptr)


def timed_replays(dev, g, reps=5):
    """Median over `reps` timed replays of graph g (HIP events on the launch
    stream, synchronized before and after each replay; the caches flushed,
    untimed, before each)."""
    t = []
    for _ in range(reps):
        flush_caches(dev)
        dev.sync()
        dev.timer_start()
        dev.graph_launch(g)
        t.append(dev.timer_stop())
    dev.sync()
    return float(np.median(t))


def graph_ms(dev, launch, steps, reps=5):
    """Per-launch ms of launch(i), i < steps, captured once and replayed."""
    g = dev.capture(lambda: [launch(i) for i in range(steps)])
    dev.graph_launch(g)  # one untimed replay
    dev.sync()
    ms = timed_replays(dev, g, reps)
    dev.graph_destroy(g)
    return ms / steps


# ---------------------------------------------------------------------------
# GEMV
# ---------------------------------------------------------------------------
def gemv_alg_bytes(qtype, n, d, nt=1):
    """Weights + Q8_0 activation + fp32 output per launch."""
    return n * synth.row_bytes(qtype, d) + nt * ((d // 32) * 34 + 4 * n)


def copy_calibration(dev, nbytes=512 << 20):
    """One pass of the plain copy kernel over a known size: the reference
    point for FETCH_SIZE / WRITE_SIZE counter runs of this same command."""
    a, b = dev.alloc(nbytes), dev.alloc(nbytes)
    for _ in range(3):  # first touch of both buffers and clocks up
        dev.copy_kernel(b.ptr, a.ptr, nbytes)
    dev.sync()
    reps = 10
    dev.timer_start()
    for _ in range(reps):
        dev.copy_kernel(b.ptr, a.ptr, nbytes)
    ms = dev.timer_stop() / reps
    a.free()
    b.free()
    return dict(bytes=nbytes, ms=ms, gbps=2 * nbytes / (ms / 1e3) / 1e9)


def bench_headline(dev, steps, warmup, copies=16):
    """Q4_K 32000 x 2048 at 1 and 4 tokens over 16 weight copies, in the tiled
    layout (qr_weights_tile, made once before timing: the same bytes permuted)
    and in the reference's row-major layout, and a plain read of the same
    bytes."""
    qtype, n, d = Q.TYPE_Q4_K, 32000, 2048
    wbytes = n * synth.row_bytes(qtype, d)
    wbuf = dev.alloc(wbytes * copies)
    tbuf = dev.alloc(wbytes * copies)
    dev.write(wbuf, synth.weights(1, n, d, qtype))
    for c in range(1, copies):
        dev.copy(wbuf.ptr + c * wbytes, wbuf.ptr, wbytes)
    for c in range(copies):
        dev.tile(qtype, wbuf.ptr + c * wbytes, tbuf.ptr + c * wbytes, n, d)
    dev.sync()
    out = {}
    for layout, buf, ty in (("tiled", tbuf, qtype | Q.TILED), ("rows", wbuf, qtype)):
        for nt in (1, 4):
            xb = dev.upload(synth.normal(2, (nt, d)))
            yb = dev.alloc(nt * n * 4)
            launch = lambda i: dev.gemv(ty, buf.ptr + (i % copies) * wbytes, xb.ptr,  # noqa: E731
                                        yb.ptr, n, d, nt)
            for i in range(warmup):
                launch(i)
            dev.sync()
            ms = graph_ms(dev, launch, steps if nt == 1 else max(steps // 2, 20))
            alg = gemv_alg_bytes(qtype, n, d, nt)
            out[(layout, nt)] = dict(ms_per_step=ms, weight_gbps=wbytes / (ms / 1e3) / 1e9,
                                     alg_bytes=alg, achieved_gbps=alg / (ms / 1e3) / 1e9)
            xb.free()
            yb.free()
    sink = dev.alloc(16)
    rd = lambda i: dev.read_kernel(wbuf.ptr + (i % copies) * wbytes, wbytes, sink.ptr)  # noqa: E731
    for i in range(warmup):
        rd(i)
    dev.sync()
    ms = graph_ms(dev, rd, steps)
    out["read"] = dict(ms_per_step=ms, bytes=wbytes, gbps=wbytes / (ms / 1e3) / 1e9)
    wbuf.free()
    tbuf.free()
    return out


def bench_sweep(dev, types, warmup, pool_bytes=600 << 20, max_steps=2048, only=None):
    """Every (type, shape, tokens) of the Q8_0 and K-quant GEMV configs (or
    only the (n, d) shapes in `only`).  Each type's weights fill a pool of
    > 590 MB (copies of its largest matrix); a launch reads n rows at a
    row-aligned offset, consecutive launches at consecutive offsets, so one
    replay streams the whole pool once."""
    res = {}
    for qtype in types:
        for d in (2048, 5632):
            shapes = [(n, dd) for (n, dd) in TINYLLAMA if dd == d]
            if qtype != Q.TYPE_Q8_0 and d == 2048:
                shapes.append((32000, 2048))  # the K-quant sweep's lm_head
            if only is not None:
                shapes = [sh for sh in shapes if sh in only]
            if not shapes:
                continue
            nmax = max(n for n, _ in shapes)
            rb = synth.row_bytes(qtype, d)
            W = synth.weights(100 + qtype + d, nmax, d, qtype)
            copies = max(1, math.ceil(pool_bytes / W.nbytes))
            pool = dev.alloc(W.nbytes * copies)
            dev.write(pool, W)
            for c in range(1, copies):
                dev.copy(pool.ptr + c * W.nbytes, pool.ptr, W.nbytes)
            prows = nmax * copies
            for n, _ in shapes:
                for nt in ((1,) if qtype == Q.TYPE_Q8_0 else (1, 4)):
                    nmat = prows // n  # row-aligned matrices in the pool
                    wb = n * rb
                    steps = int(min(max(64, nmat), max_steps))
                    xb = dev.upload(synth.normal(3 + nt, (nt, d)))
                    yb = dev.alloc(nt * n * 4)
                    launch = lambda i: dev.gemv(qtype, pool.ptr + (i % nmat) * wb, xb.ptr,  # noqa: E731
                                                yb.ptr, n, d, nt)
                    for i in range(warmup):
                        launch(i)
                    dev.sync()
                    ms = graph_ms(dev, launch, steps, reps=3)
                    alg = gemv_alg_bytes(qtype, n, d, nt)
                    key = "%s_%dx%d_t%d" % (TNAME[qtype], n, d, nt)
                    res[key] = dict(us=round(ms * 1e3, 3),
                                    weight_gbps=round(wb / (ms / 1e3) / 1e9, 1),
                                    alg_bytes=alg,
                                    achieved_gbps=round(alg / (ms / 1e3) / 1e9, 1),
                                    frac=round(alg / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                                    launches=steps)
                    log("bench: %-22s %8.2f us  %7.0f GB/s  frac %.3f" % (
                        key, ms * 1e3, alg / (ms / 1e3) / 1e9, res[key]["frac"]))
                    xb.free()
                    yb.free()
            if qtype in (Q.TYPE_Q4_K, Q.TYPE_Q5_K, Q.TYPE_Q6_K, Q.TYPE_Q8_0):
                # the same shapes in the tiled layout: a pool of tiled copies of the
                # first n rows (Q6_K: n * (d / 256) a multiple of 8)
                for n, _ in shapes:
                    if qtype == Q.TYPE_Q6_K and (n * (d // 256)) % 8:
                        continue
                    wb = n * rb
                    copies_t = max(1, math.ceil(pool_bytes / wb))
                    tpool = dev.alloc(wb * copies_t)
                    dev.tile(qtype, pool.ptr, tpool.ptr, n, d)
                    for c in range(1, copies_t):
                        dev.copy(tpool.ptr + c * wb, tpool.ptr, wb)
                    for nt in ((1,) if qtype == Q.TYPE_Q8_0 else (1, 4)):
                        steps = int(min(max(64, copies_t), max_steps))
                        xb = dev.upload(synth.normal(3 + nt, (nt, d)))
                        yb = dev.alloc(nt * n * 4)
                        launch = lambda i: dev.gemv(qtype | Q.TILED,  # noqa: E731
                                                    tpool.ptr + (i % copies_t) * wb, xb.ptr,
                                                    yb.ptr, n, d, nt)
                        for i in range(warmup):
                            launch(i)
                        dev.sync()
                        ms = graph_ms(dev, launch, steps, reps=3)
                        alg = gemv_alg_bytes(qtype, n, d, nt)
                        key = "%s_%dx%d_t%d_tiled" % (TNAME[qtype], n, d, nt)
                        res[key] = dict(us=round(ms * 1e3, 3),
                                        weight_gbps=round(wb / (ms / 1e3) / 1e9, 1),
                                        alg_bytes=alg,
                                        achieved_gbps=round(alg / (ms / 1e3) / 1e9, 1),
                                        frac=round(alg / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                                        launches=steps)
                        log("bench: %-28s %8.2f us  %7.0f GB/s  frac %.3f" % (
                            key, ms * 1e3, alg / (ms / 1e3) / 1e9, res[key]["frac"]))
                        xb.free()
                        yb.free()
                    tpool.free()
            pool.free()
    return res


def ggml_rows(seed, qtype, n, d):
    """n rows of llama.cpp-layout blocks: random bytes with finite half scales
    (d and dmin; Q6_K's d at bytes 208..209)."""
    rng = np.random.default_rng(seed)
    B = {Q.TYPE_Q4_K: 144, Q.TYPE_Q5_K: 176, Q.TYPE_Q6_K: 210}[qtype]
    nb = n * (d // 256)
    w = rng.integers(0, 256, (nb, B), dtype=np.uint8)
    half = lambda: (rng.uniform(1e-4, 2e-2, nb) * rng.choice([-1.0, 1.0], nb)).astype(  # noqa: E731
        np.float16).view(np.uint8).reshape(nb, 2)
    if qtype == Q.TYPE_Q6_K:
        w[:, 208:210] = half()
    else:
        w[:, 0:2] = half()
        w[:, 2:4] = half()
    return w.reshape(n, -1)


def bench_ggml(dev, warmup, pool_bytes=600 << 20, steps=200):
    """The llama.cpp-layout K-quant GEMV (QR_GGML, Q8_K activations) on the
    32000 x 2048 lm_head shape at 1 and 4 tokens, over > 590 MB of copies."""
    res = {}
    n, d = 32000, 2048
    for qtype in (Q.TYPE_Q4_K, Q.TYPE_Q5_K, Q.TYPE_Q6_K):
        W = ggml_rows(900 + qtype, qtype, n, d)
        copies = max(1, math.ceil(pool_bytes / W.nbytes))
        pool = dev.alloc(W.nbytes * copies)
        dev.write(pool, W)
        for c in range(1, copies):
            dev.copy(pool.ptr + c * W.nbytes, pool.ptr, W.nbytes)
        for nt in (1, 4):
            xb = dev.upload(synth.normal(5 + nt, (nt, d)))
            yb = dev.alloc(nt * n * 4)
            launch = lambda i: dev.gemv(qtype | Q.GGML, pool.ptr + (i % copies) * W.nbytes,  # noqa: E731
                                        xb.ptr, yb.ptr, n, d, nt)
            for i in range(warmup):
                launch(i)
            dev.sync()
            ms = graph_ms(dev, launch, steps, reps=3)
            alg = W.nbytes + nt * ((d // 256) * 292 + 4 * n)
            key = "%s_ggml_%dx%d_t%d" % (TNAME[qtype], n, d, nt)
            res[key] = dict(us=round(ms * 1e3, 3), weight_gbps=round(W.nbytes / (ms / 1e3) / 1e9, 1),
                            alg_bytes=alg, achieved_gbps=round(alg / (ms / 1e3) / 1e9, 1),
                            frac=round(alg / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4))
            log("bench: %-28s %8.2f us  %7.0f GB/s  frac %.3f" % (
                key, ms * 1e3, alg / (ms / 1e3) / 1e9, res[key]["frac"]))
            xb.free()
            yb.free()
        pool.free()
    return res


# ---------------------------------------------------------------------------
# MoE layers
# ---------------------------------------------------------------------------
QWEN3 = dict(dim=2048, hidden=768, E=128, K=8)
QWEN15 = dict(dim=2048, hidden=1408, E=60, K=4, sh=5632)


def build_qwen3(dev, layers):
    dim, hidden, E, K = QWEN3["dim"], QWEN3["hidden"], QWEN3["E"], QWEN3["K"]
    t0 = time.time()
    router, u, _ = synth.zipf_router(3000, E, dim)
    parts = [router,
             synth.weights(3001, E * hidden, dim, Q.TYPE_Q4_K),
             synth.weights(3002, E * hidden, dim, Q.TYPE_Q4_K),
             synth.weights(3003, E * dim, hidden, Q.TYPE_Q6_K)]
    log("bench: Qwen3 layer weights built in %.1fs" % (time.time() - t0))
    offs = np.cumsum([0] + [p.nbytes for p in parts])
    per_layer = int(offs[-1])
    slab = dev.alloc(per_layer * layers)
    for p, o in zip(parts, offs):
        dev.write(slab, p, int(o))
    for l in range(1, layers):
        dev.copy(slab.ptr + l * per_layer, slab.ptr, per_layer)
    Ls = []
    for l in range(layers):
        b = slab.ptr + l * per_layer
        Ls.append(Q.MoeLayer(dim, hidden, E, K, b, b + int(offs[1]), b + int(offs[2]),
                             b + int(offs[3]), Q.TYPE_Q4_K, Q.TYPE_Q4_K, Q.TYPE_Q6_K))
    expert_bytes = (per_layer - router.nbytes) // E
    return dict(layers=Ls, slab=slab, u=u, parts=parts, expert_bytes=expert_bytes,
                per_layer=per_layer, shape=QWEN3, shared_bytes=0,
                types=(Q.TYPE_Q4_K, Q.TYPE_Q6_K, None))


def build_qwen15(dev, layers):
    dim, hidden, E, K, SH = (QWEN15[k] for k in ("dim", "hidden", "E", "K", "sh"))
    t0 = time.time()
    parts = [synth.normal(4000, (E, dim), 0.02),
             synth.weights(4001, E * hidden, dim, Q.TYPE_Q4_K),
             synth.weights(4002, E * hidden, dim, Q.TYPE_Q4_K),
             synth.weights(4003, E * dim, hidden, Q.TYPE_Q8_0),
             synth.normal(4004, (dim,), 0.02),
             synth.weights(4005, SH, dim, Q.TYPE_Q4_K),
             synth.weights(4006, SH, dim, Q.TYPE_Q4_K),
             synth.weights(4007, dim, SH, Q.TYPE_Q4_K)]
    log("bench: Qwen1.5 layer weights built in %.1fs" % (time.time() - t0))
    offs = np.cumsum([0] + [(p.nbytes + 255) // 256 * 256 for p in parts])
    per_layer = int(offs[-1])
    slab = dev.alloc(per_layer * layers)
    for p, o in zip(parts, offs):
        dev.write(slab, p, int(o))
    for l in range(1, layers):
        dev.copy(slab.ptr + l * per_layer, slab.ptr, per_layer)
    Ls = []
    for l in range(layers):
        b = [slab.ptr + l * per_layer + int(o) for o in offs[:-1]]
        L = Q.MoeLayer(dim, hidden, E, K, b[0], b[1], b[2], b[3], Q.TYPE_Q4_K, Q.TYPE_Q4_K,
                       Q.TYPE_Q8_0)
        L.sh_hidden = SH
        L.sh_gate_inp, L.sh_up, L.sh_gate, L.sh_down = b[4], b[5], b[6], b[7]
        L.sh_up_type = L.sh_gate_type = L.sh_down_type = Q.TYPE_Q4_K
        Ls.append(L)
    expert_bytes = sum(p.nbytes for p in parts[1:4]) // E
    shared_bytes = sum(p.nbytes for p in parts[4:])
    return dict(layers=Ls, slab=slab, u=None, parts=parts, expert_bytes=expert_bytes,
                per_layer=per_layer, shape=QWEN15, shared_bytes=shared_bytes,
                types=(Q.TYPE_Q4_K, Q.TYPE_Q8_0, Q.TYPE_Q4_K))


def moe_alg_bytes(M, T, touched):
    """Router + touched experts + shared expert + activations in and out."""
    sh = M["shape"]
    return 4 * sh["E"] * sh["dim"] + touched * M["expert_bytes"] + M["shared_bytes"] + \
        2 * 4 * T * sh["dim"]


def moe_term_ops(M, T):
    """fp32 VALU operations the layer's expert products must perform at T tokens
    (one rounded operation per TERM_OPS step, per output row, token slot and unit)."""
    sh = M["shape"]
    ut, dt, st = M["types"]
    dim, hid, K = sh["dim"], sh["hidden"], sh["K"]
    ops = T * K * (2 * hid * (dim // 32) * TERM_OPS[ut] + dim * (hid // 32) * TERM_OPS[dt])
    if st is not None:
        ops += T * (2 * sh["sh"] * (dim // 32) + dim * (sh["sh"] // 32)) * TERM_OPS[st]
    return ops


def bench_moe(dev, M, T, steps, warmup, order, nbatches=8, seed=7000):
    sh = M["shape"]
    dim, E, K = sh["dim"], sh["E"], sh["K"]
    Ls = M["layers"]
    if M["u"] is not None:
        xb_all = np.concatenate([synth.zipf_tokens(seed + 31 * T + b, T, dim, M["u"])
                                 for b in range(nbatches)])
    else:
        xb_all = synth.normal(seed + 31 * T, (nbatches * T, dim))
    xbb = dev.upload(xb_all)
    xs = dev.upload(synth.normal(seed + 500 + T, (nbatches * T, dim)))
    # routing of each batch (for the algorithmic byte count: touched experts)
    idxb, wtb = dev.alloc(nbatches * T * K * 4), dev.alloc(nbatches * T * K * 4)
    dev.moe_route(Ls[0], xbb.ptr, nbatches * T, order, None, idxb.ptr, wtb.ptr)
    idx = dev.download(idxb, (nbatches, T * K), np.int32)
    touched = float(np.mean([np.unique(r).size for r in idx]))
    counts = np.bincount(idx[0], minlength=E)
    step_bytes = moe_alg_bytes(M, T, touched)

    def one(i):
        b = i % nbatches
        dev.moe_forward(Ls[i % len(Ls)], xs.ptr + b * T * dim * 4, xbb.ptr + b * T * dim * 4, T,
                        order)

    for i in range(max(warmup, 1)):
        one(i)
    dev.sync()
    ms = graph_ms(dev, one, steps)
    s = ms / 1e3
    ops = moe_term_ops(M, T)
    hbm_us = step_bytes / (HBM_PEAK_GBPS * 1e9) * 1e6
    valu_us = ops / VALU_PEAK_OPS * 1e6
    return dict(T=T, ms_per_step=ms, tokens_per_s=T / s, touched_experts=touched,
                max_tokens_per_expert=int(counts.max()), alg_bytes=int(step_bytes),
                achieved_gbps=step_bytes / s / 1e9,
                roofline_frac=step_bytes / s / 1e9 / HBM_PEAK_GBPS,
                term_ops=int(ops), hbm_bound_us=round(hbm_us, 2), valu_bound_us=round(valu_us, 2),
                bound_frac=round(max(hbm_us, valu_us) / (ms * 1e3), 4))


# ---------------------------------------------------------------------------
# Full decode step
# ---------------------------------------------------------------------------
QWEN3_DEC = dict(dim=2048, n_heads=32, n_kv_heads=4, head_dim=128, vocab=151936, prefill=4096,
                 prefill_prompt=512)


def _tiled(dev, rows_blob, n_rows):
    """A device tensor of n_rows rows made by repeating rows_blob's rows."""
    r, rb = rows_blob.shape
    buf = dev.alloc(n_rows * rb)
    dev.write(buf, rows_blob)
    done = r
    while done < n_rows:
        k = min(done, n_rows - done)
        dev.copy(buf.ptr + done * rb, buf.ptr, k * rb)
        done += k
    return buf


def build_decoder(dev, M, cap):
    """The Qwen3-30B-A3B-shaped decoder: 48 layers of attention (wq / wk / wo
    Q4_K, wv Q6_K, 32 query heads over 4 kv heads of 128) on top of the MoE
    layers M, a Q4_K embedding and a Q6_K lm_head of 151936 rows (8192
    distinct rows repeated; tiled), and a Q8_0 KV cache of `cap` positions."""
    c = QWEN3_DEC
    dim, H, KVH, hd, V = c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["vocab"]
    qd, kvd = H * hd, KVH * hd
    L = len(M["layers"])
    t0 = time.time()
    parts = [synth.weights(5001, qd, dim, Q.TYPE_Q4_K), synth.weights(5002, kvd, dim, Q.TYPE_Q4_K),
             synth.weights(5003, kvd, dim, Q.TYPE_Q6_K), synth.weights(5004, dim, qd, Q.TYPE_Q4_K),
             (1.0 + synth.normal(5005, (dim,), 0.1)).astype(np.float32),
             (1.0 + synth.normal(5006, (dim,), 0.1)).astype(np.float32)]
    offs = np.cumsum([0] + [(p.nbytes + 255) // 256 * 256 for p in parts])
    per_layer = int(offs[-1])
    slab = dev.alloc(per_layer * L)
    for p, o in zip(parts, offs):
        dev.write(slab, p, int(o))
    # wq / wk / wo (Q4_K) in the tiled layout, as qr_gguf_load stores them
    for j, (rows, cols) in ((0, (qd, dim)), (1, (kvd, dim)), (3, (dim, qd))):
        tmp = dev.upload(parts[j])
        dev.tile(Q.TYPE_Q4_K, tmp.ptr, slab.ptr + int(offs[j]), rows, cols)
        dev.sync()
        tmp.free()
    for l in range(1, L):
        dev.copy(slab.ptr + l * per_layer, slab.ptr, per_layer)
    emb = _tiled(dev, synth.weights(5010, 8192, dim, Q.TYPE_Q4_K), V)
    # the Q6_K lm_head in the tiled layout, as qr_gguf_load stores it
    wrows = _tiled(dev, synth.weights(5011, 8192, dim, Q.TYPE_Q6_K), V)
    wcls = dev.alloc(V * synth.row_bytes(Q.TYPE_Q6_K, dim))
    dev.tile(Q.TYPE_Q6_K, wrows.ptr, wcls.ptr, V, dim)
    dev.sync()
    wrows.free()
    rmsf = dev.upload((1.0 + synth.normal(5012, (dim,), 0.1)).astype(np.float32))
    log("bench: decoder weights built in %.1fs" % (time.time() - t0))
    layers = []
    for l in range(L):
        b = [slab.ptr + l * per_layer + int(o) for o in offs[:-1]]
        ml = M["layers"][l]
        layers.append(dict(wq=b[0], wk=b[1], wv=b[2], wo=b[3], rms_att=b[4], rms_ffn=b[5],
                           router=ml.router, up=ml.up, gate=ml.gate, down=ml.down))
    m = dict(dim=dim, n_heads=H, n_kv_heads=KVH, head_dim=hd, n_layers=L, vocab=V, seq_len=cap,
             rope_base=1e6, tok_embd=emb.ptr, tok_type=Q.TYPE_Q4_K, rms_final=rmsf.ptr,
             wcls=wcls.ptr, wcls_type=Q.TYPE_Q6_K | Q.TILED,
             wtype=(Q.TYPE_Q4_K | Q.TILED, Q.TYPE_Q4_K | Q.TILED, Q.TYPE_Q6_K,
                    Q.TYPE_Q4_K | Q.TILED),
             E=M["shape"]["E"], K=M["shape"]["K"], hidden=M["shape"]["hidden"],
             up_type=Q.TYPE_Q4_K, down_type=Q.TYPE_Q6_K, layers=layers)
    attn_bytes = sum(p.nbytes for p in parts[:4]) + 2 * 4 * dim
    return m, [slab, emb, wcls, rmsf], attn_bytes


def bench_decode(dev, M, steps, warmup, order):
    """tokens/s of the whole single-token decode step (graph replay), at
    positions prefill, prefill + 1, ... over a Q8_0 cache prefilled with
    seeded N(0, 1) keys and values; the token ids are a seeded random
    sequence (the step does not wait for its own argmax)."""
    c = QWEN3_DEC
    P = c["prefill"]
    cap = P + warmup + steps + 1
    m, bufs, attn_bytes = build_decoder(dev, M, cap)
    model, layers, keep = Q.upload_decode_model(dev, m)
    t0 = time.time()
    d = Q.Decoder(dev, model, layers, kv_type=Q.KV_Q8_0, order=order, page=256,
                  flags=Q.DEC_GRAPH)
    log("bench: decoder created (RoPE table, cache) in %.1fs" % (time.time() - t0))
    kvd = c["n_kv_heads"] * c["head_dim"]
    kb = dev.upload(synth.normal(5020, (P, kvd)))
    vb = dev.upload(synth.normal(5021, (P, kvd)))
    for l in range(m["n_layers"]):
        d.kv_write(l, 0, P, kb.ptr, vb.ptr)
    kb.free()
    vb.free()
    toks = np.random.default_rng(5030).integers(0, c["vocab"], size=warmup + steps)
    lg = dev.alloc(4 * c["vocab"])
    for i in range(warmup):
        d.forward(int(toks[i]), P + i, lg.ptr)
    dev.sync()
    dev.timer_start()
    for i in range(warmup, warmup + steps):
        d.forward(int(toks[i]), P + i, lg.ptr)
    ms = dev.timer_stop() / steps
    logits = dev.download(lg, c["vocab"], np.float32)
    # prompt prefill: 512 prompt tokens at positions 0 .. 511 in the default
    # chunk (qr_decoder_prefill with chunk 0; the workspace is allocated by an
    # untimed first call of the same size)
    pn = c["prefill_prompt"]
    ptoks = np.random.default_rng(5031).integers(0, c["vocab"], size=pn)
    d.prefill(ptoks, 0, lg.ptr)
    dev.sync()
    dev.timer_start()
    d.prefill(ptoks, 0, lg.ptr)
    pms = dev.timer_stop()
    d.close()
    for b in bufs:
        b.free()
    # algorithmic bytes per step: attention weights and norms, router and the
    # K experts of every layer, the KV rows read (mean position of the timed
    # steps), the embedding row and the lm_head
    L, dim = m["n_layers"], c["dim"]
    npos = P + warmup + (steps + 1) / 2.0
    rs = (kvd // 32) * 34
    sh = M["shape"]
    step_bytes = (L * (attn_bytes + 4 * sh["E"] * dim + sh["K"] * M["expert_bytes"]) +
                  L * 2 * npos * rs + synth.row_bytes(Q.TYPE_Q4_K, dim) +
                  c["vocab"] * synth.row_bytes(Q.TYPE_Q6_K, dim) + 4 * dim)
    s = ms / 1e3
    return dict(ms_per_step=ms, tokens_per_s=1.0 / s, layers=L, positions=npos,
                prefill=dict(tokens=int(pn), chunk=min(int(pn), Q.PREFILL_CHUNK), ms=round(pms, 3),
                             tokens_per_s=round(pn / (pms / 1e3), 1),
                             speedup_vs_decode=round((pn / (pms / 1e3)) * s, 2)),
                alg_bytes=int(step_bytes), achieved_gbps=step_bytes / s / 1e9,
                roofline_frac=step_bytes / s / 1e9 / HBM_PEAK_GBPS,
                finite_logits=bool(np.isfinite(logits).all()))


# ---------------------------------------------------------------------------
# CPU baseline: the reference's own code on this host
# ---------------------------------------------------------------------------
def thread_counts(cpus):
    return sorted({1, min(8, cpus), cpus})


def cpu_baseline_gemv(cpus, reps=30, copies=16):
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    n, d = 32000, 2048
    ref = O.RefLib("avx2")
    W = synth.weights(90, n, d, Q.TYPE_Q4_K)
    Ws = [W] + [W.copy() for _ in range(copies - 1)]  # 590 MB: beyond the host's caches
    x = synth.normal(91, (d,))
    wbytes = W.nbytes
    by = {}
    for th in thread_counts(cpus):
        t = ref.gemv_bench(x, Ws, Q.TYPE_Q4_K, n, d, th, 3, reps)
        by[th] = dict(gbps=round(wbytes / float(np.median(t)) / 1e9, 2),
                      ms=round(float(np.median(t)) * 1e3, 3))
        log("bench: CPU matmul_q_fused Q4_K 32000x2048, %d threads: %.1f GB/s (%.2f ms)"
            % (th, by[th]["gbps"], by[th]["ms"]))
    return dict(value=by[cpus]["gbps"], unit="GB/s", cores=cpus, kind="reference",
                sample="matmul_q_fused Q4_K 32000x2048 (oracle/_ref: the reference's sources, "
                       "-O3 -std=c99 -mavx2 -mfma, OpenMP), 16 rotating weight copies (590 MB), "
                       "3 warm-ups then the median of %d calls per thread count; %s, %d CPUs "
                       "available to this process of %d; the reference's Q4_K dot returns "
                       "invalid values but does the same work" % (reps, cpu_model(), cpus,
                                                                  os.cpu_count() or 0),
                by_threads={str(k): v for k, v in by.items()})


def cpu_baseline_moe(M, cpus, reps=24, copies=4):
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    sh = M["shape"]
    dim, hidden, E, K = sh["dim"], sh["hidden"], sh["E"], sh["K"]
    router, up, gate, down = M["parts"][:4]
    ref = O.RefLib("avx2")
    cp = lambda a: [a] + [a.copy() for _ in range(copies - 1)]  # noqa: E731
    R, U, G, D = cp(router), cp(up), cp(gate), cp(down)
    x = synth.zipf_tokens(9000, 16, dim, M["u"])
    by = {}
    for th in thread_counts(cpus):
        t = ref.moe_bench(x, dim, hidden, E, K, R, U, Q.TYPE_Q4_K, G, Q.TYPE_Q4_K, D,
                          Q.TYPE_Q6_K, O.BACKEND_AVX2, th, 3, reps)
        med = float(np.median(t))
        by[th] = dict(tokens_per_s=round(1.0 / med, 1), ms_per_token=round(med * 1e3, 3))
        log("bench: CPU MoE block (Qwen3 shape), %d threads: %.1f tokens/s (%.2f ms per token)"
            % (th, 1.0 / med, med * 1e3))
    return dict(value=by[cpus]["tokens_per_s"], unit="tokens/s", cores=cpus, kind="reference",
                sample="forward_runtime's MoE block (oracle/_ref, CI flags, OpenMP), one token per "
                       "call as the reference runs tokens (so T = 1, 16 and 512 share this rate), "
                       "layer weights rotating over %d copies (1.6 GB), set-up outside the timed "
                       "region, 3 warm-ups then the median of %d calls" % (copies, reps),
                by_threads={str(k): v for k, v in by.items()})


def cpu_baseline_decode(M, cpus, reps=10, copies=2):
    """The reference's forward_runtime per token at the nearest Qwen3-30B-A3B
    shape it runs: head_dim = dim / n_heads (64, where the model has 128), its
    fp32 KV cache, the same MoE layer, at position 4096.  One decoder layer
    per timed call (a one-layer model rotating over `copies` weight copies,
    attention weights Q8_0: the reference's Q4_K dot returns values that turn
    into NaN router logits a layer later), so a token costs 48 such calls plus
    the Q6_K lm_head, timed alone."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    sh = M["shape"]
    dim, hidden, E, K = sh["dim"], sh["hidden"], sh["E"], sh["K"]
    c = QWEN3_DEC
    H, KVH, V, P, L = c["n_heads"], c["n_kv_heads"], c["vocab"], c["prefill"], len(M["layers"])
    hd = dim // H
    kvd = KVH * hd
    router, up, gate, down = M["parts"][:4]
    ref = O.RefLib("avx2")
    cps = []
    for i in range(copies):
        cps.append(dict(wq=synth.weights(7100 + i, H * hd, dim, Q.TYPE_Q8_0),
                        wk=synth.weights(7110 + i, kvd, dim, Q.TYPE_Q8_0),
                        wv=synth.weights(7120 + i, kvd, dim, Q.TYPE_Q8_0),
                        wo=synth.weights(7130 + i, dim, H * hd, Q.TYPE_Q8_0),
                        router=router if i == 0 else router.copy(),
                        up=up if i == 0 else up.copy(), gate=gate if i == 0 else gate.copy(),
                        down=down if i == 0 else down.copy()))
    tok = synth.zipf_tokens(9001, 16, dim, M["u"])
    rms = np.ones(dim, np.float32)
    head = np.tile(synth.weights(7140, 8192, dim, Q.TYPE_Q6_K), (V // 8192 + 1, 1))[:V].copy()
    x = synth.normal(7141, (dim,))
    by = {}
    for th in thread_counts(cpus):
        tl = ref.decode_layer_bench(dim, H, KVH, hidden, E, K, P, tok, cps,
                                    (Q.TYPE_Q8_0,) * 4, Q.TYPE_Q4_K, Q.TYPE_Q6_K, rms,
                                    O.BACKEND_AVX2, th, 2, reps)
        th_head = ref.gemv_bench(x, [head], Q.TYPE_Q6_K, V, dim, th, 1, 3)
        lay, hm = float(np.median(tl)), float(np.median(th_head))
        tok_s = 1.0 / (L * lay + hm)
        by[th] = dict(tokens_per_s=round(tok_s, 3), layer_ms=round(lay * 1e3, 3),
                      lm_head_ms=round(hm * 1e3, 2))
        log("bench: CPU decode step (reference forward_runtime, %d layers at position %d), "
            "%d threads: %.2f tokens/s (%.2f ms per layer, lm_head %.1f ms)"
            % (L, P, th, tok_s, lay * 1e3, hm * 1e3))
    return dict(value=by[cpus]["tokens_per_s"], unit="tokens/s", cores=cpus, kind="reference",
                sample="forward_runtime (oracle/_ref, CI flags, OpenMP) of one decoder layer per "
                       "call at position %d over its fp32 KV cache (head_dim %d = dim / n_heads, "
                       "the reference's rule; 32 query / 4 kv heads; Q8_0 attention weights; the "
                       "MoE layer of the GPU leg), %d weight copies, 2 warm-ups then the median "
                       "of %d calls, times %d layers, plus the Q6_K 151936 x 2048 lm_head "
                       "(matmul_q_fused, median of 3)" % (P, hd, copies, reps, L),
                by_threads={str(k): v for k, v in by.items()})


# ---------------------------------------------------------------------------
def load_traffic():
    p = os.path.join(REPO, "profiles", "k_gemv_tiled_q4k_32000x2048_traffic.json")
    if not os.path.exists(p):
        return None
    try:
        return json.load(open(p)).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--sweep-types", default="Q8_0,Q4_K,Q5_K,Q6_K")
    ap.add_argument("--sweep-shapes", default="",
                    help="restrict the sweep to these NxD shapes (comma-separated; profiling runs)")
    ap.add_argument("--moe-layers", type=int, default=48)
    ap.add_argument("--moe-t", default="1,16,512",
                    help="token counts of the Qwen3 MoE leg (comma-separated)")
    ap.add_argument("--moe-steps", type=int, default=0,
                    help="layers timed per token count (0: the defaults, 100 / 100 / 20)")
    ap.add_argument("--no-qwen15", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-crossover", action="store_true",
                    help="skip the grouped-GEMV / MFMA comparison of the Qwen3 MoE leg")
    ap.add_argument("--decode-steps", type=int, default=32)
    ap.add_argument("--no-ggml", action="store_true",
                    help="skip the llama.cpp-layout K-quant GEMV leg")
    ap.add_argument("--no-gemv", action="store_true",
                    help="skip the GEMV headline (profiling runs of other legs; value is null)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: there is no multi-GPU path; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    dev = Q.Device(0)
    cal = copy_calibration(dev)
    log("bench: copy kernel %.0f GB/s (read+write) over %d MB" % (cal["gbps"], cal["bytes"] >> 20))
    h = None
    if not args.no_gemv:
        h = bench_headline(dev, args.steps, args.warmup)
        for layout in ("tiled", "rows"):
            for nt in (1, 4):
                g = h[(layout, nt)]
                log("bench: Q4_K 32000x2048 %s T=%d: %.3f us/launch, %.0f GB/s weights, "
                    "%.0f GB/s algorithmic" % (layout, nt, g["ms_per_step"] * 1e3,
                                              g["weight_gbps"], g["achieved_gbps"]))
        rd = h["read"]
        log("bench: plain read of the same %d bytes: %.3f us, %.0f GB/s" % (
            rd["bytes"], rd["ms_per_step"] * 1e3, rd["gbps"]))

    sweep = None
    if not args.no_sweep:
        names = {v: k for k, v in TNAME.items()}
        types = [names[t.strip()] for t in args.sweep_types.split(",") if t.strip()]
        only = None
        if args.sweep_shapes.strip():
            only = {tuple(int(v) for v in sh.lower().split("x"))
                    for sh in args.sweep_shapes.split(",") if sh.strip()}
        sweep = bench_sweep(dev, types, min(args.warmup, 5), only=only)
    ggml = None if args.no_ggml else bench_ggml(dev, min(args.warmup, 5))

    moe = moe15 = dec = None
    M = None
    if not args.no_moe:
        M = build_qwen3(dev, args.moe_layers)
        moe = {}
        default_steps = {1: max(args.steps, 100), 16: 100, 512: 20}
        for T in [int(t) for t in args.moe_t.split(",") if t.strip()]:
            steps = args.moe_steps or default_steps.get(T, 20)
            r = bench_moe(dev, M, T, steps, 3, Q.ORDER_AVX2)
            moe["T%d" % T] = r
            log("bench: MoE Qwen3 T=%d: %.1f us/layer, %.0f tokens/s, %.1f experts touched, "
                "%.0f GB/s (%.1f%% of HBM peak); bounds HBM %.1f us, VALU %.1f us -> frac %.3f"
                % (T, r["ms_per_step"] * 1e3, r["tokens_per_s"], r["touched_experts"],
                   r["achieved_gbps"], 100 * r["roofline_frac"], r["hbm_bound_us"],
                   r["valu_bound_us"], r["bound_frac"]))
        if not args.no_crossover:
            paths = {}
            for T in (2, 4, 8, 16, 32, 64):
                row = {}
                for name, path in (("gemv", Q.MOE_PATH_GEMV), ("mfma", Q.MOE_PATH_MFMA)):
                    dev.set_moe_path(path)
                    r = bench_moe(dev, M, T, 30, 3, Q.ORDER_AVX2)
                    row[name + "_us"] = round(r["ms_per_step"] * 1e3, 2)
                dev.set_moe_path(Q.MOE_PATH_AUTO)
                paths["T%d" % T] = row
                log("bench: MoE Qwen3 T=%d expert products: grouped GEMV %.1f us, int8 MFMA %.1f us"
                    % (T, row["gemv_us"], row["mfma_us"]))
            moe["paths"] = paths
        if not args.no_decode:
            dec = bench_decode(dev, M, args.decode_steps, 3, Q.ORDER_AVX2)
            log("bench: decode step Qwen3-30B-A3B shape, %d layers at ~%.0f positions: %.3f ms, "
                "%.1f tokens/s, %.0f GB/s algorithmic (%.1f%% of HBM peak)" % (
                    dec["layers"], dec["positions"], dec["ms_per_step"], dec["tokens_per_s"],
                    dec["achieved_gbps"], 100 * dec["roofline_frac"]))
            pf = dec["prefill"]
            log("bench: prefill of %d prompt tokens (chunks of %d): %.2f ms, %.0f tokens/s, "
                "%.1fx the decode step's rate" % (pf["tokens"], pf["chunk"], pf["ms"],
                                                   pf["tokens_per_s"], pf["speedup_vs_decode"]))
        M["slab"].free()
        if not args.no_qwen15:
            M15 = build_qwen15(dev, 8)
            moe15 = {}
            for T, steps in ((1, 100), (64, 40)):
                r = bench_moe(dev, M15, T, steps, 3, Q.ORDER_SEQ, seed=8000)
                moe15["T%d" % T] = r
                log("bench: MoE Qwen1.5 T=%d: %.1f us/layer, %.0f tokens/s, %.1f experts touched, "
                    "%.0f GB/s (%.1f%% of HBM peak)" % (T, r["ms_per_step"] * 1e3,
                                                       r["tokens_per_s"], r["touched_experts"],
                                                       r["achieved_gbps"],
                                                       100 * r["roofline_frac"]))
            M15["slab"].free()

    cpus = host_cpus()
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_gemv(cpus)
        if M is not None:
            moe["cpu_baseline"] = cpu_baseline_moe(M, cpus)
            if dec is not None:
                dec["cpu_baseline"] = cpu_baseline_decode(M, cpus)

    h1 = h[("tiled", 1)] if h else None

    def gkey(layout, nt):
        g = h[(layout, nt)]
        return {"ms_per_step": round(g["ms_per_step"], 6),
                "weight_gbps": round(g["weight_gbps"], 2), "alg_bytes": g["alg_bytes"],
                "achieved_gbps": round(g["achieved_gbps"], 2),
                "roofline_frac": round(g["achieved_gbps"] / HBM_PEAK_GBPS, 4)}
    out = {
        "metric": METRIC,
        "value": round(h1["weight_gbps"], 2) if h else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h1["ms_per_step"], 6) if h else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "Q4_K decode GEMV 32000x2048 (lm_head of the K-quant sweep), "
                               "1 token, 16 rotating weight copies in the tiled layout "
                               "(qr_weights_tile, made before timing)", "n": 32000, "d": 2048,
                   "qtype": "Q4_K", "tokens": 1, "layout": "tiled"},
        "roofline": {"bound": "hbm", "achieved": round(h1["achieved_gbps"], 2),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(h1["achieved_gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": load_traffic(),
                     "read_ceiling": {
                         "note": "a plain read of the same weight bytes, 16 rotating copies",
                         "us": round(h["read"]["ms_per_step"] * 1e3, 3),
                         "gbps": round(h["read"]["gbps"], 1),
                         "gemv_over_read": round(h["read"]["ms_per_step"] / h1["ms_per_step"],
                                                 4)}} if h else None,
        "cpu_baseline": cpu,
        "gemv_q4k_32000x2048_t4": gkey("tiled", 4) if h else None,
        "gemv_q4k_32000x2048_rows_t1": gkey("rows", 1) if h else None,
        "gemv_q4k_32000x2048_rows_t4": gkey("rows", 4) if h else None,
        "gemv_sweep": sweep,
        "gemv_ggml": ggml,
        "moe_qwen3": moe,
        "moe_qwen15": moe15,
        "decode_qwen3": dec,
        "copy_kernel_gbps": round(cal["gbps"], 1),
    }
    print(json.dumps(out), flush=True)
    dev.close()


if __name__ == "__main__":
    main()
