#!/usr/bin/env python3
"""Benchmark of the quantized GEMV + MoE hot path on one MI355X.

Headline (one JSON line on stdout): Q4_K decode GEMV weight GB/s on the
32000 x 2048 lm_head shape of the K-quant sweep, batch 1, as a fraction of the
8 TB/s HBM peak.  A step is one GEMV launch (activation quantization fused in)
over one of 16 distinct weight copies (592 MB in total, more than the 256 MB
Infinity Cache), with the activation already resident in HBM.  The K timed
steps are replayed from a HIP graph between two synchronizations and timed
with HIP events on the launch stream.

The same line carries the Qwen3-30B-A3B-shaped MoE layer (2048 wide, 128
experts top-8, ffn 768, gate/up Q4_K, down Q6_K, Zipf(1.1) expert skew) in
tokens/s at T = 1, 16 and 512, rotating over 48 layer copies like a 48-layer
decode, and the CPU baseline: the reference's own matmul_q_fused and MoE block
(oracle/_ref, its sources compiled with the CI flags) timed on this host's cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-moe] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "quantr-in-c_amd"))

import quantr_amd as Q  # noqa: E402
from quantr_amd import synth  # noqa: E402

HBM_PEAK_GBPS = 8000.0
METRIC = "Q4_K GEMV weight GB/s (% HBM peak); MoE layer tokens/s at 30B-A3B shape"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_cores():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------
# GEMV headline
# ---------------------------------------------------------------------------
def gemv_alg_bytes(qtype, n, d, nt=1):
    """Weights + Q8_0 activation + fp32 output per launch."""
    return n * synth.row_bytes(qtype, d) + nt * ((d // 32) * 34 + 4 * n)


def bench_gemv(dev, qtype, n, d, nt, steps, warmup, copies=16, seed=1):
    rb = synth.row_bytes(qtype, d)
    wbytes = n * rb
    W = synth.weights(seed, n, d, qtype)
    wbuf = dev.alloc(wbytes * copies)
    dev.write(wbuf, W)
    for c in range(1, copies):
        dev.copy(wbuf.ptr + c * wbytes, wbuf.ptr, wbytes)
    xb = dev.upload(synth.normal(seed + 1, (nt, d)))
    yb = dev.alloc(nt * n * 4)
    for i in range(warmup):
        dev.gemv(qtype, wbuf.ptr + (i % copies) * wbytes, xb.ptr, yb.ptr, n, d, nt)
    dev.sync()

    def record():
        for i in range(steps):
            dev.gemv(qtype, wbuf.ptr + (i % copies) * wbytes, xb.ptr, yb.ptr, n, d, nt)

    g = dev.capture(record)
    dev.graph_launch(g)  # one untimed replay
    dev.sync()
    ms = timed_replays(dev, g)
    dev.graph_destroy(g)
    wbuf.free()
    s = ms / 1e3 / steps
    return dict(ms_per_step=ms / steps, weight_gbps=wbytes / s / 1e9,
                alg_bytes=gemv_alg_bytes(qtype, n, d, nt),
                achieved_gbps=gemv_alg_bytes(qtype, n, d, nt) / s / 1e9)


def timed_replays(dev, g, reps=5):
    """Median over `reps` timed replays of graph g (HIP events on the launch
    stream, synchronized before and after each replay)."""
    t = []
    for _ in range(reps):
        dev.sync()
        dev.timer_start()
        dev.graph_launch(g)
        t.append(dev.timer_stop())
    dev.sync()
    return float(np.median(t))


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


# ---------------------------------------------------------------------------
# MoE layer
# ---------------------------------------------------------------------------
QWEN3 = dict(dim=2048, hidden=768, E=128, K=8)


def build_qwen3(dev, layers):
    dim, hidden, E, K = QWEN3["dim"], QWEN3["hidden"], QWEN3["E"], QWEN3["K"]
    t0 = time.time()
    router, u, _ = synth.zipf_router(3000, E, dim)
    parts = [synth.weights(3001, E * hidden, dim, Q.TYPE_Q4_K),
             synth.weights(3002, E * hidden, dim, Q.TYPE_Q4_K),
             synth.weights(3003, E * dim, hidden, Q.TYPE_Q6_K)]
    log("bench: Qwen3 layer weights built in %.1fs" % (time.time() - t0))
    sizes = [p.nbytes for p in parts]
    per_layer = sum(sizes)
    slab = dev.alloc(per_layer * layers)
    off = 0
    for p in parts:
        dev.write(slab, p, off)
        off += p.nbytes
    for l in range(1, layers):
        dev.copy(slab.ptr + l * per_layer, slab.ptr, per_layer)
    rbuf = dev.upload(router)
    Ls = []
    for l in range(layers):
        base = slab.ptr + l * per_layer
        Ls.append(Q.MoeLayer(dim, hidden, E, K, rbuf.ptr, base, base + sizes[0],
                             base + sizes[0] + sizes[1], Q.TYPE_Q4_K, Q.TYPE_Q4_K, Q.TYPE_Q6_K))
    expert_bytes = sum(sizes) // E
    return dict(layers=Ls, slab=slab, rbuf=rbuf, u=u, router=router, parts=parts,
                expert_bytes=expert_bytes, per_layer=per_layer)


def moe_alg_bytes(T, touched, expert_bytes):
    dim, E = QWEN3["dim"], QWEN3["E"]
    return 4 * E * dim + touched * expert_bytes + 2 * 4 * T * dim


def bench_moe(dev, M, T, steps, warmup, nbatches=8, order=Q.ORDER_AVX2):
    dim, E, K = QWEN3["dim"], QWEN3["E"], QWEN3["K"]
    Ls = M["layers"]
    xb_all = np.concatenate([synth.zipf_tokens(7000 + 31 * T + b, T, dim, M["u"])
                             for b in range(nbatches)])
    xbb = dev.upload(xb_all)
    xs = dev.upload(synth.normal(7500 + T, (nbatches * T, dim)))
    # routing of each batch (for the algorithmic byte count: touched experts)
    idxb, wtb = dev.alloc(nbatches * T * K * 4), dev.alloc(nbatches * T * K * 4)
    dev.moe_route(Ls[0], xbb.ptr, nbatches * T, order, None, idxb.ptr, wtb.ptr)
    idx = dev.download(idxb, (nbatches, T * K), np.int32)
    touched = float(np.mean([np.unique(r).size for r in idx]))
    counts = np.bincount(idx[0], minlength=E)
    step_bytes = moe_alg_bytes(T, touched, M["expert_bytes"])

    def one(i):
        b = i % nbatches
        dev.moe_forward(Ls[i % len(Ls)], xs.ptr + b * T * dim * 4, xbb.ptr + b * T * dim * 4, T,
                        order)

    for i in range(max(warmup, 1)):
        one(i)
    dev.sync()
    g = dev.capture(lambda: [one(i) for i in range(steps)])
    dev.graph_launch(g)
    dev.sync()
    ms = timed_replays(dev, g)
    dev.graph_destroy(g)
    s = ms / 1e3 / steps
    return dict(T=T, ms_per_step=ms / steps, tokens_per_s=T / s,
                touched_experts=touched, max_tokens_per_expert=int(counts.max()),
                alg_bytes=int(step_bytes), achieved_gbps=step_bytes / s / 1e9,
                roofline_frac=step_bytes / s / 1e9 / HBM_PEAK_GBPS)


# ---------------------------------------------------------------------------
# CPU baseline: the reference's own code on this host
# ---------------------------------------------------------------------------
def cpu_baseline_gemv(seconds, cores):
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    n, d = 32000, 2048
    try:
        ref = O.RefLib("avx2")
        kind = "reference"
        call = lambda out, x, w: ref.lib.matmul_q_fused(out, x, w.ctypes.data_as(O.C.c_void_p),  # noqa: E731
                                                         12, n, d, cores)
    except FileNotFoundError:
        orc = O.Oracle()
        kind = "port"
        call = lambda out, x, w: orc.lib.qro_matmul_q_fused_batch(  # noqa: E731
            out, x, w.ctypes.data_as(O.C.c_void_p), 12, n, d, 1, cores, O.ORDER_SEQ)
    copies = 8  # 296 MB of weights: beyond the host's last-level cache
    Ws = [synth.weights(90 + c, n, d, Q.TYPE_Q4_K) for c in range(copies)]
    x = synth.normal(91, (d,))
    out = np.zeros(n, np.float32)
    call(out, x, Ws[0])  # warm-up
    t0 = time.perf_counter()
    calls = 0
    while time.perf_counter() - t0 < seconds or calls < 3:
        call(out, x, Ws[calls % copies])
        calls += 1
    dt = (time.perf_counter() - t0) / calls
    wbytes = n * synth.row_bytes(Q.TYPE_Q4_K, d)
    return dict(value=wbytes / dt / 1e9, unit="GB/s", cores=cores, kind=kind,
                sample="%d calls of matmul_q_fused Q4_K 32000x2048 over 8 weight copies (%s, "
                       "-O3 -std=c99 -mavx2 -mfma, OpenMP %d threads, %s); the reference's "
                       "Q4_K dot returns invalid values but does the same work"
                       % (calls, "oracle/_ref" if kind == "reference" else "oracle port", cores,
                          cpu_model()),
                ms_per_call=dt * 1e3)


def cpu_baseline_moe(M, tokens, cores):
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    dim, hidden, E, K = QWEN3["dim"], QWEN3["hidden"], QWEN3["E"], QWEN3["K"]
    up, gate, down = M["parts"]
    x = synth.zipf_tokens(9000, tokens, dim, M["u"])
    try:
        ref = O.RefLib("avx2")
        t0 = time.perf_counter()
        ref.moe_layer(x, dim, hidden, E, K, M["router"], up, Q.TYPE_Q4_K, gate, Q.TYPE_Q4_K,
                      down, Q.TYPE_Q6_K, backend=O.BACKEND_AVX2, threads=cores)
        kind = "reference"
    except FileNotFoundError:
        orc = O.Oracle()
        keep = []
        L = orc.make_layer(keep, dim, hidden, E, K, M["router"], up, Q.TYPE_Q4_K, gate,
                           Q.TYPE_Q4_K, down, Q.TYPE_Q6_K)
        t0 = time.perf_counter()
        orc.moe_forward(x, x, L, order=O.ORDER_AVX2, threads=cores)
        kind = "port"
    dt = time.perf_counter() - t0
    return dict(value=tokens / dt, unit="tokens/s", cores=cores, kind=kind,
                sample="%d tokens through forward_runtime's MoE block, one token per call as "
                       "the reference runs them (Qwen3 shape, %d OpenMP threads)" % (tokens, cores))


# ---------------------------------------------------------------------------
def load_traffic():
    p = os.path.join(REPO, "profiles", "k_gemv_blk_q4k_32000x2048_traffic.json")
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
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--moe-layers", type=int, default=48)
    ap.add_argument("--moe-t", default="1,16,512",
                    help="token counts of the MoE leg (comma-separated), e.g. 16 for a profile")
    ap.add_argument("--moe-steps", type=int, default=0,
                    help="layers timed per token count (0: the defaults, 100 / 100 / 20)")
    ap.add_argument("--no-gemv", action="store_true",
                    help="skip the GEMV headline (profiling runs of the MoE leg; value is null)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: there is no multi-GPU path; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    dev = Q.Device(0)
    cal = copy_calibration(dev)
    log("bench: copy kernel %.0f GB/s (read+write) over %d MB" % (cal["gbps"], cal["bytes"] >> 20))
    g = g4 = None
    if not args.no_gemv:
        g = bench_gemv(dev, Q.TYPE_Q4_K, 32000, 2048, 1, args.steps, args.warmup)
        log("bench: Q4_K 32000x2048 T=1: %.3f us/launch, %.0f GB/s weights, %.0f GB/s algorithmic"
            % (g["ms_per_step"] * 1e3, g["weight_gbps"], g["achieved_gbps"]))
        # the same GEMV for 4 tokens (the survey's K-quant config at NT = 4): not the headline
        g4 = bench_gemv(dev, Q.TYPE_Q4_K, 32000, 2048, 4, max(args.steps // 2, 20), args.warmup)
        log("bench: Q4_K 32000x2048 T=4: %.3f us/launch, %.0f GB/s weights"
            % (g4["ms_per_step"] * 1e3, g4["weight_gbps"]))

    moe = None
    if not args.no_moe:
        M = build_qwen3(dev, args.moe_layers)
        moe = {}
        default_steps = {1: max(args.steps, 100), 16: 100, 512: 20}
        for T in [int(t) for t in args.moe_t.split(",") if t.strip()]:
            steps = args.moe_steps or default_steps.get(T, 20)
            r = bench_moe(dev, M, T, steps, 3)
            moe["T%d" % T] = r
            log("bench: MoE Qwen3 T=%d: %.1f us/layer, %.0f tokens/s, %.1f experts touched, "
                "%.0f GB/s (%.1f%% of HBM peak)" % (T, r["ms_per_step"] * 1e3, r["tokens_per_s"],
                                                   r["touched_experts"], r["achieved_gbps"],
                                                   100 * r["roofline_frac"]))

    cores = host_cores()
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_gemv(args.cpu_seconds, cores)
        log("bench: CPU baseline %.1f GB/s (%s, %d cores)" % (cpu["value"], cpu["kind"], cores))
        if moe is not None:
            cpu_moe = cpu_baseline_moe(M, 16, cores)
            moe["cpu_baseline"] = cpu_moe
            log("bench: CPU MoE baseline %.1f tokens/s (%s)" % (cpu_moe["value"], cpu_moe["kind"]))

    out = {
        "metric": METRIC,
        "value": round(g["weight_gbps"], 2) if g else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 6) if g else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "Q4_K decode GEMV 32000x2048 (lm_head of the K-quant sweep), "
                               "1 token, 16 rotating weight copies", "n": 32000, "d": 2048,
                   "qtype": "Q4_K", "tokens": 1},
        "roofline": {"bound": "hbm", "achieved": round(g["achieved_gbps"], 2),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(g["achieved_gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": load_traffic()} if g else None,
        "cpu_baseline": cpu,
        "gemv_q4k_32000x2048_t4": {
            "ms_per_step": round(g4["ms_per_step"], 6), "weight_gbps": round(g4["weight_gbps"], 2),
            "alg_bytes": g4["alg_bytes"], "achieved_gbps": round(g4["achieved_gbps"], 2),
            "roofline_frac": round(g4["achieved_gbps"] / HBM_PEAK_GBPS, 4)} if g else None,
        "moe_qwen3": moe,
        "copy_kernel_gbps": round(cal["gbps"], 1),
    }
    print(json.dumps(out), flush=True)
    dev.close()


if __name__ == "__main__":
    main()
