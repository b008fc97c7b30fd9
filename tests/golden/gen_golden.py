"""Write the golden fixtures of tests/golden/ from the compiled reference.

Runs only where the reference checkout exists: it loads oracle/_ref/libqref_*.so
(the reference's own src/quant.c, src/kernels.c, src/runtime.c, src/model.c,
src/gguf.c and src/threadpool.c, compiled where they lie by `make -C oracle ref`,
plus oracle/ref_driver.c) and records what the reference computes on the inputs
built by inputs.py.  Every number in the fixtures comes from the reference's
code; this script only feeds it and saves the results.

    make -C oracle ref && python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, HERE)

import inputs as I  # noqa: E402
from oracle import BACKEND_AVX2, BACKEND_AVX512, BACKEND_REF, RefLib  # noqa: E402


def cpu_has(flag):
    try:
        return flag in open("/proc/cpuinfo").read().split()
    except OSError:
        return False


def save(name, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrays)
    print("wrote %s (%d bytes)" % (path, os.path.getsize(path)))


def gen_fp16(r):
    import ctypes as C
    codes = np.arange(65536, dtype=np.uint32)
    codes16 = codes.astype(np.uint16)
    h2f = np.empty(65536, np.float32)
    r.lib.refdrv_h2f_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
    r.lib.refdrv_h2f_batch(codes16.ctypes.data, h2f.ctypes.data, 65536)
    h2f = h2f.view(np.uint32)
    rng = np.random.default_rng(5)
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e5, -1e5, 6.1035156e-05,
                         6.1e-05, 5.96e-08, 1e-8, 3.14159, 0.0001, 2.0 ** -14, 2.0 ** -15,
                         np.inf, -np.inf], np.float32)
    rnd = rng.integers(0, 2 ** 32, size=4096, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rnd = rnd[np.isfinite(rnd)]
    f_in = np.concatenate([specials, rnd]).astype(np.float32)
    f_out = np.array([r.lib.refdrv_f2h(float(f)) for f in f_in], np.uint16)
    save("fp16.npz", h2f_sha=np.array(I.digest(h2f)), h2f_sample_codes=codes[::97],
         h2f_sample=h2f[::97], f2h_in=f_in, f2h_out=f_out)


def gen_q8(r):
    edge = I.q8_edge_rows()
    edge_out = np.stack([r.quantize_q8_0(row) for row in edge])
    rnd = I.activations(11, 16, 2048)
    rnd_out = np.stack([r.quantize_q8_0(row) for row in rnd])
    save("q8_quant.npz", edge_in=edge, edge_out=edge_out, rand_sha=np.array(I.digest(rnd)),
         rand_out=rnd_out)


def gen_dequant(r):
    out = {}
    for t in (I.TYPE_Q8_0, I.TYPE_Q4_K, I.TYPE_Q5_K, I.TYPE_Q6_K):
        elems, bb = I.BLOCK[t]
        blob = np.concatenate([I.blocks(100 + t, t, 16), I.special_blocks(t)])
        n = (blob.size // bb) * elems
        out["in_sha_%d" % t] = np.array(I.digest(blob))
        out["out_%d" % t] = r.dequantize(blob, t, n).view(np.uint32)
    save("dequant.npz", **out)


def gen_dots(rc, ra, r5):
    out = {}
    for d in (2048, 768):
        x = I.activations(300 + d, 4, d)
        xq_c = np.stack([rc.quantize_q8_0(row) for row in x])
        xq_a = np.stack([ra.quantize_q8_0(row) for row in x])
        assert (xq_c == xq_a).all()
        out["x_sha_%d" % d] = np.array(I.digest(x))
        for t in (I.TYPE_Q8_0, I.TYPE_Q5_K, I.TYPE_Q6_K, I.TYPE_Q4_K):
            W = I.dot_set(200 + t + d, t, 15, d)
            out["w_sha_%d_%d" % (t, d)] = np.array(I.digest(W))
            Wr, tr = W, t
            if t == I.TYPE_Q4_K:
                # The reference's Q4_K dot is defective; its Q5_K dot on the same
                # blocks with a zero fifth-bit plane is the value it was meant to compute.
                Wr, tr = np.stack([I.q4k_to_q5k(row) for row in W]), I.TYPE_Q5_K
            vc = [[rc.vec_dot(tr, Wr[i], xq_c[j], d) for j in range(4)] for i in range(W.shape[0])]
            va = [[ra.vec_dot(tr, Wr[i], xq_a[j], d) for j in range(4)] for i in range(W.shape[0])]
            mc = [rc.matmul_q_fused(x[j], Wr, tr, W.shape[0], d, threads=4) for j in range(4)]
            out["dot_c99_%d_%d" % (t, d)] = np.array(vc, np.float32)
            out["dot_avx2_%d_%d" % (t, d)] = np.array(va, np.float32)
            if r5 is not None and t == I.TYPE_Q8_0:
                # the AVX-512 build updates the Q8_0 dot's 8 lanes by fused multiply-adds
                v5 = [[r5.vec_dot(tr, Wr[i], xq_c[j], d) for j in range(4)]
                      for i in range(W.shape[0])]
                out["dot_avx512_%d_%d" % (t, d)] = np.array(v5, np.float32)
            out["mm_c99_%d_%d" % (t, d)] = np.array(mc, np.float32).T.copy()
    save("dots.npz", **out)


def gen_router(rc, ra, r5):
    out = {}
    for (E, d, seed) in ((128, 2048, 400), (60, 2048, 410), (16, 2051, 420)):
        W = I.activations(seed, E, d, std=0.02)
        X = I.activations(seed + 1, 4, d)
        out["sha_%d_%d" % (E, d)] = np.array(I.digest(W, X))
        out["ref_%d_%d" % (E, d)] = np.stack([rc.matmul(BACKEND_REF, x, W, E, d) for x in X])
        out["avx2_%d_%d" % (E, d)] = np.stack([ra.matmul(BACKEND_AVX2, x, W, E, d) for x in X])
        if r5 is not None:
            out["avx512_%d_%d" % (E, d)] = np.stack([r5.matmul(BACKEND_AVX512, x, W, E, d) for x in X])
        out["softmax_%d_%d" % (E, d)] = np.stack(
            [rc.softmax(BACKEND_REF, l) for l in out["ref_%d_%d" % (E, d)]])
    save("router.npz", **out)


def gen_moe(rc, ra, r5):
    out = {}
    for name in I.MOE_CASES:
        m = I.moe_inputs(name)
        out["sha_" + name] = np.array(I.digest(m["up"], m["gate"], m["down"], m["router"], m["x"]))
        ut = m["up_type"]
        up, gate = m["up"], m["gate"]
        if ut == I.TYPE_Q4_K:  # the reference's sound Q5_K path computes corrected Q4_K
            up, gate, ut = I.q4k_to_q5k(up), I.q4k_to_q5k(gate), I.TYPE_Q5_K
        builds = [("c99", rc, BACKEND_REF), ("avx2", ra, BACKEND_AVX2)]
        if r5 is not None:
            builds.append(("avx512", r5, BACKEND_AVX512))
        for tag, lib, backend in builds:
            xb, xo = lib.moe_layer(m["x"], m["dim"], m["hidden"], m["E"], m["K"], m["router"], up, ut,
                                   gate, ut, m["down"], m["down_type"], backend=backend, threads=4)
            out["xb_%s_%s" % (name, tag)] = xb
            out["xo_%s_%s" % (name, tag)] = xo
    save("moe.npz", **out)


def gen_decode(rc, ra, r5):
    """forward_runtime of the small decode models, token by token from
    position 0, in each build, with the fp32 KV cache (kv_cache_type 0) and
    with the fp16 one (kv_cache_type 1, malloc_run_state_kv: keys logits16_*,
    x16_*)."""
    out = {}
    for name in I.DECODE_CASES:
        m = I.decode_model(name)
        out["sha_" + name] = np.array(I.decode_digest(m))
        builds = [("c99", rc, BACKEND_REF), ("avx2", ra, BACKEND_AVX2)]
        if r5 is not None:
            builds.append(("avx512", r5, BACKEND_AVX512))
        for tag, lib, backend in builds:
            lg, xs = lib.forward(m, m["tokens"], backend, threads=2)
            out["logits_%s_%s" % (name, tag)] = lg
            out["x_%s_%s" % (name, tag)] = xs
            lg, xs = lib.forward(m, m["tokens"], backend, threads=2, kv_type=1)
            out["logits16_%s_%s" % (name, tag)] = lg
            out["x16_%s_%s" % (name, tag)] = xs
    save("decode.npz", **out)


def main():
    rc, ra = RefLib("c99"), RefLib("avx2")
    assert rc.lib.refdrv_has_avx2_paths() == 0 and ra.lib.refdrv_has_avx2_paths() == 1
    r5 = RefLib("avx512") if cpu_has("avx512f") else None
    if r5 is not None:
        assert r5.lib.refdrv_has_avx512_paths() == 1
    gen_fp16(rc)
    gen_q8(rc)
    gen_dequant(rc)
    gen_dots(rc, ra, r5)
    gen_router(rc, ra, r5)
    gen_moe(rc, ra, r5)
    gen_decode(rc, ra, r5)


if __name__ == "__main__":
    main()
