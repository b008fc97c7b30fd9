"""The reference's own runtime with libqr_hip.so bound in by the linker.

oracle/_ref/libqref_gpu_<build>.so is the reference's unmodified sources
(src/runtime.c, quant.c, kernels.c, model.c, ...) compiled with one build's
flags and linked with -Wl,--wrap so that matmul_q_fused, resolve_backend and
kernels_for_backend go to the drop-ins (oracle/ref_gpu_bind.c: INTEGRATION.md's
binding, applied by the linker).  Run on BACKEND_GPU, the reference's own
forward_runtime must give what the same build computes on the CPU: the
golden fixtures written by the compiled reference, and the plain reference
build run on this host.
"""
import os

import numpy as np
import pytest

import inputs as I
from conftest import assert_bits_equal
from oracle import BACKEND_AVX2, BACKEND_AVX512, BACKEND_GPU, BACKEND_REF, HERE, RefLib
from quantr_amd import synth

pytestmark = pytest.mark.gpu

BUILDS = [("c99", 0, BACKEND_REF), ("avx2", 1, BACKEND_AVX2), ("avx512", 2, BACKEND_AVX512)]


def _host_has(flag):
    try:
        return flag in open("/proc/cpuinfo").read().split()
    except OSError:
        return False


def _builds():
    out = []
    for tag, order, backend in BUILDS:
        if tag == "avx512" and not _host_has("avx512f"):
            continue  # this host cannot run the -mavx512f build
        out.append((tag, order, backend))
    return out


_LIBS = {}


def _bound(tag, order):
    if tag not in _LIBS:
        path = os.path.join(HERE, "_ref", "libqref_gpu_%s.so" % tag)
        assert os.path.exists(path), "run __graft_entry__.build() where the reference exists"
        _LIBS[tag] = RefLib("gpu_" + tag)
    lib = _LIBS[tag]
    assert lib.lib.refgpu_bind(order) == 0
    lib.lib.refgpu_take_calls()
    return lib


@pytest.mark.parametrize("name", sorted(I.MOE_CASES))
@pytest.mark.parametrize("tag,order,backend", _builds())
def test_forward_runtime_moe_on_gpu_matches_reference_build(golden, name, tag, order, backend):
    """forward_runtime's MoE layer (src/runtime.c:202-269) with every expert
    GEMV and the router on the GPU: bit-exact with the fixture the same
    reference build wrote on the CPU."""
    g = golden("moe.npz")
    m = I.moe_inputs(name)
    up, gate, ut = m["up"], m["gate"], m["up_type"]
    if ut == I.TYPE_Q4_K:  # as the fixture: the reference's sound Q5_K path
        up, gate, ut = I.q4k_to_q5k(up), I.q4k_to_q5k(gate), I.TYPE_Q5_K
    lib = _bound(tag, order)
    xb, xo = lib.moe_layer(m["x"], m["dim"], m["hidden"], m["E"], m["K"], m["router"], up, ut,
                           gate, ut, m["down"], m["down_type"], backend=BACKEND_GPU, threads=4)
    T = m["x"].shape[0]
    assert lib.lib.refgpu_take_calls() == T * m["K"] * 3, "expert GEMVs not on the GPU"
    assert_bits_equal(xb, g["xb_%s_%s" % (name, tag)], "xb %s/%s" % (name, tag))
    assert_bits_equal(xo, g["xo_%s_%s" % (name, tag)], "forward_runtime %s/%s" % (name, tag))


@pytest.mark.parametrize("qtype", [I.TYPE_Q8_0, I.TYPE_Q5_K, I.TYPE_Q6_K])
@pytest.mark.parametrize("tag,order,backend", _builds())
def test_matmul_q_fused_through_reference_matches_cpu_build(qtype, tag, order, backend):
    """matmul_q_fused called from the reference's code goes to the GPU and
    returns what the same build returns on this host's CPU (plain
    oracle/_ref/libqref_<build>.so), at the 5632 x 2048 TinyLlama shape."""
    n, d = 5632, 2048
    W = synth.weights(6100 + qtype, n, d, qtype)
    x = synth.normal(6200, (d,))
    lib = _bound(tag, order)
    got = lib.matmul_q_fused_cross(x, W, qtype, n, d, threads=8)
    assert lib.lib.refgpu_take_calls() == 1
    cpu = RefLib(tag).matmul_q_fused_cross(x, W, qtype, n, d, threads=8)
    assert_bits_equal(got, cpu, "matmul_q_fused type %d, %s build" % (qtype, tag))


@pytest.mark.parametrize("tag,order,backend", _builds())
def test_forward_runtime_qwen3_layer_matches_cpu_build(tag, order, backend):
    """A Qwen3-30B-A3B-shaped MoE layer (128 experts top-8, ffn 768, down
    Q6_K; gate/up Q5_K, the reference's sound K-quant path) for 4 tokens
    through the GPU-bound forward_runtime and through the same build on this
    host's CPU: bit-exact."""
    dim, hidden, E, K = 2048, 768, 128, 8
    router, u, _ = synth.zipf_router(6300, E, dim)
    up = I.q4k_to_q5k(synth.weights(6301, E * hidden, dim, I.TYPE_Q4_K))
    gate = I.q4k_to_q5k(synth.weights(6302, E * hidden, dim, I.TYPE_Q4_K))
    down = synth.weights(6303, E * dim, hidden, I.TYPE_Q6_K)
    x = synth.zipf_tokens(6304, 4, dim, u)
    lib = _bound(tag, order)
    xb, xo = lib.moe_layer(x, dim, hidden, E, K, router, up, I.TYPE_Q5_K, gate, I.TYPE_Q5_K, down,
                           I.TYPE_Q6_K, backend=BACKEND_GPU, threads=8)
    assert lib.lib.refgpu_take_calls() == 4 * K * 3
    cxb, cxo = RefLib(tag).moe_layer(x, dim, hidden, E, K, router, up, I.TYPE_Q5_K, gate,
                                     I.TYPE_Q5_K, down, I.TYPE_Q6_K, backend=backend, threads=8)
    assert_bits_equal(xb, cxb, "xb")
    assert_bits_equal(xo, cxo, "forward_runtime Qwen3 layer, %s build" % tag)
