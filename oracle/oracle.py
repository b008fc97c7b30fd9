"""ctypes binding of the parity checker (test infrastructure only).

``Oracle`` wraps liboracle.so, the C99 restatement of quantr-in-c's quantized
GEMV and MoE path (oracle/qr_oracle.c).  ``RefLib`` wraps oracle/_ref/libqref_*.so,
the reference's own sources compiled where they lie plus ref_driver.c; those
files exist only where the reference checkout was present at build time.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module.  The product never does.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

TYPE_F32, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 0, 8, 12, 13, 14
ORDER_SEQ, ORDER_AVX2, ORDER_AVX512 = 0, 1, 2
# KernelBackend values (include/types.h:99-108)
BACKEND_REF, BACKEND_AVX2, BACKEND_AVX512, BACKEND_GPU = 0, 1, 2, 7

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def row_bytes(qtype, d):
    """Bytes per weight row (src/quant.c:477-484)."""
    if qtype == TYPE_Q8_0:
        return (d // 32) * 34
    if qtype == TYPE_Q4_K:
        return (d // 256) * 144
    if qtype == TYPE_Q5_K:
        return (d // 256) * 176
    if qtype == TYPE_Q6_K:
        return (d // 256) * 210
    return d * 4


class MoeLayer(C.Structure):
    _fields_ = [
        ("dim", C.c_int), ("hidden", C.c_int), ("n_experts", C.c_int), ("n_used", C.c_int),
        ("router", C.c_void_p), ("up", C.c_void_p), ("gate", C.c_void_p), ("down", C.c_void_p),
        ("up_type", C.c_uint32), ("gate_type", C.c_uint32), ("down_type", C.c_uint32),
        ("sh_hidden", C.c_int), ("sh_gate_inp", C.c_void_p), ("sh_up", C.c_void_p),
        ("sh_gate", C.c_void_p), ("sh_down", C.c_void_p),
        ("sh_up_type", C.c_uint32), ("sh_gate_type", C.c_uint32), ("sh_down_type", C.c_uint32),
    ]


class OModel(C.Structure):
    """qro_model (oracle/qr_oracle.h)."""
    _fields_ = [
        ("dim", C.c_int), ("n_layers", C.c_int), ("n_heads", C.c_int), ("n_kv_heads", C.c_int),
        ("head_dim", C.c_int), ("vocab", C.c_int), ("seq_len", C.c_int), ("rope_base", C.c_float),
        ("kv_type", C.c_int), ("tok_embd", C.c_void_p), ("tok_type", C.c_uint32),
        ("tok_row_bytes", C.c_size_t), ("rms_att", C.c_void_p), ("rms_ffn", C.c_void_p),
        ("wq", C.c_void_p), ("wk", C.c_void_p), ("wv", C.c_void_p), ("wo", C.c_void_p),
        ("wtype", C.c_void_p), ("moe", C.c_void_p), ("rms_final", C.c_void_p),
        ("wcls", C.c_void_p), ("wcls_type", C.c_uint32), ("threads", C.c_int),
    ]


KV_F32, KV_F16, KV_Q8_0 = 0, 1, 2


def oracle_threads():
    """OpenMP width for the oracle's model-sized loops: the CPUs this process
    may run on, at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _parr(keep, arrs):
    """A C array of pointers to the numpy arrays (kept alive in `keep`)."""
    arrs = [None if a is None else np.ascontiguousarray(a) for a in arrs]
    keep.extend(a for a in arrs if a is not None)
    p = (C.c_void_p * len(arrs))(*[None if a is None else a.ctypes.data for a in arrs])
    keep.append(p)
    return p


def build_oracle():
    """Compile liboracle.so (and oracle/_ref when the reference checkout exists)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if os.path.isdir("/root/reference/src"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


class Oracle:
    def __init__(self, path=None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build_oracle()
        L = self.lib = C.CDLL(path)
        L.qro_h2f.restype = C.c_float
        L.qro_h2f.argtypes = [C.c_uint16]
        L.qro_h2f_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
        L.qro_f2h.restype = C.c_uint16
        L.qro_f2h.argtypes = [C.c_float]
        L.qro_row_bytes.restype = C.c_size_t
        L.qro_row_bytes.argtypes = [C.c_uint32, C.c_int]
        L.qro_units_per_row.restype = C.c_int
        L.qro_units_per_row.argtypes = [C.c_uint32, C.c_int]
        L.qro_quantize_row_q8_0.argtypes = [_f32p, C.c_void_p, C.c_int]
        L.qro_dequantize_row.argtypes = [_f32p, C.c_void_p, C.c_uint32, C.c_int]
        L.qro_vec_dot.restype = C.c_float
        L.qro_vec_dot.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.qro_row_accum.restype = C.c_int
        L.qro_row_accum.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int, _i32p, C.c_void_p]
        L.qro_matmul_q_fused_batch.argtypes = [_f32p, _f32p, C.c_void_p, C.c_uint32, C.c_int,
                                               C.c_int, C.c_int, C.c_int, C.c_int]
        L.qro_matmul_f32.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.qro_softmax.argtypes = [_f32p, C.c_int]
        L.qro_silu.restype = C.c_float
        L.qro_silu.argtypes = [C.c_float]
        L.qro_expf_batch.argtypes = [_f32p, _f32p, C.c_size_t]
        L.qro_route.restype = C.c_int
        L.qro_route.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_void_p, C.c_void_p, _i32p, _f32p]
        L.qro_moe_forward.argtypes = [_f32p, _f32p, C.c_int, C.POINTER(MoeLayer), C.c_int,
                                      C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        L.qro_shared_expert.argtypes = [_f32p, _f32p, C.POINTER(MoeLayer), C.c_int]
        L.qro_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int]
        L.qro_rope.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.qro_rope_table.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_float]
        L.qro_kv_row_bytes.restype = C.c_size_t
        L.qro_kv_row_bytes.argtypes = [C.c_int, C.c_int]
        L.qro_attention.argtypes = [_f32p, _f32p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_int,
                                    C.c_int, C.c_int, C.c_int, C.c_int, _f32p]
        L.qro_kv_store.argtypes = [C.c_void_p, _f32p, C.c_int, C.c_int]
        L.qro_forward.argtypes = [C.POINTER(OModel), C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                  C.c_int, _f32p, _f32p]
        L.qro_moe_dispatch.restype = C.c_int
        L.qro_moe_dispatch.argtypes = [_i32p, C.c_int, C.c_int, C.c_int, _i32p, _i32p, _i32p, _i32p]
        # llama.cpp / ggml K-quant formats (qr_oracle_ggml.c)
        L.qro_ggml_h2f.restype = C.c_float
        L.qro_ggml_h2f.argtypes = [C.c_uint16]
        L.qro_ggml_h2f_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
        L.qro_ggml_block_bytes.restype = C.c_size_t
        L.qro_ggml_block_bytes.argtypes = [C.c_int]
        L.qro_ggml_scale_min.argtypes = [C.c_void_p, _i32p, _i32p]
        L.qro_ggml_dequantize_row.argtypes = [C.c_int, C.c_void_p, _f32p, C.c_int]
        L.qro_quantize_row_q8_K.argtypes = [_f32p, C.c_void_p, C.c_int]
        L.qro_ggml_block_ints.argtypes = [C.c_int, C.c_void_p, C.c_void_p, _i32p, _i32p]
        L.qro_ggml_vec_dot.restype = C.c_float
        L.qro_ggml_vec_dot.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int]
        L.qro_ggml_matmul.argtypes = [_f32p, _f32p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int]

    # --- fp16 helpers, include/quant.h:53-77
    def h2f(self, h):
        return self.lib.qro_h2f(int(h))

    def h2f_bits(self, codes):
        """uint16 codes -> uint32 float bits (NaN payloads preserved)."""
        codes = np.ascontiguousarray(codes, np.uint16)
        out = np.empty(codes.size, np.float32)
        self.lib.qro_h2f_batch(_ptr(codes), _ptr(out), codes.size)
        return out.view(np.uint32)

    def f2h(self, f):
        return self.lib.qro_f2h(float(f))

    # --- llama.cpp / ggml K-quants (not in the reference; qr_oracle_ggml.c)
    def ggml_h2f_bits(self, codes):
        codes = np.ascontiguousarray(codes, np.uint16)
        out = np.empty(codes.size, np.float32)
        self.lib.qro_ggml_h2f_batch(_ptr(codes), _ptr(out), codes.size)
        return out.view(np.uint32)

    def ggml_scale_min(self, scales12):
        sc, mn = np.zeros(8, np.int32), np.zeros(8, np.int32)
        self.lib.qro_ggml_scale_min(_ptr(np.ascontiguousarray(scales12, np.uint8)), sc, mn)
        return sc, mn

    def ggml_dequantize(self, blob, qtype, n):
        out = np.zeros(n, np.float32)
        self.lib.qro_ggml_dequantize_row(qtype, _ptr(np.ascontiguousarray(blob, np.uint8)), out, n)
        return out

    def quantize_q8_K(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        out = np.zeros((x.size // 256) * 292, np.uint8)
        self.lib.qro_quantize_row_q8_K(x, _ptr(out), x.size)
        return out

    def ggml_block_ints(self, qtype, blk, yb):
        aux, sumi = np.zeros(8, np.int32), np.zeros(1, np.int32)
        self.lib.qro_ggml_block_ints(qtype, _ptr(np.ascontiguousarray(blk, np.uint8)),
                                     _ptr(np.ascontiguousarray(yb, np.uint8)), aux, sumi)
        return aux, int(sumi[0])

    def ggml_vec_dot(self, qtype, row, q8k, d):
        return self.lib.qro_ggml_vec_dot(qtype, _ptr(np.ascontiguousarray(row, np.uint8)),
                                         _ptr(np.ascontiguousarray(q8k, np.uint8)), d)

    def ggml_matmul(self, x, w, qtype, n, d):
        """x [nt, d] fp32, w [n][d/256 * block] bytes -> [nt, n]."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, d)
        out = np.zeros((x.shape[0], n), np.float32)
        self.lib.qro_ggml_matmul(out, x, _ptr(np.ascontiguousarray(w, np.uint8)), qtype, n, d,
                                 x.shape[0])
        return out

    # --- src/quant.c:143-158
    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        out = np.zeros((x.size // 32) * 34, np.uint8)
        self.lib.qro_quantize_row_q8_0(x, _ptr(out), x.size)
        return out

    def dequantize(self, blob, qtype, n):
        out = np.zeros(n, np.float32)
        blob = np.ascontiguousarray(blob, np.uint8)
        self.lib.qro_dequantize_row(out, _ptr(blob), qtype, n)
        return out

    def vec_dot(self, qtype, row, xq8, d, order=ORDER_SEQ):
        row = np.ascontiguousarray(row, np.uint8)
        xq8 = np.ascontiguousarray(xq8, np.uint8)
        return self.lib.qro_vec_dot(qtype, _ptr(row), _ptr(xq8), d, order)

    def row_accum(self, qtype, row, xq8, d):
        units = self.lib.qro_units_per_row(qtype, d)
        isum = np.zeros(max(units, 1), np.int32)
        bsum = np.zeros(max(units, 1), np.int32)
        row = np.ascontiguousarray(row, np.uint8)
        xq8 = np.ascontiguousarray(xq8, np.uint8)
        self.lib.qro_row_accum(qtype, _ptr(row), _ptr(xq8), d, isum, _ptr(bsum))
        return isum[:units], bsum[:units]

    def matmul_q_fused(self, x, w, qtype, n, d, threads=1, order=ORDER_SEQ):
        """x: [nt, d] or [d]; returns [nt, n] or [n] (src/quant.c:441-523)."""
        x = np.ascontiguousarray(x, np.float32)
        nt = 1 if x.ndim == 1 else x.shape[0]
        out = np.zeros((nt, n), np.float32)
        wptr = None if w is None else _ptr(np.ascontiguousarray(w))
        self.lib.qro_matmul_q_fused_batch(out, x.reshape(nt, d), wptr, qtype, n, d, nt,
                                          threads, order)
        return out[0] if x.ndim == 1 else out

    def matmul_f32(self, x, w, n, d, order=ORDER_SEQ):
        out = np.zeros(n, np.float32)
        self.lib.qro_matmul_f32(out, np.ascontiguousarray(x, np.float32),
                                np.ascontiguousarray(w, np.float32), n, d, order)
        return out

    def softmax(self, x):
        x = np.array(x, np.float32)
        self.lib.qro_softmax(x, x.size)
        return x

    def expf(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self.lib.qro_expf_batch(x.ravel(), out.ravel(), x.size)
        return out

    def route(self, xb, router_w, E, K, order=ORDER_SEQ):
        dim = xb.size
        logits = np.zeros(E, np.float32)
        probs = np.zeros(E, np.float32)
        idx = np.zeros(K, np.int32)
        wts = np.zeros(K, np.float32)
        self.lib.qro_route(np.ascontiguousarray(xb, np.float32),
                           np.ascontiguousarray(router_w, np.float32), dim, E, K, order,
                           _ptr(logits), _ptr(probs), idx, wts)
        return logits, probs, idx, wts

    @staticmethod
    def make_layer(keep, dim, hidden, E, K, router, up, up_type, gate, gate_type, down, down_type,
                   shared=None):
        """Build a MoeLayer; `keep` is a list that holds the numpy buffers alive."""
        bufs = [np.ascontiguousarray(router, np.float32), np.ascontiguousarray(up),
                np.ascontiguousarray(gate), np.ascontiguousarray(down)]
        keep.extend(bufs)
        L = MoeLayer(dim, hidden, E, K, _ptr(bufs[0]), _ptr(bufs[1]), _ptr(bufs[2]),
                     _ptr(bufs[3]), up_type, gate_type, down_type)
        if shared is not None:
            sb = [np.ascontiguousarray(shared["gate_inp"], np.float32),
                  np.ascontiguousarray(shared["up"]), np.ascontiguousarray(shared["gate"]),
                  np.ascontiguousarray(shared["down"])]
            keep.extend(sb)
            L.sh_hidden = shared["hidden"]
            L.sh_gate_inp, L.sh_up, L.sh_gate, L.sh_down = [_ptr(b) for b in sb]
            L.sh_up_type = shared["up_type"]
            L.sh_gate_type = shared.get("gate_type", shared["up_type"])
            L.sh_down_type = shared["down_type"]
        return L

    def moe_forward(self, x, xb, layer, order=ORDER_SEQ, dot_order=ORDER_SEQ, threads=1):
        """Returns (x_out [T,dim], idx [T,K], wts [T,K]) (src/runtime.c:202-269 per token).
        order: router (KernelOps.matmul) order; dot_order: Q8_0 fused-dot order."""
        x = np.array(x, np.float32, copy=True)
        T, K = x.shape[0], layer.n_used
        idx = np.zeros((T, K), np.int32)
        wts = np.zeros((T, K), np.float32)
        self.lib.qro_moe_forward(x, np.ascontiguousarray(xb, np.float32), T, C.byref(layer),
                                 order, dot_order, threads, _ptr(idx), _ptr(wts))
        return x, idx, wts

    def shared_expert(self, xb, layer, threads=1):
        y = np.zeros(layer.dim, np.float32)
        self.lib.qro_shared_expert(y, np.ascontiguousarray(xb, np.float32), C.byref(layer), threads)
        return y

    # --- the decode step (oracle/qr_oracle_decode.c)
    def rmsnorm(self, x, w):
        x = np.ascontiguousarray(x, np.float32)
        o = np.zeros_like(x)
        self.lib.qro_rmsnorm(o, x, np.ascontiguousarray(w, np.float32), x.size)
        return o

    def rope(self, q, k, head_dim, n_kv_heads, pos, base):
        q = np.array(q, np.float32)
        k = np.array(k, np.float32)
        if k.size < q.size:  # apply_rope reads k up to kv_dim only
            k = np.concatenate([k, np.zeros(q.size - k.size, np.float32)])
        self.lib.qro_rope(q, k, q.size, head_dim, n_kv_heads, pos, base)
        return q, k

    def rope_table(self, qlen, head_dim, pos, base):
        cs = np.zeros(qlen, np.float32)
        self.lib.qro_rope_table(cs, qlen, head_dim, pos, base)
        return cs

    def kv_row_bytes(self, kv_type, kv_dim):
        return self.lib.qro_kv_row_bytes(kv_type, kv_dim)

    def attention(self, q, kc, vc, kv_type, pos, n_heads, n_kv_heads, head_dim):
        """kc / vc: [pos+1][row bytes] uint8 (fp32 rows as bytes for KV_F32)."""
        q = np.ascontiguousarray(q, np.float32)
        kc = np.ascontiguousarray(kc)
        vc = np.ascontiguousarray(vc)
        out = np.zeros(n_heads * head_dim, np.float32)
        att = np.zeros(n_heads * (pos + 1), np.float32)
        self.lib.qro_attention(out, q, _ptr(kc), _ptr(vc), kc.nbytes // (pos + 1), kv_type, pos,
                               n_heads, n_kv_heads, head_dim, att)
        return out, att.reshape(n_heads, pos + 1)

    @staticmethod
    def make_model(keep, m, kv_type):
        """qro_model of a decode model dict (tests/golden/inputs.py decode_model)."""
        L = m["n_layers"]
        lay = m["layers"]
        moes = (MoeLayer * L)()
        for l in range(L):
            ml = Oracle.make_layer(keep, m["dim"], m["hidden"], m["E"], m["K"], lay[l]["router"],
                                   lay[l]["up"], m["up_type"], lay[l]["gate"], m["up_type"],
                                   lay[l]["down"], m["down_type"], shared=lay[l].get("shared"))
            moes[l] = ml
        keep.append(moes)
        wtype = np.array([t for l in range(L) for t in m["wtype"]], np.uint32)
        tok = np.ascontiguousarray(m["tok_embd"])
        keep.extend([wtype, tok])
        om = OModel()
        om.dim, om.n_layers, om.n_heads = m["dim"], L, m["n_heads"]
        om.n_kv_heads, om.head_dim, om.vocab = m["n_kv_heads"], m["head_dim"], m["vocab"]
        om.seq_len, om.rope_base, om.kv_type = m["seq_len"], m["rope_base"], kv_type
        om.tok_embd, om.tok_type = tok.ctypes.data, m["tok_type"]
        om.tok_row_bytes = tok.nbytes // m["vocab"]
        om.rms_att = C.cast(_parr(keep, [x["rms_att"] for x in lay]), C.c_void_p)
        om.rms_ffn = C.cast(_parr(keep, [x["rms_ffn"] for x in lay]), C.c_void_p)
        for f in ("wq", "wk", "wv", "wo"):
            setattr(om, f, C.cast(_parr(keep, [x[f] for x in lay]), C.c_void_p))
        om.wtype = wtype.ctypes.data
        om.moe = C.cast(moes, C.c_void_p)
        rf = np.ascontiguousarray(m["rms_final"], np.float32)
        wc = np.ascontiguousarray(m["wcls"])
        keep.extend([rf, wc])
        om.rms_final, om.wcls, om.wcls_type = rf.ctypes.data, wc.ctypes.data, m["wcls_type"]
        om.threads = oracle_threads()
        return om

    def forward_seq(self, m, tokens, order, kv_type=KV_F32):
        """qro_forward for tokens at positions 0..n-1: (logits [n][vocab], x [n][dim])."""
        keep = []
        om = self.make_model(keep, m, kv_type)
        kvd = m["n_kv_heads"] * m["head_dim"]
        rs = self.kv_row_bytes(kv_type, kvd)
        kc = np.zeros(m["n_layers"] * m["seq_len"] * rs, np.uint8)
        vc = np.zeros_like(kc)
        lg = np.zeros((len(tokens), m["vocab"]), np.float32)
        xs = np.zeros((len(tokens), m["dim"]), np.float32)
        for i, tok in enumerate(tokens):
            x = np.zeros(m["dim"], np.float32)
            lo = np.zeros(m["vocab"], np.float32)
            self.lib.qro_forward(C.byref(om), _ptr(kc), _ptr(vc), int(tok), i, order, x, lo)
            lg[i], xs[i] = lo, x
        return lg, xs

    def forward_cached(self, m, kc, vc, tokens, pos0, order, kv_type):
        """qro_forward for tokens at positions pos0, pos0 + 1, ... over a cache
        that already holds positions 0 .. pos0 - 1 (kc / vc: uint8
        [n_layers * seq_len * row bytes], updated in place)."""
        keep = []
        om = self.make_model(keep, m, kv_type)
        lg = np.zeros((len(tokens), m["vocab"]), np.float32)
        xs = np.zeros((len(tokens), m["dim"]), np.float32)
        for i, tok in enumerate(tokens):
            x = np.zeros(m["dim"], np.float32)
            lo = np.zeros(m["vocab"], np.float32)
            self.lib.qro_forward(C.byref(om), _ptr(kc), _ptr(vc), int(tok), pos0 + i, order, x,
                                 lo)
            lg[i], xs[i] = lo, x
        return lg, xs

    def kv_rows(self, vals, kv_type):
        """Cache rows (uint8 [n][row bytes]) of fp32 values [n][kv_dim]:
        qro_kv_store of each row."""
        vals = np.ascontiguousarray(vals, np.float32)
        n, kvd = vals.shape
        rs = self.kv_row_bytes(kv_type, kvd)
        out = np.zeros((n, rs), np.uint8)
        for t in range(n):
            self.lib.qro_kv_store(_ptr(out[t]), vals[t], kvd, kv_type)
        return out

    def dispatch(self, idx, E):
        idx = np.ascontiguousarray(idx, np.int32)
        T, K = idx.shape
        counts = np.zeros(E, np.int32)
        offsets = np.zeros(E + 1, np.int32)
        perm = np.zeros(T * K, np.int32)
        inv = np.zeros(T * K, np.int32)
        rc = self.lib.qro_moe_dispatch(idx.ravel(), T, K, E, counts, offsets, perm, inv)
        if rc != 0:
            raise ValueError("dispatch: expert index out of range")
        return counts, offsets, perm, inv


class RefLib:
    """The reference's own code (oracle/_ref/libqref_<flavour>.so)."""

    def __init__(self, flavour="c99"):
        path = os.path.join(HERE, "_ref", "libqref_%s.so" % flavour)
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.path = path
        L = self.lib = C.CDLL(path)
        L.refdrv_h2f.restype = C.c_float
        L.refdrv_h2f.argtypes = [C.c_uint16]
        L.refdrv_f2h.restype = C.c_uint16
        L.refdrv_f2h.argtypes = [C.c_float]
        L.quantize_row_q8_0.argtypes = [_f32p, C.c_void_p, C.c_int]
        L.dequantize_row.argtypes = [_f32p, C.c_void_p, C.c_uint32, C.c_int]
        for name in ("vec_dot_q8_0_q8_0", "vec_dot_q4K_q8_0", "vec_dot_q5K_q8_0",
                     "vec_dot_q6K_q8_0"):
            f = getattr(L, name)
            f.restype = C.c_float
            f.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        L.matmul_q_fused.argtypes = [_f32p, _f32p, C.c_void_p, C.c_uint32, C.c_int, C.c_int, C.c_int]
        L.refdrv_matmul.argtypes = [C.c_int, _f32p, _f32p, _f32p, C.c_int, C.c_int]
        L.refdrv_softmax.argtypes = [C.c_int, _f32p, C.c_int]
        L.refdrv_matmul_q_fused.argtypes = [_f32p, _f32p, C.c_void_p, C.c_uint32, C.c_int,
                                            C.c_int, C.c_int]
        if hasattr(L, "refgpu_bind"):  # the GPU-bound builds (ref_gpu_bind.c)
            L.refgpu_bind.restype = C.c_int
            L.refgpu_bind.argtypes = [C.c_int]
            L.refgpu_take_calls.restype = C.c_int
            L.refgpu_take_calls.argtypes = []
        L.refdrv_moe_bench.restype = C.c_int
        L.refdrv_moe_bench.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p,
                                       C.c_uint32, C.c_void_p, C.c_uint32, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_void_p]
        L.refdrv_decode_layer_bench.restype = C.c_int
        L.refdrv_decode_layer_bench.argtypes = [C.c_int] * 8 + [C.c_void_p, C.c_int] + \
            [C.c_void_p] * 6 + [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_uint32,
                                C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p]
        L.refdrv_gemv_bench.restype = C.c_int
        L.refdrv_gemv_bench.argtypes = [_f32p, C.c_void_p, C.c_int, C.c_uint32, C.c_int, C.c_int,
                                        C.c_int, C.c_int, C.c_int, _f32p, C.c_void_p]
        L.refdrv_gguf_parse.restype = C.c_int
        L.refdrv_gguf_parse.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_int, C.c_void_p,
                                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.refdrv_gguf_vals.restype = C.c_int
        L.refdrv_gguf_vals.argtypes = [C.c_void_p, C.c_size_t, C.c_char_p, C.c_uint32, C.c_float,
                                       C.c_void_p, C.c_void_p, C.c_char_p, C.c_int]
        L.refdrv_load_gguf.restype = C.c_int
        L.refdrv_load_gguf.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p]
        L.refdrv_forward.restype = C.c_int
        L.refdrv_forward.argtypes = [C.c_int] * 7 + [C.c_float, C.c_int, C.c_int, C.c_void_p,
                                                     C.c_uint32, C.c_size_t] + \
            [C.c_void_p] * 7 + [C.c_void_p] * 4 + [C.c_uint32] * 3 + \
            [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
             _f32p, C.c_void_p]
        L.refdrv_moe_layer.restype = C.c_int
        L.refdrv_moe_layer.argtypes = [_f32p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_int, _f32p, C.c_void_p, C.c_uint32,
                                       C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32,
                                       C.c_int, C.c_int]

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        out = np.zeros((x.size // 32) * 34, np.uint8)
        self.lib.quantize_row_q8_0(x, _ptr(out), x.size)
        return out

    def dequantize(self, blob, qtype, n):
        out = np.zeros(n, np.float32)
        self.lib.dequantize_row(out, _ptr(np.ascontiguousarray(blob, np.uint8)), qtype, n)
        return out

    def vec_dot(self, qtype, row, xq8, d):
        name = {TYPE_Q8_0: "vec_dot_q8_0_q8_0", TYPE_Q4_K: "vec_dot_q4K_q8_0",
                TYPE_Q5_K: "vec_dot_q5K_q8_0", TYPE_Q6_K: "vec_dot_q6K_q8_0"}[qtype]
        return getattr(self.lib, name)(_ptr(np.ascontiguousarray(row, np.uint8)),
                                       _ptr(np.ascontiguousarray(xq8, np.uint8)), d)

    def matmul_q_fused(self, x, w, qtype, n, d, threads=1):
        out = np.zeros(n, np.float32)
        self.lib.matmul_q_fused(out, np.ascontiguousarray(x, np.float32),
                                _ptr(np.ascontiguousarray(w)), qtype, n, d, threads)
        return out

    def matmul_q_fused_cross(self, x, w, qtype, n, d, threads=1):
        """matmul_q_fused called from another file (wrapped in the GPU-bound builds)."""
        out = np.zeros(n, np.float32)
        self.lib.refdrv_matmul_q_fused(out, np.ascontiguousarray(x, np.float32),
                                       _ptr(np.ascontiguousarray(w)), qtype, n, d, threads)
        return out

    def matmul(self, backend, x, w, n, d):
        out = np.zeros(n, np.float32)
        self.lib.refdrv_matmul(backend, out, np.ascontiguousarray(x, np.float32),
                               np.ascontiguousarray(w, np.float32), n, d)
        return out

    def softmax(self, backend, x):
        x = np.array(x, np.float32)
        self.lib.refdrv_softmax(backend, x, x.size)
        return x

    def moe_layer(self, x_in, dim, hidden, E, K, router, up, up_type, gate, gate_type, down,
                  down_type, backend=BACKEND_REF, threads=1):
        x_in = np.ascontiguousarray(x_in, np.float32)
        T = x_in.shape[0]
        xb = np.zeros_like(x_in)
        xo = np.zeros_like(x_in)
        rc = self.lib.refdrv_moe_layer(x_in, _ptr(xb), _ptr(xo), T, dim, hidden, E, K,
                                       np.ascontiguousarray(router, np.float32),
                                       _ptr(np.ascontiguousarray(up)), up_type,
                                       _ptr(np.ascontiguousarray(gate)), gate_type,
                                       _ptr(np.ascontiguousarray(down)), down_type,
                                       backend, threads)
        if rc != 0:
            raise RuntimeError("refdrv_moe_layer failed: %d" % rc)
        return xb, xo

    def moe_bench(self, x_in, dim, hidden, E, K, routers, ups, up_type, gates, gate_type, downs,
                  down_type, backend, threads, warmup, reps):
        """Seconds of each timed forward_runtime call over len(ups) MoE layers."""
        x_in = np.ascontiguousarray(x_in, np.float32)
        L = len(ups)
        arr = lambda bufs: (C.c_void_p * L)(*[b.ctypes.data for b in bufs])  # noqa: E731
        times = np.zeros(reps, np.float64)
        rc = self.lib.refdrv_moe_bench(x_in, x_in.shape[0], dim, hidden, E, K, L, arr(routers),
                                       arr(ups), up_type, arr(gates), gate_type, arr(downs),
                                       down_type, backend, threads, warmup, reps,
                                       times.ctypes.data_as(C.c_void_p))
        if rc != 0:
            raise RuntimeError("refdrv_moe_bench failed: %d" % rc)
        return times

    def decode_layer_bench(self, dim, n_heads, n_kv_heads, hidden, E, K, pos, tok_embd, copies,
                           wtype, up_type, down_type, rms, backend, threads, warmup, reps):
        """Seconds of each timed one-layer forward_runtime call at position pos
        (refdrv_decode_layer_bench); copies: dicts of wq, wk, wv, wo, router,
        up, gate, down arrays."""
        n = len(copies)
        arr = lambda k: (C.c_void_p * n)(*[c[k].ctypes.data for c in copies])  # noqa: E731
        tok = np.ascontiguousarray(tok_embd, np.float32)
        wt = np.array(wtype, np.uint32)
        rms = np.ascontiguousarray(rms, np.float32)
        times = np.zeros(reps, np.float64)
        rc = self.lib.refdrv_decode_layer_bench(
            dim, n_heads, n_kv_heads, hidden, E, K, pos, n, tok.ctypes.data, tok.shape[0],
            arr("wq"), arr("wk"), arr("wv"), arr("wo"), wt.ctypes.data, arr("router"), arr("up"),
            up_type, arr("gate"), arr("down"), down_type, rms.ctypes.data, backend, threads,
            warmup, reps, times.ctypes.data_as(C.c_void_p))
        if rc != 0:
            raise RuntimeError("refdrv_decode_layer_bench failed: %d" % rc)
        return times

    def gemv_bench(self, x, copies, qtype, n, d, threads, warmup, reps):
        """Seconds of each timed matmul_q_fused call, rotating over `copies`."""
        ptrs = (C.c_void_p * len(copies))(*[c.ctypes.data for c in copies])
        out = np.zeros(n, np.float32)
        times = np.zeros(reps, np.float64)
        rc = self.lib.refdrv_gemv_bench(np.ascontiguousarray(x, np.float32), ptrs, len(copies),
                                        qtype, n, d, threads, warmup, reps, out,
                                        times.ctypes.data_as(C.c_void_p))
        if rc != 0:
            raise RuntimeError("refdrv_gemv_bench failed: %d" % rc)
        return times

    def gguf_parse(self, data, max_t=4096):
        """gguf_init_from_buffer on data: None when refused, else (hdr dict,
        list of tensor dicts with the data offset from the buffer start)."""
        buf = C.create_string_buffer(bytes(data), len(data))
        hdr = np.zeros(5, np.uint64)
        names = C.create_string_buffer(96 * max_t)
        types = np.zeros(max_t, np.uint32)
        nd = np.zeros(max_t, np.uint32)
        ne = np.zeros(4 * max_t, np.uint64)
        off = np.zeros(max_t, np.uint64)
        rc = self.lib.refdrv_gguf_parse(C.cast(buf, C.c_void_p), len(data), _ptr(hdr), max_t, names,
                                        _ptr(types), _ptr(nd), _ptr(ne), _ptr(off))
        if rc != 0:
            return None
        h = dict(version=int(hdr[0]), n_tensors=int(hdr[1]), n_kv=int(hdr[2]),
                 alignment=int(hdr[3]), data_offset=int(hdr[4]))
        ts = []
        for i in range(min(h["n_tensors"], max_t)):
            nm = names.raw[96 * i:96 * (i + 1)].split(b"\0")[0].decode()
            ts.append(dict(name=nm, type=int(types[i]), n_dims=int(nd[i]),
                           ne=[int(v) for v in ne[4 * i:4 * i + 4]], offset=int(off[i])))
        return h, ts

    def gguf_vals(self, data, key, def_u32=7, def_f32=-1.5):
        buf = C.create_string_buffer(bytes(data), len(data))
        u = np.zeros(1, np.uint32)
        f = np.zeros(1, np.float32)
        out = C.create_string_buffer(512)
        rc = self.lib.refdrv_gguf_vals(C.cast(buf, C.c_void_p), len(data), key.encode(), def_u32,
                                       def_f32, _ptr(u), _ptr(f), out, 512)
        if rc != 0:
            return None
        return int(u[0]), float(f[0]), out.value.decode()

    def load_gguf(self, path, n_layers, n_experts):
        """load_transformer of a .gguf path: (cfg, rope_base, offsets, types,
        token_embd_row_bytes) as refdrv_load_gguf lays them out."""
        cfg = np.zeros(9, np.int32)
        rope = np.zeros(1, np.float32)
        # a dense model (no experts) reports its w1 / w2 / w3 in the experts' places
        off = np.zeros(3 + 7 * n_layers + 3 * n_layers * max(n_experts, 1), np.int64)
        types = np.zeros(2 + 7 * n_layers, np.uint32)
        rb = np.zeros(1, np.uint64)
        n = self.lib.refdrv_load_gguf(path.encode(), _ptr(cfg), _ptr(rope), _ptr(off), _ptr(types),
                                      _ptr(rb))
        assert n == len(off), (n, len(off))
        return cfg, float(rope[0]), off, types, int(rb[0])

    def forward(self, m, tokens, backend, threads=1, kv_type=0):
        """The reference's forward_runtime on decode model m (tests/golden/inputs.py)
        for tokens at positions 0..n-1: (logits [n][vocab], x [n][dim])."""
        keep = []
        lay = m["layers"]
        L = m["n_layers"]
        wtype = np.array([t for l in range(L) for t in m["wtype"]], np.uint32)
        tok = np.ascontiguousarray(m["tok_embd"])
        toks = np.array(tokens, np.int32)
        keep.extend([wtype, tok, toks])
        P = lambda key: _parr(keep, [x[key] for x in lay])  # noqa: E731
        lg = np.zeros((len(tokens), m["vocab"]), np.float32)
        xs = np.zeros((len(tokens), m["dim"]), np.float32)
        rf = np.ascontiguousarray(m["rms_final"], np.float32)
        wc = np.ascontiguousarray(m["wcls"])
        keep.extend([rf, wc])
        rc = self.lib.refdrv_forward(
            m["dim"], m["hidden"], L, m["n_heads"], m["n_kv_heads"], m["vocab"], m["seq_len"],
            m["rope_base"], m["E"], m["K"], tok.ctypes.data, m["tok_type"], tok.nbytes // m["vocab"],
            P("rms_att"), P("rms_ffn"), P("wq"), P("wk"), P("wv"), P("wo"), wtype.ctypes.data,
            P("router"), P("up"), P("gate"), P("down"), m["up_type"], m["up_type"], m["down_type"],
            rf.ctypes.data, wc.ctypes.data, m["wcls_type"], toks.ctypes.data, len(tokens), kv_type,
            backend, threads, lg, xs.ctypes.data)
        if rc != 0:
            raise RuntimeError("refdrv_forward failed: %d" % rc)
        return lg, xs
