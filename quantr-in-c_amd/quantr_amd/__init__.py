"""ctypes binding of libqr_hip.so, the MI355X (gfx950) quantized GEMV + MoE
library whose C ABI is declared in include/qr_hip.h and include/qr_dropin.h.

This module only moves bytes and calls the C ABI; all arithmetic happens in the
HIP kernels.  If the library has not been built, importing works but
``load()`` raises: there is no CPU fallback.
"""
import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "lib", "libqr_hip.so")
HEADERS = [os.path.join(REPO_DIR, "include", "qr_hip.h"),
           os.path.join(REPO_DIR, "include", "qr_dropin.h")]

TYPE_F32, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 0, 8, 12, 13, 14
TILED = 0x100  # OR'ed into a Q4_K / Q5_K / Q6_K / Q8_0 type: the weights are in the tiled layout
GGML = 0x200   # OR'ed into a Q4_K / Q5_K / Q6_K type: llama.cpp's block layout, Q8_K activations
GGUF_GGML_KQUANTS = 1  # qr_gguf_load_ex: the file's K-quant tensors in llama.cpp's layouts
ORDER_SEQ, ORDER_AVX2, ORDER_AVX512 = 0, 1, 2

_vp = C.c_void_p


class QrError(RuntimeError):
    pass


class MoeLayer(C.Structure):
    """qr_moe_layer (include/qr_hip.h); pointers are device addresses."""
    _fields_ = [
        ("dim", C.c_int), ("hidden", C.c_int), ("n_experts", C.c_int), ("n_used", C.c_int),
        ("router", _vp), ("up", _vp), ("gate", _vp), ("down", _vp),
        ("up_type", C.c_uint32), ("gate_type", C.c_uint32), ("down_type", C.c_uint32),
        ("sh_hidden", C.c_int), ("sh_gate_inp", _vp), ("sh_up", _vp), ("sh_gate", _vp),
        ("sh_down", _vp),
        ("sh_up_type", C.c_uint32), ("sh_gate_type", C.c_uint32), ("sh_down_type", C.c_uint32),
    ]


class Layer(C.Structure):
    """qr_layer (include/qr_hip.h); pointers are device addresses."""
    _fields_ = [
        ("rms_att", _vp), ("rms_ffn", _vp), ("wq", _vp), ("wk", _vp), ("wv", _vp), ("wo", _vp),
        ("wq_type", C.c_uint32), ("wk_type", C.c_uint32), ("wv_type", C.c_uint32),
        ("wo_type", C.c_uint32), ("moe", MoeLayer),
    ]


class Model(C.Structure):
    """qr_model (include/qr_hip.h); `layers` is a host array of Layer."""
    _fields_ = [
        ("dim", C.c_int), ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
        ("n_layers", C.c_int), ("vocab", C.c_int), ("seq_len", C.c_int), ("rope_base", C.c_float),
        ("tok_embd", _vp), ("tok_type", C.c_uint32), ("rms_final", _vp), ("wcls", _vp),
        ("wcls_type", C.c_uint32), ("layers", C.POINTER(Layer)),
    ]


KV_F32, KV_F16, KV_Q8_0 = 0, 1, 2
MOE_PATH_AUTO, MOE_PATH_GEMV, MOE_PATH_MFMA = 0, 1, 2
DEC_GRAPH = 1
PREFILL_ALL_LOGITS = 1
PREFILL_CHUNK = 512  # QR_PREFILL_CHUNK: the chunk of qr_decoder_prefill(..., chunk=0)

_SIGS = {
    "qr_last_error": (C.c_char_p, []),
    "qr_version": (C.c_char_p, []),
    "qr_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "qr_ctx_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "qr_ctx_destroy": (C.c_int, [_vp]),
    "qr_ctx_set_stream": (C.c_int, [_vp, _vp]),
    "qr_ctx_get_stream": (_vp, [_vp]),
    "qr_ctx_set_moe_path": (C.c_int, [_vp, C.c_int]),
    "qr_sync": (C.c_int, [_vp]),
    "qr_malloc": (C.c_int, [_vp, C.c_size_t, C.POINTER(_vp)]),
    "qr_free": (C.c_int, [_vp, _vp]),
    "qr_memcpy_h2d": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "qr_memcpy_d2h": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "qr_memcpy_d2d": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "qr_memset": (C.c_int, [_vp, _vp, C.c_int, C.c_size_t]),
    "qr_timer_start": (C.c_int, [_vp]),
    "qr_timer_stop": (C.c_int, [_vp, C.POINTER(C.c_float)]),
    "qr_copy_kernel": (C.c_int, [_vp, _vp, _vp, C.c_size_t]),
    "qr_read_kernel": (C.c_int, [_vp, _vp, C.c_size_t, _vp]),
    "qr_capture_begin": (C.c_int, [_vp]),
    "qr_capture_end": (C.c_int, [_vp, C.POINTER(_vp)]),
    "qr_graph_launch": (C.c_int, [_vp, _vp]),
    "qr_graph_destroy": (C.c_int, [_vp]),
    "qr_quantize_q8_0": (C.c_int, [_vp, _vp, _vp, C.c_long]),
    "qr_quantize_q8_k": (C.c_int, [_vp, _vp, _vp, C.c_long]),
    "qr_gemv_ex": (C.c_int, [_vp, C.c_uint32, _vp, _vp, C.c_int, _vp, C.c_int, C.c_int, C.c_int,
                             C.c_int, _vp, _vp]),
    "qr_gemv": (C.c_int, [_vp, C.c_uint32, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int]),
    "qr_gemv_ord": (C.c_int, [_vp, C.c_int, C.c_uint32, _vp, _vp, C.c_int, _vp, C.c_int, C.c_int,
                              C.c_int, C.c_int, _vp, _vp]),
    "qr_gemv_rows": (C.c_int, [_vp, C.c_int, C.c_uint32, _vp, _vp, C.c_int, _vp, C.c_int, C.c_int,
                               C.c_int, C.c_int]),
    "qr_matmul_f32": (C.c_int, [_vp, C.c_int, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int]),
    "qr_softmax": (C.c_int, [_vp, _vp, C.c_int, C.c_int]),
    "qr_row_bytes": (C.c_size_t, [C.c_uint32, C.c_int]),
    "qr_moe_route": (C.c_int, [_vp, C.POINTER(MoeLayer), _vp, C.c_int, C.c_int, _vp, _vp, _vp]),
    "qr_moe_dispatch": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp]),
    "qr_moe_forward": (C.c_int, [_vp, C.POINTER(MoeLayer), _vp, _vp, C.c_int, C.c_int, _vp, _vp]),
    "qr_moe_forward_noalloc": (C.c_int, [_vp, C.POINTER(MoeLayer), _vp, _vp, C.c_int, C.c_int,
                                         _vp, _vp]),
    "qr_weights_upload": (C.c_int, [_vp, _vp, C.c_size_t, C.POINTER(_vp)]),
    "qr_weights_tile": (C.c_int, [_vp, C.c_uint32, _vp, _vp, C.c_int, C.c_int]),
    "qr_weights_untile": (C.c_int, [_vp, C.c_uint32, _vp, _vp, C.c_int, C.c_int]),
    "qr_weights_upload_parts": (C.c_int, [_vp, _vp, _vp, C.c_size_t, C.c_int, C.POINTER(_vp)]),
    "qr_weights_lookup": (C.c_int, [_vp, _vp, C.POINTER(_vp)]),
    "qr_weights_release": (C.c_int, [_vp, _vp]),
    "qr_weights_release_all": (C.c_int, [_vp]),
    "qr_test_expf": (C.c_int, [_vp, _vp, _vp, C.c_long]),
    "qr_kv_row_bytes": (C.c_size_t, [C.c_int, C.c_int]),
    "qr_dequantize": (C.c_int, [_vp, C.c_uint32, _vp, C.c_int, C.c_int, _vp]),
    "qr_rmsnorm": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int]),
    "qr_attention": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int,
                               C.c_int, C.c_int, _vp, _vp]),
    "qr_decoder_create": (C.c_int, [_vp, C.POINTER(Model), C.c_int, C.c_int, C.c_int, C.c_int,
                                    C.POINTER(_vp)]),
    "qr_decoder_destroy": (C.c_int, [_vp]),
    "qr_decoder_set_pages": (C.c_int, [_vp, _vp]),
    "qr_decoder_pages": (C.c_int, [_vp, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "qr_decoder_kv_write": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "qr_decoder_kv_rows": (C.c_int, [_vp, C.c_int, C.c_int, C.POINTER(_vp), C.POINTER(_vp)]),
    "qr_decoder_forward": (C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp]),
    "qr_decoder_prefill": (C.c_int, [_vp, C.POINTER(C.c_int32), C.c_int, C.c_int, C.c_int, _vp, _vp,
                                     C.c_int]),
    "qr_gguf_parse": (C.c_int, [_vp, C.c_size_t, C.POINTER(_vp)]),
    "qr_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "qr_gguf_close": (C.c_int, [_vp]),
    "qr_gguf_info": (C.c_int, [_vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                               C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                               C.POINTER(C.c_uint64)]),
    "qr_gguf_tensor": (C.c_int, [_vp, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32),
                                 C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(_vp)]),
    "qr_gguf_find": (C.c_int64, [_vp, C.c_char_p]),
    "qr_gguf_get_u32": (C.c_uint32, [_vp, C.c_char_p, C.c_uint32]),
    "qr_gguf_get_f32": (C.c_float, [_vp, C.c_char_p, C.c_float]),
    "qr_gguf_get_str": (C.c_char_p, [_vp, C.c_char_p]),
    "qr_gguf_get_arr_len": (C.c_int64, [_vp, C.c_char_p]),
    "qr_gguf_model_host": (C.c_int, [_vp, C.c_int, C.POINTER(Model), C.POINTER(Layer), C.c_int]),
    "qr_gguf_expert_host": (C.c_int, [_vp, C.c_int, C.c_int, C.POINTER(_vp), C.POINTER(_vp),
                                      C.POINTER(_vp)]),
    "qr_gguf_load": (C.c_int, [_vp, _vp, C.c_int, C.POINTER(_vp)]),
    "qr_gguf_load_ex": (C.c_int, [_vp, _vp, C.c_int, C.c_uint32, C.POINTER(_vp)]),
    "qr_gguf_model_get": (C.POINTER(Model), [_vp]),
    "qr_gguf_model_free": (C.c_int, [_vp]),
    # drop-ins (include/qr_dropin.h)
    "qr_dropin_init": (C.c_int, [C.c_int, C.c_int]),
    "qr_dropin_shutdown": (None, []),
    "qr_gpu_available": (C.c_int, []),
    "qr_matmul_q_fused": (None, [_vp, _vp, _vp, C.c_uint32, C.c_int, C.c_int, C.c_int]),
    "qr_quantize_row_q8_0": (None, [_vp, _vp, C.c_int]),
    "qr_ops_matmul": (None, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int]),
    "qr_ops_softmax": (None, [_vp, C.c_int]),
    "qr_moe_block": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32,
                               C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "qr_dropin_register_weights": (C.c_int, [_vp, C.c_size_t]),
    "qr_dropin_release_weights": (None, []),
}

_lib = None


def load(path=None):
    """Load libqr_hip.so (built by __graft_entry__.build() or `make`)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise QrError("libqr_hip.so is not built (%s); run __graft_entry__.build()" % path)
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    if path == LIB_PATH:
        _lib = lib
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_vp)


class DevBuf:
    """A device allocation owned by a Device."""

    def __init__(self, dev, nbytes):
        self.dev = dev
        self.nbytes = int(nbytes)
        p = _vp()
        dev._check(dev.lib.qr_malloc(dev.ctx, max(self.nbytes, 16), C.byref(p)), "qr_malloc")
        self.ptr = p.value

    def offset(self, nbytes):
        return self.ptr + int(nbytes)

    def free(self):
        if self.ptr is not None and self.dev.ctx is not None:
            self.dev.lib.qr_free(self.dev.ctx, _vp(self.ptr))
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Device:
    """One qr_ctx on one GPU."""

    def __init__(self, device=0, lib=None):
        self.lib = lib or load()
        ctx = _vp()
        self._check(self.lib.qr_ctx_create(device, C.byref(ctx)), "qr_ctx_create")
        self.ctx = ctx.value

    def _check(self, rc, what):
        if rc != 0:
            msg = self.lib.qr_last_error().decode(errors="replace")
            raise QrError("%s failed (%d): %s" % (what, rc, msg))

    def close(self):
        if self.ctx is not None:
            self.lib.qr_ctx_destroy(_vp(self.ctx))
            self.ctx = None

    def set_moe_path(self, path):
        """QR_MOE_PATH_*: 0 auto, 1 grouped GEMV, 2 int8 MFMA (T > 1)."""
        self._check(self.lib.qr_ctx_set_moe_path(self.ctx, path), "qr_ctx_set_moe_path")

    # ---- memory
    def alloc(self, nbytes):
        return DevBuf(self, nbytes)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        b = DevBuf(self, arr.nbytes)
        self._check(self.lib.qr_memcpy_h2d(self.ctx, _vp(b.ptr), _ptr(arr), arr.nbytes), "h2d")
        return b

    def download(self, buf, shape, dtype, offset=0):
        out = np.empty(shape, dtype)
        ptr = buf.ptr if isinstance(buf, DevBuf) else buf
        self._check(self.lib.qr_memcpy_d2h(self.ctx, _ptr(out), _vp(ptr + offset), out.nbytes),
                    "d2h")
        return out

    def write(self, buf, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        ptr = buf.ptr if isinstance(buf, DevBuf) else buf
        self._check(self.lib.qr_memcpy_h2d(self.ctx, _vp(ptr + offset), _ptr(arr), arr.nbytes),
                    "h2d")

    def memset(self, buf, value, nbytes):
        ptr = buf.ptr if isinstance(buf, DevBuf) else buf
        self._check(self.lib.qr_memset(self.ctx, _vp(ptr), value, nbytes), "qr_memset")

    def copy(self, dst, src, nbytes):
        self._check(self.lib.qr_memcpy_d2d(self.ctx, _vp(dst), _vp(src), nbytes), "d2d")

    def sync(self):
        self._check(self.lib.qr_sync(self.ctx), "qr_sync")

    # ---- timing on the context stream
    def timer_start(self):
        self._check(self.lib.qr_timer_start(self.ctx), "qr_timer_start")

    def timer_stop(self):
        ms = C.c_float()
        self._check(self.lib.qr_timer_stop(self.ctx, C.byref(ms)), "qr_timer_stop")
        return ms.value

    # ---- HIP graphs
    def capture(self, fn):
        """Record fn()'s enqueued work into a graph; returns the graph handle."""
        self._check(self.lib.qr_capture_begin(self.ctx), "qr_capture_begin")
        try:
            fn()
        finally:
            g = _vp()
            rc = self.lib.qr_capture_end(self.ctx, C.byref(g))
        self._check(rc, "qr_capture_end")
        return g.value

    def last_error(self):
        return self.lib.qr_last_error().decode(errors="replace")

    def graph_launch(self, g):
        self._check(self.lib.qr_graph_launch(self.ctx, _vp(g)), "qr_graph_launch")

    def graph_destroy(self, g):
        self._check(self.lib.qr_graph_destroy(_vp(g)), "qr_graph_destroy")

    # ---- ops (device pointers)
    def quantize_q8_0(self, x_ptr, y_ptr, n):
        self._check(self.lib.qr_quantize_q8_0(self.ctx, _vp(x_ptr), _vp(y_ptr), n), "qr_quantize_q8_0")

    def quantize_q8_k(self, x_ptr, y_ptr, n):
        """qr_quantize_q8_k: n / 256 ggml block_q8_K (292 bytes each)."""
        self._check(self.lib.qr_quantize_q8_k(self.ctx, _vp(x_ptr), _vp(y_ptr), n), "qr_quantize_q8_k")

    def gemv(self, qtype, w_ptr, x_ptr, y_ptr, n, d, nt=1, xstride=None, ystride=None,
             acc_ptr=None, accb_ptr=None, order=ORDER_SEQ):
        """qr_gemv_ord: `order` is the reference build (only Q8_0 depends on it)."""
        self._check(self.lib.qr_gemv_ord(self.ctx, order, qtype, _vp(w_ptr), _vp(x_ptr),
                                          xstride or d, _vp(y_ptr), ystride or n, n, d, nt,
                                          _vp(acc_ptr), _vp(accb_ptr)), "qr_gemv_ord")

    def gemv_rows(self, qtype, w_ptr, x_ptr, y_ptr, n, d, T, xstride=None, ystride=None,
                  order=ORDER_SEQ):
        """qr_gemv_rows: T tokens through one matrix as an int8 MFMA product
        (the same bits as gemv token by token)."""
        self._check(self.lib.qr_gemv_rows(self.ctx, order, qtype, _vp(w_ptr), _vp(x_ptr),
                                           xstride or d, _vp(y_ptr), ystride or n, n, d, T),
                    "qr_gemv_rows")

    def tile(self, qtype, src_ptr, dst_ptr, n, d, reverse=False):
        """qr_weights_tile (or qr_weights_untile): the tiled copy of an n x d
        Q4_K / Q5_K / Q6_K / Q8_0 matrix; pass qtype | TILED to gemv for it."""
        f = self.lib.qr_weights_untile if reverse else self.lib.qr_weights_tile
        self._check(f(self.ctx, qtype, _vp(src_ptr), _vp(dst_ptr), n, d),
                    "qr_weights_untile" if reverse else "qr_weights_tile")

    def matmul_f32(self, order, w_ptr, x_ptr, y_ptr, n, d, nt=1):
        self._check(self.lib.qr_matmul_f32(self.ctx, order, _vp(w_ptr), _vp(x_ptr), _vp(y_ptr),
                                           n, d, nt), "qr_matmul_f32")

    def softmax(self, x_ptr, rows, n):
        self._check(self.lib.qr_softmax(self.ctx, _vp(x_ptr), rows, n), "qr_softmax")

    def moe_route(self, layer, xb_ptr, T, order, probs_ptr, idx_ptr, wts_ptr):
        self._check(self.lib.qr_moe_route(self.ctx, C.byref(layer), _vp(xb_ptr), T, order,
                                          _vp(probs_ptr), _vp(idx_ptr), _vp(wts_ptr)),
                    "qr_moe_route")

    def moe_dispatch(self, idx_ptr, T, K, E, counts, offsets, perm, inv):
        self._check(self.lib.qr_moe_dispatch(self.ctx, _vp(idx_ptr), T, K, E, _vp(counts),
                                             _vp(offsets), _vp(perm), _vp(inv)), "qr_moe_dispatch")

    def moe_forward(self, layer, x_ptr, xb_ptr, T, order, idx_ptr=None, w_ptr=None):
        self._check(self.lib.qr_moe_forward(self.ctx, C.byref(layer), _vp(x_ptr), _vp(xb_ptr), T,
                                            order, _vp(idx_ptr), _vp(w_ptr)), "qr_moe_forward")

    def copy_kernel(self, dst, src, nbytes):
        self._check(self.lib.qr_copy_kernel(self.ctx, _vp(dst), _vp(src), nbytes), "qr_copy_kernel")

    def read_kernel(self, src, nbytes, sink):
        self._check(self.lib.qr_read_kernel(self.ctx, _vp(src), nbytes, _vp(sink)), "qr_read_kernel")

    def test_expf(self, x_ptr, y_ptr, n):
        self._check(self.lib.qr_test_expf(self.ctx, _vp(x_ptr), _vp(y_ptr), n), "qr_test_expf")

    def dequantize(self, qtype, src_ptr, rows, n, out_ptr):
        self._check(self.lib.qr_dequantize(self.ctx, qtype, _vp(src_ptr), rows, n, _vp(out_ptr)),
                    "qr_dequantize")

    def rmsnorm(self, o_ptr, x_ptr, w_ptr, n, add_ptr=None):
        self._check(self.lib.qr_rmsnorm(self.ctx, _vp(o_ptr), _vp(x_ptr), _vp(add_ptr), _vp(w_ptr),
                                        n), "qr_rmsnorm")

    def attention(self, q_ptr, kc_ptr, vc_ptr, ptab_ptr, page, kv_type, npos, n_heads,
                  n_kv_heads, head_dim, att_ptr, out_ptr):
        self._check(self.lib.qr_attention(self.ctx, _vp(q_ptr), _vp(kc_ptr), _vp(vc_ptr),
                                          _vp(ptab_ptr), page, kv_type, npos, n_heads, n_kv_heads,
                                          head_dim, _vp(att_ptr), _vp(out_ptr)), "qr_attention")


class Decoder:
    """qr_decoder over a model whose weights are already on the device.

    `model` is a Model whose `layers` points at a ctypes array this object
    keeps alive."""

    def __init__(self, dev, model, layers, kv_type=KV_Q8_0, order=ORDER_SEQ, page=0, flags=0):
        self.dev = dev
        self._layers = layers
        self._model = model
        h = _vp()
        dev._check(dev.lib.qr_decoder_create(dev.ctx, C.byref(model), kv_type, order, page, flags,
                                             C.byref(h)), "qr_decoder_create")
        self.h = h.value

    def pages(self):
        n, p = C.c_int(), C.c_int()
        self.dev._check(self.dev.lib.qr_decoder_pages(_vp(self.h), C.byref(n), C.byref(p)),
                        "qr_decoder_pages")
        return n.value, p.value

    def set_pages(self, table):
        t = np.ascontiguousarray(table, dtype=np.int32)
        self.dev._check(self.dev.lib.qr_decoder_set_pages(_vp(self.h), _ptr(t)),
                        "qr_decoder_set_pages")

    def kv_write(self, layer, pos0, n, k_ptr, v_ptr):
        self.dev._check(self.dev.lib.qr_decoder_kv_write(_vp(self.h), layer, pos0, n, _vp(k_ptr),
                                                         _vp(v_ptr)), "qr_decoder_kv_write")

    def kv_rows(self, layer, pos):
        k, v = _vp(), _vp()
        self.dev._check(self.dev.lib.qr_decoder_kv_rows(_vp(self.h), layer, pos, C.byref(k),
                                                        C.byref(v)), "qr_decoder_kv_rows")
        return k.value, v.value

    def forward(self, token, pos, logits_ptr, x_ptr=None):
        self.dev._check(self.dev.lib.qr_decoder_forward(_vp(self.h), token, pos,
                                                        _vp(logits_ptr), _vp(x_ptr)),
                        "qr_decoder_forward")

    def prefill(self, tokens, pos0, logits_ptr=None, x_ptr=None, chunk=0, all_logits=False):
        """qr_decoder_prefill: tokens at positions pos0 .. pos0 + len - 1."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        self.dev._check(self.dev.lib.qr_decoder_prefill(
            _vp(self.h), t.ctypes.data_as(C.POINTER(C.c_int32)), len(t), pos0, chunk,
            _vp(logits_ptr), _vp(x_ptr), PREFILL_ALL_LOGITS if all_logits else 0),
            "qr_decoder_prefill")

    def close(self):
        if self.h is not None:
            self.dev.lib.qr_decoder_destroy(_vp(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Gguf:
    """A parsed GGUF container (host only).  From bytes (kept alive here) or a
    file path (mapped read-only by the library)."""

    def __init__(self, data=None, path=None, lib=None):
        self.lib = lib or load()
        h = _vp()
        if isinstance(data, (str, os.PathLike)):
            data, path = None, os.fspath(data)
        if path is not None:
            rc = self.lib.qr_gguf_open(path.encode(), C.byref(h))
            self._buf = None
        else:
            self._buf = C.create_string_buffer(bytes(data), len(data))
            rc = self.lib.qr_gguf_parse(C.cast(self._buf, _vp), len(data), C.byref(h))
        if rc != 0:
            raise QrError("GGUF parse failed (%d): %s" % (
                rc, self.lib.qr_last_error().decode(errors="replace")))
        self.h = h.value

    @property
    def base(self):
        """Address of the parsed bytes (buffer form only)."""
        return C.addressof(self._buf) if self._buf is not None else None

    def info(self):
        v, nt, nk, al, do = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        self.lib.qr_gguf_info(_vp(self.h), C.byref(v), C.byref(nt), C.byref(nk), C.byref(al),
                              C.byref(do))
        return dict(version=v.value, n_tensors=nt.value, n_kv=nk.value, alignment=al.value,
                    data_offset=do.value)

    def tensor(self, i):
        name, typ, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
        ne, data = (C.c_uint64 * 4)(), _vp()
        rc = self.lib.qr_gguf_tensor(_vp(self.h), i, C.byref(name), C.byref(typ), C.byref(nd), ne,
                                     C.byref(data))
        if rc != 0:
            raise QrError("qr_gguf_tensor(%d) failed" % i)
        return dict(name=name.value.decode(), type=typ.value, n_dims=nd.value, ne=list(ne),
                    data=data.value)

    def tensors(self):
        return [self.tensor(i) for i in range(self.info()["n_tensors"])]

    def u32(self, key, default=0):
        return self.lib.qr_gguf_get_u32(_vp(self.h), key.encode(), default)

    def f32(self, key, default=0.0):
        return self.lib.qr_gguf_get_f32(_vp(self.h), key.encode(), default)

    def str(self, key):
        v = self.lib.qr_gguf_get_str(_vp(self.h), key.encode())
        return None if v is None else v.decode()

    def arr_len(self, key):
        return self.lib.qr_gguf_get_arr_len(_vp(self.h), key.encode())

    def model_host(self, seq_len=0):
        """(Model, Layer array) of host pointers into the buffer."""
        m = Model()
        n = self.lib.qr_gguf_model_host(_vp(self.h), seq_len, C.byref(m), None, 0)
        if n <= 0:
            raise QrError("qr_gguf_model_host failed (%d): %s" % (
                n, self.lib.qr_last_error().decode(errors="replace")))
        layers = (Layer * n)()
        n2 = self.lib.qr_gguf_model_host(_vp(self.h), seq_len, C.byref(m), layers, n)
        if n2 != n:
            raise QrError("qr_gguf_model_host failed (%d)" % n2)
        return m, layers

    def expert_host(self, layer, e):
        up, down, gate = _vp(), _vp(), _vp()
        rc = self.lib.qr_gguf_expert_host(_vp(self.h), layer, e, C.byref(up), C.byref(down),
                                          C.byref(gate))
        if rc != 0:
            raise QrError("qr_gguf_expert_host failed")
        return up.value, down.value, gate.value

    def load(self, dev, seq_len, ggml_kquants=False):
        """A GgufModel: the model uploaded to dev's GPU (ggml_kquants: its
        K-quant tensors in llama.cpp's layouts, QR_GGUF_GGML_KQUANTS)."""
        return GgufModel(dev, self, seq_len, GGUF_GGML_KQUANTS if ggml_kquants else 0)

    def close(self):
        if self.h is not None:
            self.lib.qr_gguf_close(_vp(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GgufModel:
    """qr_gguf_load: a qr_model of device pointers in one device allocation
    this object owns (the Gguf may be closed after loading)."""

    def __init__(self, dev, g, seq_len, flags=0):
        self.dev, self.g = dev, g
        h = _vp()
        dev._check(dev.lib.qr_gguf_load_ex(dev.ctx, _vp(g.h), seq_len, flags, C.byref(h)),
                   "qr_gguf_load")
        self.h = h.value
        mp = dev.lib.qr_gguf_model_get(_vp(self.h))
        self.model = mp.contents
        self.layers = self.model.layers

    def decoder(self, kv_type=KV_Q8_0, order=ORDER_SEQ, page=0, flags=0):
        return Decoder(self.dev, self.model, self, kv_type=kv_type, order=order, page=page,
                       flags=flags)

    def close(self):
        if self.h is not None:
            self.dev.lib.qr_gguf_model_free(_vp(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def upload_decode_model(dev, m):
    """Model + Layer array for a decoder from a dict of weights.

    m holds the sizes (dim, n_heads, n_kv_heads, head_dim, n_layers, vocab,
    seq_len, rope_base, E, K, hidden), the types (tok_type, wcls_type,
    wtype = (wq, wk, wv, wo), up_type (also gate), down_type) and the tensors
    (tok_embd, rms_final, wcls, and per layer rms_att, rms_ffn, wq, wk, wv,
    wo, router, up, gate, down, and optionally shared: a shared expert as
    {hidden, gate_inp, up, gate, down, up_type, down_type}).  A tensor is a numpy array (uploaded here) or
    an int device address (used as is).  E = 0 describes a dense model: up,
    gate and down are then each layer's ffn_up (w1), ffn_gate (w3) and
    ffn_down (w2), and router is empty.  Returns (model, layers, keep); keep
    holds the device buffers and must outlive the decoder."""
    keep = []

    def dptr(a):
        if a is None or (isinstance(a, np.ndarray) and a.size == 0):
            return 0  # e.g. the router of a dense layer (n_experts 0)
        if isinstance(a, (int, np.integer)):
            return int(a)
        if isinstance(a, DevBuf):
            keep.append(a)
            return a.ptr
        b = dev.upload(np.ascontiguousarray(a))
        keep.append(b)
        return b.ptr

    L = m["n_layers"]
    layers = (Layer * L)()
    wt = m["wtype"]
    for l in range(L):
        lw = m["layers"][l]
        y = layers[l]
        y.rms_att, y.rms_ffn = dptr(lw["rms_att"]), dptr(lw["rms_ffn"])
        y.wq, y.wk, y.wv, y.wo = (dptr(lw[k]) for k in ("wq", "wk", "wv", "wo"))
        y.wq_type, y.wk_type, y.wv_type, y.wo_type = wt
        e = y.moe
        e.dim, e.hidden, e.n_experts, e.n_used = m["dim"], m["hidden"], m["E"], m["K"]
        e.router = dptr(lw["router"])
        e.up, e.gate, e.down = dptr(lw["up"]), dptr(lw["gate"]), dptr(lw["down"])
        e.up_type = e.gate_type = m["up_type"]
        e.down_type = m["down_type"]
        sh = lw.get("shared")
        if sh is not None:  # a shared expert with its sigmoid gate
            e.sh_hidden = sh["hidden"]
            e.sh_gate_inp, e.sh_up = dptr(sh["gate_inp"]), dptr(sh["up"])
            e.sh_gate, e.sh_down = dptr(sh["gate"]), dptr(sh["down"])
            e.sh_up_type = e.sh_gate_type = sh["up_type"]
            e.sh_down_type = sh["down_type"]
    mo = Model()
    mo.dim, mo.n_heads, mo.n_kv_heads = m["dim"], m["n_heads"], m["n_kv_heads"]
    mo.head_dim, mo.n_layers, mo.vocab = m["head_dim"], L, m["vocab"]
    mo.seq_len, mo.rope_base = m["seq_len"], m["rope_base"]
    mo.tok_embd, mo.tok_type = dptr(m["tok_embd"]), m["tok_type"]
    mo.rms_final = dptr(m["rms_final"])
    mo.wcls, mo.wcls_type = dptr(m["wcls"]), m["wcls_type"]
    mo.layers = C.cast(layers, C.POINTER(Layer))
    keep.append(layers)
    return mo, layers, keep


def declared_symbols():
    """Function names declared in include/qr_hip.h and include/qr_dropin.h."""
    import re
    names = []
    for h in HEADERS:
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"\b(qr_[a-z0-9_]+)\s*\(", src):
            if m.group(1) not in names:
                names.append(m.group(1))
    return names
