// qr_runtime.hip -- context, memory, weight registry, timing and the C-ABI
// entry points of libqr_hip.so.  Argument checking happens here, on the host,
// before any kernel is launched: every launch below has had its sizes,
// alignments and types validated against what the kernel assumes.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "qr_common.h"
#include "qr_internal.h"
#include "qr_tokens.h"

// A registered weight tensor: its device copy, its size, and a 64-bit digest
// of what it was uploaded from (the first and last up to 64 bytes of each
// host range, and for gathered tensors the part pointers and size).
struct RegEntry {
  void* dev = nullptr;
  size_t bytes = 0;
  uint64_t digest = 0;
  bool gathered = false;
};

// FNV-1a over `n` bytes, continuing from h.
static uint64_t fnv(uint64_t h, const void* p, size_t n) {
  const uint8_t* b = static_cast<const uint8_t*>(p);
  for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 0x100000001B3ull;
  return h;
}

// Digest of host range [host, host + bytes): its length and its two ends.
static uint64_t range_digest(uint64_t h, const void* host, size_t bytes) {
  const size_t n = bytes < 64 ? bytes : 64;
  h = fnv(h, &bytes, sizeof(bytes));
  h = fnv(h, host, n);
  return fnv(h, static_cast<const uint8_t*>(host) + bytes - n, n);
}

static uint64_t parts_digest(const void* const* parts, size_t part_bytes, int nparts) {
  uint64_t h = 0xCBF29CE484222325ull;
  for (int i = 0; i < nparts; i++) {
    h = fnv(h, &parts[i], sizeof(parts[i]));
    h = range_digest(h, parts[i], part_bytes);
  }
  return h;
}

struct qr_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  std::mutex mu;
  std::unordered_map<const void*, RegEntry> registry;
  // Device scratch of the MoE and router calls.  A buffer that a larger call
  // supersedes is retired, not freed: graphs captured earlier may still
  // point at it.  Retired buffers are freed by qr_ctx_destroy.
  void* work = nullptr;
  size_t work_bytes = 0;
  std::vector<void*> retired;
  // Device address of this GPU's copy of the static `scratch` array
  // (qr_moe_forward_noalloc).
  void* static_scratch = nullptr;
  // QR_MOE_PATH_* for this context's MoE calls with T > 1.
  int moe_path = QR_MOE_PATH_AUTO;
};

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(QR_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define QR_HIP(call, what)                     \
  do {                                         \
    hipError_t e_ = (call);                    \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

bool known_type(uint32_t t) {
  return t == QR_T_F32 || t == QR_T_Q8_0 || t == QR_T_Q4_K || t == QR_T_Q5_K || t == QR_T_Q6_K;
}

int set_device(qr_ctx* c) {
  QR_HIP(hipSetDevice(c->device), "hipSetDevice");
  return QR_OK;
}

// True while the context's stream is being captured into a graph.  Calls that
// would allocate, free, synchronize or record a memset node refuse then.
bool capturing(qr_ctx* c) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(c->stream, &st) != hipSuccess) return false;
  return st != hipStreamCaptureStatusNone;
}

#define QR_NO_CAPTURE(c, who)                                                               \
  do {                                                                                      \
    if (capturing(c))                                                                       \
      return fail(QR_ERR_INVALID, "%s: not allowed while the stream is being captured "    \
                  "(it allocates, synchronizes or sets memory)", who);                      \
  } while (0)

// At least `need` bytes of context scratch.  Growing is refused under capture;
// the superseded buffer is retired (freed at qr_ctx_destroy), and the new one
// is at least 1.5 x the old, so at most a few buffers are ever retired.
int ctx_scratch(qr_ctx* c, size_t need, const char* who, void** out) {
  if (need > c->work_bytes) {
    if (capturing(c))
      return fail(QR_ERR_INVALID,
                  "%s: needs %zu bytes of scratch, more than any earlier call; run it once "
                  "outside graph capture first",
                  who, need);
    if (set_device(c) != QR_OK) return QR_ERR_HIP;
    size_t want = c->work_bytes + c->work_bytes / 2;
    if (want < need) want = need;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) return fail(QR_ERR_NOMEM, "%s: scratch of %zu bytes: %s", who, want,
                                     hipGetErrorString(e));
    if (c->work) c->retired.push_back(c->work);
    c->work = p;
    c->work_bytes = want;
  }
  *out = c->work;
  return QR_OK;
}

// ---- the static scratch of qr_moe_forward_noalloc ---------------------------
// A file-scope device array: every GPU the library runs on holds its own copy
// (QR_NOALLOC_SCRATCH_BYTES) from code-object load until the process ends.
// Host code never uses the name `scratch` as an address (on the host it is a
// stand-in, not device memory): qr_ctx_create looks up this device's copy
// with hipGetSymbolAddress, once per device, and every use goes through that
// pointer.  Calls on one GPU share the array; it keeps the last call's
// contents (the MoE kernels write every scratch word they read, so nothing
// has to start at zero).
__device__ __align__(256) uint8_t scratch[QR_NOALLOC_SCRATCH_BYTES];

std::mutex g_sym_mu;
void* g_sym_ptr[64] = {};  // per device; set once, with that device current

// This device's address of `scratch`; c's device is current.
int static_scratch_addr(int device, void** out) {
  if (device < 0 || device >= 64) return fail(QR_ERR_INVALID, "device %d out of range", device);
  std::lock_guard<std::mutex> lk(g_sym_mu);
  if (!g_sym_ptr[device]) {
    void* p = nullptr;
    QR_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) return fail(QR_ERR_HIP, "hipGetSymbolAddress(scratch): null address");
    g_sym_ptr[device] = p;
  }
  *out = g_sym_ptr[device];
  return QR_OK;
}

// ---- small kernels ---------------------------------------------------------
// out[t * stride + i] = 0 for i < n, t < rows: the zero output of a call with
// no weights, as a kernel (no memset node in a captured graph).
__global__ void k_zero_rows(float* __restrict__ out, int n, int rows, int stride) {
  const long total = (long)n * rows;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long)gridDim.x * blockDim.x) {
    const int t = (int)(i / n);
    out[(size_t)t * stride + (i - (long)t * n)] = 0.0f;
  }
}

// dst[i] = v for i < n bytes: qr_memset under graph capture.
__global__ void k_fill_u8(uint8_t* __restrict__ dst, uint8_t v, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = v;
}

__global__ void k_copy16(uint4* __restrict__ dst, const uint4* __restrict__ src, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

// A plain read of n16 16-byte chunks: one non-temporal load per thread, one
// short-lived workgroup per 256 chunks -- the fastest of the plain-read forms
// measured on MI355X (6.6 us for 36.9 MB, against 7.0-8.4 us for grid-stride
// loops and for several loads per thread): the achievable-rate reference for
// a kernel that streams the same bytes once.  The XOR of what was read is
// stored only if it equals `never` (a value the caller's data cannot produce
// in practice), so the loads cannot be dropped.
__global__ void k_read16(const uint4* __restrict__ src, size_t n16, uint32_t never,
                         uint32_t* __restrict__ sink) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n16) return;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + i));
  const uint32_t acc = v.x ^ v.y ^ v.z ^ v.w;
  if (acc == never) sink[0] = acc;
}

// Both device forms of expf: the memory-table one and the register-table one
// the latency-critical kernels use; they must agree with each other (and the
// test compares with the host C library).
__global__ void k_test_expf(const float* __restrict__ x, float* __restrict__ y, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const float v = i < n ? x[i] : 0.0f;
  const float a = qr_expf_w(v, qr_expf_tab());  // every lane
  const float b = qr_expf(v);
  if (i < n) y[i] = __builtin_bit_cast(uint32_t, a) == __builtin_bit_cast(uint32_t, b)
                        ? a
                        : __builtin_bit_cast(float, 0x7FC0DEADu);  // flags a disagreement
}

}  // namespace

// Context internals for the other translation units (qr_internal.h).
// The host C layer's (host/qr_gguf.c) way to set qr_last_error(); local to
// the library (not a qr_* symbol, so the export map keeps it hidden).
extern "C" int qrint_set_error(int code, const char* msg) { return fail(code, "%s", msg); }

namespace qr {
int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}
hipStream_t ctx_stream(qr_ctx* c) { return c->stream; }
int ctx_device(qr_ctx* c) { return c->device; }
bool ctx_capturing(qr_ctx* c) { return capturing(c); }
}  // namespace qr

extern "C" {

const char* qr_last_error(void) { return g_err; }

const char* qr_version(void) { return "qr_hip 0.1 gfx950"; }

int qr_device_count(int* count) {
  if (!count) return fail(QR_ERR_INVALID, "qr_device_count: null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *count = 0;
    return hip_fail(e, "hipGetDeviceCount");
  }
  *count = n;
  return QR_OK;
}

int qr_ctx_create(int device, qr_ctx** out) {
  if (!out) return fail(QR_ERR_INVALID, "qr_ctx_create: null out");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return fail(QR_ERR_NODEV, "qr_ctx_create: no HIP device");
  if (device < 0 || device >= n)
    return fail(QR_ERR_INVALID, "qr_ctx_create: device %d of %d", device, n);
  hipDeviceProp_t prop;
  QR_HIP(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(QR_ERR_NODEV, "qr_ctx_create: device %d is %s, this library is built for gfx950",
                device, prop.gcnArchName);
  qr_ctx* c = new qr_ctx();
  c->device = device;
  if (set_device(c) != QR_OK) {
    delete c;
    return QR_ERR_HIP;
  }
  hipError_t e = hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&c->ev0);
  if (e == hipSuccess) e = hipEventCreate(&c->ev1);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "qr_ctx_create");
  }
  c->stream = c->own;
  const int rs = static_scratch_addr(device, &c->static_scratch);
  if (rs != QR_OK) {
    (void)hipEventDestroy(c->ev0);
    (void)hipEventDestroy(c->ev1);
    (void)hipStreamDestroy(c->own);
    delete c;
    return rs;
  }
  *out = c;
  return QR_OK;
}

int qr_ctx_destroy(qr_ctx* c) {
  if (!c) return QR_OK;
  set_device(c);
  (void)hipStreamSynchronize(c->stream);
  for (auto& kv : c->registry) (void)hipFree(kv.second.dev);
  if (c->work) (void)hipFree(c->work);
  for (void* p : c->retired) (void)hipFree(p);
  if (c->ev0) (void)hipEventDestroy(c->ev0);
  if (c->ev1) (void)hipEventDestroy(c->ev1);
  if (c->own) (void)hipStreamDestroy(c->own);
  delete c;
  return QR_OK;
}

int qr_ctx_set_moe_path(qr_ctx* c, int path) {
  if (!c) return fail(QR_ERR_INVALID, "qr_ctx_set_moe_path: null ctx");
  if (path < QR_MOE_PATH_AUTO || path > QR_MOE_PATH_MFMA)
    return fail(QR_ERR_INVALID, "qr_ctx_set_moe_path: path %d", path);
  c->moe_path = path;
  return QR_OK;
}

int qr_ctx_set_stream(qr_ctx* c, void* s) {
  if (!c) return fail(QR_ERR_INVALID, "qr_ctx_set_stream: null ctx");
  c->stream = s ? static_cast<hipStream_t>(s) : c->own;
  return QR_OK;
}

void* qr_ctx_get_stream(qr_ctx* c) { return c ? (void*)c->stream : nullptr; }

int qr_sync(qr_ctx* c) {
  if (!c) return fail(QR_ERR_INVALID, "qr_sync: null ctx");
  QR_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return QR_OK;
}

int qr_malloc(qr_ctx* c, size_t bytes, void** p) {
  if (!c || !p) return fail(QR_ERR_INVALID, "qr_malloc: null argument");
  *p = nullptr;
  QR_NO_CAPTURE(c, "qr_malloc");
  if (set_device(c) != QR_OK) return QR_ERR_HIP;
  hipError_t e = hipMalloc(p, bytes ? bytes : 16);
  if (e != hipSuccess) return fail(QR_ERR_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  return QR_OK;
}

int qr_free(qr_ctx* c, void* p) {
  if (!c) return fail(QR_ERR_INVALID, "qr_free: null ctx");
  if (!p) return QR_OK;
  QR_NO_CAPTURE(c, "qr_free");
  QR_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  QR_HIP(hipFree(p), "hipFree");
  return QR_OK;
}

int qr_memcpy_h2d(qr_ctx* c, void* dst, const void* src, size_t n) {
  if (!c || (n && (!dst || !src))) return fail(QR_ERR_INVALID, "qr_memcpy_h2d: null argument");
  if (!n) return QR_OK;
  QR_NO_CAPTURE(c, "qr_memcpy_h2d");
  QR_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync H2D");
  QR_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return QR_OK;
}

int qr_memcpy_d2h(qr_ctx* c, void* dst, const void* src, size_t n) {
  if (!c || (n && (!dst || !src))) return fail(QR_ERR_INVALID, "qr_memcpy_d2h: null argument");
  if (!n) return QR_OK;
  QR_NO_CAPTURE(c, "qr_memcpy_d2h");
  QR_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync D2H");
  QR_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return QR_OK;
}

int qr_memcpy_d2d(qr_ctx* c, void* dst, const void* src, size_t n) {
  if (!c || (n && (!dst || !src))) return fail(QR_ERR_INVALID, "qr_memcpy_d2d: null argument");
  if (!n) return QR_OK;
  QR_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, c->stream), "hipMemcpyAsync D2D");
  return QR_OK;
}

int qr_memset(qr_ctx* c, void* dst, int v, size_t n) {
  if (!c || (n && !dst)) return fail(QR_ERR_INVALID, "qr_memset: null argument");
  if (!n) return QR_OK;
  if (capturing(c)) {  // a fill kernel: no memset node in the graph
    size_t grid = (n + 255) / 256;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(k_fill_u8, dim3((unsigned)grid), dim3(256), 0, c->stream,
                       static_cast<uint8_t*>(dst), (uint8_t)v, n);
    QR_HIP(hipGetLastError(), "k_fill_u8");
    return QR_OK;
  }
  QR_HIP(hipMemsetAsync(dst, v, n, c->stream), "hipMemsetAsync");
  return QR_OK;
}

int qr_timer_start(qr_ctx* c) {
  if (!c) return fail(QR_ERR_INVALID, "qr_timer_start: null ctx");
  QR_HIP(hipEventRecord(c->ev0, c->stream), "hipEventRecord");
  return QR_OK;
}

int qr_timer_stop(qr_ctx* c, float* ms) {
  if (!c || !ms) return fail(QR_ERR_INVALID, "qr_timer_stop: null argument");
  QR_NO_CAPTURE(c, "qr_timer_stop");
  QR_HIP(hipEventRecord(c->ev1, c->stream), "hipEventRecord");
  QR_HIP(hipEventSynchronize(c->ev1), "hipEventSynchronize");
  QR_HIP(hipEventElapsedTime(ms, c->ev0, c->ev1), "hipEventElapsedTime");
  return QR_OK;
}

int qr_capture_begin(qr_ctx* c) {
  if (!c) return fail(QR_ERR_INVALID, "qr_capture_begin: null ctx");
  QR_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  return QR_OK;
}

int qr_capture_end(qr_ctx* c, void** graph) {
  if (!c || !graph) return fail(QR_ERR_INVALID, "qr_capture_end: null argument");
  *graph = nullptr;
  hipGraph_t g = nullptr;
  QR_HIP(hipStreamEndCapture(c->stream, &g), "hipStreamEndCapture");
  hipGraphExec_t ex = nullptr;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
  *graph = ex;
  return QR_OK;
}

int qr_graph_launch(qr_ctx* c, void* graph) {
  if (!c || !graph) return fail(QR_ERR_INVALID, "qr_graph_launch: null argument");
  QR_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), c->stream), "hipGraphLaunch");
  return QR_OK;
}

int qr_graph_destroy(void* graph) {
  if (!graph) return QR_OK;
  QR_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)), "hipGraphExecDestroy");
  return QR_OK;
}

int qr_copy_kernel(qr_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || !dst || !src) return fail(QR_ERR_INVALID, "qr_copy_kernel: null argument");
  if (!aligned(dst, 16) || !aligned(src, 16) || (bytes & 15))
    return fail(QR_ERR_INVALID, "qr_copy_kernel: needs 16-byte aligned pointers and size");
  const size_t n16 = bytes / 16;
  if (!n16) return QR_OK;
  size_t grid = (n16 + 255) / 256;
  if (grid > 8192) grid = 8192;
  hipLaunchKernelGGL(k_copy16, dim3((unsigned)grid), dim3(256), 0, c->stream,
                     static_cast<uint4*>(dst), static_cast<const uint4*>(src), n16);
  QR_HIP(hipGetLastError(), "k_copy16");
  return QR_OK;
}

int qr_read_kernel(qr_ctx* c, const void* src, size_t bytes, void* sink) {
  if (!c || !src || !sink) return fail(QR_ERR_INVALID, "qr_read_kernel: null argument");
  if (!aligned(src, 16) || (bytes & 15) || !aligned(sink, 4))
    return fail(QR_ERR_INVALID, "qr_read_kernel: needs 16-byte aligned src and size");
  const size_t n16 = bytes / 16;
  if (!n16) return QR_OK;
  const size_t grid = (n16 + 255) / 256;
  if (grid > 0x7FFFFFFFu) return fail(QR_ERR_INVALID, "qr_read_kernel: too large");
  hipLaunchKernelGGL(k_read16, dim3((unsigned)grid), dim3(256), 0, c->stream,
                     static_cast<const uint4*>(src), n16, 0x9E3779B9u, static_cast<uint32_t*>(sink));
  QR_HIP(hipGetLastError(), "k_read16");
  return QR_OK;
}

size_t qr_row_bytes(uint32_t type, int d) {
  // the tiled layout keeps the row size; ggml's K-quant blocks have the
  // reference's sizes (144 / 176 / 210 bytes)
  type &= ~(uint32_t)(QR_TILED | QR_GGML);
  if (d < 0 || !known_type(type)) return 0;
  return qr_wrow_bytes((int)type, d);
}

static int tile_args(uint32_t type, const void* src, void* dst, int n, int d, const char* who) {
  if (type != QR_T_Q4_K && type != QR_T_Q5_K && type != QR_T_Q6_K && type != QR_T_Q8_0)
    return fail(QR_ERR_UNSUPPORTED, "%s: type %u has no tiled layout (Q4_K, Q5_K, Q6_K, Q8_0)", who,
                type);
  if (n < 0 || d <= 0 || (d & 255) || (d >> 8) > 64)
    return fail(QR_ERR_UNSUPPORTED, "%s: shape %d x %d (d a multiple of 256, at most 16384)", who,
                n, d);
  if (type == QR_T_Q6_K && ((long)n * (d >> 8)) % 8)
    return fail(QR_ERR_UNSUPPORTED,
                "%s: tiled Q6_K needs n * (d / 256) a multiple of 8 (%d x %d)", who, n, d);
  if (n > 0 && (!src || !dst)) return fail(QR_ERR_INVALID, "%s: null pointer", who);
  if (!aligned(src, 16) || !aligned(dst, 16))
    return fail(QR_ERR_INVALID, "%s: src and dst must be 16-byte aligned", who);
  const size_t bytes = qr_wrow_bytes((int)type, d) * (size_t)n;
  const uintptr_t a = reinterpret_cast<uintptr_t>(src), b = reinterpret_cast<uintptr_t>(dst);
  if (n > 0 && a < b + bytes && b < a + bytes)
    return fail(QR_ERR_INVALID, "%s: src and dst overlap", who);
  return QR_OK;
}

int qr_weights_tile(qr_ctx* c, uint32_t type, const void* src, void* dst, int n, int d) {
  if (!c) return fail(QR_ERR_INVALID, "qr_weights_tile: null ctx");
  int rc = tile_args(type, src, dst, n, d, "qr_weights_tile");
  if (rc) return rc;
  QR_HIP(qr::tile_pack_launch((int)type, src, dst, n, d, false, c->stream), "k_tile_pack");
  return QR_OK;
}

int qr_weights_untile(qr_ctx* c, uint32_t type, const void* src, void* dst, int n, int d) {
  if (!c) return fail(QR_ERR_INVALID, "qr_weights_untile: null ctx");
  int rc = tile_args(type, src, dst, n, d, "qr_weights_untile");
  if (rc) return rc;
  QR_HIP(qr::tile_pack_launch((int)type, src, dst, n, d, true, c->stream), "k_tile_pack");
  return QR_OK;
}

int qr_quantize_q8_k(qr_ctx* c, const float* x, void* y, long n) {
  if (!c) return fail(QR_ERR_INVALID, "qr_quantize_q8_k: null ctx");
  if (n < 0) return fail(QR_ERR_INVALID, "qr_quantize_q8_k: negative size");
  const long nb = n / 256;
  if (nb == 0) return QR_OK;
  if (!x || !y) return fail(QR_ERR_INVALID, "qr_quantize_q8_k: null pointer");
  QR_HIP(qr::quantize_q8k_launch(x, y, nb, c->stream), "k_quantize_q8k");
  return QR_OK;
}

int qr_quantize_q8_0(qr_ctx* c, const float* x, void* y, long n) {
  if (!c) return fail(QR_ERR_INVALID, "qr_quantize_q8_0: null ctx");
  if (n < 0) return fail(QR_ERR_INVALID, "qr_quantize_q8_0: negative size");
  const long nb = n / 32;
  if (nb == 0) return QR_OK;
  if (!x || !y) return fail(QR_ERR_INVALID, "qr_quantize_q8_0: null pointer");
  QR_HIP(qr::quantize_q8_0_launch(x, y, nb, c->stream), "k_quantize_q8_0");
  return QR_OK;
}

int qr_gemv_ord(qr_ctx* c, int order, uint32_t type, const void* w, const float* x, int xstride,
                float* y, int ystride, int n, int d, int nt, int32_t* acc, int32_t* accb) {
  if (!c) return fail(QR_ERR_INVALID, "qr_gemv: null ctx");
  if (order < QR_ORDER_SEQ || order > QR_ORDER_AVX512)
    return fail(QR_ERR_INVALID, "qr_gemv: order %d", order);
  const bool tiled = (type & QR_TILED) != 0;
  const bool ggml = (type & QR_GGML) != 0;
  type &= ~(uint32_t)(QR_TILED | QR_GGML);
  if (!known_type(type)) return fail(QR_ERR_INVALID, "qr_gemv: unknown type %u", type);
  if (ggml && (tiled || (type != QR_T_Q4_K && type != QR_T_Q5_K && type != QR_T_Q6_K)))
    return fail(QR_ERR_UNSUPPORTED, "qr_gemv: ggml type %u (Q4_K, Q5_K, Q6_K; not tiled)", type);
  if (n < 0 || d < 0) return fail(QR_ERR_INVALID, "qr_gemv: negative size");
  if (!(nt == 1 || nt == 2 || nt == 3 || nt == 4 || nt == 8))
    return fail(QR_ERR_UNSUPPORTED, "qr_gemv: nt=%d (supported 1,2,3,4,8)", nt);
  if (n == 0) return QR_OK;
  if (!x || !y) return fail(QR_ERR_INVALID, "qr_gemv: null x or y");
  if (xstride < d || ystride < n) return fail(QR_ERR_INVALID, "qr_gemv: stride below size");
  if (!w) {  // src/quant.c:443-446: no weights -> zero output
    const long total = (long)n * nt;
    long grid = (total + 255) / 256;
    if (grid > 1024) grid = 1024;
    hipLaunchKernelGGL(k_zero_rows, dim3((unsigned)grid), dim3(256), 0, c->stream, y, n, nt,
                       ystride);
    QR_HIP(hipGetLastError(), "k_zero_rows");
    return QR_OK;
  }
  if (tiled && type != QR_T_Q4_K && type != QR_T_Q5_K && type != QR_T_Q6_K && type != QR_T_Q8_0)
    return fail(QR_ERR_UNSUPPORTED, "qr_gemv: type %u has no tiled layout", type);
  if (type == QR_T_F32) {
    if (acc || accb) return fail(QR_ERR_INVALID, "qr_gemv: F32 has no integer sums");
    QR_HIP(qr::gemv_f32_launch(QR_ORDER_SEQ, static_cast<const float*>(w), x, y, n, d, nt,
                               xstride, ystride, c->stream), "k_gemv_f32");
    return QR_OK;
  }
  if (!aligned(w, 16)) return fail(QR_ERR_INVALID, "qr_gemv: weights must be 16-byte aligned");
  if (!aligned(x, 16) || (nt > 1 && (xstride & 3)))
    return fail(QR_ERR_INVALID, "qr_gemv: x must be 16-byte aligned (and xstride a multiple of 4)");
  if (ggml) {
    if (acc || accb) return fail(QR_ERR_UNSUPPORTED, "qr_gemv: no integer sums on ggml weights");
    if (!qr::gemv_ggml_ok((int)type, d, nt))
      return fail(QR_ERR_UNSUPPORTED, "qr_gemv: ggml type %u at d=%d nt=%d", type, d, nt);
    QR_HIP(qr::gemv_ggml_launch((int)type, w, x, y, n, d, nt, xstride, ystride, c->stream),
           "k_gemv_ggml");
    return QR_OK;
  }
  if (tiled) {
    if (acc || accb) return fail(QR_ERR_UNSUPPORTED, "qr_gemv: no integer sums on tiled weights");
    if (!qr::gemv_tiled_ok((int)type, n, d, nt, order))
      return fail(QR_ERR_UNSUPPORTED, "qr_gemv: tiled type %u at d=%d nt=%d order %d", type, d, nt,
                  order);
    QR_HIP(qr::gemv_tiled_launch((int)type, w, x, y, n, d, nt, xstride, ystride, c->stream, order),
           "k_gemv_tiled");
    return QR_OK;
  }
  const int R = qr::gemv_rows_per_wg((int)type, order, n, d, nt);
  if (!qr::gemv_blk_ok((int)type, d, nt) && !qr::gemv_stream_ok((int)type, order, d, nt) &&
      qr::gemv_lds_bytes((int)type, order, d, nt, R) > 64 * 1024)
    return fail(QR_ERR_UNSUPPORTED, "qr_gemv: d=%d nt=%d exceeds the LDS budget", d, nt);
  QR_HIP(qr::gemv_launch((int)type, order, w, x, y, n, d, nt, xstride, ystride, acc, accb,
                         c->stream),
         "k_gemv");
  return QR_OK;
}

int qr_gemv_ex(qr_ctx* c, uint32_t type, const void* w, const float* x, int xstride, float* y,
               int ystride, int n, int d, int nt, int32_t* acc, int32_t* accb) {
  return qr_gemv_ord(c, QR_ORDER_SEQ, type, w, x, xstride, y, ystride, n, d, nt, acc, accb);
}

int qr_gemv(qr_ctx* c, uint32_t type, const void* w, const float* x, float* y, int n, int d,
            int nt) {
  return qr_gemv_ex(c, type, w, x, d, y, n, n, d, nt, nullptr, nullptr);
}

int qr_gemv_rows(qr_ctx* c, int order, uint32_t type, const void* w, const float* x, int xstride,
                 float* y, int ystride, int n, int d, int T) {
  if (!c) return fail(QR_ERR_INVALID, "qr_gemv_rows: null ctx");
  if (order < QR_ORDER_SEQ || order > QR_ORDER_AVX512)
    return fail(QR_ERR_INVALID, "qr_gemv_rows: order %d", order);
  const bool tiled = (type & QR_TILED) != 0;
  const uint32_t base = type & ~(uint32_t)QR_TILED;
  if (n < 0 || d <= 0 || T < 0) return fail(QR_ERR_INVALID, "qr_gemv_rows: bad size");
  if (n == 0 || T == 0) return QR_OK;
  if (!w || !x || !y) return fail(QR_ERR_INVALID, "qr_gemv_rows: null pointer");
  if (xstride < d || ystride < n || (xstride & 3))
    return fail(QR_ERR_INVALID, "qr_gemv_rows: strides (xstride >= d, a multiple of 4; ystride >= n)");
  if ((type & QR_GGML) || !qr::mfma_type_ok((int)base) || d % 256 || (d >> 8) > 64 ||
      (tiled && base != QR_T_Q4_K && base != QR_T_Q5_K))
    return fail(QR_ERR_UNSUPPORTED,
                "qr_gemv_rows: type %u at d=%d (Q4_K / Q5_K row-major or tiled, Q6_K, Q8_0; d a "
                "multiple of 256, at most 16384)", type, d);
  if (base == QR_T_Q8_0 && order != QR_ORDER_SEQ)
    return fail(QR_ERR_UNSUPPORTED, "qr_gemv_rows: Q8_0 in a lane order (use qr_gemv_ord)");
  if (!aligned(w, 16) || !aligned(x, 16))
    return fail(QR_ERR_INVALID, "qr_gemv_rows: w and x must be 16-byte aligned");
  const size_t slice = qr_wrow_bytes((int)base, d) * (size_t)n;
  if (slice >= ((size_t)1 << 32)) return fail(QR_ERR_UNSUPPORTED, "qr_gemv_rows: matrix of 4 GiB or more");
  // scratch: the rows' activation records, then the single-"expert" dispatch
  const size_t rec = (((size_t)T * (d / 32) * qr::kXQ) + 255) & ~(size_t)255;
  void* base_p = nullptr;
  int rc = ctx_scratch(c, rec + 16 + 4 * (size_t)T + 16, "qr_gemv_rows", &base_p);
  if (rc) return rc;
  uint8_t* recp = static_cast<uint8_t*>(base_p);
  int32_t* off = reinterpret_cast<int32_t*>(recp + rec);
  int32_t* tiles = off + 4;
  int32_t* perm = tiles + 4;
  const int tile = 16;
  QR_HIP(qr::rows_dispatch_launch(T, tile, off, perm, tiles, c->stream), "k_rows_dispatch");
  QR_HIP(qr::quant_rows_launch(x, xstride, T, d, base != QR_T_Q8_0, recp, c->stream),
         "k_quant_rows");
  QR_HIP(qr::expert_mfma_launch((int)base, false, static_cast<const uint8_t*>(w), nullptr, slice,
                                1, 1, n, d, recp, 1, off, perm, tiles, y, ystride,
                                (T + tile - 1) / tile + 1, tile, nullptr, false, c->stream, tiled),
         "k_expert_mfma");
  return QR_OK;
}

int qr_matmul_f32(qr_ctx* c, int order, const float* w, const float* x, float* y, int n, int d,
                  int nt) {
  if (!c) return fail(QR_ERR_INVALID, "qr_matmul_f32: null ctx");
  if (order < QR_ORDER_SEQ || order > QR_ORDER_AVX512)
    return fail(QR_ERR_INVALID, "qr_matmul_f32: order %d", order);
  if (n < 0 || d < 0 || nt < 1) return fail(QR_ERR_INVALID, "qr_matmul_f32: bad size");
  if (n == 0) return QR_OK;
  if (!w || !x || !y) return fail(QR_ERR_INVALID, "qr_matmul_f32: null pointer");
  QR_HIP(qr::gemv_f32_launch(order, w, x, y, n, d, nt, d, n, c->stream), "k_gemv_f32");
  return QR_OK;
}

int qr_softmax(qr_ctx* c, float* x, int rows, int n) {
  if (!c) return fail(QR_ERR_INVALID, "qr_softmax: null ctx");
  if (rows < 0 || n < 0) return fail(QR_ERR_INVALID, "qr_softmax: bad size");
  if (rows == 0 || n == 0) return QR_OK;
  if (!x) return fail(QR_ERR_INVALID, "qr_softmax: null pointer");
  QR_HIP(qr::softmax_launch(x, rows, n, c->stream), "k_softmax");
  return QR_OK;
}

int qr_test_expf(qr_ctx* c, const float* x, float* y, long n) {
  if (!c || (n > 0 && (!x || !y))) return fail(QR_ERR_INVALID, "qr_test_expf: null argument");
  if (n <= 0) return QR_OK;
  const long grid = (n + 255) / 256;
  hipLaunchKernelGGL(k_test_expf, dim3((unsigned)grid), dim3(256), 0, c->stream, x, y, n);
  QR_HIP(hipGetLastError(), "k_test_expf");
  return QR_OK;
}

// ---- MoE --------------------------------------------------------------------
static int check_layer(const qr_moe_layer* L, const char* who) {
  if (!L) return fail(QR_ERR_INVALID, "%s: null layer", who);
  if (L->dim <= 0 || L->n_experts <= 0 || L->n_used <= 0 || L->hidden <= 0)
    return fail(QR_ERR_INVALID, "%s: bad layer sizes", who);
  // src/runtime.c:204 and 208 hold the logits and the choice on the stack.
  if (L->n_experts > 256 || L->n_used > 16 || L->n_used > L->n_experts)
    return fail(QR_ERR_INVALID, "%s: E=%d K=%d (E <= 256, K <= 16, K <= E)", who, L->n_experts,
                L->n_used);
  if (!L->router) return fail(QR_ERR_INVALID, "%s: null router", who);
  if (L->dim % 32) return fail(QR_ERR_INVALID, "%s: dim must be a multiple of 32", who);
  return QR_OK;
}

static int check_experts(const qr_moe_layer* L, const char* who) {
  const uint32_t ts[3] = {L->up_type, L->gate_type, L->down_type};
  const void* ps[3] = {L->up, L->gate, L->down};
  const int ng = ((ts[0] & QR_GGML) != 0) + ((ts[1] & QR_GGML) != 0) + ((ts[2] & QR_GGML) != 0);
  if (ng) {  // llama.cpp-layout experts: all three, on ggml's Q8_K dot
    if (ng != 3 || L->up_type != L->gate_type)
      return fail(QR_ERR_UNSUPPORTED, "%s: ggml experts need ggml up, gate and down (up = gate)",
                  who);
    if (!qr::gemv_ggml_ok((int)(L->up_type & ~(uint32_t)QR_GGML), L->dim, 1) ||
        !qr::gemv_ggml_ok((int)(L->down_type & ~(uint32_t)QR_GGML), L->hidden, 1))
      return fail(QR_ERR_UNSUPPORTED, "%s: ggml expert types %u / %u at dim %d, hidden %d", who,
                  L->up_type, L->down_type, L->dim, L->hidden);
    for (int i = 0; i < 3; i++) {
      if (!ps[i]) return fail(QR_ERR_INVALID, "%s: null expert tensor", who);
      if (!aligned(ps[i], 16))
        return fail(QR_ERR_INVALID, "%s: expert tensors must be 16-byte aligned", who);
    }
    const size_t su = qr_row_bytes(L->up_type, L->dim) * (size_t)L->hidden;
    const size_t sd = qr_row_bytes(L->down_type, L->hidden) * (size_t)L->dim;
    if ((su & 15) || (sd & 15))
      return fail(QR_ERR_UNSUPPORTED, "%s: expert slice not 16-byte aligned", who);
    if (L->sh_hidden > 0)
      return fail(QR_ERR_UNSUPPORTED, "%s: no shared expert beside ggml experts", who);
    return QR_OK;
  }
  for (int i = 0; i < 3; i++) {
    if (ts[i] == QR_T_F32 || !known_type(ts[i]))
      return fail(QR_ERR_UNSUPPORTED, "%s: expert type %u (quantized types only)", who, ts[i]);
    if (!ps[i]) return fail(QR_ERR_INVALID, "%s: null expert tensor", who);
    if (!aligned(ps[i], 16)) return fail(QR_ERR_INVALID, "%s: expert tensors must be 16-byte aligned", who);
  }
  if (L->up_type != L->gate_type)
    return fail(QR_ERR_UNSUPPORTED, "%s: up and gate must share a type", who);
  if (L->hidden % 32) return fail(QR_ERR_INVALID, "%s: hidden must be a multiple of 32", who);
  // expert slices must stay 16-byte aligned
  const size_t su = qr_row_bytes(L->up_type, L->dim) * (size_t)L->hidden;
  const size_t sd = qr_row_bytes(L->down_type, L->hidden) * (size_t)L->dim;
  if ((su & 15) || (sd & 15)) return fail(QR_ERR_UNSUPPORTED, "%s: expert slice not 16-byte aligned", who);
  if (L->sh_hidden > 0) {
    if (!L->sh_gate_inp || !L->sh_up || !L->sh_gate || !L->sh_down)
      return fail(QR_ERR_INVALID, "%s: null shared-expert tensor", who);
    if (L->sh_up_type != L->sh_gate_type || L->sh_up_type == QR_T_F32 ||
        L->sh_down_type == QR_T_F32 || !known_type(L->sh_up_type) || !known_type(L->sh_down_type))
      return fail(QR_ERR_UNSUPPORTED, "%s: shared expert types", who);
    if (L->sh_hidden % 32) return fail(QR_ERR_INVALID, "%s: sh_hidden must be a multiple of 32", who);
    if (!aligned(L->sh_up, 16) || !aligned(L->sh_gate, 16) || !aligned(L->sh_down, 16))
      return fail(QR_ERR_INVALID, "%s: shared tensors must be 16-byte aligned", who);
  }
  return QR_OK;
}

}  // extern "C"

namespace qr {
int moe_check(const qr_moe_layer* L, const char* who) {
  const int rc = check_layer(L, who);
  return rc ? rc : check_experts(L, who);
}

int gemv_check(uint32_t type, int order, const void* w, int n, int d, const char* who) {
  if (type & QR_GGML) {
    type &= ~(uint32_t)QR_GGML;
    if (n <= 0 || d <= 0) return fail(QR_ERR_INVALID, "%s: weight shape %d x %d", who, n, d);
    if (!gemv_ggml_ok((int)type, d, 1))
      return fail(QR_ERR_UNSUPPORTED, "%s: ggml type %u at d=%d (Q4_K, Q5_K, Q6_K; not tiled)",
                  who, type, d);
    if (w && !aligned(w, 16)) return fail(QR_ERR_INVALID, "%s: weights must be 16-byte aligned", who);
    return QR_OK;
  }
  if (type & QR_TILED) {
    type &= ~(uint32_t)QR_TILED;
    if (n <= 0 || d <= 0) return fail(QR_ERR_INVALID, "%s: weight shape %d x %d", who, n, d);
    if (!gemv_tiled_ok((int)type, n, d, 1, order))
      return fail(QR_ERR_UNSUPPORTED, "%s: tiled type %u at %d x %d (order %d)", who, type, n, d,
                  order);
    if (w && !aligned(w, 16)) return fail(QR_ERR_INVALID, "%s: weights must be 16-byte aligned", who);
    return QR_OK;
  }
  if (!known_type(type)) return fail(QR_ERR_INVALID, "%s: unknown weight type %u", who, type);
  if (n <= 0 || d <= 0) return fail(QR_ERR_INVALID, "%s: weight shape %d x %d", who, n, d);
  if (type == QR_T_F32) return QR_OK;
  if (d % qr_block_elems((int)type))
    return fail(QR_ERR_INVALID, "%s: d=%d is not whole blocks of type %u", who, d, type);
  if (w && !aligned(w, 16)) return fail(QR_ERR_INVALID, "%s: weights must be 16-byte aligned", who);
  const int R = gemv_rows_per_wg((int)type, order, n, d, 1);
  if (!gemv_blk_ok((int)type, d, 1) && !gemv_stream_ok((int)type, order, d, 1) &&
      gemv_lds_bytes((int)type, order, d, 1, R) > 64 * 1024)
    return fail(QR_ERR_UNSUPPORTED, "%s: d=%d exceeds the GEMV's LDS budget", who, d);
  return QR_OK;
}
}  // namespace qr

extern "C" {

int qr_moe_route(qr_ctx* c, const qr_moe_layer* L, const float* xb, int T, int order,
                 float* probs, int32_t* idx, float* wts) {
  if (!c) return fail(QR_ERR_INVALID, "qr_moe_route: null ctx");
  int rc = check_layer(L, "qr_moe_route");
  if (rc) return rc;
  if (order < QR_ORDER_SEQ || order > QR_ORDER_AVX512)
    return fail(QR_ERR_INVALID, "qr_moe_route: order %d", order);
  if (T < 0) return fail(QR_ERR_INVALID, "qr_moe_route: T < 0");
  if (T == 0) return QR_OK;
  if (!xb || !idx || !wts) return fail(QR_ERR_INVALID, "qr_moe_route: null pointer");
  void* logits = nullptr;
  rc = ctx_scratch(c, (size_t)T * L->n_experts * 4, "qr_moe_route", &logits);
  if (rc) return rc;
  QR_HIP(qr::moe_route_launch(L, xb, T, order, static_cast<float*>(logits), probs, idx, wts,
                              c->stream),
         "moe_route");
  return QR_OK;
}

int qr_moe_dispatch(qr_ctx* c, const int32_t* idx, int T, int K, int E, int32_t* counts,
                    int32_t* offsets, int32_t* perm, int32_t* inv) {
  if (!c) return fail(QR_ERR_INVALID, "qr_moe_dispatch: null ctx");
  if (T < 0 || K <= 0 || E <= 0 || E > 256 || K > 16)
    return fail(QR_ERR_INVALID, "qr_moe_dispatch: T=%d K=%d E=%d (E <= 256, K <= 16)", T, K, E);
  if (!counts || !offsets || (T > 0 && (!idx || !perm || !inv)))
    return fail(QR_ERR_INVALID, "qr_moe_dispatch: null pointer");
  QR_HIP(qr::moe_dispatch_launch(idx, T, K, E, 1, counts, offsets, nullptr, perm, inv, c->stream),
         "moe_dispatch");
  return QR_OK;
}

int qr_moe_forward(qr_ctx* c, const qr_moe_layer* L, float* x, const float* xb, int T, int order,
                   int32_t* idx_out, float* w_out) {
  if (!c) return fail(QR_ERR_INVALID, "qr_moe_forward: null ctx");
  int rc = check_layer(L, "qr_moe_forward");
  if (rc) return rc;
  rc = check_experts(L, "qr_moe_forward");
  if (rc) return rc;
  if (order < QR_ORDER_SEQ || order > QR_ORDER_AVX512)
    return fail(QR_ERR_INVALID, "qr_moe_forward: order %d", order);
  if (T < 0) return fail(QR_ERR_INVALID, "qr_moe_forward: T < 0");
  if (T == 0) return QR_OK;
  if (!x || !xb) return fail(QR_ERR_INVALID, "qr_moe_forward: null x / xb");
  if (!aligned(xb, 16) || !aligned(x, 16)) return fail(QR_ERR_INVALID, "qr_moe_forward: x/xb alignment");
  void* base = nullptr;
  rc = ctx_scratch(c, qr::moe_scratch_bytes(L, T), "qr_moe_forward", &base);
  if (rc) return rc;
  qr::MoeScratch s;
  qr::moe_scratch_carve(base, L, T, &s);
  QR_HIP(qr::moe_forward_launch(L, x, xb, T, order, s, c->stream, c->moe_path), "moe_forward");
  const size_t kb = (size_t)T * L->n_used;
  if (idx_out) QR_HIP(hipMemcpyAsync(idx_out, s.idx, kb * 4, hipMemcpyDeviceToDevice, c->stream), "copy idx");
  if (w_out) QR_HIP(hipMemcpyAsync(w_out, s.wts, kb * 4, hipMemcpyDeviceToDevice, c->stream), "copy wts");
  return QR_OK;
}

int qr_moe_forward_noalloc(qr_ctx* c, const qr_moe_layer* L, float* x, const float* xb, int T,
                           int order, int32_t* idx_out, float* w_out) {
  if (!c) return fail(QR_ERR_INVALID, "qr_moe_forward_noalloc: null ctx");
  int rc = check_layer(L, "qr_moe_forward_noalloc");
  if (rc) return rc;
  rc = check_experts(L, "qr_moe_forward_noalloc");
  if (rc) return rc;
  if (order < QR_ORDER_SEQ || order > QR_ORDER_AVX512)
    return fail(QR_ERR_INVALID, "qr_moe_forward_noalloc: order %d", order);
  if (T < 0) return fail(QR_ERR_INVALID, "qr_moe_forward_noalloc: T < 0");
  if (T == 0) return QR_OK;
  if (!x || !xb) return fail(QR_ERR_INVALID, "qr_moe_forward_noalloc: null x / xb");
  if (!aligned(xb, 16) || !aligned(x, 16))
    return fail(QR_ERR_INVALID, "qr_moe_forward_noalloc: x/xb alignment");
  const size_t need = qr::moe_scratch_bytes(L, T);
  if (need > (size_t)QR_NOALLOC_SCRATCH_BYTES)
    return fail(QR_ERR_INVALID,
                "qr_moe_forward_noalloc: T=%d on this layer needs %zu bytes of scratch, above "
                "the fixed %d (use qr_moe_forward, or fewer tokens per call)",
                T, need, (int)QR_NOALLOC_SCRATCH_BYTES);
  if (!c->static_scratch) return fail(QR_ERR_HIP, "qr_moe_forward_noalloc: no scratch address");
  qr::MoeScratch s;
  qr::moe_scratch_carve(c->static_scratch, L, T, &s);
  QR_HIP(qr::moe_forward_launch(L, x, xb, T, order, s, c->stream, c->moe_path), "moe_forward");
  const size_t kb = (size_t)T * L->n_used;
  if (idx_out) QR_HIP(hipMemcpyAsync(idx_out, s.idx, kb * 4, hipMemcpyDeviceToDevice, c->stream), "copy idx");
  if (w_out) QR_HIP(hipMemcpyAsync(w_out, s.wts, kb * 4, hipMemcpyDeviceToDevice, c->stream), "copy wts");
  return QR_OK;
}

// ---- registry -----------------------------------------------------------------
int qr_weights_upload(qr_ctx* c, const void* host, size_t bytes, const void** dev) {
  if (!c || !host || !dev) return fail(QR_ERR_INVALID, "qr_weights_upload: null argument");
  QR_NO_CAPTURE(c, "qr_weights_upload");
  std::lock_guard<std::mutex> lk(c->mu);
  auto it = c->registry.find(host);
  if (it != c->registry.end()) {
    const RegEntry& r = it->second;
    if (!r.gathered && r.bytes == bytes &&
        r.digest == range_digest(0xCBF29CE484222325ull, host, bytes)) {
      *dev = it->second.dev;
      return QR_OK;
    }
    (void)hipStreamSynchronize(c->stream);  // work still reading the old copy
    (void)hipFree(it->second.dev);
    c->registry.erase(it);
  }
  if (set_device(c) != QR_OK) return QR_ERR_HIP;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
  if (e != hipSuccess) return fail(QR_ERR_NOMEM, "qr_weights_upload: hipMalloc(%zu)", bytes);
  e = hipMemcpyAsync(p, host, bytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(e, "qr_weights_upload: copy");
  }
  RegEntry r;
  r.dev = p;
  r.bytes = bytes;
  r.digest = range_digest(0xCBF29CE484222325ull, host, bytes);
  c->registry[host] = r;
  *dev = p;
  return QR_OK;
}

int qr_weights_upload_parts(qr_ctx* c, const void* key, const void* const* parts,
                            size_t part_bytes, int nparts, const void** dev) {
  if (!c || !key || !parts || !dev || nparts <= 0)
    return fail(QR_ERR_INVALID, "qr_weights_upload_parts: bad argument");
  for (int i = 0; i < nparts; i++)
    if (!parts[i]) return fail(QR_ERR_INVALID, "qr_weights_upload_parts: null part %d", i);
  const size_t bytes = part_bytes * (size_t)nparts;
  QR_NO_CAPTURE(c, "qr_weights_upload_parts");
  std::lock_guard<std::mutex> lk(c->mu);
  auto it = c->registry.find(key);
  if (it != c->registry.end()) {
    const RegEntry& r = it->second;
    if (r.gathered && r.bytes == bytes && r.digest == parts_digest(parts, part_bytes, nparts)) {
      *dev = r.dev;
      return QR_OK;
    }
    (void)hipStreamSynchronize(c->stream);  // work still reading the old copy
    (void)hipFree(r.dev);
    c->registry.erase(it);
  }
  if (set_device(c) != QR_OK) return QR_ERR_HIP;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
  if (e != hipSuccess) return fail(QR_ERR_NOMEM, "qr_weights_upload_parts: hipMalloc(%zu)", bytes);
  for (int i = 0; i < nparts && e == hipSuccess; i++)
    e = hipMemcpyAsync(static_cast<uint8_t*>(p) + (size_t)i * part_bytes, parts[i], part_bytes,
                       hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(e, "qr_weights_upload_parts: copy");
  }
  RegEntry r;
  r.dev = p;
  r.bytes = bytes;
  r.digest = parts_digest(parts, part_bytes, nparts);
  r.gathered = true;
  c->registry[key] = r;
  *dev = p;
  return QR_OK;
}

int qr_weights_lookup(qr_ctx* c, const void* host, const void** dev) {
  if (!c || !host || !dev) return fail(QR_ERR_INVALID, "qr_weights_lookup: null argument");
  std::lock_guard<std::mutex> lk(c->mu);
  auto it = c->registry.find(host);
  if (it == c->registry.end()) {
    *dev = nullptr;
    return fail(QR_ERR_INVALID, "qr_weights_lookup: %p not registered", host);
  }
  *dev = it->second.dev;
  return QR_OK;
}

int qr_weights_release(qr_ctx* c, const void* host) {
  if (!c || !host) return fail(QR_ERR_INVALID, "qr_weights_release: null argument");
  std::lock_guard<std::mutex> lk(c->mu);
  auto it = c->registry.find(host);
  if (it == c->registry.end()) return QR_OK;
  (void)hipStreamSynchronize(c->stream);
  (void)hipFree(it->second.dev);
  c->registry.erase(it);
  return QR_OK;
}

int qr_weights_release_all(qr_ctx* c) {
  if (!c) return fail(QR_ERR_INVALID, "qr_weights_release_all: null ctx");
  std::lock_guard<std::mutex> lk(c->mu);
  (void)hipStreamSynchronize(c->stream);
  for (auto& kv : c->registry) (void)hipFree(kv.second.dev);
  c->registry.clear();
  return QR_OK;
}

}  // extern "C"
