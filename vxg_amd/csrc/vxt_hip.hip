// vxt_hip.hip -- C ABI, context, upload (device-residency re-layout) and
// dispatch for the compressed-weight matmul engine.  See include/vxt_hip.h.
//
// Reference boundary mirrored here: vxt_metal_create / upload / run_multi /
// free_buffer / destroy (crates/vxg-tensor/src/metal_ffi.rs:27-49,
// native/metal_gemv.mm:258-475) and the engine calls built on them
// (metal.rs:393-557).  Errors are reported as negative codes plus a message in
// the caller's buffer; nothing throws across the boundary.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <limits>
#include <memory>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <set>
#include <string>
#include <unordered_set>
#include <vector>

#include "../../include/vxt_hip.h"
#include "common.hpp"

namespace vxt {
hipError_t launch_gemv(const DevTensor& t, const void* x, bool x_bf16, bool x_vec, uint32_t m,
                       void* y, bool y_bf16, hipStream_t s);
size_t gemm_workspace_bytes(const DevTensor& t, uint32_t m, bool x_bf16, int mode);
hipError_t launch_gemm(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y, bool y_bf16, void* ws,
                       size_t ws_bytes, hipStream_t s, int mode);
hipError_t launch_dequant(const DevTensor& t, uint32_t row0, uint32_t nrows, float* out,
                          hipStream_t s);
hipError_t launch_gemv_norm(const DevTensor& t, const NormIn& nin, int epi, void* y, bool y_bf16, uint32_t y_stride,
                            hipStream_t s);
hipError_t launch_gemv_glu(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* act, bool act_bf16,
                           uint32_t act_stride, bool gelu, hipStream_t s);
hipError_t launch_glu_act(const float* gu, uint32_t m, uint32_t n_ff, bool gelu, void* act, bool act_bf16,
                          uint32_t act_stride, hipStream_t s);
hipError_t launch_rms_norm(float* cur, const float* delta, const float* w, void* out, bool out_bf16, uint32_t dim,
                           uint32_t stride, uint32_t m, float eps, hipStream_t s);
hipError_t launch_embed(const DevTensor& t, const uint32_t* tokens, uint32_t batch_m, float scale, bool scale_on,
                        float* out, uint32_t stride, hipStream_t s);
hipError_t launch_kv_append(const KvQ8Dev& c, const float* k, const float* v, uint32_t pos, hipStream_t s);
hipError_t launch_gqa_prep(const KvQ8Dev& c, GqaPrep a, uint32_t rope_dim, float freq_base, uint32_t batch,
                           hipStream_t s);
size_t attn_workspace_bytes(uint32_t n_head, uint32_t seq_len, uint32_t n_kv, uint32_t hd, uint32_t batch);
hipError_t launch_attn(const KvQ8Dev& c, const float* q, uint32_t n_head, uint32_t seq0, uint32_t batch,
                       const float* gate, float* out, void* ws, hipStream_t s);
hipError_t launch_attn_step(const KvQ8Dev& c, GqaPrep pp, uint32_t rope_dim, float freq_base, float* out, void* ws,
                            hipStream_t s);
size_t attn_prefill_workspace_bytes(uint32_t n_head, uint32_t hd, uint32_t pos0, uint32_t batch);
hipError_t launch_attn_prefill(const KvQ8Dev& c, const float* q, const float* gate, float* out, uint32_t n_head,
                               uint32_t pos0, uint32_t batch, void* ws, hipStream_t s);
size_t greedy_state_bytes();
hipError_t launch_greedy(const float* logits, uint32_t n, void* state, uint32_t* out, hipStream_t s);
hipError_t launch_read_probe(const void* p, size_t bytes, uint32_t* sink, uint32_t key, hipStream_t s);
void blas_acquire_device(int dev);
void blas_release_device(int dev);
}  // namespace vxt

// Scratch memory of the allocation-free matmul entry point
// (vxt_hip_matmul_noalloc_dev): one array per GPU, in the code object, so
// calls through that entry point never allocate.  Host code reaches it only
// through the device address hipGetSymbolAddress returns for the current
// device (kept per context); the name itself is a host-side stand-in.
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

using vxt::DevTensor;

struct Ctx;

struct Tensor {
  Ctx* ctx = nullptr;
  uint32_t kind = 0, rows = 0, cols = 0, kp = 0;
  void* arena = nullptr;
  size_t bytes = 0;
  size_t off_p0 = 0, off_p1 = 0, off_rp = 0, off_out = 0;
  uint32_t nnz = 0;
  uint32_t split0 = 0, split1 = 0;
  float cent[48] = {};
  uint32_t tail_nonfinite = 0;   // g64: see DevTensor::tail_nonfinite
  size_t off_rx = 0;             // cb4: row exponents of the decode-in-loop GEMM (0: not eligible)

  DevTensor dev() const {
    DevTensor d{};
    const char* base = static_cast<const char*>(arena);
    d.kind = kind;
    d.rows = rows;
    d.cols = cols;
    d.kp = kp;
    d.p0 = base + off_p0;
    d.p1 = reinterpret_cast<const uint16_t*>(base + off_p1);
    d.tail_nonfinite = tail_nonfinite;
    if (kind == VXT_KIND_CB4) {
      d.row_ptr = reinterpret_cast<const uint32_t*>(base + off_rp);
      d.outliers = reinterpret_cast<const uint32_t*>(base + off_out);
      d.split0 = split0;
      d.split1 = split1;
      std::memcpy(d.cent, cent, sizeof(cent));
      if (off_rx) d.rexp = reinterpret_cast<const int8_t*>(base + off_rx);
    }
    return d;
  }
};

struct Graph;
struct Runner;
void release_runner(Runner* r);   // with the context's lock held, or unneeded

struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double last_ms = 0.0;
  void* d_x = nullptr;
  size_t d_x_cap = 0;
  void* d_y = nullptr;
  size_t d_y_cap = 0;
  void* ws = nullptr;           // workspace: GEMM panel, partial sums, staging
  size_t ws_cap = 0;
  std::vector<void*> retired;   // replaced workspaces, kept until destroy
  void* greedy = nullptr;  // greedy-selection state words (zero between calls)
  void* scratch = nullptr; // device address of `scratch` on this context's device
  int gemm_mode = vxt::kGemmAuto;
  std::mutex mu;
  std::set<Tensor*> tensors;
  std::set<void*> buffers;
  std::set<Graph*> graphs;
  std::set<Runner*> runners;
  bool capturing = false;
};

struct Graph {
  Ctx* ctx = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

// Live handles (contexts, tensors, graphs).  A handle is checked here before
// use, so releasing a tensor or graph after its context was destroyed (which
// already released it), or releasing twice, is a no-op instead of a use
// after free.
std::mutex g_reg_mu;
std::unordered_set<const void*> g_live;

void reg_add(const void* p) {
  std::lock_guard<std::mutex> g(g_reg_mu);
  g_live.insert(p);
}
bool reg_live(const void* p) {
  std::lock_guard<std::mutex> g(g_reg_mu);
  return g_live.count(p) != 0;
}
bool reg_take(const void* p) {   // removes; true if it was live
  std::lock_guard<std::mutex> g(g_reg_mu);
  return g_live.erase(p) != 0;
}

// ---- error plumbing ---------------------------------------------------------

void set_err(char* err, size_t cap, const char* fmt, ...) {
  if (!err || cap == 0) return;
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(err, cap, fmt, ap);
  va_end(ap);
}

void clear_err(char* err, size_t cap) {
  if (err && cap) err[0] = '\0';
}

struct Fail {
  int code;
  std::string msg;
};

#define VXT_HIP_CHECK(expr)                                                                   \
  do {                                                                                        \
    hipError_t e_ = (expr);                                                                   \
    if (e_ != hipSuccess)                                                                     \
      throw Fail{VXT_E_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)};            \
  } while (0)

[[noreturn]] void fail(int code, const std::string& msg) { throw Fail{code, msg}; }

template <typename F>
int guarded(char* err, size_t cap, F&& f) {
  clear_err(err, cap);
  try {
    f();
    return VXT_OK;
  } catch (const Fail& e) {
    set_err(err, cap, "%s", e.msg.c_str());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_err(err, cap, "host allocation failed");
    return VXT_E_DEVICE;
  } catch (...) {
    set_err(err, cap, "unexpected internal error");
    return VXT_E_DEVICE;
  }
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

void use_device(Ctx* c) { VXT_HIP_CHECK(hipSetDevice(c->device)); }

void ensure(void** buf, size_t* cap, size_t need) {
  if (*cap >= need) return;
  if (*buf) VXT_HIP_CHECK(hipFree(*buf));
  *buf = nullptr;
  *cap = 0;
  size_t n = std::max<size_t>(need, 1 << 20);
  VXT_HIP_CHECK(hipMalloc(buf, n));
  *cap = n;
}

Tensor* new_tensor(Ctx* c, uint32_t kind, uint32_t rows, uint32_t cols, uint32_t kp,
                   const std::vector<char>& host_arena) {
  Tensor* t = new Tensor();
  t->ctx = c;
  t->kind = kind;
  t->rows = rows;
  t->cols = cols;
  t->kp = kp;
  t->bytes = host_arena.size();
  hipError_t e = hipMalloc(&t->arena, t->bytes);
  if (e != hipSuccess) {
    delete t;
    fail(VXT_E_DEVICE, std::string("hipMalloc of weight arena failed: ") + hipGetErrorString(e));
  }
  e = hipMemcpy(t->arena, host_arena.data(), t->bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(t->arena);
    delete t;
    fail(VXT_E_DEVICE, std::string("weight upload failed: ") + hipGetErrorString(e));
  }
  return t;
}

void register_tensor(Ctx* c, Tensor* t) {
  {
    std::lock_guard<std::mutex> g(c->mu);
    c->tensors.insert(t);
  }
  reg_add(t);
}

Tensor* as_tensor(void* p) {
  if (!p) fail(VXT_E_ARG, "null tensor handle");
  if (!reg_live(p)) fail(VXT_E_ARG, "released or unknown tensor handle");
  return static_cast<Tensor*>(p);
}

Ctx* as_ctx(void* p) {
  if (!p) fail(VXT_E_ARG, "null context handle");
  if (!reg_live(p)) fail(VXT_E_ARG, "destroyed or unknown context handle");
  return static_cast<Ctx*>(p);
}

// Releases one graph (its context's lock held by the caller or unneeded).
void release_graph(Graph* g) {
  (void)hipSetDevice(g->ctx->device);
  (void)hipStreamSynchronize(g->ctx->stream);
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  delete g;
}

// Plane checks of one CodebookMatrix view, as the archive reader does
// (format.rs:423-440, :565-574).
void validate_cb4(const VxtCb4View* v) {
  if (v->bits != 4) fail(VXT_E_UNSUPPORTED, "only 4-bit codebooks run on the device");
  if (v->rows == 0 || v->cols == 0) fail(VXT_E_SHAPE, "rows and cols must be positive");
  if (v->padded_cols < v->cols || v->padded_cols % 128u != 0)
    fail(VXT_E_FORMAT, "invalid codebook padded_cols");
  if (v->cols > 65536u && v->n_outliers != 0) fail(VXT_E_FORMAT, "outliers need cols <= 65536");
  if (!v->centroids || !v->scales_f16 || !v->packed_words || !v->outlier_row_ptr ||
      (v->n_outliers && !v->outliers_packed))
    fail(VXT_E_ARG, "null codebook plane");
  const size_t groups = (size_t)v->rows * (v->padded_cols / 128u);
  if (v->n_scales != groups || v->n_words != groups * 16u || v->n_row_ptr != (size_t)v->rows + 1u ||
      v->outlier_row_ptr[v->rows] != v->n_outliers)
    fail(VXT_E_FORMAT, "corrupt VXT codebook plane lengths");
  if (v->outlier_row_ptr[0] != 0) fail(VXT_E_FORMAT, "invalid VXT outlier CSR indices");
  for (size_t r = 0; r < v->rows; ++r)
    if (v->outlier_row_ptr[r] > v->outlier_row_ptr[r + 1] || v->outlier_row_ptr[r + 1] > v->n_outliers)
      fail(VXT_E_FORMAT, "invalid VXT outlier CSR indices");
  for (size_t i = 0; i < v->n_outliers; ++i)
    if ((v->outliers_packed[i] & 0xffffu) >= v->cols) fail(VXT_E_FORMAT, "invalid VXT outlier CSR indices");
}

bool dtype_ok(uint32_t d) { return d == VXT_DTYPE_F32 || d == VXT_DTYPE_BF16; }

// Shared argument checks for the device matmul entry points.
void check_matmul(Ctx* c, Tensor* t, const void* x, uint32_t x_dtype, uint32_t m, const void* y,
                  uint32_t y_dtype) {
  if (t->ctx != c) fail(VXT_E_ARG, "tensor belongs to another context");
  if (!x || !y) fail(VXT_E_ARG, "null activation or output pointer");
  if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) fail(VXT_E_ARG, "unknown dtype");
  if (m == 0) fail(VXT_E_SHAPE, "batch_m must be >= 1");
}

// The context workspace (GEMM weight panel and split-K partial sums, gated-FFN
// staging, attention partial sums) is shared by every call of this context
// (calls are ordered on one stream, or the caller orders them).  It grows only
// outside a capture, at least doubling, and a replaced buffer is kept until
// the context is destroyed: any graph captured earlier -- through
// vxt_hip_capture_begin or the caller's own stream capture -- recorded that
// buffer's address and may replay it later.  (Doubling bounds the kept
// buffers by the current one.)
void ensure_ws(Ctx* c, size_t need, hipStream_t s) {
  if (need <= c->ws_cap) return;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (c->capturing || (hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone))
    fail(VXT_E_ARG, "workspace too small inside a capture: run this shape once before capturing");
  const size_t n = std::max(need, 2 * c->ws_cap);
  void* p = nullptr;
  VXT_HIP_CHECK(hipMalloc(&p, n));
  if (c->ws) c->retired.push_back(c->ws);
  c->ws = p;
  c->ws_cap = n;
}

void run_matmul(Ctx* c, Tensor* t, const void* x, uint32_t x_dtype, uint32_t m, void* y,
                uint32_t y_dtype, hipStream_t s) {
  const DevTensor d = t->dev();
  const bool xb = x_dtype == VXT_DTYPE_BF16;
  const bool yb = y_dtype == VXT_DTYPE_BF16;
  hipError_t e;
  if (m <= 8) {
    const size_t esz = xb ? 2 : 4;
    const bool x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && ((size_t)t->cols * esz) % 16 == 0;
    e = vxt::launch_gemv(d, x, xb, x_vec, m, y, yb, s);
  } else {
    const size_t need = vxt::gemm_workspace_bytes(d, m, xb, c->gemm_mode);
    ensure_ws(c, need, s);
    e = vxt::launch_gemm(d, x, xb, m, y, yb, c->ws, c->ws_cap, s, c->gemm_mode);
  }
  if (e == hipErrorNotSupported) fail(VXT_E_UNSUPPORTED, "batch_m > 8 GEMM not available for this tensor");
  if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("kernel launch failed: ") + hipGetErrorString(e));
  (void)c;
}

}  // namespace

// ============================================================================
// C ABI
// ============================================================================

extern "C" {

void* vxt_hip_create(int32_t device, char* dev_name, size_t dev_name_cap, char* err,
                     size_t err_cap) {
  Ctx* c = nullptr;
  int rc = guarded(err, err_cap, [&] {
    int n = 0;
    VXT_HIP_CHECK(hipGetDeviceCount(&n));
    if (n <= 0) fail(VXT_E_DEVICE, "no HIP device");
    int dev = device;
    if (dev < 0) VXT_HIP_CHECK(hipGetDevice(&dev));
    if (dev >= n) fail(VXT_E_ARG, "device index out of range");
    hipDeviceProp_t prop;
    VXT_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      fail(VXT_E_UNSUPPORTED, std::string("kernels are built for gfx950, device is ") + prop.gcnArchName);
    c = new Ctx();
    c->device = dev;
    try {
      VXT_HIP_CHECK(hipSetDevice(dev));
      VXT_HIP_CHECK(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
      VXT_HIP_CHECK(hipEventCreate(&c->ev0));
      VXT_HIP_CHECK(hipEventCreate(&c->ev1));
      VXT_HIP_CHECK(hipMalloc(&c->greedy, vxt::greedy_state_bytes()));
      VXT_HIP_CHECK(hipMemset(c->greedy, 0, vxt::greedy_state_bytes()));
      VXT_HIP_CHECK(hipGetSymbolAddress(&c->scratch, HIP_SYMBOL(scratch)));   // with `dev` current
    } catch (...) {
      if (c->greedy) (void)hipFree(c->greedy);
      if (c->ev1) (void)hipEventDestroy(c->ev1);
      if (c->ev0) (void)hipEventDestroy(c->ev0);
      if (c->stream) (void)hipStreamDestroy(c->stream);
      delete c;
      c = nullptr;
      throw;
    }
    if (dev_name && dev_name_cap)
      std::snprintf(dev_name, dev_name_cap, "%s (%s)", prop.name, prop.gcnArchName);
  });
  if (rc != VXT_OK) return nullptr;
  vxt::blas_acquire_device(c->device);
  reg_add(c);
  return c;
}

void vxt_hip_destroy(void* ctx) {
  if (!ctx || !reg_take(ctx)) return;   // null, unknown or already destroyed
  Ctx* c = static_cast<Ctx*>(ctx);
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  {
    // Everything the context handed out goes with it; those handles become
    // stale (their release calls are then no-ops).
    std::lock_guard<std::mutex> g(c->mu);
    for (Runner* r : c->runners) {
      reg_take(r);
      release_runner(r);
    }
    c->runners.clear();
    for (Graph* gr : c->graphs) {
      reg_take(gr);
      release_graph(gr);
    }
    c->graphs.clear();
    for (Tensor* t : c->tensors) {
      reg_take(t);
      (void)hipFree(t->arena);
      delete t;
    }
    c->tensors.clear();
    for (void* b : c->buffers) (void)hipFree(b);
    c->buffers.clear();
  }
  if (c->d_x) (void)hipFree(c->d_x);
  if (c->d_y) (void)hipFree(c->d_y);
  if (c->ws) (void)hipFree(c->ws);
  for (void* b : c->retired) (void)hipFree(b);
  if (c->greedy) (void)hipFree(c->greedy);
  (void)hipEventDestroy(c->ev0);
  (void)hipEventDestroy(c->ev1);
  (void)hipStreamDestroy(c->stream);
  vxt::blas_release_device(c->device);
  delete c;
}

void* vxt_hip_upload_q8_0(void* ctx, uint32_t rows, uint32_t cols, const uint8_t* blocks,
                          size_t n_bytes, char* err, size_t err_cap) {
  Tensor* out = nullptr;
  guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!blocks) fail(VXT_E_ARG, "null Q8_0 byte pointer");
    if (rows == 0 || cols == 0) fail(VXT_E_SHAPE, "rows and cols must be positive");
    const size_t kb = (cols + 31u) / 32u;
    if (n_bytes != (size_t)rows * kb * 34u)
      fail(VXT_E_FORMAT, "Q8_0 byte length != rows * ceil(cols/32) * 34");
    const uint32_t kp = (uint32_t)(kb * 32u);
    // Split each 34-byte block into an int8 plane and an f16 scale plane so
    // every lane's 16-byte load is aligned and contiguous.
    // The scale plane keeps 16 bytes after its last scale (zero), so a
    // 16-byte load of 8 scales that starts at any scale stays inside the
    // allocation (the fused GEMM reads a chunk's 8 scales per row at once).
    const size_t qs_bytes = align256((size_t)rows * kp);
    const size_t d_bytes = align256((size_t)rows * kb * 2u + 16u);
    std::vector<char> h(qs_bytes + d_bytes, 0);
    int8_t* qs = reinterpret_cast<int8_t*>(h.data());
    uint16_t* d = reinterpret_cast<uint16_t*>(h.data() + qs_bytes);
    for (size_t r = 0; r < rows; ++r) {
      for (size_t b = 0; b < kb; ++b) {
        const uint8_t* blk = blocks + (r * kb + b) * 34u;
        d[r * kb + b] = (uint16_t)(blk[0] | (blk[1] << 8));
        std::memcpy(qs + r * kp + b * 32u, blk + 2, 32);
      }
    }
    use_device(c);
    Tensor* t = new_tensor(c, VXT_KIND_Q8_0, rows, cols, kp, h);
    t->off_p0 = 0;
    t->off_p1 = qs_bytes;
    register_tensor(c, t);
    out = t;
  });
  return out;
}

void* vxt_hip_upload_q4_0(void* ctx, uint32_t rows, uint32_t cols, uint32_t padded_cols, const uint16_t* scales_f16,
                          size_t n_scales, const uint32_t* qs_words, size_t n_words, char* err, size_t err_cap) {
  Tensor* out = nullptr;
  guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!scales_f16 || !qs_words) fail(VXT_E_ARG, "null Q4_0 plane pointer");
    if (rows == 0 || cols == 0) fail(VXT_E_SHAPE, "rows and cols must be positive");
    // format.rs:453-462
    const size_t kb = (cols + 31u) / 32u;
    if ((size_t)padded_cols != kb * 32u) fail(VXT_E_FORMAT, "invalid VXT Q4_0 padded_cols");
    if (n_scales != (size_t)rows * kb || n_words != (size_t)rows * kb * 4u)
      fail(VXT_E_FORMAT, "corrupt VXT Q4_0 plane lengths");
    // The planes as they are (the little-endian words are the block bytes in
    // order): 16 nibble bytes per block, row after row, then the f16 scales.
    const uint32_t kp = (uint32_t)(kb * 32u);
    const size_t qs_bytes = align256((size_t)rows * kb * 16u);
    const size_t d_bytes = align256((size_t)rows * kb * 2u);
    std::vector<char> h(qs_bytes + d_bytes, 0);
    std::memcpy(h.data(), qs_words, (size_t)rows * kb * 16u);
    std::memcpy(h.data() + qs_bytes, scales_f16, (size_t)rows * kb * 2u);
    use_device(c);
    Tensor* t = new_tensor(c, VXT_KIND_Q4_0, rows, cols, kp, h);
    t->off_p0 = 0;
    t->off_p1 = qs_bytes;
    register_tensor(c, t);
    out = t;
  });
  return out;
}

namespace {

float host_f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1f) return m ? std::numeric_limits<float>::quiet_NaN() : (s ? -INFINITY : INFINITY);
  const float v = e ? std::ldexp((float)(m | 0x400u), (int)e - 25) : std::ldexp((float)m, -24);
  return s ? -v : v;
}

}  // namespace

// Whether the decode-in-loop GEMM can take a cb4 tensor, and its per-row
// exponents if so: every centroid, scale and residual finite; each row's
// residual columns strictly increasing and inside the row; at most
// kCb4TileResCap residuals per block of 128 rows (the block's list is staged
// in LDS); e with bound * 2^e in [2^14, 2^15) for bound = largest |scale| x
// largest |centroid| + largest |residual| of the row (so every w * 2^e, and
// its hi/lo f16 split, stays inside the f16 range).
constexpr uint32_t kCb4TileResCap = 16384;

static bool cb4_tile_exponents(const VxtCb4View* subs, uint32_t n_subs, const uint32_t* rp, const uint32_t* outl,
                               const uint16_t* scales, std::vector<int8_t>& rex) {
  size_t rows = 0;
  for (uint32_t i = 0; i < n_subs; ++i) rows += subs[i].rows;
  const uint32_t cols = subs[0].cols, gpr = subs[0].padded_cols / 128u;
  rex.assign(rows, 0);
  size_t r = 0;
  for (uint32_t i = 0; i < n_subs; ++i) {
    double cmax = 0.0;
    for (int q = 0; q < 16; ++q) {
      const float c = subs[i].centroids[q];
      if (!std::isfinite(c)) return rex.clear(), false;
      cmax = std::max(cmax, (double)std::fabs(c));
    }
    for (size_t rr = 0; rr < subs[i].rows; ++rr, ++r) {
      double smax = 0.0, emax = 0.0;
      for (uint32_t g = 0; g < gpr; ++g) {
        const float sc = host_f16_to_f32(scales[r * gpr + g]);
        if (!std::isfinite(sc)) return rex.clear(), false;
        smax = std::max(smax, (double)std::fabs(sc));
      }
      int64_t prev = -1;
      for (uint32_t k = rp[r]; k < rp[r + 1]; ++k) {
        const uint32_t col = outl[k] & 0xffffu;
        const float v = host_f16_to_f32((uint16_t)(outl[k] >> 16));
        if (col >= cols || (int64_t)col <= prev || !std::isfinite(v)) return rex.clear(), false;
        prev = col;
        emax = std::max(emax, (double)std::fabs(v));
      }
      const double bound = smax * cmax + emax;
      int e = 0;
      if (bound > 0.0) {
        e = 14 - std::ilogb(bound);
        if (e < -100 || e > 100) return rex.clear(), false;
      }
      rex[r] = (int8_t)e;
    }
  }
  for (size_t b = 0; b < rows; b += 128)
    if (rp[std::min(rows, b + 128)] - rp[b] > kCb4TileResCap) return rex.clear(), false;
  return true;
}

void* vxt_hip_upload_cb4(void* ctx, const VxtCb4View* v, char* err, size_t err_cap) {
  return vxt_hip_upload_cb4_concat(ctx, v, 1u, err, err_cap);
}

void* vxt_hip_upload_cb4_concat(void* ctx, const VxtCb4View* subs, uint32_t n_subs, char* err,
                                size_t err_cap) {
  Tensor* out = nullptr;
  guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!subs) fail(VXT_E_ARG, "null codebook view");
    if (n_subs == 0 || n_subs > 3) fail(VXT_E_ARG, "a concatenated codebook tensor has 1 to 3 parts");
    size_t rows = 0, nnz = 0, n_words = 0, n_scales = 0;
    for (uint32_t i = 0; i < n_subs; ++i) {
      validate_cb4(&subs[i]);
      if (subs[i].cols != subs[0].cols || subs[i].padded_cols != subs[0].padded_cols)
        fail(VXT_E_SHAPE, "concatenated codebook parts must share cols and padded_cols");
      rows += subs[i].rows;
      nnz += subs[i].n_outliers;
      n_words += subs[i].n_words;
      n_scales += subs[i].n_scales;
    }
    if (rows > 0xffffffffu || nnz > 0xffffffffu) fail(VXT_E_SHAPE, "concatenated tensor too large");
    // One arena: words, scales, row_ptr (rebased per part), outliers, each
    // plane 256-byte aligned (metal_cb4_fast.mm:140-171 concatenates the same way).
    const size_t w_bytes = align256(n_words * 4u);
    const size_t s_bytes = align256(n_scales * 2u);
    const size_t rp_bytes = align256((rows + 1u) * 4u);
    const size_t o_bytes = align256(std::max<size_t>(nnz, 1) * 4u);
    std::vector<char> h(w_bytes + s_bytes + rp_bytes + o_bytes, 0);
    uint32_t* rp = reinterpret_cast<uint32_t*>(h.data() + w_bytes + s_bytes);
    size_t wo = 0, so = 0, ro = 0, oo = 0;
    for (uint32_t i = 0; i < n_subs; ++i) {
      const VxtCb4View& v = subs[i];
      std::memcpy(h.data() + wo * 4u, v.packed_words, v.n_words * 4u);
      std::memcpy(h.data() + w_bytes + so * 2u, v.scales_f16, v.n_scales * 2u);
      for (size_t r = 0; r < v.rows; ++r) rp[ro + r] = (uint32_t)(oo + v.outlier_row_ptr[r]);
      if (v.n_outliers)
        std::memcpy(h.data() + w_bytes + s_bytes + rp_bytes + oo * 4u, v.outliers_packed, v.n_outliers * 4u);
      wo += v.n_words;
      so += v.n_scales;
      ro += v.rows;
      oo += v.n_outliers;
    }
    rp[rows] = (uint32_t)nnz;
    // Decode-in-loop GEMM (gemm_tile.hip, tile_cb4_kernel): per-row exponents
    // appended to the arena when the tensor suits it.
    std::vector<int8_t> rex;
    if (cb4_tile_exponents(subs, n_subs, rp, reinterpret_cast<const uint32_t*>(h.data() + w_bytes + s_bytes + rp_bytes),
                           reinterpret_cast<const uint16_t*>(h.data() + w_bytes), rex)) {
      const size_t at = h.size();
      h.resize(at + align256(rows));
      std::memcpy(h.data() + at, rex.data(), rows);
    }
    const size_t rx_at = rex.empty() ? 0 : w_bytes + s_bytes + rp_bytes + o_bytes;
    use_device(c);
    Tensor* t = new_tensor(c, VXT_KIND_CB4, (uint32_t)rows, subs[0].cols, subs[0].padded_cols, h);
    t->off_rx = rx_at;
    t->off_p0 = 0;
    t->off_p1 = w_bytes;
    t->off_rp = w_bytes + s_bytes;
    t->off_out = w_bytes + s_bytes + rp_bytes;
    t->nnz = (uint32_t)nnz;
    // Table i serves rows [split(i), split(i+1)); unused tables repeat the last part's.
    uint32_t split[2] = {(uint32_t)rows, (uint32_t)rows};
    uint32_t acc = 0;
    for (uint32_t i = 0; i < 3; ++i) {
      const VxtCb4View& v = subs[i < n_subs ? i : n_subs - 1];
      std::memcpy(t->cent + 16 * i, v.centroids, 16 * sizeof(float));
      if (i < n_subs) {
        acc += v.rows;
        if (i < 2 && i + 1 < n_subs) split[i] = acc;
      }
    }
    t->split0 = split[0];
    t->split1 = split[1];
    register_tensor(c, t);
    out = t;
  });
  return out;
}

void* vxt_hip_upload_cb4_g64(void* ctx, const VxtCb4G64View* v, char* err, size_t err_cap) {
  Tensor* out = nullptr;
  guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!v) fail(VXT_E_ARG, "null g64 view");
    if (!v->idx || !v->lut_f16) fail(VXT_E_ARG, "null g64 plane");
    if (v->rows == 0 || v->cols == 0) fail(VXT_E_SHAPE, "rows and cols must be positive");
    if (v->padded_cols < v->cols || v->padded_cols % 64u != 0) fail(VXT_E_FORMAT, "invalid g64 padded_cols");
    const size_t n_idx = (size_t)v->rows * v->padded_cols / 2u;
    const size_t n_lut = (size_t)v->rows * (v->padded_cols / 64u) * 16u;
    if (v->n_idx != n_idx || v->n_lut != n_lut) fail(VXT_E_FORMAT, "corrupt g64 plane lengths");
    const size_t i_bytes = align256(n_idx);
    const size_t l_bytes = align256(n_lut * 2u);
    std::vector<char> h(i_bytes + l_bytes, 0);
    std::memcpy(h.data(), v->idx, n_idx);
    std::memcpy(h.data() + i_bytes, v->lut_f16, n_lut * 2u);
    use_device(c);
    // Padding columns multiply zero activations: they add nothing unless the
    // entry they index is Inf/NaN, which the kernels that do not mask them
    // must know about.
    uint32_t tail_nonfinite = 0;
    if (v->cols % 64u != 0) {
      const size_t gpr = v->padded_cols / 64u;
      for (size_t r = 0; r < v->rows && !tail_nonfinite; ++r)
        for (size_t e = 0; e < 16; ++e)
          if ((v->lut_f16[(r * gpr + gpr - 1) * 16 + e] & 0x7c00u) == 0x7c00u) tail_nonfinite = 1;
    }
    Tensor* t = new_tensor(c, VXT_KIND_CB4_G64, v->rows, v->cols, v->padded_cols, h);
    t->off_p0 = 0;
    t->off_p1 = i_bytes;
    t->tail_nonfinite = tail_nonfinite;
    register_tensor(c, t);
    out = t;
  });
  return out;
}

void* vxt_hip_clone_tensor(void* tensor, char* err, size_t err_cap) {
  Tensor* out = nullptr;
  guarded(err, err_cap, [&] {
    Tensor* s = as_tensor(tensor);
    Ctx* c = s->ctx;
    use_device(c);
    Tensor* t = new Tensor(*s);
    t->arena = nullptr;
    hipError_t e = hipMalloc(&t->arena, t->bytes);
    if (e != hipSuccess) {
      delete t;
      fail(VXT_E_DEVICE, std::string("hipMalloc for clone failed: ") + hipGetErrorString(e));
    }
    e = hipMemcpy(t->arena, s->arena, t->bytes, hipMemcpyDeviceToDevice);
    if (e != hipSuccess) {
      (void)hipFree(t->arena);
      delete t;
      fail(VXT_E_DEVICE, std::string("clone copy failed: ") + hipGetErrorString(e));
    }
    register_tensor(c, t);
    out = t;
  });
  return out;
}

void vxt_hip_free_tensor(void* tensor) {
  if (!tensor || !reg_take(tensor)) return;   // released already (or with its context)
  Tensor* t = static_cast<Tensor*>(tensor);
  Ctx* c = t->ctx;
  (void)hipSetDevice(c->device);
  // Work queued on the context stream may still read the arena.
  (void)hipStreamSynchronize(c->stream);
  {
    std::lock_guard<std::mutex> g(c->mu);
    c->tensors.erase(t);
  }
  (void)hipFree(t->arena);
  delete t;
}

int vxt_hip_tensor_info(void* tensor, uint32_t* kind, uint32_t* rows, uint32_t* cols,
                        uint64_t* device_bytes) {
  if (!tensor || !reg_live(tensor)) return VXT_E_ARG;
  Tensor* t = static_cast<Tensor*>(tensor);
  if (kind) *kind = t->kind;
  if (rows) *rows = t->rows;
  if (cols) *cols = t->cols;
  if (device_bytes) *device_bytes = t->bytes;
  return VXT_OK;
}

int vxt_hip_matmul_dev(void* ctx, void* tensor, const void* x, uint32_t x_dtype, uint32_t batch_m,
                       void* y, uint32_t y_dtype, void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    Tensor* t = as_tensor(tensor);
    check_matmul(c, t, x, x_dtype, batch_m, y, y_dtype);
    run_matmul(c, t, x, x_dtype, batch_m, y, y_dtype, static_cast<hipStream_t>(stream));
  });
}

int vxt_hip_matmul_noalloc_dev(void* ctx, void* tensor, const void* x, uint32_t x_dtype, uint32_t batch_m,
                               void* y, uint32_t y_dtype, void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    Tensor* t = as_tensor(tensor);
    check_matmul(c, t, x, x_dtype, batch_m, y, y_dtype);
    const DevTensor d = t->dev();
    const bool xb = x_dtype == VXT_DTYPE_BF16, yb = y_dtype == VXT_DTYPE_BF16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (batch_m <= 8) {   // the GEMV kernels use no workspace
      const size_t esz = xb ? 2 : 4;
      const bool x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && ((size_t)t->cols * esz) % 16 == 0;
      e = vxt::launch_gemv(d, x, xb, x_vec, batch_m, y, yb, s);
    } else {
      // The context's path choice, with the library's dense phase replaced by
      // the own kernel (the library allocates descriptors on first use).
      const int mode = c->gemm_mode == vxt::kGemmAuto    ? vxt::kGemmAutoOwn
                       : c->gemm_mode == vxt::kGemmLibrary ? vxt::kGemmPanel
                                                           : c->gemm_mode;
      const size_t need = vxt::gemm_workspace_bytes(d, batch_m, xb, mode);
      if (need > kScratchBytes)
        fail(VXT_E_SHAPE, "this GEMM needs " + std::to_string(need) + " bytes of scratch; the allocation-free entry "
                          "point has " + std::to_string(kScratchBytes) + " (use vxt_hip_matmul_dev)");
      e = vxt::launch_gemm(d, x, xb, batch_m, y, yb, c->scratch, kScratchBytes, s, mode);
    }
    if (e == hipErrorNotSupported) fail(VXT_E_UNSUPPORTED, "batch_m > 8 GEMM not available for this tensor");
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("kernel launch failed: ") + hipGetErrorString(e));
  });
}

int vxt_hip_matmul_multi_dev(void* ctx, void* const* tensors, uint32_t n, const void* x,
                             uint32_t x_dtype, uint32_t batch_m, void* const* ys, uint32_t y_dtype,
                             void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!tensors || !ys) fail(VXT_E_ARG, "null tensor or output array");
    uint32_t cols = 0;
    for (uint32_t i = 0; i < n; ++i) {
      Tensor* t = as_tensor(tensors[i]);
      check_matmul(c, t, x, x_dtype, batch_m, ys[i], y_dtype);
      if (i == 0) cols = t->cols;
      if (t->cols != cols) fail(VXT_E_SHAPE, "tensors sharing x must have equal cols");
    }
    for (uint32_t i = 0; i < n; ++i)
      run_matmul(c, static_cast<Tensor*>(tensors[i]), x, x_dtype, batch_m, ys[i], y_dtype,
                 static_cast<hipStream_t>(stream));
  });
}

int vxt_hip_run_multi(void* ctx, const float* x, uint32_t x_elems, const VxtHipJob* jobs,
                      uint32_t n_jobs, uint32_t iters, double* gpu_ms, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (gpu_ms) *gpu_ms = 0.0;
    if (n_jobs == 0) return;
    if (!x || !jobs) fail(VXT_E_ARG, "null x or job array");
    size_t y_total = 0;
    for (uint32_t i = 0; i < n_jobs; ++i) {
      Tensor* t = as_tensor(jobs[i].tensor);
      if (t->ctx != c) fail(VXT_E_ARG, "tensor belongs to another context");
      if (!jobs[i].y) fail(VXT_E_ARG, "null job output");
      if (x_elems < t->cols) fail(VXT_E_SHAPE, "x shorter than a job's cols");
      y_total += align256((size_t)t->rows * 4u);
    }
    use_device(c);
    ensure(&c->d_x, &c->d_x_cap, (size_t)x_elems * 4u);
    ensure(&c->d_y, &c->d_y_cap, y_total);
    VXT_HIP_CHECK(hipMemcpyAsync(c->d_x, x, (size_t)x_elems * 4u, hipMemcpyHostToDevice, c->stream));
    const uint32_t runs = std::max<uint32_t>(iters, 1u);
    VXT_HIP_CHECK(hipEventRecord(c->ev0, c->stream));
    for (uint32_t it = 0; it < runs; ++it) {
      size_t off = 0;
      for (uint32_t i = 0; i < n_jobs; ++i) {
        Tensor* t = static_cast<Tensor*>(jobs[i].tensor);
        run_matmul(c, t, c->d_x, VXT_DTYPE_F32, 1, static_cast<char*>(c->d_y) + off, VXT_DTYPE_F32,
                   c->stream);
        off += align256((size_t)t->rows * 4u);
      }
    }
    VXT_HIP_CHECK(hipEventRecord(c->ev1, c->stream));
    size_t off = 0;
    for (uint32_t i = 0; i < n_jobs; ++i) {
      Tensor* t = static_cast<Tensor*>(jobs[i].tensor);
      VXT_HIP_CHECK(hipMemcpyAsync(jobs[i].y, static_cast<char*>(c->d_y) + off, (size_t)t->rows * 4u,
                                   hipMemcpyDeviceToHost, c->stream));
      off += align256((size_t)t->rows * 4u);
    }
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
    float ms = 0.0f;
    VXT_HIP_CHECK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
    c->last_ms = ms;
    if (gpu_ms) *gpu_ms = ms;
  });
}

int vxt_hip_gemm(void* ctx, void* tensor, const float* x_batch, uint32_t batch_m, float* y_batch,
                 double* gpu_ms, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    Tensor* t = as_tensor(tensor);
    if (gpu_ms) *gpu_ms = 0.0;
    if (t->ctx != c) fail(VXT_E_ARG, "tensor belongs to another context");
    if (batch_m == 0) return;  // llm_prefill.rs:163-165
    if (!x_batch || !y_batch) fail(VXT_E_ARG, "null x_batch or y_batch");
    use_device(c);
    const size_t xb = (size_t)batch_m * t->cols * 4u;
    const size_t yb = (size_t)batch_m * t->rows * 4u;
    ensure(&c->d_x, &c->d_x_cap, xb);
    ensure(&c->d_y, &c->d_y_cap, yb);
    VXT_HIP_CHECK(hipMemcpyAsync(c->d_x, x_batch, xb, hipMemcpyHostToDevice, c->stream));
    VXT_HIP_CHECK(hipEventRecord(c->ev0, c->stream));
    run_matmul(c, t, c->d_x, VXT_DTYPE_F32, batch_m, c->d_y, VXT_DTYPE_F32, c->stream);
    VXT_HIP_CHECK(hipEventRecord(c->ev1, c->stream));
    VXT_HIP_CHECK(hipMemcpyAsync(y_batch, c->d_y, yb, hipMemcpyDeviceToHost, c->stream));
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
    float ms = 0.0f;
    VXT_HIP_CHECK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
    c->last_ms = ms;
    if (gpu_ms) *gpu_ms = ms;
  });
}

int vxt_hip_dequant_rows_dev(void* ctx, void* tensor, uint32_t row0, uint32_t nrows, float* out,
                             void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    Tensor* t = as_tensor(tensor);
    if (t->ctx != c) fail(VXT_E_ARG, "tensor belongs to another context");
    if (!out && nrows) fail(VXT_E_ARG, "null output");
    if ((uint64_t)row0 + nrows > t->rows) fail(VXT_E_SHAPE, "row range outside the tensor");
    const DevTensor d = t->dev();
    for (uint32_t done = 0; done < nrows;) {
      const uint32_t n = std::min<uint32_t>(nrows - done, 32768u);
      hipError_t e = vxt::launch_dequant(d, row0 + done, n, out + (size_t)done * t->cols,
                                         static_cast<hipStream_t>(stream));
      if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("dequant launch failed: ") + hipGetErrorString(e));
      done += n;
    }
  });
}

int vxt_hip_dequant_rows(void* ctx, void* tensor, uint32_t row0, uint32_t nrows, float* out,
                         char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    Tensor* t = as_tensor(tensor);
    if (t->ctx != c) fail(VXT_E_ARG, "tensor belongs to another context");
    if (!out && nrows) fail(VXT_E_ARG, "null output");
    if ((uint64_t)row0 + nrows > t->rows) fail(VXT_E_SHAPE, "row range outside the tensor");
    if (nrows == 0) return;
    use_device(c);
    const size_t ob = (size_t)nrows * t->cols * 4u;
    ensure(&c->d_y, &c->d_y_cap, ob);
    char e2[256];
    int rc = vxt_hip_dequant_rows_dev(ctx, tensor, row0, nrows, static_cast<float*>(c->d_y), c->stream,
                                      e2, sizeof(e2));
    if (rc != VXT_OK) fail(rc, e2);
    VXT_HIP_CHECK(hipMemcpyAsync(out, c->d_y, ob, hipMemcpyDeviceToHost, c->stream));
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int vxt_hip_ffn_glu_dev(void* ctx, void* tensor, const void* x, uint32_t x_dtype, uint32_t batch_m, void* act,
                        uint32_t act_dtype, uint32_t act_stride, uint32_t activation, void* stream, char* err,
                        size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    Tensor* t = as_tensor(tensor);
    check_matmul(c, t, x, x_dtype, batch_m, act, act_dtype);
    if (t->rows % 2 != 0) fail(VXT_E_SHAPE, "a [gate; up] tensor has an even row count");
    if (activation > VXT_ACT_GELU_TANH) fail(VXT_E_ARG, "unknown activation");
    const uint32_t n_ff = t->rows / 2;
    if (act_stride < n_ff) fail(VXT_E_SHAPE, "act_stride < rows / 2");
    const bool xb = x_dtype == VXT_DTYPE_BF16, ab = act_dtype == VXT_DTYPE_BF16;
    const bool gelu = activation == VXT_ACT_GELU_TANH;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const DevTensor d = t->dev();
    hipError_t e;
    if (batch_m <= 2) {
      e = vxt::launch_gemv_glu(d, x, xb, batch_m, act, ab, act_stride, gelu, s);
    } else {
      // Gate and up rows into f32 staging after the GEMM's own workspace,
      // then the element-wise activation.
      const size_t gemm_ws =
          batch_m > 8 ? (vxt::gemm_workspace_bytes(d, batch_m, xb, c->gemm_mode) + 255) / 256 * 256 : 0;
      const size_t stage = (size_t)batch_m * t->rows * sizeof(float);
      ensure_ws(c, gemm_ws + stage, s);
      float* gu = reinterpret_cast<float*>(static_cast<char*>(c->ws) + gemm_ws);
      if (batch_m <= 8) {
        e = vxt::launch_gemv(d, x, xb, false, batch_m, gu, false, s);
      } else {
        e = vxt::launch_gemm(d, x, xb, batch_m, gu, false, c->ws, gemm_ws, s, c->gemm_mode);
      }
      if (e == hipSuccess) e = vxt::launch_glu_act(gu, batch_m, n_ff, gelu, act, ab, act_stride, s);
    }
    if (e == hipErrorNotSupported) fail(VXT_E_UNSUPPORTED, "batch_m > 8 GEMM not available for this tensor");
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("gated FFN launch failed: ") + hipGetErrorString(e));
  });
}

int vxt_hip_norm_matmul_dev(void* ctx, void* tensor, const float* cur, const float* delta, const float* norm_w,
                            float eps, float* cur_out, uint32_t mode, void* y, uint32_t y_dtype, uint32_t y_stride,
                            void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    Tensor* t = as_tensor(tensor);
    if (t->ctx != c) fail(VXT_E_ARG, "tensor belongs to another context");
    if (!cur || !norm_w || !y) fail(VXT_E_ARG, "null pointer");
    if (!dtype_ok(y_dtype)) fail(VXT_E_ARG, "unknown dtype");
    if (mode > VXT_NORM_GLU_GELU_TANH) fail(VXT_E_ARG, "unknown mode");
    if (delta && (!cur_out || cur_out == cur || cur_out == delta))
      fail(VXT_E_ARG, "with delta, cur_out must be a separate buffer");
    if (t->cols > 4096) fail(VXT_E_UNSUPPORTED, "the norm prologue takes cols <= 4096");
    const bool gated = mode != VXT_NORM_PLAIN;
    if (gated && t->rows % 2 != 0) fail(VXT_E_SHAPE, "a [gate; up] tensor has an even row count");
    if (gated && y_stride < t->rows / 2) fail(VXT_E_SHAPE, "y_stride < rows / 2");
    vxt::NormIn nin{cur, delta, norm_w, delta ? cur_out : nullptr, eps};
    const int epi = mode == VXT_NORM_PLAIN ? 0 : mode == VXT_NORM_GLU_SILU ? 1 : 2;
    hipError_t e = vxt::launch_gemv_norm(t->dev(), nin, epi, y, y_dtype == VXT_DTYPE_BF16, gated ? y_stride : t->rows,
                                         static_cast<hipStream_t>(stream));
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("norm matmul launch failed: ") + hipGetErrorString(e));
  });
}

namespace {
vxt::KvQ8Dev kv_cache_dev(const VxtKvQ8Cache* kc) {
  if (!kc) fail(VXT_E_ARG, "null cache");
  if (!kc->k_qs || !kc->k_d || !kc->v_qs || !kc->v_d) fail(VXT_E_ARG, "null cache plane");
  if (kc->head_dim != 32 && kc->head_dim != 64 && kc->head_dim != 128 && kc->head_dim != 256)
    fail(VXT_E_UNSUPPORTED, "head_dim must be 32, 64, 128 or 256");
  if (kc->n_kv == 0 || kc->max_seq == 0) fail(VXT_E_SHAPE, "empty cache");
  if (((uintptr_t)kc->k_qs | (uintptr_t)kc->v_qs) % 16 || ((uintptr_t)kc->k_d | (uintptr_t)kc->v_d) % 2)
    fail(VXT_E_ARG, "value planes must be 16-byte aligned, scale planes 2-byte aligned");
  return vxt::KvQ8Dev{static_cast<int8_t*>(kc->k_qs), static_cast<uint16_t*>(kc->k_d),
                      static_cast<int8_t*>(kc->v_qs), static_cast<uint16_t*>(kc->v_d), kc->max_seq, kc->n_kv,
                      kc->head_dim};
}
}  // namespace

int vxt_hip_kv_q8_append_dev(void* ctx, const VxtKvQ8Cache* cache, const float* k, const float* v, uint32_t pos,
                             void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    (void)as_ctx(ctx);
    const vxt::KvQ8Dev c = kv_cache_dev(cache);
    if (!k || !v) fail(VXT_E_ARG, "null k or v");
    if (pos >= c.max_seq) fail(VXT_E_SHAPE, "pos >= max_seq");
    hipError_t e = vxt::launch_kv_append(c, k, v, pos, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("kv append launch failed: ") + hipGetErrorString(e));
  });
}

int vxt_hip_attn_q8_dev(void* ctx, const VxtKvQ8Cache* cache, const float* q, uint32_t n_head, uint32_t seq_len,
                        const float* gate, float* out, void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    const vxt::KvQ8Dev kc = kv_cache_dev(cache);
    if (!q || !out) fail(VXT_E_ARG, "null q or out");
    if (seq_len == 0 || seq_len > kc.max_seq) fail(VXT_E_SHAPE, "need 1 <= seq_len <= max_seq");
    if (n_head == 0 || n_head % kc.n_kv != 0) fail(VXT_E_SHAPE, "n_head must be a multiple of n_kv");
    if (n_head / kc.n_kv > 8) fail(VXT_E_UNSUPPORTED, "at most 8 query heads per kv head");
    ensure_ws(c, vxt::attn_workspace_bytes(n_head, seq_len, kc.n_kv, kc.hd, 1), static_cast<hipStream_t>(stream));
    hipError_t e = vxt::launch_attn(kc, q, n_head, seq_len, 1, gate, out, c->ws, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("attention launch failed: ") + hipGetErrorString(e));
  });
}

namespace {
// Batches of at least this many tokens take the MFMA prefill attention.
constexpr uint32_t kPrefillMfmaMin = 16;

// Checks shared by the prep and the whole step; fills the device arguments
// (q_out / gate_out left to the caller).
vxt::GqaPrep gqa_prep_args(const vxt::KvQ8Dev& kc, const VxtGqaParams* p, const float* q_raw, uint32_t q_stride,
                           const float* k_cur, const float* v_cur, uint32_t kv_stride, uint32_t batch_m, uint32_t pos,
                           uint32_t rope_pos) {
  if (!p) fail(VXT_E_ARG, "null params");
  if (!q_raw || !k_cur || !v_cur) fail(VXT_E_ARG, "null q_raw, k_cur or v_cur");
  if (p->n_head == 0) fail(VXT_E_SHAPE, "n_head must be >= 1");
  if (p->gated_q > 1 || p->rope_neox > 1) fail(VXT_E_ARG, "gated_q and rope_neox are 0 or 1");
  if (batch_m == 0 || batch_m > 65535u) fail(VXT_E_SHAPE, "need 1 <= batch_m <= 65535");
  if (pos >= kc.max_seq || batch_m > kc.max_seq - pos) fail(VXT_E_SHAPE, "pos + batch_m > max_seq");
  if (rope_pos > UINT32_MAX - (batch_m - 1)) fail(VXT_E_SHAPE, "rope_pos + batch_m - 1 overflows");
  const uint64_t q_rows = (uint64_t)p->n_head * kc.hd * (p->gated_q ? 2u : 1u);
  if (batch_m > 1 && q_stride < q_rows) fail(VXT_E_SHAPE, "q_stride < q_rows");
  if (batch_m > 1 && kv_stride < kc.n_kv * kc.hd) fail(VXT_E_SHAPE, "kv_stride < n_kv * head_dim");
  if (!(p->eps >= 0.0f) || !std::isfinite(p->rope_freq_base)) fail(VXT_E_ARG, "eps or rope_freq_base out of range");
  vxt::GqaPrep a{};
  a.q_raw = q_raw;
  a.k_cur = k_cur;
  a.v_cur = v_cur;
  a.q_norm = p->q_norm;
  a.k_norm = p->k_norm;
  a.q_bias = p->q_bias;
  a.k_bias = p->k_bias;
  a.v_bias = p->v_bias;
  a.q_stride = q_stride;
  a.kv_stride = kv_stride;
  a.n_head = p->n_head;
  a.gated = p->gated_q;
  a.neox = p->rope_neox;
  a.pos = pos;
  a.rope_pos = rope_pos;
  a.eps = p->eps;
  return a;
}
}  // namespace

int vxt_hip_attn_prep_q8_dev(void* ctx, const VxtKvQ8Cache* cache, const VxtGqaParams* params, const float* q_raw,
                             uint32_t q_stride, const float* k_cur, const float* v_cur, uint32_t kv_stride,
                             uint32_t batch_m, uint32_t pos, uint32_t rope_pos, float* q_out, float* gate_out,
                             void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    (void)as_ctx(ctx);
    const vxt::KvQ8Dev kc = kv_cache_dev(cache);
    vxt::GqaPrep a = gqa_prep_args(kc, params, q_raw, q_stride, k_cur, v_cur, kv_stride, batch_m, pos, rope_pos);
    if (!q_out) fail(VXT_E_ARG, "null q_out");
    if (params->gated_q && !gate_out) fail(VXT_E_ARG, "a gated q needs gate_out");
    a.q_out = q_out;
    a.gate_out = params->gated_q ? gate_out : nullptr;
    hipError_t e = vxt::launch_gqa_prep(kc, a, params->rope_dim, params->rope_freq_base, batch_m,
                                        static_cast<hipStream_t>(stream));
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("attention prep launch failed: ") + hipGetErrorString(e));
  });
}

int vxt_hip_attn_step_q8_dev(void* ctx, const VxtKvQ8Cache* cache, const VxtGqaParams* params, const float* q_raw,
                             uint32_t q_stride, const float* k_cur, const float* v_cur, uint32_t kv_stride,
                             uint32_t batch_m, uint32_t pos, uint32_t rope_pos, float* out, void* stream, char* err,
                             size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    const vxt::KvQ8Dev kc = kv_cache_dev(cache);
    vxt::GqaPrep a = gqa_prep_args(kc, params, q_raw, q_stride, k_cur, v_cur, kv_stride, batch_m, pos, rope_pos);
    if (!out) fail(VXT_E_ARG, "null out");
    const uint32_t n_head = params->n_head;
    if (n_head % kc.n_kv != 0) fail(VXT_E_SHAPE, "n_head must be a multiple of n_kv");
    if (n_head / kc.n_kv > 8) fail(VXT_E_UNSUPPORTED, "at most 8 query heads per kv head");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (batch_m == 1) {
      // decode: the prep runs inside the attention's chunk kernel
      ensure_ws(c, vxt::attn_workspace_bytes(n_head, pos + 1, kc.n_kv, kc.hd, 1), s);
      hipError_t e = vxt::launch_attn_step(kc, a, params->rope_dim, params->rope_freq_base, out, c->ws, s);
      if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("attention step launch failed: ") + hipGetErrorString(e));
      return;
    }
    // Workspace: q (and gate) of every token, then (batches below
    // kPrefillMfmaMin tokens, or head_dim 256) the partial sums of one group
    // of tokens at a time, groups sized to keep that part near 16 MiB.
    const size_t q_bytes = (size_t)batch_m * n_head * kc.hd * sizeof(float);
    const size_t qg_bytes = (q_bytes * (params->gated_q ? 2u : 1u) + 255u) & ~(size_t)255u;
    if (batch_m >= kPrefillMfmaMin && kc.hd <= 128) {
      // prep, then the MFMA attention over position segments, in token
      // groups whose segment partial sums stay near 256 MiB
      const size_t per_tok = vxt::attn_prefill_workspace_bytes(n_head, kc.hd, pos, batch_m) / batch_m;
      const uint32_t group_t = (uint32_t)std::max<size_t>(
          1, std::min<size_t>(batch_m, ((size_t)256 << 20) / std::max<size_t>(per_tok, 1)));
      ensure_ws(c, qg_bytes + per_tok * group_t, s);
      float* q_ws = static_cast<float*>(c->ws);
      a.q_out = q_ws;
      a.gate_out = params->gated_q ? q_ws + (size_t)batch_m * n_head * kc.hd : nullptr;
      void* part = static_cast<char*>(c->ws) + qg_bytes;
      hipError_t e = vxt::launch_gqa_prep(kc, a, params->rope_dim, params->rope_freq_base, batch_m, s);
      const size_t row = (size_t)n_head * kc.hd;
      for (uint32_t t = 0; t < batch_m && e == hipSuccess; t += group_t) {
        const uint32_t nb = std::min(group_t, batch_m - t);
        e = vxt::launch_attn_prefill(kc, q_ws + t * row, a.gate_out ? a.gate_out + t * row : nullptr, out + t * row,
                                     n_head, pos + t, nb, part, s);
      }
      if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("prefill attention launch failed: ") + hipGetErrorString(e));
      return;
    }
    const size_t per_tok = vxt::attn_workspace_bytes(n_head, pos + batch_m, kc.n_kv, kc.hd, 1);
    const uint32_t group_m =
        (uint32_t)std::max<size_t>(1, std::min<size_t>(batch_m, ((size_t)16 << 20) / std::max<size_t>(per_tok, 1)));
    ensure_ws(c, qg_bytes + vxt::attn_workspace_bytes(n_head, pos + batch_m - group_m + 1, kc.n_kv, kc.hd, group_m),
              s);
    float* q_ws = static_cast<float*>(c->ws);
    float* g_ws = params->gated_q ? q_ws + (size_t)batch_m * n_head * kc.hd : nullptr;
    void* part = static_cast<char*>(c->ws) + qg_bytes;
    a.q_out = q_ws;
    a.gate_out = g_ws;
    hipError_t e = vxt::launch_gqa_prep(kc, a, params->rope_dim, params->rope_freq_base, batch_m, s);
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("attention prep launch failed: ") + hipGetErrorString(e));
    const size_t row = (size_t)n_head * kc.hd;
    for (uint32_t t = 0; t < batch_m; t += group_m) {
      const uint32_t nb = std::min(group_m, batch_m - t);
      e = vxt::launch_attn(kc, q_ws + t * row, n_head, pos + t + 1, nb, g_ws ? g_ws + t * row : nullptr,
                           out + t * row, part, s);
      if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("attention launch failed: ") + hipGetErrorString(e));
    }
  });
}

int vxt_hip_rms_norm_dev(void* ctx, float* cur, const float* delta, const float* weight, void* out,
                         uint32_t out_dtype, uint32_t dim, uint32_t stride, uint32_t batch_m, float eps,
                         void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    (void)as_ctx(ctx);
    if (batch_m == 0) return;
    if (!cur || !weight || !out) fail(VXT_E_ARG, "null pointer");
    if (!dtype_ok(out_dtype)) fail(VXT_E_ARG, "unknown dtype");
    if (dim == 0 || stride < dim) fail(VXT_E_SHAPE, "need 0 < dim <= stride");
    if (out_dtype == VXT_DTYPE_BF16 && (out == cur || out == delta))
      fail(VXT_E_ARG, "a bf16 output cannot overwrite an f32 input");
    if (delta && out == delta) fail(VXT_E_ARG, "out may alias cur, not delta");
    hipError_t e = vxt::launch_rms_norm(cur, delta, weight, out, out_dtype == VXT_DTYPE_BF16, dim, stride, batch_m,
                                        eps, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("rms_norm launch failed: ") + hipGetErrorString(e));
  });
}

int vxt_hip_embed_dev(void* ctx, void* tensor, const uint32_t* tokens, uint32_t batch_m, float embed_scale,
                      float* out, uint32_t out_stride, void* stream, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    Tensor* t = as_tensor(tensor);
    if (t->ctx != c) fail(VXT_E_ARG, "tensor belongs to another context");
    if (batch_m == 0) return;
    if (!tokens || !out) fail(VXT_E_ARG, "null tokens or output");
    if (out_stride < t->cols) fail(VXT_E_SHAPE, "out_stride < cols");
    if (batch_m > 65535) fail(VXT_E_SHAPE, "batch_m > 65535");
    if (!std::isfinite(embed_scale)) fail(VXT_E_ARG, "embed_scale is not finite");
    // llm_cpu.rs:226: the scale applies when it differs from 1 by more than 1e-7.
    const bool scale_on = std::fabs(embed_scale - 1.0f) > 1e-7f;
    hipError_t e = vxt::launch_embed(t->dev(), tokens, batch_m, embed_scale, scale_on, out, out_stride,
                                     static_cast<hipStream_t>(stream));
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("embed launch failed: ") + hipGetErrorString(e));
  });
}

int vxt_hip_greedy_dev(void* ctx, const float* logits, uint32_t n, uint32_t* out, void* stream, char* err,
                       size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!out) fail(VXT_E_ARG, "null output");
    if (!logits && n) fail(VXT_E_ARG, "null logits");
    if ((reinterpret_cast<uintptr_t>(logits) & 3u) != 0) fail(VXT_E_ARG, "logits must be 4-byte aligned");
    if ((reinterpret_cast<uintptr_t>(out) & 3u) != 0) fail(VXT_E_ARG, "out must be 4-byte aligned");
    if (n > 0x7fffffffu) fail(VXT_E_SHAPE, "more than 2^31 - 1 logits");
    hipError_t e = vxt::launch_greedy(logits, n, c->greedy, out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("greedy launch failed: ") + hipGetErrorString(e));
  });
}

int vxt_hip_read_probe_dev(void* ctx, const void* p, size_t bytes, uint32_t key, void* stream, char* err,
                           size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!p) fail(VXT_E_ARG, "null pointer");
    if (bytes < 16 || bytes % 16 != 0) fail(VXT_E_SHAPE, "bytes must be a positive multiple of 16");
    // the sink word: the greedy state's last word, never written by the probe
    uint32_t* sink = reinterpret_cast<uint32_t*>(static_cast<char*>(c->greedy) + vxt::greedy_state_bytes()) - 1;
    const hipError_t e = vxt::launch_read_probe(p, bytes, sink, key, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) fail(VXT_E_DEVICE, std::string("probe launch failed: ") + hipGetErrorString(e));
  });
}

void* vxt_hip_device_alloc(void* ctx, size_t bytes, char* err, size_t err_cap) {
  void* out = nullptr;
  guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    use_device(c);
    void* p = nullptr;
    VXT_HIP_CHECK(hipMalloc(&p, std::max<size_t>(bytes, 256)));
    std::lock_guard<std::mutex> g(c->mu);
    c->buffers.insert(p);
    out = p;
  });
  return out;
}

void vxt_hip_device_free(void* ctx, void* dev_ptr) {
  if (!ctx || !dev_ptr || !reg_live(ctx)) return;   // a destroyed context freed its buffers
  Ctx* c = static_cast<Ctx*>(ctx);
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  std::lock_guard<std::mutex> g(c->mu);
  if (c->buffers.erase(dev_ptr)) (void)hipFree(dev_ptr);
}

int vxt_hip_memcpy(void* ctx, void* dst, const void* src, size_t bytes, uint32_t kind, char* err,
                   size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (bytes == 0) return;
    if (!dst || !src) fail(VXT_E_ARG, "null copy pointer");
    hipMemcpyKind k;
    switch (kind) {
      case 0: k = hipMemcpyHostToDevice; break;
      case 1: k = hipMemcpyDeviceToHost; break;
      case 2: k = hipMemcpyDeviceToDevice; break;
      default: fail(VXT_E_ARG, "unknown copy kind");
    }
    use_device(c);
    VXT_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, k, c->stream));
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

void* vxt_hip_stream(void* ctx) {
  if (!ctx || !reg_live(ctx)) return nullptr;
  return static_cast<Ctx*>(ctx)->stream;
}

int vxt_hip_synchronize(void* ctx, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    use_device(c);
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int vxt_hip_capture_begin(void* ctx, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (c->capturing) fail(VXT_E_ARG, "capture already in progress");
    use_device(c);
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
    VXT_HIP_CHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
  });
}

void* vxt_hip_capture_end(void* ctx, char* err, size_t err_cap) {
  Graph* out = nullptr;
  guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!c->capturing) fail(VXT_E_ARG, "no capture in progress");
    use_device(c);
    c->capturing = false;
    hipGraph_t g = nullptr;
    VXT_HIP_CHECK(hipStreamEndCapture(c->stream, &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      (void)hipGraphDestroy(g);
      fail(VXT_E_DEVICE, std::string("hipGraphInstantiate failed: ") + hipGetErrorString(e));
    }
    out = new Graph{c, g, ex};
    {
      std::lock_guard<std::mutex> lk(c->mu);
      c->graphs.insert(out);
    }
    reg_add(out);
  });
  return out;
}

int vxt_hip_graph_launch(void* ctx, void* graph, uint32_t replays, double* gpu_ms, char* err,
                         size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!graph) fail(VXT_E_ARG, "null graph");
    if (!reg_live(graph)) fail(VXT_E_ARG, "released or unknown graph handle");
    Graph* g = static_cast<Graph*>(graph);
    if (g->ctx != c) fail(VXT_E_ARG, "graph belongs to another context");
    use_device(c);
    VXT_HIP_CHECK(hipEventRecord(c->ev0, c->stream));
    for (uint32_t i = 0; i < replays; ++i) VXT_HIP_CHECK(hipGraphLaunch(g->exec, c->stream));
    VXT_HIP_CHECK(hipEventRecord(c->ev1, c->stream));
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
    float ms = 0.0f;
    VXT_HIP_CHECK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
    c->last_ms = ms;
    if (gpu_ms) *gpu_ms = ms;
  });
}

void vxt_hip_graph_free(void* graph) {
  if (!graph || !reg_take(graph)) return;   // released already (or with its context)
  Graph* g = static_cast<Graph*>(graph);
  {
    std::lock_guard<std::mutex> lk(g->ctx->mu);
    g->ctx->graphs.erase(g);
  }
  release_graph(g);
}

int vxt_hip_last_kernel_ms(void* ctx, double* ms) {
  if (!ctx || !ms || !reg_live(ctx)) return VXT_E_ARG;
  *ms = static_cast<Ctx*>(ctx)->last_ms;
  return VXT_OK;
}

int vxt_hip_set_gemm_path(void* ctx, uint32_t path) {
  if (!ctx || path > VXT_GEMM_LIBRARY || !reg_live(ctx)) return VXT_E_ARG;
  Ctx* c = static_cast<Ctx*>(ctx);
  std::lock_guard<std::mutex> lk(c->mu);
  c->gemm_mode = (int)path;
  return VXT_OK;
}


// ============================================================================
// Decode-step runner (see include/vxt_hip.h): the layer sequence of
// llm_cpu.rs:395-482 over the entry points above, one KV cache per layer,
// and a captured single-token step whose attention reads the position from
// device memory.

// After a captured step: the greedy id and its flag into the history row of
// the step's position, then the position (and rope position) advanced.  One
// thread; the host keeps the position below max_seq.
__global__ void runner_advance_kernel(uint32_t* __restrict__ dpos, const uint32_t* __restrict__ tok,
                                      uint32_t* __restrict__ hist, uint32_t max_seq) {
  if (threadIdx.x != 0) return;
  const uint32_t p = dpos[0];
  if (p < max_seq) {
    hist[2u * p] = tok[0];
    hist[2u * p + 1u] = tok[1];
  }
  dpos[0] = p + 1u;
  dpos[1] = dpos[1] + 1u;
}

namespace {

struct Runner {
  Ctx* ctx = nullptr;
  VxtRunnerConfig cfg{};
  std::vector<VxtRunnerLayer> layers;
  const float* out_norm = nullptr;
  void* head = nullptr;
  void* embed = nullptr;
  void* arena = nullptr;
  float* cur = nullptr;        // [max_batch][hidden] residual stream
  float* cur2 = nullptr;       // [hidden] its other buffer in the single-token step (norms inside GEMVs)
  float* delta = nullptr;      // [max_batch][hidden]
  uint16_t* normed = nullptr;  // [max_batch][hidden] bf16
  float* qkv = nullptr;        // [max_batch][qkv_rows]
  float* attn = nullptr;       // [max_batch][n_head * head_dim]
  uint16_t* act = nullptr;     // [max_batch][ffn] bf16
  float* logits = nullptr;     // [vocab]
  uint32_t* tok_in = nullptr;  // [max_batch] ids of a batched step
  uint32_t* tok = nullptr;     // [2] greedy id and flag; the single-token step embeds tok[0]
  uint32_t* dpos = nullptr;    // [2] position, rope position of the single-token step
  uint32_t* hist = nullptr;    // [max_seq][2] greedy id and flag per position
  std::vector<VxtKvQ8Cache> caches;
  uint32_t q_rows = 0, kvd = 0, qkv_rows = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  uint32_t seed[4] = {};       // host words copied into tok / dpos before a step
};

// A failed entry point call inside the runner: its code and message.
void call_ok(int rc, const char* what, const char* err) {
  if (rc != VXT_OK) fail(rc, std::string(what) + ": " + err);
}

VxtGqaParams runner_params(const Runner& r, uint32_t layer) {
  VxtGqaParams p{};
  p.q_norm = r.layers[layer].q_norm;
  p.k_norm = r.layers[layer].k_norm;
  p.n_head = r.cfg.n_head;
  p.gated_q = r.cfg.gated_q;
  p.rope_dim = r.cfg.rope_dim;
  p.rope_neox = r.cfg.rope_neox;
  p.rope_freq_base = r.cfg.rope_freq_base;
  p.eps = r.cfg.eps;
  return p;
}

// Whether the single-token step builds its two norms per layer inside the
// projections that read them (vxt_hip_norm_matmul_dev: one launch fewer
// each, the residual stream alternating between cur and cur2).
bool runner_fused_norms(const Runner& r) { return r.cfg.hidden <= 4096; }

// The layers and the head for m tokens whose embeddings are in cur; the
// attention at host position pos (m tokens) or, with dpos, at the device
// position (m == 1).  logits of the last token.
void runner_layers(Runner& r, uint32_t m, uint32_t pos, bool device_pos, hipStream_t s) {
  Ctx* c = r.ctx;
  void* ctx = c;
  const VxtRunnerConfig& g = r.cfg;
  char e[256];
  const size_t H = g.hidden;
  const bool fused = m == 1 && runner_fused_norms(r);
  float* res[2] = {r.cur, r.cur2};   // fused: the residual stream, ping-pong
  int rc = 0;
  for (uint32_t l = 0; l < g.n_layers; ++l) {
    const VxtRunnerLayer& L = r.layers[l];
    if (fused) {
      call_ok(vxt_hip_norm_matmul_dev(ctx, L.w_in, res[rc], l ? r.delta : nullptr, L.attn_norm, g.eps,
                                      l ? res[rc ^ 1] : nullptr, VXT_NORM_PLAIN, r.qkv, VXT_DTYPE_F32, r.qkv_rows, s,
                                      e, sizeof e),
              "attention norm + qkv projection", e);
      if (l) rc ^= 1;
    } else {
      call_ok(vxt_hip_rms_norm_dev(ctx, r.cur, l ? r.delta : nullptr, L.attn_norm, r.normed, VXT_DTYPE_BF16,
                                   g.hidden, g.hidden, m, g.eps, s, e, sizeof e),
              "attention norm", e);
      call_ok(vxt_hip_matmul_dev(ctx, L.w_in, r.normed, VXT_DTYPE_BF16, m, r.qkv, VXT_DTYPE_F32, s, e, sizeof e),
              "qkv projection", e);
    }
    const VxtGqaParams p = runner_params(r, l);
    const float* k = r.qkv + r.q_rows;
    const float* v = r.qkv + r.q_rows + r.kvd;
    if (device_pos) {
      const vxt::KvQ8Dev kc = kv_cache_dev(&r.caches[l]);
      vxt::GqaPrep a = gqa_prep_args(kc, &p, r.qkv, r.qkv_rows, k, v, r.qkv_rows, 1, 0, 0);
      a.dpos = r.dpos;
      const hipError_t he = vxt::launch_attn_step(kc, a, p.rope_dim, p.rope_freq_base, r.attn, c->ws, s);
      if (he != hipSuccess) fail(VXT_E_DEVICE, std::string("attention step launch failed: ") + hipGetErrorString(he));
    } else {
      call_ok(vxt_hip_attn_step_q8_dev(ctx, &r.caches[l], &p, r.qkv, r.qkv_rows, k, v, r.qkv_rows, m, pos, pos,
                                       r.attn, s, e, sizeof e),
              "attention", e);
    }
    call_ok(vxt_hip_matmul_dev(ctx, L.w_out, r.attn, VXT_DTYPE_F32, m, r.delta, VXT_DTYPE_F32, s, e, sizeof e),
            "output projection", e);
    if (fused) {
      const uint32_t mode = g.activation == VXT_ACT_GELU_TANH ? VXT_NORM_GLU_GELU_TANH : VXT_NORM_GLU_SILU;
      call_ok(vxt_hip_norm_matmul_dev(ctx, L.w_ffn_gu, res[rc], r.delta, L.post_attn_norm, g.eps, res[rc ^ 1], mode,
                                      r.act, VXT_DTYPE_BF16, g.ffn, s, e, sizeof e),
              "post-attention norm + gated FFN", e);
      rc ^= 1;
    } else {
      call_ok(vxt_hip_rms_norm_dev(ctx, r.cur, r.delta, L.post_attn_norm, r.normed, VXT_DTYPE_BF16, g.hidden,
                                   g.hidden, m, g.eps, s, e, sizeof e),
              "post-attention norm", e);
      call_ok(vxt_hip_ffn_glu_dev(ctx, L.w_ffn_gu, r.normed, VXT_DTYPE_BF16, m, r.act, VXT_DTYPE_BF16, g.ffn,
                                  g.activation, s, e, sizeof e),
              "gated FFN", e);
    }
    call_ok(vxt_hip_matmul_dev(ctx, L.w_ffn_dn, r.act, VXT_DTYPE_BF16, m, r.delta, VXT_DTYPE_F32, s, e, sizeof e),
            "down projection", e);
  }
  // the last token only: its final norm and the head
  float* cur_last = fused ? res[rc] : r.cur + (size_t)(m - 1) * H;
  const float* delta_last = r.delta + (size_t)(m - 1) * H;
  uint16_t* normed_last = r.normed + (size_t)(m - 1) * H;
  call_ok(vxt_hip_rms_norm_dev(ctx, cur_last, g.n_layers ? delta_last : nullptr, r.out_norm, normed_last,
                               VXT_DTYPE_BF16, g.hidden, g.hidden, 1, g.eps, s, e, sizeof e),
          "output norm", e);
  call_ok(vxt_hip_matmul_dev(ctx, r.head, normed_last, VXT_DTYPE_BF16, 1, r.logits, VXT_DTYPE_F32, s, e, sizeof e),
          "head", e);
}

// The single-token step as captured: embedding of tok[0], the layers at the
// device position, the head, the greedy id into tok, the history row and the
// position advanced.
void runner_enqueue_token(Runner& r, hipStream_t s) {
  char e[256];
  call_ok(vxt_hip_embed_dev(r.ctx, r.embed, r.tok, 1, r.cfg.embed_scale, r.cur, r.cfg.hidden, s, e, sizeof e),
          "embedding", e);
  runner_layers(r, 1, 0, true, s);
  call_ok(vxt_hip_greedy_dev(r.ctx, r.logits, r.cfg.vocab, r.tok, s, e, sizeof e), "greedy", e);
  hipLaunchKernelGGL(runner_advance_kernel, dim3(1), dim3(64), 0, s, r.dpos, r.tok, r.hist, r.cfg.max_seq);
  const hipError_t he = hipGetLastError();
  if (he != hipSuccess) fail(VXT_E_DEVICE, std::string("runner advance launch failed: ") + hipGetErrorString(he));
}

void release_runner(Runner* r) {
  (void)hipSetDevice(r->ctx->device);
  (void)hipStreamSynchronize(r->ctx->stream);
  if (r->exec) (void)hipGraphExecDestroy(r->exec);
  if (r->graph) (void)hipGraphDestroy(r->graph);
  if (r->arena) (void)hipFree(r->arena);
  delete r;
}

Runner* as_runner(void* p) {
  if (!p) fail(VXT_E_ARG, "null runner handle");
  if (!reg_live(p)) fail(VXT_E_ARG, "destroyed or unknown runner handle");
  return static_cast<Runner*>(p);
}

// Puts the host position into dpos (both words) and the token into tok[0].
void runner_seed(Runner& r, uint32_t token, uint32_t pos) {
  r.seed[0] = token;
  r.seed[1] = 0u;
  r.seed[2] = pos;
  r.seed[3] = pos;
  VXT_HIP_CHECK(hipMemcpyAsync(r.tok, r.seed, 2 * sizeof(uint32_t), hipMemcpyHostToDevice, r.ctx->stream));
  VXT_HIP_CHECK(hipMemcpyAsync(r.dpos, r.seed + 2, 2 * sizeof(uint32_t), hipMemcpyHostToDevice, r.ctx->stream));
}

}  // namespace

void* vxt_hip_runner_create(void* ctx, const VxtRunnerConfig* cfg, const VxtRunnerLayer* layers,
                            const float* output_norm, void* lm_head, void* embed, char* err, size_t err_cap) {
  Runner* out = nullptr;
  guarded(err, err_cap, [&] {
    Ctx* c = as_ctx(ctx);
    if (!cfg || (!layers && cfg->n_layers)) fail(VXT_E_ARG, "null config or layers");
    if (!output_norm) fail(VXT_E_ARG, "null output norm");
    const VxtRunnerConfig g = *cfg;
    if (g.hidden == 0 || g.n_head == 0 || g.n_kv == 0 || g.ffn == 0 || g.vocab == 0 || g.max_seq == 0 ||
        g.max_batch == 0)
      fail(VXT_E_SHAPE, "hidden, n_head, n_kv, ffn, vocab, max_seq and max_batch must be positive");
    if (g.head_dim != 32 && g.head_dim != 64 && g.head_dim != 128 && g.head_dim != 256)
      fail(VXT_E_UNSUPPORTED, "head_dim must be 32, 64, 128 or 256");
    if (g.n_head % g.n_kv != 0) fail(VXT_E_SHAPE, "n_head must be a multiple of n_kv");
    if (g.n_head / g.n_kv > 8) fail(VXT_E_UNSUPPORTED, "at most 8 query heads per kv head");
    if (g.gated_q > 1 || g.rope_neox > 1 || g.activation > VXT_ACT_GELU_TANH)
      fail(VXT_E_ARG, "gated_q, rope_neox or activation out of range");
    if (g.max_batch > 65535 || g.max_seq > (1u << 24)) fail(VXT_E_SHAPE, "max_batch or max_seq too large");
    if (!(g.eps >= 0.0f) || !std::isfinite(g.rope_freq_base) || !std::isfinite(g.embed_scale))
      fail(VXT_E_ARG, "eps, rope_freq_base or embed_scale out of range");
    auto shape = [&](void* h, uint32_t rows, uint32_t cols, const char* what) {
      Tensor* t = as_tensor(h);
      if (t->ctx != c) fail(VXT_E_ARG, std::string(what) + " belongs to another context");
      if (t->rows != rows || t->cols != cols) fail(VXT_E_SHAPE, std::string(what) + " has the wrong shape");
    };
    const uint32_t q_rows = g.n_head * g.head_dim * (g.gated_q ? 2u : 1u);
    const uint32_t kvd = g.n_kv * g.head_dim, attn_w = g.n_head * g.head_dim;
    for (uint32_t l = 0; l < g.n_layers; ++l) {
      const VxtRunnerLayer& L = layers[l];
      shape(L.w_in, q_rows + 2u * kvd, g.hidden, "w_in");
      shape(L.w_out, g.hidden, attn_w, "w_out");
      shape(L.w_ffn_gu, 2u * g.ffn, g.hidden, "w_ffn_gu");
      shape(L.w_ffn_dn, g.hidden, g.ffn, "w_ffn_dn");
      if (!L.attn_norm || !L.post_attn_norm) fail(VXT_E_ARG, "null layer norm");
    }
    shape(lm_head, g.vocab, g.hidden, "lm_head");
    {
      Tensor* t = as_tensor(embed);
      if (t->ctx != c) fail(VXT_E_ARG, "embed belongs to another context");
      if (t->cols != g.hidden) fail(VXT_E_SHAPE, "embed width != hidden");
    }
    use_device(c);
    std::unique_ptr<Runner> r(new Runner());
    r->ctx = c;
    r->cfg = g;
    r->layers.assign(layers, layers + g.n_layers);
    r->out_norm = output_norm;
    r->head = lm_head;
    r->embed = embed;
    r->q_rows = q_rows;
    r->kvd = kvd;
    r->qkv_rows = q_rows + 2u * kvd;
    // One arena: activations, ids, then per layer K / V values and scales.
    const size_t B = g.max_batch;
    size_t off = 0;
    auto take = [&](size_t bytes) {
      const size_t o = off;
      off += align256(bytes);
      return o;
    };
    const size_t o_cur = take(B * g.hidden * 4), o_cur2 = take((size_t)g.hidden * 4);
    const size_t o_delta = take(B * g.hidden * 4), o_normed = take(B * g.hidden * 2);
    const size_t o_qkv = take(B * r->qkv_rows * 4), o_attn = take(B * attn_w * 4), o_act = take(B * g.ffn * 2);
    const size_t o_logits = take((size_t)g.vocab * 4), o_tin = take(B * 4), o_tok = take(8), o_dpos = take(8);
    const size_t o_hist = take((size_t)g.max_seq * 8);
    std::vector<size_t> o_kv(4 * (size_t)g.n_layers);
    for (uint32_t l = 0; l < g.n_layers; ++l) {
      o_kv[4 * l] = take((size_t)g.max_seq * kvd);
      o_kv[4 * l + 1] = take((size_t)g.max_seq * (kvd / 32) * 2);
      o_kv[4 * l + 2] = take((size_t)g.max_seq * kvd);
      o_kv[4 * l + 3] = take((size_t)g.max_seq * (kvd / 32) * 2);
    }
    VXT_HIP_CHECK(hipMalloc(&r->arena, off));
    VXT_HIP_CHECK(hipMemsetAsync(r->arena, 0, off, c->stream));
    char* base = static_cast<char*>(r->arena);
    r->cur = reinterpret_cast<float*>(base + o_cur);
    r->cur2 = reinterpret_cast<float*>(base + o_cur2);
    r->delta = reinterpret_cast<float*>(base + o_delta);
    r->normed = reinterpret_cast<uint16_t*>(base + o_normed);
    r->qkv = reinterpret_cast<float*>(base + o_qkv);
    r->attn = reinterpret_cast<float*>(base + o_attn);
    r->act = reinterpret_cast<uint16_t*>(base + o_act);
    r->logits = reinterpret_cast<float*>(base + o_logits);
    r->tok_in = reinterpret_cast<uint32_t*>(base + o_tin);
    r->tok = reinterpret_cast<uint32_t*>(base + o_tok);
    r->dpos = reinterpret_cast<uint32_t*>(base + o_dpos);
    r->hist = reinterpret_cast<uint32_t*>(base + o_hist);
    for (uint32_t l = 0; l < g.n_layers; ++l)
      r->caches.push_back(VxtKvQ8Cache{base + o_kv[4 * l], base + o_kv[4 * l + 1], base + o_kv[4 * l + 2],
                                       base + o_kv[4 * l + 3], g.max_seq, g.n_kv, g.head_dim, 0});
    // The single-token step's attention partial sums for the whole cache,
    // then the capture (nothing in it allocates).
    ensure_ws(c, vxt::attn_workspace_bytes(g.n_head, g.max_seq, g.n_kv, g.head_dim, 1), c->stream);
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
    if (c->capturing) fail(VXT_E_ARG, "a capture is in progress on this context");
    VXT_HIP_CHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    try {
      runner_enqueue_token(*r, c->stream);
    } catch (...) {
      c->capturing = false;
      hipGraph_t junk = nullptr;
      (void)hipStreamEndCapture(c->stream, &junk);
      if (junk) (void)hipGraphDestroy(junk);
      (void)hipFree(r->arena);
      r->arena = nullptr;
      throw;
    }
    c->capturing = false;
    VXT_HIP_CHECK(hipStreamEndCapture(c->stream, &r->graph));
    const hipError_t ie = hipGraphInstantiate(&r->exec, r->graph, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
      (void)hipGraphDestroy(r->graph);
      (void)hipFree(r->arena);
      fail(VXT_E_DEVICE, std::string("hipGraphInstantiate failed: ") + hipGetErrorString(ie));
    }
    out = r.release();
    {
      std::lock_guard<std::mutex> lk(c->mu);
      c->runners.insert(out);
    }
    reg_add(out);
  });
  return out;
}

int vxt_hip_runner_step(void* runner, const uint32_t* tok_ids, uint32_t batch_m, uint32_t pos_base,
                        float* logits_out, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Runner* r = as_runner(runner);
    Ctx* c = r->ctx;
    const VxtRunnerConfig& g = r->cfg;
    if (!tok_ids) fail(VXT_E_ARG, "null token ids");
    if (batch_m == 0 || batch_m > g.max_batch) fail(VXT_E_SHAPE, "need 1 <= batch_m <= max_batch");
    if (pos_base >= g.max_seq || batch_m > g.max_seq - pos_base) fail(VXT_E_SHAPE, "pos_base + batch_m > max_seq");
    for (uint32_t i = 0; i < batch_m; ++i)
      if (tok_ids[i] >= g.vocab) fail(VXT_E_ARG, "token id out of vocabulary range");
    if (c->capturing) fail(VXT_E_ARG, "a capture is in progress on this context");
    use_device(c);
    if (batch_m == 1) {
      runner_seed(*r, tok_ids[0], pos_base);
      VXT_HIP_CHECK(hipGraphLaunch(r->exec, c->stream));
    } else {
      char e[256];
      VXT_HIP_CHECK(hipMemcpyAsync(r->tok_in, tok_ids, (size_t)batch_m * 4, hipMemcpyHostToDevice, c->stream));
      call_ok(vxt_hip_embed_dev(c, r->embed, r->tok_in, batch_m, g.embed_scale, r->cur, g.hidden, c->stream, e,
                                sizeof e),
              "embedding", e);
      runner_layers(*r, batch_m, pos_base, false, c->stream);
    }
    if (logits_out)
      VXT_HIP_CHECK(hipMemcpyAsync(logits_out, r->logits, (size_t)g.vocab * 4, hipMemcpyDeviceToHost, c->stream));
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int vxt_hip_runner_generate(void* runner, uint32_t token, uint32_t pos_base, uint32_t n_steps, uint32_t* tokens_out,
                            uint32_t* flags_out, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    Runner* r = as_runner(runner);
    Ctx* c = r->ctx;
    const VxtRunnerConfig& g = r->cfg;
    if (n_steps == 0) return;
    if (!tokens_out) fail(VXT_E_ARG, "null tokens_out");
    if (token >= g.vocab) fail(VXT_E_ARG, "token id out of vocabulary range");
    if (pos_base >= g.max_seq || n_steps > g.max_seq - pos_base) fail(VXT_E_SHAPE, "pos_base + n_steps > max_seq");
    if (c->capturing) fail(VXT_E_ARG, "a capture is in progress on this context");
    use_device(c);
    runner_seed(*r, token, pos_base);
    for (uint32_t i = 0; i < n_steps; ++i) VXT_HIP_CHECK(hipGraphLaunch(r->exec, c->stream));
    std::vector<uint32_t> h(2 * (size_t)n_steps);
    VXT_HIP_CHECK(hipMemcpyAsync(h.data(), r->hist + 2 * (size_t)pos_base, h.size() * 4, hipMemcpyDeviceToHost,
                                 c->stream));
    VXT_HIP_CHECK(hipStreamSynchronize(c->stream));
    for (uint32_t i = 0; i < n_steps; ++i) {
      tokens_out[i] = h[2 * i];
      if (flags_out) flags_out[i] = h[2 * i + 1];
    }
  });
}

void vxt_hip_runner_destroy(void* runner) {
  if (!runner || !reg_take(runner)) return;   // released already (or with its context)
  Runner* r = static_cast<Runner*>(runner);
  {
    std::lock_guard<std::mutex> lk(r->ctx->mu);
    r->ctx->runners.erase(r);
  }
  release_runner(r);
}

}  // extern "C"
