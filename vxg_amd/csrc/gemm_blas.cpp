// gemm_blas.cpp -- the dense phase of the two-phase prefill GEMM on
// hipBLASLt, for the pinned comparison path only.
//
// Built as its own shared library (libvxt_hip_blas.so, next to
// libvxt_hip.so), which libvxt_hip.so opens the first time a caller runs the
// pinned library path (blas_plugin.cpp): the matmul library itself does not
// link or load hipBLASLt.
//
// Once the weights are decoded into an f16 panel (gemm_panel.hip), what is
// left is a plain f16 x f16 -> f32 GEMM, D[M][N] = alpha * A[M][K] * B[N][K]^T
// + beta * D, both operands K-contiguous.  Column-major, that is
// D^T (N x M) = op_T(B as K x N) * (A as K x M): hipBLASLt's "TN" case.
// Handles are per device; the descriptors and the heuristic's first
// algorithm are cached per shape.  A call can also split K into `batch`
// equal slices run as one strided batch (slice b of A and B starts b * K
// columns in, its D is the b-th M x N block), so a product with few output
// tiles still fills the GPU; the caller adds the blocks.  No workspace is offered to the library, so
// the algorithms it picks never clear one (a clearing node recorded into a
// captured graph is not replayed reliably on this platform).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace vxt {

namespace {

struct Entry {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

using Key = std::tuple<int, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t>;   // device, M, N, K, lda, ldb, batch

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<Key, Entry> g_entries;
constexpr size_t kMaxEntries = 512;

void destroy_entry(Entry& en) {
  if (en.ld) hipblasLtMatrixLayoutDestroy(en.ld);
  if (en.lb) hipblasLtMatrixLayoutDestroy(en.lb);
  if (en.la) hipblasLtMatrixLayoutDestroy(en.la);
  if (en.op) hipblasLtMatmulDescDestroy(en.op);
}

hipError_t status(hipblasStatus_t st) {
  if (st == HIPBLAS_STATUS_SUCCESS) return hipSuccess;
  return st == HIPBLAS_STATUS_NOT_SUPPORTED ? hipErrorNotSupported : hipErrorUnknown;
}

// The cached entry for this shape on the current device (created on first
// use, outside any capture: the caller's eager call sizes the workspace
// before a capture is allowed).
hipError_t entry_for(int dev, uint32_t M, uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb, uint32_t batch,
                     hipblasLtHandle_t* h, const Entry** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto hi = g_handles.find(dev);
  if (hi == g_handles.end()) {
    hipblasLtHandle_t nh = nullptr;
    hipError_t e = status(hipblasLtCreate(&nh));
    if (e != hipSuccess) return e;
    hi = g_handles.emplace(dev, nh).first;
  }
  *h = hi->second;
  const Key key{dev, M, N, K, lda, ldb, batch};
  auto it = g_entries.find(key);
  if (it != g_entries.end()) {
    *out = &it->second;
    return hipSuccess;
  }
  if (g_entries.size() >= kMaxEntries) return hipErrorNotSupported;
  Entry en;
  hipError_t e = status(hipblasLtMatmulDescCreate(&en.op, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (e == hipSuccess)
    e = status(hipblasLtMatmulDescSetAttribute(en.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
  if (e == hipSuccess)
    e = status(hipblasLtMatmulDescSetAttribute(en.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
  if (e == hipSuccess) e = status(hipblasLtMatrixLayoutCreate(&en.la, HIP_R_16F, K, N, ldb));   // weights
  if (e == hipSuccess) e = status(hipblasLtMatrixLayoutCreate(&en.lb, HIP_R_16F, K, M, lda));   // activations
  if (e == hipSuccess) e = status(hipblasLtMatrixLayoutCreate(&en.ld, HIP_R_32F, N, M, N));
  if (batch > 1) {
    const int32_t bc = (int32_t)batch;
    const int64_t kstride = K, dstride = (int64_t)M * N;
    for (hipblasLtMatrixLayout_t l : {en.la, en.lb, en.ld}) {
      const int64_t stride = l == en.ld ? dstride : kstride;
      if (e == hipSuccess)
        e = status(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc)));
      if (e == hipSuccess)
        e = status(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &stride,
                                                     sizeof(stride)));
    }
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  if (e == hipSuccess) e = status(hipblasLtMatmulPreferenceCreate(&pref));
  const uint64_t no_ws = 0;
  if (e == hipSuccess)
    e = status(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_ws,
                                                     sizeof(no_ws)));
  hipblasLtMatmulHeuristicResult_t res{};
  int nres = 0;
  if (e == hipSuccess) e = status(hipblasLtMatmulAlgoGetHeuristic(*h, en.op, en.la, en.lb, en.ld, en.ld, pref, 1,
                                                                  &res, &nres));
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (e == hipSuccess && nres < 1) e = hipErrorNotSupported;
  if (e != hipSuccess) {
    destroy_entry(en);
    return e;
  }
  en.algo = res.algo;
  *out = &g_entries.emplace(key, en).first->second;
  return hipSuccess;
}

}  // namespace

}  // namespace vxt

// Releases the library handle and cached descriptors of a device; called by
// libvxt_hip.so when the last context on that device is destroyed (the
// handle is shared by the device's contexts).
extern "C" __attribute__((visibility("default"))) void vxt_blas_release_device(int dev) {
  using namespace vxt;
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto it = g_entries.begin(); it != g_entries.end();) {
    if (std::get<0>(it->first) == dev) {
      destroy_entry(it->second);
      it = g_entries.erase(it);
    } else {
      ++it;
    }
  }
  auto h = g_handles.find(dev);
  if (h != g_handles.end()) {
    int cur = 0;
    const bool restore = hipGetDevice(&cur) == hipSuccess;
    (void)hipSetDevice(dev);
    hipblasLtDestroy(h->second);
    g_handles.erase(h);
    if (restore) (void)hipSetDevice(cur);
  }
}

// D_b[M][N] (f32, row-major; block b at D + b * M * N) = alpha * A_b[M][K] *
// B_b[N][K]^T + beta * D_b for b < batch, where A_b and B_b are the columns
// [b K, (b + 1) K) of A and B (f16 row-major, row strides lda, ldb elements).
extern "C" __attribute__((visibility("default"))) hipError_t vxt_blas_gemm_f16_tn(
    const uint16_t* A, uint32_t lda, const uint16_t* B, uint32_t ldb, uint32_t M, uint32_t N, uint32_t K,
    uint32_t batch, float alpha, float beta, float* D, hipStream_t s) {
  using namespace vxt;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipblasLtHandle_t h = nullptr;
  const Entry* en = nullptr;
  e = entry_for(dev, M, N, K, lda, ldb, batch, &h, &en);
  if (e != hipSuccess) return e;
  return status(hipblasLtMatmul(h, en->op, &alpha, B, en->la, A, en->lb, &beta, D, en->ld, D, en->ld, &en->algo,
                                nullptr, 0, s));
}
