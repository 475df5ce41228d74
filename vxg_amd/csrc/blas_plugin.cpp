// blas_plugin.cpp -- the pinned library path's access to hipBLASLt.
//
// The dense phase on hipBLASLt (gemm_blas.cpp) is a comparison path that no
// automatic route takes, so it lives in its own shared library,
// libvxt_hip_blas.so, in the directory of libvxt_hip.so.  It is opened the
// first time a caller runs the pinned library path and stays loaded until the
// process ends; a process that never pins it never loads hipBLASLt.  Without
// the plugin the pinned path fails with hipErrorNotSupported (reported as
// VXT_E_UNSUPPORTED by the C ABI).
//
// Contexts register per device here whether or not the plugin is loaded; the
// last context of a device to go releases the plugin's handle for it.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>

namespace vxt {

namespace {

using GemmFn = hipError_t (*)(const uint16_t*, uint32_t, const uint16_t*, uint32_t, uint32_t, uint32_t, uint32_t,
                              uint32_t, float, float, float*, hipStream_t);
using ReleaseFn = void (*)(int);

std::mutex g_mu;
std::map<int, int> g_users;   // contexts alive per device
bool g_tried = false;
GemmFn g_gemm = nullptr;
ReleaseFn g_release = nullptr;

// The plugin's path: libvxt_hip_blas.so beside the library holding this code.
std::string plugin_path() {
  Dl_info info{};
  if (!dladdr(reinterpret_cast<void*>(&plugin_path), &info) || !info.dli_fname) return "libvxt_hip_blas.so";
  std::string p = info.dli_fname;
  const size_t slash = p.rfind('/');
  return (slash == std::string::npos ? std::string() : p.substr(0, slash + 1)) + "libvxt_hip_blas.so";
}

// Called with g_mu held.
void load_locked() {
  if (g_tried) return;
  g_tried = true;
  void* h = dlopen(plugin_path().c_str(), RTLD_NOW | RTLD_LOCAL);
  if (!h) return;
  g_gemm = reinterpret_cast<GemmFn>(dlsym(h, "vxt_blas_gemm_f16_tn"));
  g_release = reinterpret_cast<ReleaseFn>(dlsym(h, "vxt_blas_release_device"));
  if (!g_gemm || !g_release) {
    g_gemm = nullptr;
    g_release = nullptr;
  }
}

}  // namespace

void blas_acquire_device(int dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  ++g_users[dev];
}

void blas_release_device(int dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto u = g_users.find(dev);
  if (u == g_users.end() || --u->second > 0) return;
  g_users.erase(u);
  if (g_release) g_release(dev);
}

// D_b[M][N] (f32, row-major; block b at D + b * M * N) = alpha * A_b[M][K] *
// B_b[N][K]^T + beta * D_b for b < batch, where A_b and B_b are the columns
// [b K, (b + 1) K) of A and B (f16 row-major, row strides lda, ldb elements),
// on hipBLASLt through the plugin.
hipError_t blas_gemm_f16_tn(const uint16_t* A, uint32_t lda, const uint16_t* B, uint32_t ldb, uint32_t M, uint32_t N,
                            uint32_t K, uint32_t batch, float alpha, float beta, float* D, hipStream_t s) {
  GemmFn fn;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    load_locked();
    fn = g_gemm;
  }
  if (!fn) return hipErrorNotSupported;
  return fn(A, lda, B, ldb, M, N, K, batch, alpha, beta, D, s);
}

}  // namespace vxt
