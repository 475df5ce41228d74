// gemm.hip -- prefill dequantise + GEMM (batch_m > 8): MFMA kernels go here.
#include "common.hpp"

namespace vxt {

hipError_t launch_gemm(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y,
                       bool y_bf16, hipStream_t s) {
  (void)t; (void)x; (void)x_bf16; (void)m; (void)y; (void)y_bf16; (void)s;
  return hipErrorNotSupported;
}

}  // namespace vxt
