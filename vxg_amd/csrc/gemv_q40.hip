// gemv_q40.hip -- instantiates the decode GEMV (gemv_impl.hpp) for one
// weight kind, so the kinds compile in parallel.
#include "gemv_impl.hpp"

namespace vxt {

hipError_t launch_gemv_q40(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y,
                        bool y_bf16, hipStream_t s) {
  return gv::launch_kind<KIND_Q40>(t, x, x_bf16, m, y, y_bf16, s);
}

hipError_t launch_glu_q40(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, uint32_t n_ff, void* y,
                        bool y_bf16, uint32_t y_stride, bool gelu, hipStream_t s) {
  return gv::launch_glu_kind<KIND_Q40>(t, x, x_bf16, m, n_ff, y, y_bf16, y_stride, gelu, s);
}

hipError_t launch_norm_q40(const DevTensor& t, const NormIn& nin, int epi, void* y, bool y_bf16,
                         uint32_t y_stride, hipStream_t s) {
  return gv::launch_norm_kind<KIND_Q40>(t, nin, epi, y, y_bf16, y_stride, s);
}

}  // namespace vxt
