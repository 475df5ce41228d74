// gemv.hip -- dispatch of the decode GEMV (batch_m 1..8) by weight kind.
// The kernels live in gemv_impl.hpp and are instantiated in gemv_{q8,q40,cb4,g64}.hip.
#include "common.hpp"

namespace vxt {

hipError_t launch_gemv_q8(const DevTensor&, const void*, bool, uint32_t, void*, bool, hipStream_t);
hipError_t launch_gemv_q40(const DevTensor&, const void*, bool, uint32_t, void*, bool, hipStream_t);
hipError_t launch_gemv_cb4(const DevTensor&, const void*, bool, uint32_t, void*, bool, hipStream_t);
hipError_t launch_gemv_g64(const DevTensor&, const void*, bool, uint32_t, void*, bool, hipStream_t);
hipError_t launch_norm_q8(const DevTensor&, const NormIn&, int, void*, bool, uint32_t, hipStream_t);
hipError_t launch_norm_q40(const DevTensor&, const NormIn&, int, void*, bool, uint32_t, hipStream_t);
hipError_t launch_norm_cb4(const DevTensor&, const NormIn&, int, void*, bool, uint32_t, hipStream_t);
hipError_t launch_norm_g64(const DevTensor&, const NormIn&, int, void*, bool, uint32_t, hipStream_t);
hipError_t launch_glu_q8(const DevTensor&, const void*, bool, uint32_t, uint32_t, void*, bool, uint32_t, bool,
                         hipStream_t);
hipError_t launch_glu_q40(const DevTensor&, const void*, bool, uint32_t, uint32_t, void*, bool, uint32_t, bool,
                          hipStream_t);
hipError_t launch_glu_cb4(const DevTensor&, const void*, bool, uint32_t, uint32_t, void*, bool, uint32_t, bool,
                          hipStream_t);
hipError_t launch_glu_g64(const DevTensor&, const void*, bool, uint32_t, uint32_t, void*, bool, uint32_t, bool,
                          hipStream_t);

// x_vec (x rows 16-byte aligned) is accepted for the ABI layer; the kernels
// stage activations through LDS or read them element-wise.
hipError_t launch_gemv(const DevTensor& t, const void* x, bool x_bf16, bool x_vec, uint32_t m, void* y,
                       bool y_bf16, hipStream_t s) {
  (void)x_vec;
  switch (t.kind) {
    case KIND_Q8: return launch_gemv_q8(t, x, x_bf16, m, y, y_bf16, s);
    case KIND_Q40: return launch_gemv_q40(t, x, x_bf16, m, y, y_bf16, s);
    case KIND_CB4: return launch_gemv_cb4(t, x, x_bf16, m, y, y_bf16, s);
    case KIND_G64: return launch_gemv_g64(t, x, x_bf16, m, y, y_bf16, s);
    default: return hipErrorInvalidValue;
  }
}

// Gated gate/up GEMV (batch_m 1..8): t is [gate; up] with t.rows = 2 * n_ff.
hipError_t launch_gemv_glu(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* act, bool act_bf16,
                           uint32_t act_stride, bool gelu, hipStream_t s) {
  const uint32_t n_ff = t.rows / 2;
  switch (t.kind) {
    case KIND_Q8: return launch_glu_q8(t, x, x_bf16, m, n_ff, act, act_bf16, act_stride, gelu, s);
    case KIND_Q40: return launch_glu_q40(t, x, x_bf16, m, n_ff, act, act_bf16, act_stride, gelu, s);
    case KIND_CB4: return launch_glu_cb4(t, x, x_bf16, m, n_ff, act, act_bf16, act_stride, gelu, s);
    case KIND_G64: return launch_glu_g64(t, x, x_bf16, m, n_ff, act, act_bf16, act_stride, gelu, s);
    default: return hipErrorInvalidValue;
  }
}

// Batch-1 GEMV whose x is bf16(rms_norm(cur [+ delta]) * w), built in each
// workgroup.  epi 0: y = W x; 1 / 2: gated SiLU / GELU-tanh over [gate; up].
hipError_t launch_gemv_norm(const DevTensor& t, const NormIn& nin, int epi, void* y, bool y_bf16, uint32_t y_stride,
                            hipStream_t s) {
  switch (t.kind) {
    case KIND_Q8: return launch_norm_q8(t, nin, epi, y, y_bf16, y_stride, s);
    case KIND_Q40: return launch_norm_q40(t, nin, epi, y, y_bf16, y_stride, s);
    case KIND_CB4: return launch_norm_cb4(t, nin, epi, y, y_bf16, y_stride, s);
    case KIND_G64: return launch_norm_g64(t, nin, epi, y, y_bf16, y_stride, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vxt
