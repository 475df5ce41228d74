// dequant.hip -- bit-exact dequantisation of resident weights to f32 rows.
//
// The probe the reference uses to prove GPU dequant matches decode_row bit
// for bit (vxt_embedding_cb4_exact, vxt_llm_ops.metal:547-567, checked by
// metal_llm_tests.rs:95-139).  Values:
//   CB4: dst[c] = f32(sc) * cent[q] (one f32 rounding, no contraction), then
//        the row's CSR residuals added in CSR order for col < cols
//        (codebook.rs:285-337);
//   Q8:  dst[c] = (float)q * f32(d)                (gguf.rs:223-229, exact);
//   Q4_0: dst[c] = (float)(q - 8) * f32(d)         (q4_0.rs:89-93, exact);
//   G64: dst[c] = f32(lut[q])                      (exact).
// f16 scales and tables are widened with the integer rule of fp16.rs:6-29 so
// NaN payloads match as well.
#include "common.hpp"

namespace vxt {

#pragma clang fp contract(off)

__global__ __launch_bounds__(256) void dequant_dense_kernel(DevTensor t, uint32_t row0, uint32_t nrows,
                                                           float* __restrict__ out) {
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  const uint32_t rr = blockIdx.y;
  if (c >= t.cols || rr >= nrows) return;
  const size_t row = (size_t)row0 + rr;
  float v;
  if (t.kind == KIND_Q8) {
    const int8_t q = static_cast<const int8_t*>(t.p0)[row * t.kp + c];
    v = (float)q * f16_to_f32_exact(t.p1[row * (t.kp / 32) + c / 32]);
  } else if (t.kind == KIND_Q40) {   // q4_0.rs:89-93: ((nibble as i32) - 8) as f32 * d
    const uint8_t b = static_cast<const uint8_t*>(t.p0)[row * (t.kp / 2) + (c / 32) * 16 + c % 16];
    const int32_t q = (int32_t)((c % 32 < 16 ? b : b >> 4) & 0xfu) - 8;
    v = (float)q * f16_to_f32_exact(t.p1[row * (t.kp / 32) + c / 32]);
  } else if (t.kind == KIND_CB4) {
    const uint32_t w = static_cast<const uint32_t*>(t.p0)[row * (t.kp / 8) + c / 8];
    const uint32_t q = (w >> ((c % 8) * 4)) & 0xfu;
    const float sc = f16_to_f32_exact(t.p1[row * (t.kp / 128) + c / 128]);
    v = sc * t.cent[16u * cent_table(t, row) + q];
  } else {
    const uint8_t b = static_cast<const uint8_t*>(t.p0)[row * (t.kp / 2) + c / 2];
    const uint32_t q = (b >> ((c & 1) * 4)) & 0xfu;
    v = f16_to_f32_exact(t.p1[(row * (t.kp / 64) + c / 64) * 16 + q]);
  }
  out[(size_t)rr * t.cols + c] = v;
}

// One thread per row walks that row's CSR range in order, so duplicate
// columns accumulate in the reference's order.
__global__ __launch_bounds__(256) void dequant_outlier_kernel(DevTensor t, uint32_t row0,
                                                             uint32_t nrows, float* __restrict__ out) {
  const uint32_t rr = blockIdx.x * 256 + threadIdx.x;
  if (rr >= nrows) return;
  const uint32_t row = row0 + rr;
  const uint32_t os = t.row_ptr[row], oe = t.row_ptr[row + 1];
  float* dst = out + (size_t)rr * t.cols;
  for (uint32_t i = os; i < oe; ++i) {
    const uint32_t pk = t.outliers[i];
    const uint32_t col = pk & 0xffffu;
    if (col < t.cols) dst[col] = dst[col] + f16_to_f32_exact(pk >> 16);
  }
}

// Embedding gather: out[m][c] = decode_row(token m)[c] (times embed_scale when
// scale_on), zero for cols <= c < stride.  Token ids come from device memory;
// an id past the last row reads the last row.  One thread per element;
// a cb4 element adds every CSR residual of its row that names its column, in
// CSR order (the per-element form of vxt_cb4_embed_exact_batch,
// vxt_cb4_fast_ops.metal:22-113), so the scale multiply follows the full
// decode as in llm_cpu.rs:224-229.
__global__ __launch_bounds__(256) void embed_kernel(DevTensor t, const uint32_t* __restrict__ tokens, uint32_t stride,
                                                   float scale, uint32_t scale_on, float* __restrict__ out) {
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  const uint32_t m = blockIdx.y;
  if (c >= stride) return;
  float* dst = out + (size_t)m * stride;
  if (c >= t.cols) {
    dst[c] = 0.0f;
    return;
  }
  const size_t row = min(tokens[m], t.rows - 1u);
  float v;
  if (t.kind == KIND_Q8) {
    const int8_t q = static_cast<const int8_t*>(t.p0)[row * t.kp + c];
    v = (float)q * f16_to_f32_exact(t.p1[row * (t.kp / 32) + c / 32]);
  } else if (t.kind == KIND_Q40) {   // q4_0.rs:89-93: ((nibble as i32) - 8) as f32 * d
    const uint8_t b = static_cast<const uint8_t*>(t.p0)[row * (t.kp / 2) + (c / 32) * 16 + c % 16];
    const int32_t q = (int32_t)((c % 32 < 16 ? b : b >> 4) & 0xfu) - 8;
    v = (float)q * f16_to_f32_exact(t.p1[row * (t.kp / 32) + c / 32]);
  } else if (t.kind == KIND_CB4) {
    const uint32_t w = static_cast<const uint32_t*>(t.p0)[row * (t.kp / 8) + c / 8];
    const uint32_t q = (w >> ((c % 8) * 4)) & 0xfu;
    const float sc = f16_to_f32_exact(t.p1[row * (t.kp / 128) + c / 128]);
    v = sc * t.cent[16u * cent_table(t, (uint32_t)row) + q];
    const uint32_t os = t.row_ptr[row], oe = t.row_ptr[row + 1];
    for (uint32_t i = os; i < oe; ++i) {
      const uint32_t pk = t.outliers[i];
      if ((pk & 0xffffu) == c) v = v + f16_to_f32_exact(pk >> 16);
    }
  } else {
    const uint8_t b = static_cast<const uint8_t*>(t.p0)[row * (t.kp / 2) + c / 2];
    const uint32_t q = (b >> ((c & 1) * 4)) & 0xfu;
    v = f16_to_f32_exact(t.p1[(row * (t.kp / 64) + c / 64) * 16 + q]);
  }
  dst[c] = scale_on ? v * scale : v;
}

hipError_t launch_embed(const DevTensor& t, const uint32_t* tokens, uint32_t batch_m, float scale, bool scale_on,
                        float* out, uint32_t stride, hipStream_t s) {
  if (batch_m == 0 || stride == 0) return hipSuccess;
  hipLaunchKernelGGL(embed_kernel, dim3((stride + 255) / 256, batch_m), dim3(256), 0, s, t, tokens, stride, scale,
                     (uint32_t)scale_on, out);
  return hipGetLastError();
}

hipError_t launch_dequant(const DevTensor& t, uint32_t row0, uint32_t nrows, float* out,
                          hipStream_t s) {
  if (nrows == 0) return hipSuccess;
  dim3 grid((t.cols + 255) / 256, nrows);
  hipLaunchKernelGGL(dequant_dense_kernel, grid, dim3(256), 0, s, t, row0, nrows, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || t.kind != KIND_CB4) return e;
  hipLaunchKernelGGL(dequant_outlier_kernel, dim3((nrows + 255) / 256), dim3(256), 0, s, t, row0,
                     nrows, out);
  return hipGetLastError();
}

}  // namespace vxt
