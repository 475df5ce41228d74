// ffn.hip -- element-wise FFN activation and the residual-add + RMSNorm of
// the decode step.
//
// glu_act_kernel: act[m][i] = act(gu[m][i]) * gu[m][n_ff + i] for i < n_ff,
//   zero for n_ff <= i < act_stride: the activation pass of the device
//   runner (vxt_cb4_swiglu_batch, vxt_cb4_fast_ops.metal:236-262) for the
//   batches the fused gate/up GEMV does not take.
//
// rms_norm_kernel: one workgroup per token.
//   with delta:  cur[i] += delta[i] (written back), then
//   out[i] = cur[i] * scale * w[i],  scale = 1 / sqrt(sum(cur^2) / dim + eps)
//   for i < dim, zero for dim <= i < stride -- rms_norm of llm_ops.rs:48-57
//   after the residual add of llm_cpu.rs:443-446 (the runner fuses the two,
//   vxt_cb4_add_rms_norm_batch, vxt_cb4_fast_ops.metal:196-234); without delta,
//   rms_norm alone (vxt_cb4_rms_norm_batch, :160-194).  The sum of squares is
//   an fp32 FMA per element in a different order from the CPU's sequential
//   chain; every other operation rounds as the source does.
#include "act.hpp"
#include "common.hpp"

namespace vxt {

namespace {

constexpr uint32_t kNormThreads = 256;

__global__ __launch_bounds__(256) void glu_act_kernel(const float* __restrict__ gu, uint32_t n_ff, uint32_t gelu,
                                                     void* __restrict__ act, uint32_t act_bf16, uint32_t act_stride) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  const uint32_t m = blockIdx.y;
  if (i >= act_stride) return;
  float v = 0.0f;
  if (i < n_ff) {
    const float* row = gu + (size_t)m * 2u * n_ff;
    v = gated_act(row[i], row[n_ff + i], gelu != 0);
  }
  const size_t at = (size_t)m * act_stride + i;
  if (act_bf16)
    static_cast<uint16_t*>(act)[at] = f32_to_bf16(v);
  else
    static_cast<float*>(act)[at] = v;
}

// Values stay in registers (NP per thread, dim <= 256 * NP): cur, delta and w
// are all requested before the first use, so the kernel makes one trip to
// memory.  The sum runs in the order described at the top of this file; the
// norm-prologue GEMV (gemv_impl.hpp) repeats it step for step.
template <uint32_t NP>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(float* __restrict__ cur, const float* __restrict__ delta,
                                                                const float* __restrict__ w, void* __restrict__ out,
                                                                uint32_t out_bf16, uint32_t dim, uint32_t stride,
                                                                float eps) {
#pragma clang fp contract(off)
  const uint32_t tid = threadIdx.x;
  float* c = cur + (size_t)blockIdx.x * stride;
  const float* d = delta ? delta + (size_t)blockIdx.x * stride : nullptr;
  float v[NP], dv[NP], wv[NP];
#pragma unroll
  for (uint32_t j = 0; j < NP; ++j) {
    const uint32_t i = tid + kNormThreads * j;
    const uint32_t ic = i < dim ? i : dim - 1;
    v[j] = c[ic];
    wv[j] = w[ic];
    dv[j] = d ? d[ic] : 0.0f;
  }
  float sq = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < NP; ++j) {
    const uint32_t i = tid + kNormThreads * j;
    if (d) v[j] = v[j] + dv[j];
    if (i < dim) {
      if (d) c[i] = v[j];
      sq = __builtin_fmaf(v[j], v[j], sq);
    }
  }
  __shared__ float s_part[kNormThreads / 64];
  sq = wave_sum(sq);
  if ((tid & 63u) == 0) s_part[tid >> 6] = sq;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < kNormThreads / 64; ++k) total += s_part[k];
  const float scale = 1.0f / sqrtf(total / (float)dim + eps);
#pragma unroll
  for (uint32_t j = 0; j < NP; ++j) {
    const uint32_t i = tid + kNormThreads * j;
    if (i >= stride) break;
    const float o = i < dim ? v[j] * scale * wv[j] : 0.0f;
    const size_t at = (size_t)blockIdx.x * stride + i;
    if (out_bf16)
      static_cast<uint16_t*>(out)[at] = f32_to_bf16(o);
    else
      static_cast<float*>(out)[at] = o;
  }
  for (uint32_t i = tid + kNormThreads * NP; i < stride; i += kNormThreads) {   // padding past the held range
    const size_t at = (size_t)blockIdx.x * stride + i;
    if (out_bf16)
      static_cast<uint16_t*>(out)[at] = 0;
    else
      static_cast<float*>(out)[at] = 0.0f;
  }
}

// Any dim: the strided loop (values re-read for the output pass).
__global__ __launch_bounds__(kNormThreads) void rms_norm_wide_kernel(float* __restrict__ cur,
                                                                     const float* __restrict__ delta,
                                                                     const float* __restrict__ w, void* __restrict__ out,
                                                                     uint32_t out_bf16, uint32_t dim, uint32_t stride,
                                                                     float eps) {
#pragma clang fp contract(off)
  const uint32_t tid = threadIdx.x;
  float* c = cur + (size_t)blockIdx.x * stride;
  const float* d = delta ? delta + (size_t)blockIdx.x * stride : nullptr;
  float sq = 0.0f;
  for (uint32_t i = tid; i < dim; i += kNormThreads) {
    float v = c[i];
    if (d) {
      v = v + d[i];
      c[i] = v;
    }
    sq = __builtin_fmaf(v, v, sq);
  }
  __shared__ float s_part[kNormThreads / 64];
  sq = wave_sum(sq);
  if ((tid & 63u) == 0) s_part[tid >> 6] = sq;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < kNormThreads / 64; ++k) total += s_part[k];
  const float scale = 1.0f / sqrtf(total / (float)dim + eps);
  for (uint32_t i = tid; i < stride; i += kNormThreads) {
    const float v = i < dim ? c[i] * scale * w[i] : 0.0f;
    const size_t at = (size_t)blockIdx.x * stride + i;
    if (out_bf16)
      static_cast<uint16_t*>(out)[at] = f32_to_bf16(v);
    else
      static_cast<float*>(out)[at] = v;
  }
}

}  // namespace

hipError_t launch_glu_act(const float* gu, uint32_t m, uint32_t n_ff, bool gelu, void* act, bool act_bf16,
                          uint32_t act_stride, hipStream_t s) {
  if (m == 0 || act_stride == 0) return hipSuccess;
  hipLaunchKernelGGL(glu_act_kernel, dim3((act_stride + 255) / 256, m), dim3(256), 0, s, gu, n_ff,
                     (uint32_t)gelu, act, (uint32_t)act_bf16, act_stride);
  return hipGetLastError();
}

hipError_t launch_rms_norm(float* cur, const float* delta, const float* w, void* out, bool out_bf16, uint32_t dim,
                           uint32_t stride, uint32_t m, float eps, hipStream_t s) {
  if (m == 0) return hipSuccess;
  if (dim <= kNormThreads * 8)
    hipLaunchKernelGGL(rms_norm_kernel<8>, dim3(m), dim3(kNormThreads), 0, s, cur, delta, w, out,
                       (uint32_t)out_bf16, dim, stride, eps);
  else if (dim <= kNormThreads * 16)
    hipLaunchKernelGGL(rms_norm_kernel<16>, dim3(m), dim3(kNormThreads), 0, s, cur, delta, w, out,
                       (uint32_t)out_bf16, dim, stride, eps);
  else
    hipLaunchKernelGGL(rms_norm_wide_kernel, dim3(m), dim3(kNormThreads), 0, s, cur, delta, w, out,
                       (uint32_t)out_bf16, dim, stride, eps);
  return hipGetLastError();
}

}  // namespace vxt
