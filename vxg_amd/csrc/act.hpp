// act.hpp -- the FFN activations of the reference's CPU decode step, in f32
// with the source's rounding order (no contraction into FMA):
//   silu(x)       = x / (1 + exp(-x))                       (llm_ops.rs:39-41)
//   gelu_tanh(g)  = 0.5 g (1 + tanh(0.7978846 (g + 0.044715 g^3))), tanh via
//                   e2 = exp(-2|z|), (1 - e2) / (1 + e2) with z's sign
//                                                           (llm_prefill.rs:66-71)
//   gated(g, u)   = act(g) * u                              (llm_cpu.rs:457-464)
// exp is the device library's expf (not the fast approximation).
#pragma once
#include <hip/hip_runtime.h>

namespace vxt {

__device__ __forceinline__ float silu_f32(float g) {
#pragma clang fp contract(off)
  return g / (1.0f + expf(-g));
}

__device__ __forceinline__ float gelu_tanh_f32(float g) {
#pragma clang fp contract(off)
  const float z = 0.7978846f * (g + 0.044715f * g * g * g);
  const float e2 = expf(-2.0f * fabsf(z));
  const float th = copysignf((1.0f - e2) / (1.0f + e2), z);
  return 0.5f * g * (1.0f + th);
}

__device__ __forceinline__ float gated_act(float g, float u, bool gelu) {
#pragma clang fp contract(off)
  return (gelu ? gelu_tanh_f32(g) : silu_f32(g)) * u;
}

}  // namespace vxt
