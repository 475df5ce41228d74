// probe.hip -- the HBM streaming floor: a kernel that only reads.
//
// Every 16-byte piece of [p, p + bytes) is read once with a non-temporal
// load, one wave reading one contiguous KiB per load instruction, all of a
// wave's loads issued before the first wait -- the access pattern of the
// decode GEMV without its arithmetic.  Timed at a GEMV's size (and with the
// same weight-copy rotation), it is the floor a single launch of that size
// can reach on this part: launch ramp, first-byte latency and drain included.
// The words read are folded into one value per lane that is stored only if it
// equals a key the caller passes (the compiler cannot prove it false, so no
// load is dead code); the host picks a key the buffer's contents cannot give.
#include "common.hpp"

namespace vxt {

namespace {

constexpr int kLoads = 2;   // 16-byte loads per lane (2 KiB per wave)

__global__ __launch_bounds__(256) void read_probe_kernel(const u32x4* __restrict__ p, size_t n16,
                                                         uint32_t* __restrict__ sink, uint32_t key) {
  const size_t wave = ((size_t)blockIdx.x * 256 + threadIdx.x) / 64;
  const uint32_t lane = threadIdx.x & 63;
  const size_t base = wave * kLoads * 64 + lane;
  u32x4 v[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const size_t idx = base + (size_t)i * 64;
    v[i] = __builtin_nontemporal_load(p + (idx < n16 ? idx : n16 - 1));
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < kLoads; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (acc == key) sink[0] = acc;   // the host passes a key no fold of the data equals
}

}  // namespace

hipError_t launch_read_probe(const void* p, size_t bytes, uint32_t* sink, uint32_t key, hipStream_t s) {
  const size_t n16 = bytes / 16;
  if (n16 == 0) return hipErrorInvalidValue;
  const size_t waves = (n16 + kLoads * 64 - 1) / (kLoads * 64);
  const size_t blocks = (waves * 64 + 255) / 256;
  if (blocks > 0x7fffffffu) return hipErrorInvalidValue;
  hipLaunchKernelGGL(read_probe_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, static_cast<const u32x4*>(p), n16,
                     sink, key);
  return hipGetLastError();
}

}  // namespace vxt
