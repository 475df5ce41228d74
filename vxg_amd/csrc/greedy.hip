// greedy.hip -- exact greedy token selection over f32 logits.
//
// Result (the reference's vxt_greedy_exact, vxt_llm_ops.metal:569-600, and
// the greedy branch of sample_logits_top_k_p, llm_ops.rs:318-327):
//   id        = the lowest index i whose logit equals the largest non-NaN
//               logit, when that logit is above -inf; otherwise 0 (an empty
//               input, all -inf, all NaN).  -0 and +0 are equal values, so the
//               lower index wins between them.
//   nonfinite = 1 when any logit is NaN or +-inf, else 0.
//
// One pass over the logits.  Each element becomes a 64-bit key whose
// unsigned order is the selection order: the float's bits mapped to an
// order-preserving u32 in the high word, the complemented index in the low
// word (larger value first, then lower index).  NaN takes no key.  Each block
// reduces its slice to one key and a flag.  Then:
//   up to kOneKernelBlocks blocks: the block folds its key into a
//     device-scope atomic maximum; the last block to finish (counted by an
//     acquire-release atomic add) writes the result and zeroes the state
//     words for the next call -- one launch;
//   more blocks: each block stores its key and flag in a partials array and a
//     one-block kernel reduces them -- no atomics.  The acquire-release add
//     costs about 25 ns per block (serialised), so beyond a few dozen blocks
//     the second launch is cheaper.
// Neither path needs a memset, so both can sit inside a captured graph.
#include "common.hpp"

#include <algorithm>

namespace vxt {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kLoads = 4;            // loads in flight per thread per pass
constexpr uint32_t kMaxBlocks = 1024;

constexpr uint32_t kOneKernelBlocks = 48;

struct GreedyState {
  unsigned long long key;   // running maximum key (0 = nothing seen); zero between calls
  uint32_t nonfinite;       // zero between calls
  uint32_t done;            // blocks finished in this call; zero between calls
  unsigned long long part_key[kMaxBlocks];
  uint32_t part_nonfinite[kMaxBlocks];
};

// Integer tests only, so the result does not depend on the denormal mode.
__device__ __forceinline__ unsigned long long key_of(float v, uint32_t i) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7fffffffu) == 0u) b = 0u;
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)ord << 32) | (uint32_t)~i;
}

__device__ __forceinline__ void take(float v, uint32_t i, unsigned long long& best, uint32_t& nf) {
  const uint32_t b = __float_as_uint(v);
  nf |= (b & 0x7f800000u) == 0x7f800000u;
  const unsigned long long k = (b & 0x7fffffffu) <= 0x7f800000u ? key_of(v, i) : 0ull;
  best = k > best ? k : best;
}

__device__ __forceinline__ unsigned long long wave_max(unsigned long long k) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)k, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(k >> 32), off, 64);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    k = o > k ? o : k;
  }
  return k;
}

// This thread's best key and non-finite flag over the block's slices.
// VEC: logits is 16-byte aligned; units are float4 (the n % 4 tail is read
// singly by block 0).  Otherwise units are single floats.
template <bool VEC>
__device__ __forceinline__ void scan(const float* __restrict__ logits, uint32_t n, unsigned long long& best,
                                     uint32_t& nf) {
  const uint32_t tid = threadIdx.x;
  const uint32_t units = VEC ? n / 4u : n;
  const uint32_t per_pass = kThreads * kLoads;
  for (uint32_t base = blockIdx.x * per_pass; base < units; base += gridDim.x * per_pass) {
    if (VEC) {
      float4 v[kLoads];
#pragma unroll
      for (uint32_t r = 0; r < kLoads; ++r) {
        const uint32_t u = min(base + r * kThreads + tid, units - 1u);
        v[r] = reinterpret_cast<const float4*>(logits)[u];
      }
#pragma unroll
      for (uint32_t r = 0; r < kLoads; ++r) {
        const uint32_t u = base + r * kThreads + tid;
        if (u < units) {
          take(v[r].x, 4u * u, best, nf);
          take(v[r].y, 4u * u + 1u, best, nf);
          take(v[r].z, 4u * u + 2u, best, nf);
          take(v[r].w, 4u * u + 3u, best, nf);
        }
      }
    } else {
      float v[kLoads];
#pragma unroll
      for (uint32_t r = 0; r < kLoads; ++r) v[r] = logits[min(base + r * kThreads + tid, units - 1u)];
#pragma unroll
      for (uint32_t r = 0; r < kLoads; ++r) {
        const uint32_t u = base + r * kThreads + tid;
        if (u < units) take(v[r], u, best, nf);
      }
    }
  }
  if (VEC && blockIdx.x == 0 && tid < n % 4u) {
    const uint32_t i = (n & ~3u) + tid;
    take(logits[i], i, best, nf);
  }
}

// Block-wide reduction; thread 0 returns true holding the block's key and flag.
__device__ __forceinline__ bool block_reduce(unsigned long long& best, uint32_t& nf) {
  __shared__ unsigned long long s_key[kThreads / 64];
  __shared__ uint32_t s_nf[kThreads / 64];
  const uint32_t tid = threadIdx.x;
  best = wave_max(best);
  const uint32_t any_nf = __any(nf) ? 1u : 0u;
  if ((tid & 63u) == 0) {
    s_key[tid >> 6] = best;
    s_nf[tid >> 6] = any_nf;
  }
  __syncthreads();
  if (tid != 0) return false;
  best = s_key[0];
  nf = s_nf[0];
#pragma unroll
  for (uint32_t w = 1; w < kThreads / 64; ++w) {
    best = s_key[w] > best ? s_key[w] : best;
    nf |= s_nf[w];
  }
  return true;
}

__device__ __forceinline__ void write_result(unsigned long long k, uint32_t nf, uint32_t* __restrict__ out) {
  const unsigned long long floor = key_of(-__builtin_inff(), 0u);   // nothing above -inf -> index 0
  k = k > floor ? k : floor;
  out[0] = ~(uint32_t)k;
  out[1] = nf;
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void greedy_one_kernel(const float* __restrict__ logits, uint32_t n,
                                                              GreedyState* __restrict__ st,
                                                              uint32_t* __restrict__ out) {
  unsigned long long best = 0ull;
  uint32_t nf = 0u;
  scan<VEC>(logits, n, best, nf);
  if (!block_reduce(best, nf)) return;
  if (best) __hip_atomic_fetch_max(&st->key, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (nf) __hip_atomic_fetch_or(&st->nonfinite, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t finished = __hip_atomic_fetch_add(&st->done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  if (finished != gridDim.x - 1u) return;
  // Last block: every other block's atomics happened before its release.
  write_result(__hip_atomic_load(&st->key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
               __hip_atomic_load(&st->nonfinite, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), out);
  __hip_atomic_store(&st->key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&st->nonfinite, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&st->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void greedy_partial_kernel(const float* __restrict__ logits, uint32_t n,
                                                                  GreedyState* __restrict__ st) {
  unsigned long long best = 0ull;
  uint32_t nf = 0u;
  scan<VEC>(logits, n, best, nf);
  if (!block_reduce(best, nf)) return;
  st->part_key[blockIdx.x] = best;
  st->part_nonfinite[blockIdx.x] = nf;
}

__global__ __launch_bounds__(kThreads) void greedy_final_kernel(uint32_t blocks, const GreedyState* __restrict__ st,
                                                                uint32_t* __restrict__ out) {
  unsigned long long best = 0ull;
  uint32_t nf = 0u;
  for (uint32_t b = threadIdx.x; b < blocks; b += kThreads) {
    const unsigned long long k = st->part_key[b];
    best = k > best ? k : best;
    nf |= st->part_nonfinite[b];
  }
  if (block_reduce(best, nf)) write_result(best, nf, out);
}

}  // namespace

size_t greedy_state_bytes() { return sizeof(GreedyState); }

// `state` must hold greedy_state_bytes() zeroed bytes before the first call;
// each call leaves its first 16 bytes zeroed again.  Calls that share a state
// must not overlap in time.
hipError_t launch_greedy(const float* logits, uint32_t n, void* state, uint32_t* out, hipStream_t s) {
  const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0;
  const uint32_t units = vec ? n / 4u : n;
  const uint32_t per_pass = kThreads * kLoads;
  uint32_t blocks = (units + per_pass - 1u) / per_pass;
  blocks = std::max(1u, std::min(blocks, kMaxBlocks));
  GreedyState* st = static_cast<GreedyState*>(state);
  if (blocks <= kOneKernelBlocks) {
    if (vec)
      hipLaunchKernelGGL(greedy_one_kernel<true>, dim3(blocks), dim3(kThreads), 0, s, logits, n, st, out);
    else
      hipLaunchKernelGGL(greedy_one_kernel<false>, dim3(blocks), dim3(kThreads), 0, s, logits, n, st, out);
    return hipGetLastError();
  }
  if (vec)
    hipLaunchKernelGGL(greedy_partial_kernel<true>, dim3(blocks), dim3(kThreads), 0, s, logits, n, st);
  else
    hipLaunchKernelGGL(greedy_partial_kernel<false>, dim3(blocks), dim3(kThreads), 0, s, logits, n, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(greedy_final_kernel, dim3(1), dim3(kThreads), 0, s, blocks, st, out);
  return hipGetLastError();
}

}  // namespace vxt
