// chain.hip -- the matmuls of one decode step (batch 1) in one persistent launch.
//
// A decode step is a chain of dependent GEMVs: each projection reads (a
// slice of) an earlier one's output.  Launched one kernel per projection,
// every launch pays its own ramp-up and its first weight bytes' full HBM
// latency (about 3 us even for a 4 MB matrix), and nothing overlaps.  Weights,
// however, do not depend on activations: one cooperative launch walks all
// projections in order and keeps the next rows' weight loads in flight while
// the current projection finishes.
//
// Work: wave g of W walks rows g, g + W, ... of every op, in op order, one
// K step (2048 columns) at a time, and the weight loads of the next kDepth
// steps (of this op or later ops) are issued before the current one is
// computed.  Op boundaries, per workgroup:
//   1. wait until every workgroup has finished op o-1: wave 0 polls 32
//      device-scope completion counters;
//   2. stage op o's bf16 activations (and cb4 centroids) in LDS;
//   3. the waves compute their rows of op o;
//   4. wait for this block's stores, block barrier, and thread 0 adds one to
//      counter o[block % 32].
// Data that crosses workgroups (outputs, activations, counters) moves with
// device-coherent (sc1) stores, loads and atomics, so no L2-wide writeback
// or invalidate is needed: the L2s of the eight XCDs are not coherent, and an
// agent-scope fence per wave and op cost more than the matmuls.
// A workgroup reaches op o's count only after it waited for op o-1, so op o
// complete implies every earlier op complete: an op may read any earlier
// op's output and may overwrite a buffer that only earlier ops read.
//
// Per-row arithmetic is gemv_kernel's at M = 1 (same lane mapping, FMA order,
// group scale, residual order and wave reduction), so each output is
// bit-identical to the per-projection launch.
//
// Termination: every wait is bounded by a spin limit.  A wait that runs out
// sets the status word; from then on workgroups skip arithmetic and only
// signal, so every wave reaches the end and the grid drains.
#include <algorithm>
#include <cstring>

#include "gemv_impl.hpp"

namespace vxt {

namespace ch {

using gv::kChunk;
using gv::kPairStride;
using gv::kSlotBytes;
using gv::kStep;
using gv::lds_addr;

constexpr int kWaves = 12;                     // one block per CU, 3 waves per SIMD
constexpr int kThreads = kWaves * 64;
constexpr int kMaxSteps = 3;                    // K <= 6144 per op
constexpr uint32_t kMaxK = kMaxSteps * kStep;
constexpr int kCounters = 32;                   // completion counters per op
constexpr uint32_t kCounterStride = 32;         // words: one 128-byte line per counter
constexpr int kDepth = 3;                       // row steps in flight ahead of the current one
constexpr int kCoherent = 16;                   // buffer cache policy sc1: device-coherent access

struct ChainOp {
  DevTensor t;
  const uint16_t* x;   // bf16 [cols]
  void* y;             // [rows], f32 or bf16
  uint32_t y_bf16;
  uint32_t nsteps;     // ceil(kp / kStep) <= kMaxSteps
  uint32_t nnz;        // cb4 residual count
  uint32_t pad;
};

// Raw weight words of one row-step, any kind (the loads of gv::load_chunk).
struct Raw {
  u32x4 a, b;
  uint32_t c;
};

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return __builtin_nontemporal_load(static_cast<const u32x4*>(p));
}

__device__ __forceinline__ void load_raw(const DevTensor& t, uint32_t row, uint32_t s, uint32_t lane, Raw& r) {
  const uint32_t kp = t.kp;
  const uint32_t k0 = s * kStep + lane * kChunk;
  const uint32_t k0c = k0 < kp ? k0 : kp - kChunk;
  if (t.kind == KIND_Q8) {
    const int8_t* p = static_cast<const int8_t*>(t.p0) + (size_t)row * kp + k0c;
    r.a = ld16(p);
    r.b = ld16(p + 16);
    r.c = t.p1[(size_t)row * (kp / 32) + k0c / 32];
  } else if (t.kind == KIND_CB4) {
    r.a = ld16(static_cast<const uint32_t*>(t.p0) + (size_t)row * (kp / 8) + k0c / 8);
    r.c = t.p1[(size_t)row * (kp / 128) + k0c / 128];
  } else {
    const uint32_t gmax = kp / 64 - 1;
    const uint32_t g = s * 32 + (lane >> 1);
    r.a = ld16(static_cast<const uint8_t*>(t.p0) + (size_t)row * (kp / 2) + k0c / 2);
    r.b = ld16(t.p1 + ((size_t)row * (kp / 64) + (g < gmax ? g : gmax)) * 16 + (lane & 1) * 8);
  }
}

__device__ __forceinline__ uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

// A unit of work: K step `step` of row `row` of op `op` (op == n_ops: none).
struct Task {
  uint32_t op, row, step;
};

// The task after t for wave gw of W: next step of the row, else the wave's
// next row (rows gw, gw + W, ...), skipping ops with no row for the wave.
__device__ __forceinline__ Task advance(const ChainOp* ops, uint32_t n_ops, uint32_t gw, uint32_t W, Task t) {
  if (t.op >= n_ops) return t;
  if (t.step + 1 < ops[t.op].nsteps) return Task{t.op, t.row, t.step + 1};
  uint32_t op = t.op, row = t.row + W;
  while (op < n_ops && row >= ops[op].t.rows) {
    ++op;
    row = gw;
  }
  return Task{op, row, 0};
}

__device__ __forceinline__ void issue(const ChainOp* ops, uint32_t n_ops, Task tk, uint32_t lane, Raw& r) {
  if (tk.op < n_ops) load_raw(ops[tk.op].t, tk.row, tk.step, lane, r);
}

template <uint32_t KIND>
__device__ __forceinline__ gv::WChunk<KIND> as_chunk(const Raw& r) {
  gv::WChunk<KIND> c;
  if constexpr (KIND == KIND_Q8) {
    c.a = make_uint4(r.a.x, r.a.y, r.a.z, r.a.w);
    c.b = make_uint4(r.b.x, r.b.y, r.b.z, r.b.w);
    c.d = r.c;
  } else if constexpr (KIND == KIND_CB4) {
    c.q = make_uint4(r.a.x, r.a.y, r.a.z, r.a.w);
    c.sc = r.c;
  } else {
    c.q = make_uint4(r.a.x, r.a.y, r.a.z, r.a.w);
    c.lut = make_uint4(r.b.x, r.b.y, r.b.z, r.b.w);
  }
  return c;
}

// CSR words read through the constant address space with wave-uniform
// indices: scalar loads, which have their own wait counter and so do not
// wait behind the vector weight loads in flight.
typedef __attribute__((address_space(4))) const uint32_t* const_u32_ptr;

__device__ __forceinline__ uint32_t cload(const uint32_t* base, uint32_t i) {
  return reinterpret_cast<const_u32_ptr>(reinterpret_cast<uintptr_t>(base))[i];
}

// One K step of one row (M = 1): gemv_kernel's per-step arithmetic, x from LDS.
template <uint32_t KIND>
__device__ __forceinline__ float step_dot(const DevTensor& t, uint32_t step, const Raw& r, const uint16_t* s_x,
                                          uint32_t cbase, uint32_t slot, uint32_t lane) {
  const uint32_t k0 = step * kStep + lane * kChunk;
  const bool kin = k0 < t.kp;
  float xv[kChunk];
  const u32x4* xs = reinterpret_cast<const u32x4*>(s_x + k0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 u = xs[i];
    const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv[8 * i + 2 * j] = __uint_as_float(w4[j] << 16);
      xv[8 * i + 2 * j + 1] = __uint_as_float(w4[j] & 0xffff0000u);
    }
  }
  const gv::WChunk<KIND> c = as_chunk<KIND>(r);
  if constexpr (KIND == KIND_G64)
    *(__attribute__((address_space(3))) u32x4*)(size_t)(slot + (lane >> 1) * kPairStride + (lane & 1) * 16) = r.b;
  float w[kChunk];
  gv::dequant_chunk<KIND>(c, cbase, slot, lane, w);
  float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
  for (int j = 0; j < kChunk; j += 2) {
    p0 = __builtin_fmaf(w[j], xv[j], p0);
    p1 = __builtin_fmaf(w[j + 1], xv[j + 1], p1);
  }
  float p = p0 + p1;
  if constexpr (KIND == KIND_Q8) {
    p *= f16_to_f32(c.d);
  } else if constexpr (KIND == KIND_CB4) {
    const float sc = f16_to_f32(c.sc);   // codebook.rs:384-386
    p = sc != 0.0f ? sc * p : 0.0f;
  }
  return kin ? p : 0.0f;
}

// cb4 residuals of a row (codebook.rs:409-415): entry e of the row goes to
// lane e % 64, in order, as in gemv_kernel.
__device__ __forceinline__ float residuals(const DevTensor& t, uint32_t row, const uint16_t* s_x, uint32_t lane,
                                           float acc) {
  const uint32_t os = cload(t.row_ptr, row), oe = cload(t.row_ptr, row + 1);
  for (uint32_t e0 = os; e0 < oe; e0 += 16) {
    uint32_t pk[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) pk[i] = cload(t.outliers, e0 + i < oe ? e0 + i : oe - 1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t e = e0 + i;
      const uint32_t col = pk[i] & 0xffffu;
      if (e < oe && col < t.cols && lane == ((e - os) & 63u))
        acc = __builtin_fmaf(f16_to_f32(pk[i] >> 16), bf16_to_f32(s_x[col]), acc);
    }
  }
  return acc;
}

__global__ __launch_bounds__(kThreads) void chain_kernel(const ChainOp* __restrict__ ops, uint32_t n_ops,
                                                         uint32_t* __restrict__ counters, uint32_t* __restrict__ status,
                                                         uint32_t epoch, uint32_t spin_limit) {
  __shared__ __attribute__((aligned(16))) uint16_t s_x[kMaxK];
  __shared__ __attribute__((aligned(64))) float s_cent[48];
  __shared__ __attribute__((aligned(64))) uint4 s_slot[kWaves * kSlotBytes / 16];
  __shared__ uint32_t s_abort;

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = uni(tid >> 6);
  const uint32_t G = gridDim.x;
  const uint32_t W = G * kWaves;
  const uint32_t gw = blockIdx.x * kWaves + wave;
  const uint32_t slot = lds_addr(s_slot) + wave * kSlotBytes;
  if (tid == 0) s_abort = 0;

  // Work in flight: q[0] is computed next, q[1..kDepth] are requested.
  Task q[kDepth + 1];
  Raw rq[kDepth + 1];
  q[0] = Task{0, gw, 0};
  while (q[0].op < n_ops && q[0].row >= ops[q[0].op].t.rows) ++q[0].op;
#pragma unroll
  for (int d = 1; d <= kDepth; ++d) q[d] = advance(ops, n_ops, gw, W, q[d - 1]);
#pragma unroll
  for (int d = 0; d <= kDepth; ++d) issue(ops, n_ops, q[d], lane, rq[d]);
  float acc = 0.0f;

  for (uint32_t o = 0; o < n_ops; ++o) {
    const ChainOp& op = ops[o];
    // 1. op o-1 finished everywhere
    if (o > 0 && wave == 0) {
      uint32_t* cn = counters + (size_t)(o - 1) * kCounters * kCounterStride;
      const uint32_t c = lane & (kCounters - 1);
      const uint32_t need = (epoch + 1u) * (G / kCounters + (c < G % kCounters ? 1u : 0u));
      bool abort = false;
      for (uint32_t it = 0;; ++it) {
        const uint32_t v = __hip_atomic_load(cn + c * kCounterStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t st = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (st != 0u) {
          abort = true;
          break;
        }
        if (__all(v >= need)) break;
        if (it >= spin_limit) {
          abort = true;
          if (lane == 0) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (lane == 0 && abort) s_abort = 1u;
    }
    __syncthreads();
    const bool aborted = s_abort != 0u;

    // 2. stage x (bf16, zero past cols) and the cb4 centroid tables
    const uint32_t cols = op.t.cols, kp = op.t.kp;
    if (!aborted) {
      const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(op.x), (short)0,
                                                                           (int)(cols * 2u), 0x00020000);
      if (cols % 8u == 0u) {
        for (uint32_t p = tid; p < kp / 8u; p += kThreads)
          *reinterpret_cast<u32x4*>(&s_x[p * 8u]) = __builtin_amdgcn_raw_buffer_load_b128(xr, p * 16u, 0, kCoherent);
      } else {
        for (uint32_t cc = tid; cc < kp; cc += kThreads)
          s_x[cc] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(xr, cc * 2u, 0, kCoherent);
      }
      if (op.t.kind == KIND_CB4 && tid < 48) s_cent[tid] = op.t.cent[tid];
    }
    __syncthreads();

    // 3. this wave's row steps of op o
    const uint32_t kind = uni(op.t.kind);
    const uint32_t ns = uni(op.nsteps);
    while (q[0].op == o) {
      if (!aborted) {
        const uint32_t row = uni(q[0].row), step = uni(q[0].step);
        if (kind == KIND_G64)
          acc += step_dot<KIND_G64>(op.t, step, rq[0], s_x, 0, slot, lane);
        else if (kind == KIND_CB4)
          acc += step_dot<KIND_CB4>(op.t, step, rq[0], s_x, lds_addr(s_cent) + 64u * cent_table(op.t, row), slot, lane);
        else
          acc += step_dot<KIND_Q8>(op.t, step, rq[0], s_x, 0, slot, lane);
        if (step + 1 == ns) {   // row complete
          if (kind == KIND_CB4) acc = residuals(op.t, row, s_x, lane, acc);
          const float v = wave_sum(acc);
          if (lane == 0) {   // device-coherent store: read by other workgroups in this launch
            const uint32_t esz = op.y_bf16 ? 2u : 4u;
            const __amdgpu_buffer_rsrc_t yr =
                __builtin_amdgcn_make_buffer_rsrc(op.y, (short)0, (int)(op.t.rows * esz), 0x00020000);
            if (op.y_bf16)
              __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), yr, row * 2u, 0, kCoherent);
            else
              __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yr, row * 4u, 0, kCoherent);
          }
          acc = 0.0f;
        }
      }
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        q[d] = q[d + 1];
        rq[d] = rq[d + 1];
      }
      q[kDepth] = advance(ops, n_ops, gw, W, q[kDepth]);
      issue(ops, n_ops, q[kDepth], lane, rq[kDepth]);
    }

    // 4. op o done in this block: its (device-coherent) output stores are
    //    complete before the block is counted
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
      __hip_atomic_fetch_add(counters + ((size_t)o * kCounters + blockIdx.x % kCounters) * kCounterStride, 1u,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace ch

// ---- host side ---------------------------------------------------------------

struct ChainLaunch {
  const void* ops;
  uint32_t n_ops;
  uint32_t* counters;
  uint32_t* status;
};

size_t chain_op_bytes() { return sizeof(ch::ChainOp); }
size_t chain_counter_bytes(uint32_t n_ops) { return (size_t)n_ops * ch::kCounters * ch::kCounterStride * 4u; }
uint32_t chain_max_k() { return ch::kMaxK; }

// Fills the device op record for one projection.
void chain_fill_op(void* dst, const DevTensor& t, uint32_t nnz, const void* x, void* y, bool y_bf16) {
  ch::ChainOp op{};
  op.t = t;
  op.x = static_cast<const uint16_t*>(x);
  op.y = y;
  op.y_bf16 = y_bf16 ? 1u : 0u;
  op.nsteps = (t.kp + gv::kStep - 1) / gv::kStep;
  op.nnz = nnz;
  std::memcpy(dst, &op, sizeof(op));
}

// Workgroups that can be resident at once (the grid of the cooperative launch).
hipError_t chain_grid(uint32_t* grid) {
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&ch::chain_kernel),
                                                   ch::kThreads, 0);
  if (e != hipSuccess) return e;
  *grid = (uint32_t)std::max(1, cus * std::min(per_cu, 1));
  return hipSuccess;
}

hipError_t chain_launch(const ChainLaunch& l, uint32_t grid, uint32_t epoch, uint32_t spin_limit, hipStream_t s) {
  const ch::ChainOp* ops = static_cast<const ch::ChainOp*>(l.ops);
  uint32_t n_ops = l.n_ops;
  uint32_t* counters = l.counters;
  uint32_t* status = l.status;
  void* args[] = {&ops, &n_ops, &counters, &status, &epoch, &spin_limit};
  return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&ch::chain_kernel), dim3(grid),
                                    dim3(ch::kThreads), args, 0, s);
}

}  // namespace vxt
