// common.hpp -- device-side descriptors and helpers shared by the kernels.
//
// Device-resident layouts (built by vxt_hip.hip at upload time):
//
//   Q8_0   qs    int8  [rows][kp]        kp = 32 * ceil(cols/32), 16-B rows
//          d     f16   [rows][kp/32]
//   CB4    words u32   [rows][kp/8]      nibble c%8 of word c/8 (as uploaded)
//          sc    f16   [rows][kp/128]
//          cent  f32   [3][16]           (kernel argument; table t serves rows
//                                     [split(t), split(t+1)) of a row-concatenated
//                                     matrix, split(0)=0, split(3)=rows)
//          CSR   row_ptr u32[rows+1], outliers u32[nnz] (col | f16 << 16)
//   G64    idx   u8    [rows][kp/2]      low nibble = even column
//          lut   f16   [rows][kp/64][16]
//   Q4_0   qs    u8    [rows][kp/2]      kp = 32 * ceil(cols/32); block b of a
//                                      row is bytes 16 b .. 16 b + 15, byte j
//                                      holding column 32 b + j (low nibble) and
//                                      32 b + j + 16 (high nibble), value q - 8
//          d     f16   [rows][kp/32]
//
// Every plane starts 256-byte aligned inside one arena allocation per tensor.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vxt {

enum Kind : uint32_t { KIND_CB4 = 2u, KIND_Q40 = 4u, KIND_Q8 = 8u, KIND_G64 = 9u };

struct DevTensor {
  uint32_t kind;
  uint32_t rows;
  uint32_t cols;
  uint32_t kp;          // padded cols of the resident layout
  const void* p0;       // Q8: qs      CB4: words     G64: idx   Q4_0: nibbles
  const uint16_t* p1;   // Q8: d       CB4: scales    G64: lut   Q4_0: d
  const uint32_t* row_ptr;   // CB4 only
  const uint32_t* outliers;  // CB4 only
  uint32_t split0, split1;   // CB4: first rows served by tables 1 and 2
  float cent[48];            // CB4 only: 3 centroid tables of 16
  uint32_t tail_nonfinite;   // G64: cols % 64 != 0 and some row's last table holds Inf/NaN
  // CB4 only, null unless the decode-in-loop GEMM takes the tensor: per row,
  // the exponent e with (the row's largest |w| bound) * 2^e in [2^14, 2^15).
  const int8_t* rexp;
};

// Prefill GEMM path (batch_m > 8): chosen per call, or pinned by the caller.
// kGemmAutoOwn chooses like kGemmAuto but never the vendor library (whose
// first call for a shape allocates descriptors).
enum GemmMode : int { kGemmAuto = 0, kGemmPanel = 1, kGemmFused = 2, kGemmLibrary = 3, kGemmAutoOwn = 4 };

// Centroid table serving `row` (rows of up to 3 concatenated sub-matrices).
__device__ __forceinline__ uint32_t cent_table(const DevTensor& t, uint32_t row) {
  return (uint32_t)(row >= t.split0) + (uint32_t)(row >= t.split1);
}

// ---- memory ----------------------------------------------------------------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (weights are read once per call: non-temporal hint).
__device__ __forceinline__ uint4 load_nt16(const void* p) {
  u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- conversions ---------------------------------------------------------

// Exact f16 -> f32 in integer arithmetic: the reference's rule
// (fp16.rs:6-29), including its NaN payload (sign | 0x7f800000 | mant << 13).
__device__ __forceinline__ float f16_to_f32_exact(uint32_t h) {
  uint32_t sign = (h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t out;
  if (e == 0u) {
    if (m == 0u) {
      out = sign;
    } else {
      uint32_t sh = (uint32_t)__clz((int)m) - 21u;  // shifts until bit 10 is set
      out = sign | ((113u - sh) << 23) | (((m << sh) & 0x3ffu) << 13);
    }
  } else if (e == 31u) {
    out = sign | 0x7f800000u | (m << 13);
  } else {
    out = sign | ((e + 112u) << 23) | (m << 13);
  }
  return __uint_as_float(out);
}

// Hardware f16 -> f32 (v_cvt_f32_f16); identical to the exact rule for every
// non-NaN input.  Used on the compute paths.
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// f32 -> bf16 with the reference's rule (fp16.rs:113-120): NaN keeps its top
// bits with the quiet bit set, everything else rounds to nearest even.  The
// hardware conversion (v_cvt_pk_bf16_f32) gives exactly these bits for each
// of the 2^32 f32 inputs -- checked exhaustively on MI355X against the
// integer rule ((b + 0x7fff + lsb) >> 16, NaN -> (b >> 16) | 0x40), normal,
// subnormal, infinite and NaN inputs alike -- at one instruction per pair.
typedef float vxt_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 vxt_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_pack(float lo, float hi) {
  const vxt_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, vxt_bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float v) { return (uint16_t)bf16x2_pack(v, 0.0f); }

// A hi/lo pair of GEMM accumulators, acc + accl * 2^-11.  An Inf activation
// x puts hi * x = +-Inf in acc -- the sign of w * x, as hi carries w's sign
// -- and lo * x in accl, which is NaN where lo = 0 and may be an Inf of the
// other sign; gemm_cpu gives acc's Inf, so an infinite acc is the result.
__device__ __forceinline__ float hilo_combine(float acc, float accl) {
  return __builtin_isinf(acc) ? acc : __builtin_fmaf(accl, 1.0f / 2048.0f, acc);
}

// Inputs of a GEMV whose activations are an RMSNorm of the residual stream
// (batch 1): x = bf16(rms_norm(cur [+ delta]) * w).
struct NormIn {
  const float* cur;
  const float* delta;    // null: x = norm(cur), nothing stored
  const float* w;
  float* cur_out;        // with delta: receives cur + delta (must not alias cur or delta)
  float eps;
};

// One layer's Q8_0 KV cache (the planes of VxtKvQ8Cache): row t holds
// position t, n_kv * hd int8 values and n_kv * hd / 32 f16 scales per plane.
struct KvQ8Dev {
  int8_t* k_qs;
  uint16_t* k_d;
  int8_t* v_qs;
  uint16_t* v_d;
  uint32_t max_seq, n_kv, hd;
};

// The q / k preparation of an attention step for a batch of tokens: token m
// reads q_raw + m * q_stride, k_cur / v_cur + m * kv_stride, writes cache row
// pos + m and q_out / gate_out + m * n_head * hd, and rotates at rope_pos + m.
struct GqaPrep {
  const float* q_raw;
  const float* k_cur;
  const float* v_cur;
  const float* q_norm;   // null: no norm
  const float* k_norm;
  const float* q_bias;   // null: no bias
  const float* k_bias;
  const float* v_bias;
  float* q_out;
  float* gate_out;       // gated only
  uint32_t q_stride, kv_stride, n_head, gated, half, neox, pos, rope_pos;
  float eps;
  // Decode step only: null, or device words {pos, rope_pos} read by the
  // kernels in place of pos / rope_pos (pos clamped to the cache), so one
  // captured graph serves every position.
  const uint32_t* dpos;
};

// Workgroup barrier that orders LDS traffic only.  __syncthreads() also
// waits for every global load the wave has in flight (its release fence
// drains the vector memory counter); this one waits for the wave's LDS and
// scalar operations, then meets the other waves, so loads issued before it
// stay in flight.  Global memory written before it is not made visible by it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---- wave64 reductions ----------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Lane-group reductions with no LDS traffic (every lane active): DPP
// quad_perm xor 1 / xor 2, row_half_mirror and row_mirror pair the lanes of
// aligned groups of 2..16; v_permlane16_swap / v_permlane32_swap called with
// v as both operands return v and its xor-16 (xor-32) partner, one in each
// result, so combining the pair gives the group of 32 (64).
__device__ __forceinline__ float xor16_pair(float v, bool mx) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return mx ? fmaxf(a, b) : a + b;
}
__device__ __forceinline__ float xor32_pair(float v, bool mx) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return mx ? fmaxf(a, b) : a + b;
}

// Sum (MAX: maximum) over aligned groups of N consecutive lanes, N a power of
// two <= 64, returned in every lane of the group.
template <int N, bool MAX = false>
__device__ __forceinline__ float lane_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  if constexpr (N >= 2) v = op(v, dpp_mov<0xB1>(v));    // quad_perm [1,0,3,2]
  if constexpr (N >= 4) v = op(v, dpp_mov<0x4E>(v));    // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v = op(v, dpp_mov<0x141>(v));   // row_half_mirror
  if constexpr (N >= 16) v = op(v, dpp_mov<0x140>(v));  // row_mirror
  if constexpr (N >= 32) v = xor16_pair(v, MAX);
  if constexpr (N >= 64) v = xor32_pair(v, MAX);
  return v;
}

// Sum over the lanes that share lane % S (S a power of two <= 16), returned
// in every lane: row_ror by S, 2S, .. 8 inside each 16-lane row, then across
// rows and halves.
template <int S>
__device__ __forceinline__ float stride_sum(float v) {
  if constexpr (S <= 1) v += dpp_mov<0x121>(v);   // row_ror:1
  if constexpr (S <= 2) v += dpp_mov<0x122>(v);   // row_ror:2
  if constexpr (S <= 4) v += dpp_mov<0x124>(v);   // row_ror:4
  if constexpr (S <= 8) v += dpp_mov<0x128>(v);   // row_ror:8
  v = xor16_pair(v, false);
  return xor32_pair(v, false);
}

// Sum over the 64 lanes, returned in every lane (uniform).  DPP butterflies
// inside each 16-lane row (quad_perm xor 1, xor 2, half-mirror, mirror), then
// the four row sums are read out with v_readlane.  No LDS round trips.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);   // row_half_mirror
  v += dpp_mov<0x140>(v);   // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

}  // namespace vxt
