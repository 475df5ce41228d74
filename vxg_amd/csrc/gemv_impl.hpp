// gemv_impl.hpp -- fused dequantise + GEMV for M = 1..8 tokens (decode path).
//
// Reference behaviour: CodebookMatrix::gemv_cpu (codebook.rs:350-417), the Q8
// block-dot composition (llm_prefill.rs:45-54, :336-340) and the Metal GEMV
// kernels (vxt_gemv.metal:297-381, vxt_cb4_fast.metal:104-209).
//
// A decode GEMV moves a few MB per call, so its time is set by how early every
// byte is requested.  Mapping on CDNA4 (wave64):
//   * one wave owns RPW output rows; a K "step" covers 2048 columns, 32 per
//     lane, so each weight load is one contiguous 16-byte load per lane (a
//     fully coalesced 1 KiB per wave for the 4-bit kinds, 2 KiB for Q8);
//   * a batch of up to S steps x RPW rows is requested at once, together with
//     the activations those steps need, before the first wait.  Every load is
//     branch-free from a clamped, always-valid address; lanes outside the
//     matrix are masked after the arithmetic.  (A predicated load makes the
//     compiler drain the memory counter, and the vector memory counter drains
//     in order, so one such wait serialises every load issued before it.);
//   * activations are read straight from global memory (they are L2-resident
//     after the first wave touches them), 16 bytes at a time;
//   * cb4: the 16-entry centroid tables (up to 3 for row-concatenated
//     matrices) live in LDS, staged before any load is issued; g64: each lane loads 16 bytes of its group's codebook
//     (coalesced) and the two lanes of a 64-group exchange halves through a
//     per-wave LDS slot laid out against bank conflicts;
//   * partial sums are reduced across the wave with DPP at the end.
// Sums are fp32; the order differs from the CPU reference, so results agree
// to fp32 rounding (the parity bar is relative error, not bits).
#pragma once
#include <algorithm>
#include <cstdlib>

#include "act.hpp"
#include "common.hpp"

namespace vxt {

namespace gv {

constexpr int kWaves = 4;
constexpr int kChunk = 32;           // K columns per lane per step
constexpr int kStep = 64 * kChunk;   // K columns per wave per step

template <uint32_t KIND>
struct WChunk;
template <>
struct WChunk<KIND_Q8> {
  uint4 a, b;     // 32 int8
  uint32_t d;     // f16 scale bits
};
template <>
struct WChunk<KIND_CB4> {
  uint4 q;        // 32 nibbles
  uint32_t sc;    // f16 scale bits
};
template <>
struct WChunk<KIND_Q40> {
  uint4 q;        // one block: byte j = column j (low nibble) | column j + 16 (high nibble)
  uint32_t d;     // f16 scale bits
};
template <>
struct WChunk<KIND_G64> {
  uint4 q;        // 32 nibbles
  uint4 lut;      // this lane's half of the group's 16-entry f16 table
};

// Unconditional loads of one row-step (row and k0 already clamped in range).
template <uint32_t KIND>
__device__ __forceinline__ void load_chunk(const DevTensor& t, uint32_t row, uint32_t k0, uint32_t g,
                                           uint32_t half, WChunk<KIND>& c) {
  if constexpr (KIND == KIND_Q8) {
    const int8_t* p = static_cast<const int8_t*>(t.p0) + (size_t)row * t.kp + k0;
    c.a = load_nt16(p);
    c.b = load_nt16(p + 16);
    c.d = t.p1[(size_t)row * (t.kp / 32) + k0 / 32];
  } else if constexpr (KIND == KIND_CB4) {
    c.q = load_nt16(static_cast<const uint32_t*>(t.p0) + (size_t)row * (t.kp / 8) + k0 / 8);
    c.sc = t.p1[(size_t)row * (t.kp / 128) + k0 / 128];
  } else if constexpr (KIND == KIND_Q40) {   // k0 is a block start (lanes take 32 columns)
    c.q = load_nt16(static_cast<const uint8_t*>(t.p0) + (size_t)row * (t.kp / 2) + k0 / 2);
    c.d = t.p1[(size_t)row * (t.kp / 32) + k0 / 32];
  } else {
    c.q = load_nt16(static_cast<const uint8_t*>(t.p0) + (size_t)row * (t.kp / 2) + k0 / 2);
    c.lut = load_nt16(t.p1 + ((size_t)row * (t.kp / 64) + g) * 16 + half * 8);
  }
}

// Raw activation chunk of one token: 32 values at k0 (bf16 bits or f32),
// loaded 16 bytes at a time from a clamped address; `live` marks pieces of 8
// columns inside [0, cols).  Requires cols % 8 == 0 and 16-byte rows (vec).
template <bool XBF16>
struct XChunk {
  uint4 u[XBF16 ? 4 : 8];
  uint32_t live;   // bit i: piece i (8 columns) is inside the row
};

template <bool XBF16>
__device__ __forceinline__ void load_x(const void* __restrict__ x, uint32_t cols, int m, uint32_t k0,
                                       XChunk<XBF16>& c) {
  const uint32_t last = cols / 8 - 1;   // last full piece
  c.live = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t piece = k0 / 8 + i;
    c.live |= (piece <= last ? 1u : 0u) << i;
    const uint32_t pc = piece <= last ? piece : last;
    if constexpr (XBF16) {
      c.u[i] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + (size_t)m * cols + pc * 8);
    } else {
      const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(x) + (size_t)m * cols + pc * 8);
      c.u[2 * i] = p[0];
      c.u[2 * i + 1] = p[1];
    }
  }
}

// Element-wise fallback for unaligned rows or cols % 8 != 0.
template <bool XBF16>
__device__ __forceinline__ void load_x_scalar(const void* __restrict__ x, uint32_t cols, int m, uint32_t k0,
                                              float (&xv)[kChunk]) {
#pragma unroll
  for (int j = 0; j < kChunk; ++j) {
    const uint32_t c = k0 + j;
    const uint32_t cc = c < cols ? c : cols - 1;
    float v;
    if constexpr (XBF16)
      v = bf16_to_f32(static_cast<const uint16_t*>(x)[(size_t)m * cols + cc]);
    else
      v = static_cast<const float*>(x)[(size_t)m * cols + cc];
    xv[j] = c < cols ? v : 0.0f;
  }
}

template <bool XBF16>
__device__ __forceinline__ void unpack_x(const XChunk<XBF16>& c, float (&xv)[kChunk]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool live = (c.live >> i) & 1u;
    if constexpr (XBF16) {
      const uint32_t w[4] = {c.u[i].x, c.u[i].y, c.u[i].z, c.u[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xv[8 * i + 2 * j] = live ? __uint_as_float(w[j] << 16) : 0.0f;
        xv[8 * i + 2 * j + 1] = live ? __uint_as_float(w[j] & 0xffff0000u) : 0.0f;
      }
    } else {
      const uint4 a = c.u[2 * i], b = c.u[2 * i + 1];
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[8 * i + j] = live ? __uint_as_float(w[j]) : 0.0f;
    }
  }
}

// g64 codebooks in LDS, laid out so that no lookup conflicts on LDS banks:
// each wave owns 4 KiB blocks of 16 x 64 words, and entry e of lane l's
// table is word e * 64 + l of its block (the low half for one row, the high
// half for the row after it).  The 64 lanes of a wave always read 64
// different words in 64 different banks, whatever the indices; with one
// table per pair of lanes at a fixed stride, random indices put up to ~4
// lanes on one bank.  A table address is then byte 0 = 4 l (+2 for the high
// half), byte 1 = 16 * block | q, which one v_perm_b32 assembles from the
// nibble byte and the lane's base: a lookup costs one VALU operation.
// Blocks must lie below 64 KiB of LDS and start 4 KiB aligned.
constexpr uint32_t kTabBlock = 4096;

// The g64 tables are stored and read through may_alias types: with plain
// types (lookups _Float16, stores uint16_t), type-based alias analysis let the
// compiler move lookups above the stores that fill the table.
typedef uint16_t __attribute__((may_alias)) u16_alias_t;
typedef uint32_t __attribute__((may_alias)) u32_alias_t;
typedef __attribute__((address_space(3))) u16_alias_t lds_u16_t;
typedef __attribute__((address_space(3))) u32_alias_t lds_u32a_t;
typedef __attribute__((address_space(3))) float lds_float_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)((const lds_float_t*)p);
}

// Dequantised chunk -> w[32] (f32).  Scale / validity applied by the caller.
// Table reads use byte addresses base | (q << k) with an aligned base, so the
// address costs one shift and one v_and_or_b32.
template <uint32_t KIND>
__device__ __forceinline__ void dequant_chunk(const WChunk<KIND>& c, uint32_t cbase, uint32_t slot,
                                              uint32_t lane, float (&w)[kChunk]) {
  if constexpr (KIND == KIND_Q8) {
    const uint32_t qa[8] = {c.a.x, c.a.y, c.a.z, c.a.w, c.b.x, c.b.y, c.b.z, c.b.w};
#pragma unroll
    for (int j = 0; j < kChunk; ++j) w[j] = (float)(int8_t)((qa[j >> 2] >> ((j & 3) * 8)) & 0xffu);
  } else if constexpr (KIND == KIND_Q40) {
    // q - 8 of four nibbles at once as signed bytes: (n | 0x80) - 8 stays in
    // its byte (no borrow), and ^ 0x80 turns 0x80 + (n - 8) into n - 8; the
    // byte then converts with one sign-extending SDWA conversion.
    const uint32_t wd[4] = {c.q.x, c.q.y, c.q.z, c.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (((wd[i] & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
      const uint32_t hi = ((((wd[i] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        w[4 * i + k] = (float)(int8_t)((lo >> (8 * k)) & 0xffu);        // column 4 i + k
        w[16 + 4 * i + k] = (float)(int8_t)((hi >> (8 * k)) & 0xffu);   // column 16 + 4 i + k
      }
    }
  } else if constexpr (KIND == KIND_CB4) {
    const uint32_t wd[4] = {c.q.x, c.q.y, c.q.z, c.q.w};
    const uint32_t base = cbase;   // 64-byte aligned table for this row
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const int sh = (j & 7) * 4 - 2;
      const uint32_t off = sh < 0 ? ((wd[j >> 3] << 2) & 0x3cu) : ((wd[j >> 3] >> sh) & 0x3cu);
      w[j] = *(lds_float_t*)(size_t)(base | off);
    }
  } else {
    // slot = the lane's table address for this row: block + 4 lane (+2).
    (void)lane;
    const uint32_t wd[4] = {c.q.x, c.q.y, c.q.z, c.q.w};
    const uint32_t lbyte = slot & 0xffu;
    const uint32_t rep = ((slot >> 8) & 0xffu) * 0x01010101u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t we = (wd[i] & 0x0F0F0F0Fu) | rep;          // nibbles 0, 2, 4, 6 | block
      const uint32_t wo = ((wd[i] >> 4) & 0x0F0F0F0Fu) | rep;   // nibbles 1, 3, 5, 7 | block
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t sel = 0x0c0c0000u | ((4u + k) << 8);   // [lane byte, nibble byte k, 0, 0]
        w[8 * i + 2 * k] = f16_to_f32(*(lds_u16_t*)(size_t)__builtin_amdgcn_perm(we, lbyte, sel));
        w[8 * i + 2 * k + 1] = f16_to_f32(*(lds_u16_t*)(size_t)__builtin_amdgcn_perm(wo, lbyte, sel));
      }
    }
  }
}

// Stores the g64 tables of one row (low halves) or two rows (`b`: high
// halves) into block `blk`.  The two lanes of a 64-group each hold half of
// the group's table (entries 8 (l & 1) ..) and each writes its half into both
// lanes' columns, so no lane exchange is needed.
__device__ __forceinline__ void store_g64_tables(uint32_t blk, uint32_t lane, const WChunk<KIND_G64>& a,
                                                 const WChunk<KIND_G64>* b) {
  const uint32_t half = (lane & 1u) * 2048u;                          // entries 8 (l & 1) .. : words 512 (l & 1) ..
  lds_u32a_t* own = (lds_u32a_t*)(size_t)(blk + lane * 4u + half);    // word e of the column: own[64 e]
  lds_u32a_t* other = (lds_u32a_t*)(size_t)(blk + (lane ^ 1u) * 4u + half);
  const uint32_t A[4] = {a.lut.x, a.lut.y, a.lut.z, a.lut.w};
  uint32_t B[4] = {0, 0, 0, 0};
  if (b) {
    B[0] = b->lut.x; B[1] = b->lut.y; B[2] = b->lut.z; B[3] = b->lut.w;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {   // entry 2j: low halves of A, B; entry 2j + 1: high halves
    const uint32_t ev = b ? __builtin_amdgcn_perm(B[j], A[j], 0x05040100u) : A[j];
    const uint32_t od = b ? __builtin_amdgcn_perm(B[j], A[j], 0x07060302u) : A[j] >> 16;
    own[(2 * j) * 64] = ev;
    own[(2 * j + 1) * 64] = od;
    other[(2 * j) * 64] = ev;
    other[(2 * j + 1) * 64] = od;
  }
}

// Output epilogues.  kEpiPlain: y[m][row] = sum.  kEpiSilu / kEpiGelu: the
// matrix is [gate; up] (rows = 2 * n_ff) and the output is the gated
// activation act[m][i] = f(gate_i) * up_i for i < n_ff, zero for
// n_ff <= i < y_stride -- the fused gate/up kernel of the device runner
// (vxt_cb4_ffn_gu_nr2_m1, vxt_cb4_fast.metal:212-287) with the CPU step's
// activation (llm_cpu.rs:457-464).
enum Epi : int { kEpiPlain = 0, kEpiSilu = 1, kEpiGelu = 2 };

template <int EPI>
__device__ __forceinline__ float gated(float g, float u) {
  return gated_act(g, u, EPI == kEpiGelu);
}

// Output rows of one wave.  Plain: RPW consecutive rows from `first`.  Gated:
// RPW / 2 outputs from `first`, i.e. gate rows first.. and up rows
// n_ff + first..; rows past the end are clamped to a valid row (`valid`
// false), so every load stays in bounds.
template <int EPI, int RPW>
__device__ __forceinline__ void wave_rows(uint32_t first, uint32_t rows, uint32_t n_ff, uint32_t (&rr)[RPW],
                                          bool (&valid)[RPW]) {
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    if constexpr (EPI == kEpiPlain) {
      valid[r] = first + r < rows;
      rr[r] = valid[r] ? first + r : rows - 1;
    } else {
      constexpr int H = RPW / 2;
      const uint32_t o = first + (r % H);
      valid[r] = o < n_ff;
      rr[r] = (r < H ? 0u : n_ff) + (valid[r] ? o : n_ff - 1);
    }
  }
}

// Norm prologue (batch 1): x is not read from memory but built by every
// workgroup as bf16(rms_norm(cur [+ delta]) * w), with the reduction of the
// stand-alone RMSNorm kernel (ffn.hip) step for step -- element i = tid +
// 256 j summed by FMA in ascending j, the DPP wave sum, the four wave sums
// added in order -- so x is bit-identical to that kernel's bf16 output.
// Workgroup 0 also stores cur + delta to cur_out (the residual stream).
// Inputs: NormIn (common.hpp).
constexpr uint32_t kNormPer = 16;   // most elements per thread: cols <= 4096

// The norm arithmetic on the values the caller loaded (element i = tid +
// 256 j), then x in LDS: bf16 for i < cols, zero up to xlen.  Ends with a
// barrier, so the caller reads s_xn right after.
template <uint32_t NP>
__device__ __forceinline__ void norm_prologue(const NormIn& nin, uint32_t cols, uint32_t xlen, const float (&c)[NP],
                                              const float (&d)[NP], const float (&w)[NP], uint16_t* s_xn) {
#pragma clang fp contract(off)
  __shared__ float s_part[kWaves];
  const uint32_t tid = threadIdx.x;
  const bool add = nin.delta != nullptr;
  float v[NP];
  float sq = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < NP; ++j) {
    v[j] = add ? c[j] + d[j] : c[j];
    if (tid + 256u * j < cols) sq = __builtin_fmaf(v[j], v[j], sq);
  }
  sq = wave_sum(sq);
  if ((tid & 63u) == 0) s_part[tid >> 6] = sq;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < kWaves; ++k) total += s_part[k];
  const float scale = 1.0f / sqrtf(total / (float)cols + nin.eps);
  const bool store = add && blockIdx.x == 0;
#pragma unroll
  for (uint32_t j = 0; j < NP; ++j) {
    const uint32_t i = tid + 256u * j;
    if (i < cols) {
      s_xn[i] = f32_to_bf16(v[j] * scale * w[j]);
      if (store) nin.cur_out[i] = v[j];
    } else if (i < xlen) {
      s_xn[i] = 0;
    }
  }
  for (uint32_t i = tid + 256u * NP; i < xlen; i += 256u) s_xn[i] = 0;
  __syncthreads();
}

// 32 bf16 activations at k0 from the LDS copy (64 bytes, 16-byte aligned).
__device__ __forceinline__ void read_x_lds(const uint16_t* s_xn, uint32_t k0, float (&xv)[kChunk]) {
  typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
  const uint32_t base = lds_addr(s_xn) + k0 * 2u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 q = *(lds_u32x4*)(size_t)(base + 16u * i);
    const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv[8 * i + 2 * j] = __uint_as_float(wv[j] << 16);
      xv[8 * i + 2 * j + 1] = __uint_as_float(wv[j] & 0xffff0000u);
    }
  }
}

// Kernel: MT tokens (MT in {1,2,4,8}; m >= M_rt are padding), RPW rows per
// wave, up to S steps per batch.  Gated epilogues take n_ff and the output
// row stride; the plain epilogue ignores both.  NORM: the norm prologue above
// (MT = 1, bf16 x staged in dynamic LDS of nsteps * kStep elements).
// KS > 1 (split K): the workgroup's KS waves share its RPW rows, wave w
// taking the K steps w, w + KS, ...; their sums are added through LDS in
// wave order (deterministic), so a matrix of few rows and long K spreads over
// KS times more waves, each with a KS times shorter chain after its data.
template <uint32_t KIND, int MT, int RPW, int S, bool XBF16, int EPI = kEpiPlain, bool NORM = false,
          uint32_t NP = kNormPer, int KS = 1>
__global__ __launch_bounds__(kWaves * 64) void gemv_kernel(DevTensor t, const void* __restrict__ x,
                                                          void* __restrict__ y, uint32_t M_rt,
                                                          uint32_t y_bf16, uint32_t x_vec, uint32_t n_ff = 0,
                                                          uint32_t y_stride = 0, NormIn nin = {}) {
  static_assert(EPI == kEpiPlain || RPW % 2 == 0, "gated rows come in gate/up pairs");
  static_assert(!NORM || (MT == 1 && XBF16), "the norm prologue serves one token with bf16 x");
  static_assert(KS == 1 || (S == 1 && EPI == kEpiPlain && !NORM && KS <= kWaves), "split K: plain, one step a batch");
  extern __shared__ __attribute__((aligned(16))) uint16_t s_xn[];
  __shared__ __attribute__((aligned(64))) float s_cent[48];
  constexpr int NB = (RPW + 1) / 2;   // g64 table blocks per wave
  static_assert(kWaves * NB * kTabBlock + kTabBlock <= 65536u, "g64 table blocks must stay below 64 KiB of LDS");
  __shared__ __attribute__((aligned(KIND == KIND_G64 ? 4096 : 16))) uint32_t s_tab[KIND == KIND_G64 ? kWaves * NB * kTabBlock / 4 : 1];

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = threadIdx.x >> 6;
  constexpr uint32_t kOut = EPI == kEpiPlain ? RPW : RPW / 2;   // outputs per wave
  const uint32_t first = KS > 1 ? blockIdx.x * kOut : (blockIdx.x * kWaves + wave) * kOut;
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t nsteps = (kp + kStep - 1) / kStep;
  constexpr bool kLateX = MT >= 4;
  uint32_t rr[RPW];
  bool rv[RPW];
  wave_rows<EPI, RPW>(first, rows, n_ff, rr, rv);

  if constexpr (KIND == KIND_CB4) {   // before any global load is in flight
    if (threadIdx.x < 48) s_cent[threadIdx.x] = t.cent[threadIdx.x];
    __syncthreads();
  }
  const uint32_t tab = lds_addr(s_tab) + (KIND == KIND_G64 ? wave * NB * kTabBlock : 0);

  // cb4 residuals: each row's CSR bounds are requested before anything else
  // and each lane's first entry right after the first batch of weights, so
  // only the activation read of the residual is left after the last weight.
  uint32_t os[RPW], oe[RPW], pk0[RPW];
  if constexpr (KIND == KIND_CB4) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      os[r] = t.row_ptr[rr[r]];
      oe[r] = t.row_ptr[rr[r] + 1];
    }
  }

  // Norm inputs are requested before any weight, so waiting for them leaves
  // the weight loads in flight.
  float n_c[NORM ? NP : 1], n_d[NORM ? NP : 1], n_w[NORM ? NP : 1];
  if constexpr (NORM) {
#pragma unroll
    for (uint32_t j = 0; j < NP; ++j) {
      const uint32_t i = threadIdx.x + 256u * j;
      const uint32_t ic = i < cols ? i : cols - 1;
      n_c[j] = nin.cur[ic];
      n_w[j] = nin.w[ic];
    }
    if (nin.delta) {
#pragma unroll
      for (uint32_t j = 0; j < NP; ++j) {
        const uint32_t i = threadIdx.x + 256u * j;
        n_d[j] = nin.delta[i < cols ? i : cols - 1];
      }
    }
  }

  float acc[RPW][MT];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

  for (uint32_t s0 = KS > 1 ? wave : 0u; s0 < nsteps; s0 += KS > 1 ? (uint32_t)KS : (uint32_t)S) {
    const uint32_t ns = nsteps - s0 < (uint32_t)S ? nsteps - s0 : (uint32_t)S;   // uniform
    // ---- issue: activations, then weights, for every step of the batch
    XChunk<XBF16> xc[kLateX ? 1 : S][kLateX ? 1 : MT];
    WChunk<KIND> wc[S][RPW];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (!NORM && !kLateX && (uint32_t)s < ns && x_vec) {
        const uint32_t k0 = (s0 + s) * kStep + lane * kChunk;
#pragma unroll
        for (int m = 0; m < MT; ++m)
          load_x<XBF16>(x, cols, (uint32_t)m < M_rt ? m : 0, k0, xc[kLateX ? 0 : s][kLateX ? 0 : m]);
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if ((uint32_t)s < ns) {
        const uint32_t k0 = (s0 + s) * kStep + lane * kChunk;
        const uint32_t k0c = k0 < kp ? k0 : kp - kChunk;
        const uint32_t gmax = kp / 64 - 1;
        const uint32_t g = (s0 + s) * 32 + (lane >> 1);
#pragma unroll
        for (int r = 0; r < RPW; ++r) load_chunk<KIND>(t, rr[r], k0c, g < gmax ? g : gmax, lane & 1, wc[s][r]);
      }
    }
    if constexpr (KIND == KIND_CB4) {
      if (s0 == (KS > 1 ? wave : 0u)) {   // clamped, unconditional (the CSR stream holds at least one word)
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const uint32_t i = os[r] + (KS > 1 ? wave * 64u : 0u) + lane;
          const uint32_t last = oe[r] > 0 ? oe[r] - 1 : 0;
          pk0[r] = t.outliers[i < oe[r] ? i : (os[r] < oe[r] ? last : 0)];
        }
      }
    }
    if constexpr (NORM) {
      if (s0 == 0) norm_prologue<NP>(nin, cols, nsteps * kStep, n_c, n_d, n_w, s_xn);
    }
    // ---- consume
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if ((uint32_t)s >= ns) break;
      const uint32_t k0 = (s0 + s) * kStep + lane * kChunk;
      const bool kin = k0 < kp;
      // Early x: every token unpacked once per step.  Late x (MT >= 4): each
      // token is loaded and unpacked where it is used, so the registers hold
      // one token's 32 values at a time.
      float xv[kLateX ? 1 : MT][kChunk];
      if constexpr (NORM) {
        read_x_lds(s_xn, k0, xv[0]);
      } else if constexpr (!kLateX) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (x_vec)
            unpack_x<XBF16>(xc[s][m], xv[m]);
          else
            load_x_scalar<XBF16>(x, cols, (uint32_t)m < M_rt ? m : 0, k0, xv[m]);
        }
      }
      if constexpr (KIND == KIND_G64) {   // this step's tables; a wave's LDS operations run in
#pragma unroll                         // order, so the previous step's lookups are done first
        for (int p = 0; p < NB; ++p)
          store_g64_tables(tab + p * kTabBlock, lane, wc[s][2 * p], 2 * p + 1 < RPW ? &wc[s][2 * p + 1] : nullptr);
      }
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const uint32_t sl = tab + (r / 2) * kTabBlock + lane * 4u + (r & 1) * 2u;
        uint32_t cbase = 0;
        if constexpr (KIND == KIND_CB4) cbase = lds_addr(s_cent) + 64u * cent_table(t, rr[r]);
        float w[kChunk];
        dequant_chunk<KIND>(wc[s][r], cbase, sl, lane, w);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float* xm = xv[kLateX ? 0 : m];
          if constexpr (kLateX) {
            const uint32_t mm = (uint32_t)m < M_rt ? m : 0;
            if (x_vec) {
              XChunk<XBF16> c;
              load_x<XBF16>(x, cols, mm, k0, c);
              unpack_x<XBF16>(c, xv[0]);
            } else {
              load_x_scalar<XBF16>(x, cols, mm, k0, xv[0]);
            }
          }
          float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
          for (int j = 0; j < kChunk; j += 2) {
            p0 = __builtin_fmaf(w[j], xm[j], p0);
            p1 = __builtin_fmaf(w[j + 1], xm[j + 1], p1);
          }
          float p = p0 + p1;
          if constexpr (KIND == KIND_Q8 || KIND == KIND_Q40) {
            p *= f16_to_f32(wc[s][r].d);
          } else if constexpr (KIND == KIND_CB4) {
            // codebook.rs:384-386: a zero scale skips the group.
            const float sc = f16_to_f32(wc[s][r].sc);
            p = sc != 0.0f ? sc * p : 0.0f;
          }
          acc[r][m] += kin ? p : 0.0f;
        }
      }
    }
  }

  if constexpr (KIND == KIND_CB4) {
    // CSR residuals (codebook.rs:409-415): y += f16(res) * x[col]; lane l
    // takes entries l, l + 64, ... of the row, in that order (split K: wave
    // w takes entries 64 w + l, stepping by 64 KS).
    const uint32_t r_first = KS > 1 ? wave * 64u : 0u;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      if (!rv[r]) {
        if constexpr (EPI == kEpiPlain) break;   // later rows are past the end too
        continue;
      }
      for (uint32_t i = os[r] + r_first + lane; i < oe[r]; i += 64u * KS) {
        const uint32_t pk = i < os[r] + r_first + 64 ? pk0[r] : t.outliers[i];
        const uint32_t col = pk & 0xffffu;
        if (col >= cols) continue;
        const float val = f16_to_f32(pk >> 16);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const uint32_t mm = (uint32_t)m < M_rt ? m : 0;
          float xc;
          if constexpr (NORM)
            xc = bf16_to_f32(s_xn[col]);
          else if constexpr (XBF16)
            xc = bf16_to_f32(static_cast<const uint16_t*>(x)[(size_t)mm * cols + col]);
          else
            xc = static_cast<const float*>(x)[(size_t)mm * cols + col];
          acc[r][m] = __builtin_fmaf(val, xc, acc[r][m]);
        }
      }
    }
  }

  if constexpr (KS > 1) {   // the waves' sums, added in wave order
    __shared__ float s_part[KS > 1 ? KS * RPW * MT : 1];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float v = wave_sum(acc[r][m]);
        if (lane == 0) s_part[(wave * RPW + r) * MT + m] = v;
      }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float v = s_part[r * MT + m];
#pragma unroll
        for (int w = 1; w < KS; ++w) v += s_part[(w * RPW + r) * MT + m];
        if (lane == 0 && rv[r] && (uint32_t)m < M_rt) {
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * rows + rr[r]] = f32_to_bf16(v);
          else
            static_cast<float*>(y)[(size_t)m * rows + rr[r]] = v;
        }
      }
  } else if constexpr (EPI == kEpiPlain) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float v = wave_sum(acc[r][m]);
        if (lane == 0 && rv[r] && (uint32_t)m < M_rt) {
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * rows + rr[r]] = f32_to_bf16(v);
          else
            static_cast<float*>(y)[(size_t)m * rows + rr[r]] = v;
        }
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < (int)kOut; ++h) {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float g = wave_sum(acc[h][m]);
        const float u = wave_sum(acc[h + kOut][m]);
        if (lane == 0 && rv[h] && (uint32_t)m < M_rt) {
          const float v = gated<EPI>(g, u);
          const size_t at = (size_t)m * y_stride + first + h;
          if (y_bf16)
            static_cast<uint16_t*>(y)[at] = f32_to_bf16(v);
          else
            static_cast<float*>(y)[at] = v;
        }
      }
    }
    if (blockIdx.x == 0) {   // zero padding columns [n_ff, y_stride) of every token
      for (uint32_t m = 0; m < M_rt; ++m)
        for (uint32_t c = n_ff + threadIdx.x; c < y_stride; c += kWaves * 64) {
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * y_stride + c] = 0;
          else
            static_cast<float*>(y)[(size_t)m * y_stride + c] = 0.0f;
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Q8 weights x bf16 activations: packed bf16 dot products.
//
// An int8 weight is exact in bf16 (at most 8 significant bits), and bf16 x
// needs no conversion, so each pair of columns costs one v_dot2_f32_bf16 per
// token (the products are exact, the sum is fp32) instead of two FMAs plus
// two unpacks.  Weights are converted once per row-step (int8 -> f32 via
// SDWA, then the high halves of two f32 packed by one v_perm), and x stays in
// its packed bf16 form in registers.  Block scale, masking and the final
// wave reduction are as in gemv_kernel.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

// Columns (2j, 2j+1) of a Q8 chunk as a packed bf16 pair (low half = even column).
__device__ __forceinline__ void q8_pairs(const WChunk<KIND_Q8>& c, uint32_t (&qp)[kChunk / 2]) {
  const uint32_t wd[8] = {c.a.x, c.a.y, c.a.z, c.a.w, c.b.x, c.b.y, c.b.z, c.b.w};
#pragma unroll
  for (int j = 0; j < kChunk / 2; ++j) {
    const uint32_t w = wd[j >> 1];
    const int sh = (j & 1) * 16;
    const float lo = (float)(int8_t)((w >> sh) & 0xffu);
    const float hi = (float)(int8_t)((w >> (sh + 8)) & 0xffu);
    qp[j] = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
  }
}

// One token's 32 bf16 activations at k0 as 16 packed pairs, zero outside
// [0, cols).  The token's row is a raw buffer (base and byte size in SGPRs):
// offsets are 32-bit per lane, and the hardware returns zeros for any part
// of a load at or past the row's end, so no clamping or masking is needed.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t x_row_rsrc(const uint16_t* x, uint32_t cols, uint32_t m) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x + (size_t)m * cols), (short)0,
                                           (int)(cols * 2u), 0x00020000);
}

__device__ __forceinline__ void load_x_pairs(__amdgpu_buffer_rsrc_t r, uint32_t k0, uint32_t x_vec,
                                             uint32_t (&xp)[kChunk / 2]) {
  if (x_vec) {   // cols % 8 == 0: each 16-byte piece is wholly inside or outside the row
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (k0 + 8u * i) * 2u, 0, 0);
      xp[4 * i + 0] = v.x;
      xp[4 * i + 1] = v.y;
      xp[4 * i + 2] = v.z;
      xp[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kChunk / 2; ++j) {
      const uint32_t v0 = __builtin_amdgcn_raw_buffer_load_b16(r, (k0 + 2u * j) * 2u, 0, 0);
      const uint32_t v1 = __builtin_amdgcn_raw_buffer_load_b16(r, (k0 + 2u * j + 1u) * 2u, 0, 0);
      xp[j] = (v0 & 0xffffu) | (v1 << 16);
    }
  }
}

template <int MT, int RPW, int S>
__global__ __launch_bounds__(kWaves * 64) void gemv_q8_dot2_kernel(DevTensor t, const uint16_t* __restrict__ x,
                                                                  void* __restrict__ y, uint32_t M_rt,
                                                                  uint32_t y_bf16, uint32_t x_vec) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t row0 = (blockIdx.x * kWaves + wave) * RPW;
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t nsteps = (kp + kStep - 1) / kStep;

  float acc[RPW][MT];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

  for (uint32_t s0 = 0; s0 < nsteps; s0 += S) {
    const uint32_t ns = nsteps - s0 < (uint32_t)S ? nsteps - s0 : (uint32_t)S;   // uniform
    // Per step: the activations, then the weights, so that consuming step s
    // waits only for loads issued up to step s (the memory counter drains in
    // issue order).
    uint32_t xp[S][MT][kChunk / 2];
    WChunk<KIND_Q8> wc[S][RPW];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if ((uint32_t)s < ns) {
        const uint32_t k0 = (s0 + s) * kStep + lane * kChunk;
#pragma unroll
        for (int m = 0; m < MT; ++m) load_x_pairs(x_row_rsrc(x, cols, (uint32_t)m < M_rt ? m : 0), k0, x_vec, xp[s][m]);
        const uint32_t k0c = k0 < kp ? k0 : kp - kChunk;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const uint32_t row = row0 + r < rows ? row0 + r : rows - 1;
          load_chunk<KIND_Q8>(t, row, k0c, 0, 0, wc[s][r]);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if ((uint32_t)s >= ns) break;
      const bool kin = (s0 + s) * kStep + lane * kChunk < kp;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        uint32_t qp[kChunk / 2];
        q8_pairs(wc[s][r], qp);
        const float d = f16_to_f32(wc[s][r].d);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
          for (int j = 0; j < kChunk / 2; j += 2) {
            p0 = dot2_bf16(qp[j], xp[s][m][j], p0);
            p1 = dot2_bf16(qp[j + 1], xp[s][m][j + 1], p1);
          }
          acc[r][m] += kin ? (p0 + p1) * d : 0.0f;
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint32_t row = row0 + r;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float v = wave_sum(acc[r][m]);
      if (lane == 0 && row < rows && (uint32_t)m < M_rt) {
        if (y_bf16)
          static_cast<uint16_t*>(y)[(size_t)m * rows + row] = f32_to_bf16(v);
        else
          static_cast<float*>(y)[(size_t)m * rows + row] = v;
      }
    }
  }
}

// Larger batches (M >= 4): the same dot2 arithmetic with the activations
// staged in LDS once per workgroup.  Reading x straight from L2 costs
// M * K * 2 bytes per wave, which at M = 8 is four times the weight bytes a
// wave streams, and L2 bandwidth, not HBM, sets the time.  Workgroups are
// persistent: each stages x (all M tokens, all of K: kp <= 3 * kStep) once and
// then walks row blocks with a stride of the grid size.
template <int MT, int RPW, int WAVES, int NS>
__global__ __launch_bounds__(WAVES * 64) void gemv_q8_lds_kernel(DevTensor t, const uint16_t* __restrict__ x,
                                                                void* __restrict__ y, uint32_t M_rt,
                                                                uint32_t y_bf16, uint32_t x_vec) {
  extern __shared__ __attribute__((aligned(16))) uint32_t s_x[];   // [MT][kp / 2] packed bf16 pairs
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t kpw = kp / 2;
  const uint32_t nblocks = (rows + WAVES * RPW - 1) / (WAVES * RPW);

  // First row block's weights go out before the activations are staged.
  WChunk<KIND_Q8> wc[NS][RPW];
  auto issue = [&](uint32_t b) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint32_t k0 = s * kStep + lane * kChunk;
      const uint32_t k0c = k0 < kp ? k0 : kp - kChunk;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const uint32_t row = (b * WAVES + wave) * RPW + r;
        load_chunk<KIND_Q8>(t, row < rows ? row : rows - 1, k0c, 0, 0, wc[s][r]);
      }
    }
  };
  if (blockIdx.x < nblocks) issue(blockIdx.x);

  // Stage x: 8-column pieces, zero outside [0, cols) (raw-buffer bounds).
  const uint32_t ppr = kp / 8;   // pieces per token row
  for (uint32_t p = tid; p < MT * ppr; p += WAVES * 64) {
    const uint32_t m = p / ppr, pc = p - m * ppr;
    const __amdgpu_buffer_rsrc_t r = x_row_rsrc(x, cols, m < M_rt ? m : 0);
    u32x4 v;
    if (x_vec) {
      v = __builtin_amdgcn_raw_buffer_load_b128(r, pc * 16u, 0, 0);
    } else {
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = __builtin_amdgcn_raw_buffer_load_b16(r, (pc * 8u + j) * 2u, 0, 0) & 0xffffu;
      v = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    }
    *reinterpret_cast<u32x4*>(&s_x[m * kpw + pc * 4]) = v;
  }
  __syncthreads();

  for (uint32_t b = blockIdx.x; b < nblocks; b += gridDim.x) {
    float acc[RPW][MT];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint32_t k0 = s * kStep + lane * kChunk;
      const bool kin = k0 < kp;
      const uint32_t k0c = kin ? k0 : kp - kChunk;
      uint32_t qp[RPW][kChunk / 2];
      float d[RPW];
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        q8_pairs(wc[s][r], qp[r]);
        d[r] = f16_to_f32(wc[s][r].d);
      }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        uint32_t xp[kChunk / 2];
        const u32x4* src = reinterpret_cast<const u32x4*>(&s_x[m * kpw + k0c / 2]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 v = src[i];
          xp[4 * i] = v.x;
          xp[4 * i + 1] = v.y;
          xp[4 * i + 2] = v.z;
          xp[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
          for (int j = 0; j < kChunk / 2; j += 2) {
            p0 = dot2_bf16(qp[r][j], xp[j], p0);
            p1 = dot2_bf16(qp[r][j + 1], xp[j + 1], p1);
          }
          acc[r][m] += kin ? (p0 + p1) * d[r] : 0.0f;
        }
      }
    }
    const uint32_t row0 = (b * WAVES + wave) * RPW;
    if (b + gridDim.x < nblocks) issue(b + gridDim.x);   // next block's weights in flight during the reduction
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const uint32_t row = row0 + r;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float v = wave_sum(acc[r][m]);
        if (lane == 0 && row < rows && (uint32_t)m < M_rt) {
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * rows + row] = f32_to_bf16(v);
          else
            static_cast<float*>(y)[(size_t)m * rows + row] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Q8 weights x f32 (or bf16) activations, one token, 1..3 K steps
// (K <= 6144; config 0 is 4096 x 4096 with f32 activations).  With the activations read straight from L2, every wave
// of the generic kernel re-reads the whole f32 row (16 KB at K = 4096, as many
// bytes as its four weight rows) and waits for 30-odd loads at once; a timed
// trace of that kernel on MI355X showed no wave holding all its data before
// 4.4 us of an 8 us call.  Here the workgroup stages the row once into LDS
// (16-byte pieces, zero past `cols` by the raw-buffer bounds), each wave
// holds RPW rows, every load is unconditional (clamped rows and columns), and
// step s is multiplied as soon as its own weights have landed.  Lane l reads
// the 32 columns it multiplies as 8 pieces, piece i of lane l stored at slot
// 8 l + (i ^ ((l >> 1) & 7)) of its step's block, so 16 consecutive lanes
// reading piece i touch 16 different 16-byte bank groups.  Products and the
// order of the sums are those of the generic kernel (two fp32 chains per
// lane, the block scale on their sum, steps in order, the wave sum).
// The same kernel serves Q4_0 weights (KB = KIND_Q40): 16 bytes of nibbles
// and one scale per lane and block instead of 32 int8 values.
template <int RPW, int WAVES, int NS, bool XBF16 = false, uint32_t KB = KIND_Q8>
__global__ __launch_bounds__(WAVES * 64) void gemv_q8_m1_kernel(DevTensor t, const void* __restrict__ x,
                                                                 void* __restrict__ y, uint32_t y_bf16) {
  static_assert(NS >= 1 && NS <= 3, "K steps staged in LDS");
  static_assert(KB == KIND_Q8 || KB == KIND_Q40, "block kinds");
  __shared__ __attribute__((aligned(16))) float s_x[NS * kStep];
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t row0 = (blockIdx.x * WAVES + wave) * RPW;

  // Activations first (their wait then leaves the weights in flight).  A
  // load piece is 16 bytes: 4 f32 or 8 bf16 columns (bf16 is widened to f32,
  // exactly, as it is stored: two LDS pieces).
  constexpr uint32_t kCols = XBF16 ? 8 : 4;
  constexpr uint32_t kPieces = NS * kStep / kCols;
  constexpr uint32_t kPer = (kPieces + WAVES * 64 - 1) / (WAVES * 64);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(x), (short)0,
                                                                     (int)(cols * (XBF16 ? 2u : 4u)), 0x00020000);
  u32x4 xv[kPer];
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t p = std::min(tid + WAVES * 64 * j, kPieces - 1);   // repeats write the same value
    xv[j] = __builtin_amdgcn_raw_buffer_load_b128(xr, p * 16u, 0, 0);
  }
  WChunk<KB> wc[NS][RPW];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t k0 = s * kStep + lane * kChunk;
    const uint32_t k0c = k0 < kp ? k0 : kp - kChunk;
#pragma unroll
    for (int r = 0; r < RPW; ++r) load_chunk<KB>(t, std::min(row0 + r, rows - 1), k0c, 0, 0, wc[s][r]);
  }
  // Nothing that uses a loaded value may be scheduled above the last load:
  // a conversion hoisted there makes the wave wait for the loads before it.
  __builtin_amdgcn_sched_barrier(0);
  auto put = [&](uint32_t p, const u32x4& v) {   // f32 piece p (4 columns) to its slot
    const uint32_t blk = p / 512u, l = (p % 512u) / 8u, i = p % 8u;
    *reinterpret_cast<u32x4*>(&s_x[(blk * 512u + 8u * l + (i ^ ((l >> 1) & 7u))) * 4u]) = v;
  };
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t p = std::min(tid + WAVES * 64 * j, kPieces - 1);
    if constexpr (XBF16) {
      const u32x4 v = xv[j];
      put(2 * p, u32x4{v.x << 16, v.x & 0xffff0000u, v.y << 16, v.y & 0xffff0000u});
      put(2 * p + 1, u32x4{v.z << 16, v.z & 0xffff0000u, v.w << 16, v.w & 0xffff0000u});
    } else {
      put(p, xv[j]);
    }
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);   // the barrier waits for the activations only

  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  const uint32_t swl = (lane >> 1) & 7u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool kin = s * kStep + lane * kChunk < kp;
    float xf[kChunk];
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&s_x[(s * 512u + 8u * lane + (i ^ swl)) * 4u]);
      xf[4 * i] = __uint_as_float(v.x);
      xf[4 * i + 1] = __uint_as_float(v.y);
      xf[4 * i + 2] = __uint_as_float(v.z);
      xf[4 * i + 3] = __uint_as_float(v.w);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float w[kChunk];
      dequant_chunk<KB>(wc[s][r], 0, 0, lane, w);
      float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
      for (int j = 0; j < kChunk; j += 2) {
        p0 = __builtin_fmaf(w[j], xf[j], p0);
        p1 = __builtin_fmaf(w[j + 1], xf[j + 1], p1);
      }
      const float p = (p0 + p1) * f16_to_f32(wc[s][r].d);
      acc[r] += kin ? p : 0.0f;
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float v = wave_sum(acc[r]);
    const uint32_t row = row0 + r;
    if (lane == 0 && row < rows) {
      if (y_bf16)
        static_cast<uint16_t*>(y)[row] = f32_to_bf16(v);
      else
        static_cast<float*>(y)[row] = v;
    }
  }
}

// An empty asm that takes the four words: the compiler cannot move a use of
// them (or the wait for the load that produced them) above this point.
__device__ __forceinline__ void opaque4(uint4& v) {
  uint32_t a = v.x, b = v.y, c = v.z, d = v.w;
  asm volatile("" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
  v = make_uint4(a, b, c, d);
}

// ---------------------------------------------------------------------------
// cb4-g64 weights x bf16 (or f32) activations, one token, 1..3 K steps: the
// structure of gemv_q8_m1_kernel (activations staged once per workgroup,
// widened to f32 in swizzled LDS; every load unconditional; RPW rows per
// wave) with the g64 decode of gemv_kernel (each wave's transposed table
// blocks in LDS, one v_perm_b32 address per lookup).  Products and summation
// order are those of gemv_kernel.
template <int RPW, int WAVES, int NS, bool XBF16 = true>
__global__ __launch_bounds__(WAVES * 64) void gemv_g64_m1_kernel(DevTensor t, const void* __restrict__ x,
                                                                void* __restrict__ y, uint32_t y_bf16) {
  static_assert(NS >= 1 && NS <= 3, "K steps staged in LDS");
  constexpr int NB = (RPW + 1) / 2;   // table blocks per wave
  static_assert(WAVES * NB * kTabBlock <= 65536u, "g64 table blocks must stay below 64 KiB of LDS");
  // One array, so the table blocks start at LDS offset 0 (a lookup address
  // keeps only its low 16 bits) and the activations follow them.
  __shared__ __attribute__((aligned(4096))) uint32_t s_mem[WAVES * NB * kTabBlock / 4 + NS * kStep];
  uint32_t* const s_tab = s_mem;
  float* const s_x = reinterpret_cast<float*>(s_mem + WAVES * NB * kTabBlock / 4);
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t row0 = (blockIdx.x * WAVES + wave) * RPW;

  constexpr uint32_t kXB = XBF16 ? 2u : 4u;                 // bytes per activation
  constexpr uint32_t kPieces = NS * kStep * kXB / 16u;      // 16-byte pieces of activations
  constexpr uint32_t kPer = (kPieces + WAVES * 64 - 1) / (WAVES * 64);
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(x), (short)0, (int)(cols * kXB), 0x00020000);
  u32x4 xv[kPer];
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t p = std::min(tid + WAVES * 64 * j, kPieces - 1);   // repeats write the same value
    xv[j] = __builtin_amdgcn_raw_buffer_load_b128(xr, p * 16u, 0, 0);
  }
  WChunk<KIND_G64> wc[NS][RPW];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t k0 = s * kStep + lane * kChunk;
    const uint32_t k0c = k0 < kp ? k0 : kp - kChunk;
    const uint32_t gmax = kp / 64 - 1;
    const uint32_t g = s * 32 + (lane >> 1);
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      load_chunk<KIND_G64>(t, std::min(row0 + r, rows - 1), k0c, g < gmax ? g : gmax, lane & 1, wc[s][r]);
  }
  // Nothing that uses a loaded value may be scheduled above the last load.
  __builtin_amdgcn_sched_barrier(0);
  auto put = [&](uint32_t p, const u32x4& v) {   // f32 piece p (4 columns) to its slot
    const uint32_t blk = p / 512u, l = (p % 512u) / 8u, i = p % 8u;
    *reinterpret_cast<u32x4*>(&s_x[(blk * 512u + 8u * l + (i ^ ((l >> 1) & 7u))) * 4u]) = v;
  };
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t p = std::min(tid + WAVES * 64 * j, kPieces - 1);
    const u32x4 v = xv[j];
    if constexpr (XBF16) {
      put(2 * p, u32x4{v.x << 16, v.x & 0xffff0000u, v.y << 16, v.y & 0xffff0000u});
      put(2 * p + 1, u32x4{v.z << 16, v.z & 0xffff0000u, v.w << 16, v.w & 0xffff0000u});
    } else {
      put(p, v);
    }
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);   // the barrier waits for the activations only

  const uint32_t tab = lds_addr(s_tab) + wave * NB * kTabBlock;
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  const uint32_t swl = (lane >> 1) & 7u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool kin = s * kStep + lane * kChunk < kp;
    // The step's activations first: they are in LDS already, so their reads
    // go out before the wait for this step's weights.
    float xf[kChunk];
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&s_x[(s * 512u + 8u * lane + (i ^ swl)) * 4u]);
      xf[4 * i] = __uint_as_float(v.x);
      xf[4 * i + 1] = __uint_as_float(v.y);
      xf[4 * i + 2] = __uint_as_float(v.z);
      xf[4 * i + 3] = __uint_as_float(v.w);
    }
    // The weights enter the computation only here (an empty asm that takes
    // them), so nothing derived from them -- and no wait for them -- is
    // placed above the activation reads.
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      opaque4(wc[s][r].q);
      opaque4(wc[s][r].lut);
    }
    __builtin_amdgcn_sched_barrier(0);
    // this step's tables (the wave's LDS operations run in order, so the
    // previous step's lookups are done first)
#pragma unroll
    for (int p = 0; p < NB; ++p)
      store_g64_tables(tab + p * kTabBlock, lane, wc[s][2 * p], 2 * p + 1 < RPW ? &wc[s][2 * p + 1] : nullptr);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const uint32_t sl = tab + (r / 2) * kTabBlock + lane * 4u + (r & 1) * 2u;
      float w[kChunk];
      dequant_chunk<KIND_G64>(wc[s][r], 0, sl, lane, w);
      float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
      for (int j = 0; j < kChunk; j += 2) {
        p0 = __builtin_fmaf(w[j], xf[j], p0);
        p1 = __builtin_fmaf(w[j + 1], xf[j + 1], p1);
      }
      acc[r] += kin ? p0 + p1 : 0.0f;
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float v = wave_sum(acc[r]);
    const uint32_t row = row0 + r;
    if (lane == 0 && row < rows) {
      if (y_bf16)
        static_cast<uint16_t*>(y)[row] = f32_to_bf16(v);
      else
        static_cast<float*>(y)[row] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Q8 weights x bf16 activations, MT tokens (2..8), 1..3 K steps: the
// structure of gemv_q8_m1_kernel (every token's row staged once per workgroup
// in LDS, as packed bf16 pairs; every load unconditional; RPW rows per wave)
// with the arithmetic of gemv_q8_dot2_kernel (v_dot2_f32_bf16 on int8 pairs
// widened to bf16, the block scale on the two chains' sum).  Lane l reads its
// 32 columns of a token as 4 pieces, piece i stored at slot
// 4 l + (i ^ ((l >> 2) & 3)) of the token's step block, so 16 consecutive
// lanes reading piece i touch 16 different 16-byte bank groups.
template <int MT, int RPW, int WAVES, int NS>
__global__ __launch_bounds__(WAVES * 64) void gemv_q8_mt_kernel(DevTensor t, const uint16_t* __restrict__ x,
                                                               void* __restrict__ y, uint32_t M_rt, uint32_t y_bf16) {
  static_assert(NS >= 1 && NS <= 3 && MT >= 2 && MT <= 8, "tokens and K steps staged in LDS");
  constexpr uint32_t kBlk = kStep / 8;   // 16-byte pieces of one token's step block
  __shared__ __attribute__((aligned(16))) uint32_t s_x[MT * NS * kStep / 2];
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t row0 = (blockIdx.x * WAVES + wave) * RPW;

  constexpr uint32_t kPieces = MT * NS * kBlk;
  constexpr uint32_t kPer = (kPieces + WAVES * 64 - 1) / (WAVES * 64);
  u32x4 xv[kPer];
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t p = std::min(tid + WAVES * 64 * j, kPieces - 1);   // repeats write the same value
    const uint32_t m = p / (NS * kBlk), q = p % (NS * kBlk);
    xv[j] = __builtin_amdgcn_raw_buffer_load_b128(x_row_rsrc(x, cols, m < M_rt ? m : 0), q * 16u, 0, 0);
  }
  WChunk<KIND_Q8> wc[NS][RPW];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t k0 = s * kStep + lane * kChunk;
    const uint32_t k0c = k0 < kp ? k0 : kp - kChunk;
#pragma unroll
    for (int r = 0; r < RPW; ++r) load_chunk<KIND_Q8>(t, std::min(row0 + r, rows - 1), k0c, 0, 0, wc[s][r]);
  }
  // Nothing that uses a loaded value may be scheduled above the last load.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t p = std::min(tid + WAVES * 64 * j, kPieces - 1);
    const uint32_t mb = p / kBlk, q = p % kBlk, l = q / 4u, i = q % 4u;   // mb = token * NS + step
    *reinterpret_cast<u32x4*>(&s_x[(mb * kBlk + 4u * l + (i ^ ((l >> 2) & 3u))) * 4u]) = xv[j];
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);   // the barrier waits for the activations only

  float acc[RPW][MT];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
  const uint32_t swl = (lane >> 2) & 3u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool kin = s * kStep + lane * kChunk < kp;
    uint32_t qp[RPW][kChunk / 2];
    float d[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      q8_pairs(wc[s][r], qp[r]);
      d[r] = f16_to_f32(wc[s][r].d);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      uint32_t xp[kChunk / 2];
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(&s_x[((m * NS + s) * kBlk + 4u * lane + (i ^ swl)) * 4u]);
        xp[4 * i] = v.x;
        xp[4 * i + 1] = v.y;
        xp[4 * i + 2] = v.z;
        xp[4 * i + 3] = v.w;
      }
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
        for (int j = 0; j < kChunk / 2; j += 2) {
          p0 = dot2_bf16(qp[r][j], xp[j], p0);
          p1 = dot2_bf16(qp[r][j + 1], xp[j + 1], p1);
        }
        acc[r][m] += kin ? (p0 + p1) * d[r] : 0.0f;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint32_t row = row0 + r;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float v = wave_sum(acc[r][m]);
      if (lane == 0 && row < rows && (uint32_t)m < M_rt) {
        if (y_bf16)
          static_cast<uint16_t*>(y)[(size_t)m * rows + row] = f32_to_bf16(v);
        else
          static_cast<float*>(y)[(size_t)m * rows + row] = v;
      }
    }
  }
}

template <int MT, int RPW, int WAVES, int NS>
hipError_t launch_q8_mt_t(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  if (m > (uint32_t)MT || reinterpret_cast<uintptr_t>(x) % 16 != 0 || t.cols % 8 != 0 ||
      (t.kp + kStep - 1) / kStep != (uint32_t)NS)
    return hipErrorInvalidValue;
  const uint32_t per_block = WAVES * RPW;
  hipLaunchKernelGGL((gemv_q8_mt_kernel<MT, RPW, WAVES, NS>), dim3((t.rows + per_block - 1) / per_block),
                     dim3(WAVES * 64), 0, s, t, static_cast<const uint16_t*>(x), y, m, (uint32_t)(y_bf16 ? 1u : 0u));
  return hipGetLastError();
}

// Epilogue of the one-token kernels: plain (y[row] = sum) or gated (the
// wave's gate / up pair, y[first] = f(gate) * up, and workgroup 0 zeroes the
// padding columns [n_ff, y_stride)), as gemv_kernel writes them.
template <int EPI, int RPW, int WAVES>
__device__ __forceinline__ void m1_epilogue(const float (&acc)[RPW], const uint32_t (&rr)[RPW], const bool (&rv)[RPW],
                                            uint32_t first, uint32_t lane, uint32_t rows, uint32_t n_ff,
                                            uint32_t y_stride, void* y, uint32_t y_bf16) {
  if constexpr (EPI == kEpiPlain) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const float v = wave_sum(acc[r]);
      if (lane == 0 && rv[r]) {
        if (y_bf16)
          static_cast<uint16_t*>(y)[rr[r]] = f32_to_bf16(v);
        else
          static_cast<float*>(y)[rr[r]] = v;
      }
    }
  } else {
    const float g = wave_sum(acc[0]);
    const float u = wave_sum(acc[1]);
    if (lane == 0 && rv[0]) {
      const float v = gated<EPI>(g, u);
      if (y_bf16)
        static_cast<uint16_t*>(y)[first] = f32_to_bf16(v);
      else
        static_cast<float*>(y)[first] = v;
    }
    if (blockIdx.x == 0) {   // zero padding columns [n_ff, y_stride)
      for (uint32_t c = n_ff + threadIdx.x; c < y_stride; c += WAVES * 64) {
        if (y_bf16)
          static_cast<uint16_t*>(y)[c] = 0;
        else
          static_cast<float*>(y)[c] = 0.0f;
      }
    }
  }
  (void)rows;
}

// ---------------------------------------------------------------------------
// Norm prologue of the one-token LDS-staged kernels (NORM): x is built by
// every workgroup as bf16(rms_norm(cur [+ delta]) * w) with the reduction of
// norm_prologue (threads 0..255, element i = tid + 256 j by FMA in ascending
// j, the DPP wave sum, the four wave sums in order; the workgroup's other
// waves add zeros after them), so x is bit-identical to the stand-alone
// RMSNorm's bf16 output, and is written widened to f32 in the swizzled
// 4-column slots the kernels read (zero past cols up to xlen).  Workgroup 0
// also stores cur + delta to cur_out.  Ends with a barrier.
template <uint32_t NP, int WAVES>
__device__ __forceinline__ void norm_stage_m1(const NormIn& nin, uint32_t cols, uint32_t xlen, const float (&c)[NP],
                                              const float (&d)[NP], const float (&w)[NP], float* s_x,
                                              float* s_part) {
#pragma clang fp contract(off)
  const uint32_t tid = threadIdx.x;
  const bool add = nin.delta != nullptr, mine = tid < 256u;
  float v[NP];
  float sq = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < NP; ++j) {
    v[j] = add ? c[j] + d[j] : c[j];
    if (mine && tid + 256u * j < cols) sq = __builtin_fmaf(v[j], v[j], sq);
  }
  sq = wave_sum(sq);
  if ((tid & 63u) == 0) s_part[tid >> 6] = sq;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int k = 0; k < WAVES; ++k) total += s_part[k];
  const float scale = 1.0f / sqrtf(total / (float)cols + nin.eps);
  auto slot = [&](uint32_t i) {   // f32 index of column i
    const uint32_t q = i / 4u, blk = q / 512u, l = (q % 512u) / 8u, pi = q % 8u;
    return (blk * 512u + 8u * l + (pi ^ ((l >> 1) & 7u))) * 4u + i % 4u;
  };
  if (mine) {
    const bool store = add && blockIdx.x == 0;
#pragma unroll
    for (uint32_t j = 0; j < NP; ++j) {
      const uint32_t i = tid + 256u * j;
      if (i < cols) {
        s_x[slot(i)] = bf16_to_f32(f32_to_bf16(v[j] * scale * w[j]));
        if (store) nin.cur_out[i] = v[j];
      }
    }
  }
  for (uint32_t i = cols + tid; i < xlen; i += WAVES * 64u) s_x[slot(i)] = 0.0f;
  __syncthreads();
}

// ---------------------------------------------------------------------------
// cb4 (reference layout) weights, one token, 1..3 K steps: the structure of
// gemv_q8_m1_kernel with the cb4 decode of gemv_kernel (centroid tables in
// LDS, the group scale on the 32-column partial sum, the zero-scale group
// skip of codebook.rs:384-386, CSR residuals after the dense part in lane
// order).  The residuals' activations come from the staged row in LDS, so the
// call does not end on a dependent global read.  Products and summation order
// are those of gemv_kernel.
//
// EPI: the plain or a gated epilogue of gemv_kernel (rows in gate / up pairs,
// RPW = 2: one output per wave).  NORM: x built by norm_stage_m1 from
// cur [+ delta] and the norm weight instead of read from memory (bf16; at
// most 16 elements per thread of the first 256).
template <int RPW, int WAVES, int NS, bool XBF16, int EPI = kEpiPlain, bool NORM = false, uint32_t NP = 8>
__global__ __launch_bounds__(WAVES * 64) void gemv_cb4_m1_kernel(DevTensor t, const void* __restrict__ x,
                                                                void* __restrict__ y, uint32_t y_bf16,
                                                                uint32_t n_ff = 0, uint32_t y_stride = 0,
                                                                NormIn nin = {}) {
  static_assert(NS >= 1 && NS <= 3, "K steps staged in LDS");
  static_assert(EPI == kEpiPlain || RPW == 2, "gated: one gate / up row pair per wave");
  static_assert(!NORM || (XBF16 && NS <= 2 && WAVES >= 4), "the norm prologue: bf16, cols <= 4096");
  __shared__ __attribute__((aligned(64))) float s_cent[48];
  __shared__ __attribute__((aligned(16))) float s_x[NS * kStep];
  __shared__ float s_part[WAVES];
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  constexpr uint32_t kOut = EPI == kEpiPlain ? RPW : RPW / 2;   // outputs per wave
  const uint32_t first = (blockIdx.x * WAVES + wave) * kOut;
  uint32_t rr[RPW];
  bool rv[RPW];
  wave_rows<EPI, RPW>(first, rows, n_ff, rr, rv);

  // Load order (the vector loads count in one in-order counter, so a wait for
  // a load also waits for every load issued before it): each row's CSR
  // bounds first (lane-varying vector loads: a scalar load would share its
  // counter with the LDS traffic and hold back the activation barrier), then
  // the activations and the weights; each lane's first residual entry after
  // them, when its bounds have landed.
  uint32_t rpv[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) rpv[r] = t.row_ptr[rr[r] + (lane & 1u)];   // lane 0: start, lane 1: end
  __builtin_amdgcn_sched_barrier(0);   // keeps these loads ahead of the rest
  constexpr uint32_t kCols = XBF16 ? 8 : 4;
  constexpr uint32_t kPieces = NS * kStep / kCols;
  constexpr uint32_t kPer = NORM ? 1 : (kPieces + WAVES * 64 - 1) / (WAVES * 64);
  u32x4 xv[kPer];
  float n_c[NORM ? NP : 1], n_d[NORM ? NP : 1], n_w[NORM ? NP : 1];
  if constexpr (NORM) {   // norm inputs (clamped, unconditional), before the weights
#pragma unroll
    for (uint32_t j = 0; j < NP; ++j) {
      const uint32_t i = std::min(std::min(tid, 255u) + 256u * j, cols - 1);
      n_c[j] = nin.cur[i];
      n_w[j] = nin.w[i];
      n_d[j] = nin.delta ? nin.delta[i] : 0.0f;
    }
  } else {
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(x), (short)0,
                                                                       (int)(cols * (XBF16 ? 2u : 4u)), 0x00020000);
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
      const uint32_t p = std::min(tid + WAVES * 64 * j, kPieces - 1);   // repeats write the same value
      xv[j] = __builtin_amdgcn_raw_buffer_load_b128(xr, p * 16u, 0, 0);
    }
  }
  WChunk<KIND_CB4> wc[NS][RPW];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t k0 = s * kStep + lane * kChunk;
    const uint32_t k0c = k0 < kp ? k0 : kp - kChunk;
#pragma unroll
    for (int r = 0; r < RPW; ++r) load_chunk<KIND_CB4>(t, rr[r], k0c, 0, 0, wc[s][r]);
  }
  // Nothing that uses a loaded value may be scheduled above the last load.
  __builtin_amdgcn_sched_barrier(0);
  if (tid == 0) {   // the centroid tables come with the kernel arguments (scalar loads)
#pragma unroll
    for (int c = 0; c < 48; c += 4)
      *reinterpret_cast<float4*>(&s_cent[c]) = make_float4(t.cent[c], t.cent[c + 1], t.cent[c + 2], t.cent[c + 3]);
  }
  // Each lane's first residual entry: its bounds were the first loads, so
  // they have landed by the time the activations are waited for below.
  uint32_t os[RPW], oe[RPW], pk0[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {   // clamped, unconditional (the CSR stream holds at least one word)
    os[r] = __builtin_amdgcn_readlane(rpv[r], 0);
    oe[r] = __builtin_amdgcn_readlane(rpv[r], 1);
    const uint32_t i = os[r] + lane;
    const uint32_t last = oe[r] > 0 ? oe[r] - 1 : 0;
    pk0[r] = t.outliers[i < oe[r] ? i : (os[r] < oe[r] ? last : 0)];
  }
  if constexpr (NORM) {
    norm_stage_m1<NP, WAVES>(nin, cols, NS * kStep, n_c, n_d, n_w, s_x, s_part);
  } else {
    auto put = [&](uint32_t p, const u32x4& v) {   // f32 piece p (4 columns) to its slot
      const uint32_t blk = p / 512u, l = (p % 512u) / 8u, i = p % 8u;
      *reinterpret_cast<u32x4*>(&s_x[(blk * 512u + 8u * l + (i ^ ((l >> 1) & 7u))) * 4u]) = v;
    };
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
      const uint32_t p = std::min(tid + WAVES * 64 * j, kPieces - 1);
      const u32x4 v = xv[j];
      if constexpr (XBF16) {
        put(2 * p, u32x4{v.x << 16, v.x & 0xffff0000u, v.y << 16, v.y & 0xffff0000u});
        put(2 * p + 1, u32x4{v.z << 16, v.z & 0xffff0000u, v.w << 16, v.w & 0xffff0000u});
      } else {
        put(p, v);
      }
    }
    __syncthreads();
  }
  __builtin_amdgcn_sched_barrier(0);   // the barrier waits for the activations only

  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  const uint32_t swl = (lane >> 1) & 7u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool kin = s * kStep + lane * kChunk < kp;
    float xf[kChunk];
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(&s_x[(s * 512u + 8u * lane + (i ^ swl)) * 4u]);
      xf[4 * i] = __uint_as_float(v.x);
      xf[4 * i + 1] = __uint_as_float(v.y);
      xf[4 * i + 2] = __uint_as_float(v.z);
      xf[4 * i + 3] = __uint_as_float(v.w);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float w[kChunk];
      dequant_chunk<KIND_CB4>(wc[s][r], lds_addr(s_cent) + 64u * cent_table(t, rr[r]), 0, lane, w);
      float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
      for (int j = 0; j < kChunk; j += 2) {
        p0 = __builtin_fmaf(w[j], xf[j], p0);
        p1 = __builtin_fmaf(w[j + 1], xf[j + 1], p1);
      }
      float p = p0 + p1;
      const float sc = f16_to_f32(wc[s][r].sc);   // codebook.rs:384-386: a zero scale skips the group
      p = sc != 0.0f ? sc * p : 0.0f;
      acc[r] += kin ? p : 0.0f;
    }
  }
  // CSR residuals (codebook.rs:409-415): lane l takes entries l, l + 64, ...
  // of the row, in that order; the activation comes from the staged row.
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    if (!rv[r]) continue;
    for (uint32_t i = os[r] + lane; i < oe[r]; i += 64u) {
      const uint32_t pk = i < os[r] + 64u ? pk0[r] : t.outliers[i];
      const uint32_t col = pk & 0xffffu;
      if (col >= cols) continue;
      const uint32_t q = col / 4u, blk = q / 512u, l = (q % 512u) / 8u, pi = q % 8u;
      const float xc = s_x[(blk * 512u + 8u * l + (pi ^ ((l >> 1) & 7u))) * 4u + col % 4u];
      acc[r] = __builtin_fmaf(f16_to_f32(pk >> 16), xc, acc[r]);
    }
  }
  m1_epilogue<EPI, RPW, WAVES>(acc, rr, rv, first, lane, rows, n_ff, y_stride, y, y_bf16);
}

// ---------------------------------------------------------------------------
// Q8 weights x bf16 activations at M = 5..8 on MFMA.
//
// v_mfma_f32_16x16x32_bf16 with the activations as the A operand (rows =
// tokens; rows past M are zero) and 16 weight rows as the B operand.  An int8
// weight is exact in bf16, so every product is exact and two MFMAs sum one
// Q8 block (32 columns) of 16 rows for every token in fp32; the lane's output
// column is one weight row, so the block scale is applied per lane as
// acc += d * block (gguf.rs:223-229: w = q * d).  The dot2 kernels spend one
// VALU instruction per column pair per token; here a block costs its int8 ->
// bf16 conversion and four FMAs per lane whatever M is.
//
// Lane l (row c = l % 16 of the tile, group g = l / 16) loads 16 weight bytes
// and 16 activations at column 64 p + 16 g of a block pair p, so each load
// instruction reads 64 contiguous bytes of 16 weight rows.  Groups 0-1 then
// hold block 2p, groups 2-3 block 2p + 1: each block's MFMAs take the
// activations of its own groups and zeros in the others (the k slots of one
// MFMA must share a block scale).  The tile's block scales are staged in LDS
// by coalesced loads.  A workgroup is WAVES waves over the same 16 rows, each
// summing a contiguous range of block pairs with all loads of up to
// kQ8MfmaPairs pairs issued before the first MFMA; the waves' fragments are
// added in LDS in wave order, so the result does not depend on timing.
// D register i holds token 4 g + i of weight row row0 + c.  Requires 16-byte
// aligned activation rows (cols % 8 == 0 and an aligned x) and at most
// 4 x DI x WAVES scales per row (kQ8MfmaMaxNb).
constexpr int kQ8MfmaPairs = 8;

// Block scales per row the staging loop covers: DI loads per thread.
template <int WAVES, int DI>
constexpr uint32_t kQ8MfmaMaxNb = (uint32_t)DI * WAVES * 4u;

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// Eight int8 weights (two dwords) as eight bf16 (exact).
__device__ __forceinline__ bf16x8_t q8_bf16x8(uint32_t a, uint32_t b) {
  const uint32_t wd[2] = {a, b};
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = wd[j >> 1];
    const int sh = (j & 1) * 16;
    const float lo = (float)(int8_t)((w >> sh) & 0xffu);
    const float hi = (float)(int8_t)((w >> (sh + 8)) & 0xffu);
    r[j] = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
  }
  return __builtin_bit_cast(bf16x8_t, r);
}

template <int WAVES, int DI>
__global__ __launch_bounds__(WAVES * 64) void gemv_q8_mfma_kernel(DevTensor t, const uint16_t* __restrict__ x,
                                                                 void* __restrict__ y, uint32_t M_rt,
                                                                 uint32_t y_bf16) {
  __shared__ f32x4_t s_red[WAVES][32];
  __shared__ uint16_t s_d[16 * kQ8MfmaMaxNb<WAVES, DI>];
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // in SGPRs: pair ranges and guards are scalar
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t nb = kp / 32, np = (nb + 1) / 2;
  const uint32_t row0 = blockIdx.x * 16;
  const uint32_t c16 = lane & 15, grp = lane >> 4;
  const bool lo_half = grp < 2;   // groups 0-1: first block of a pair

  // The tile's scales (rows row0.., contiguous in the plane), clamped loads first.
  const uint32_t dn = 16 * nb;
  const size_t dlast = (size_t)rows * nb - 1;
  uint16_t dv[DI];
#pragma unroll
  for (int i = 0; i < DI; ++i) {
    const size_t idx = (size_t)row0 * nb + tid + (uint32_t)i * (WAVES * 64);
    dv[i] = t.p1[idx < dlast ? idx : dlast];
  }

  const uint32_t row = row0 + c16 < rows ? row0 + c16 : rows - 1;
  const bool tok_live = c16 < M_rt;
  const uint16_t* xr = x + (size_t)(tok_live ? c16 : 0) * cols;
  const uint8_t* wr = static_cast<const uint8_t*>(t.p0) + (size_t)row * kp;
  const uint32_t p_begin = wave * np / WAVES, p_end = (wave + 1) * np / WAVES;   // uniform per wave
  const u32x4 z = {0u, 0u, 0u, 0u};
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  bool staged = false;
  for (uint32_t p0 = p_begin; p0 < p_end; p0 += kQ8MfmaPairs) {
    u32x4 wv[kQ8MfmaPairs], xa[kQ8MfmaPairs], xb[kQ8MfmaPairs];
#pragma unroll
    for (int i = 0; i < kQ8MfmaPairs; ++i) {   // clamped, unconditional loads
      const uint32_t p = p0 + i < p_end ? p0 + i : p_end - 1;
      const uint32_t k = p * 64 + 16 * grp;
      // A missing second block (odd nb) re-reads the first block's bytes; its
      // activations are past cols (zero) and its scale is never applied.
      wv[i] = *reinterpret_cast<const u32x4*>(wr + (k < kp ? k : k - 32));
      xa[i] = *reinterpret_cast<const u32x4*>(xr + (k < cols ? k : cols - 8));
      xb[i] = *reinterpret_cast<const u32x4*>(xr + (k + 8 < cols ? k + 8 : cols - 8));
    }
    if (!staged) {   // first batch only (uniform): scales to LDS behind the loads above
#pragma unroll
      for (int i = 0; i < DI; ++i) {
        const uint32_t j = tid + (uint32_t)i * (WAVES * 64);
        if (j < dn) s_d[j] = dv[i];
      }
      lds_barrier();
      staged = true;
    }
#pragma unroll
    for (int i = 0; i < kQ8MfmaPairs; ++i) {
      const uint32_t p = p0 + i;
      if (p >= p_end) continue;   // uniform
      const uint32_t k = p * 64 + 16 * grp;   // activation pieces past cols (or padding tokens) are zero
      const u32x4 va = tok_live && k < cols ? xa[i] : z, vb = tok_live && k + 8 < cols ? xb[i] : z;
      const bf16x8_t wlo = q8_bf16x8(wv[i].x, wv[i].y), whi = q8_bf16x8(wv[i].z, wv[i].w);
      const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, lo_half ? va : z);
      const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, lo_half ? vb : z);
      const bf16x8_t a2 = __builtin_bit_cast(bf16x8_t, lo_half ? z : va);
      const bf16x8_t a3 = __builtin_bit_cast(bf16x8_t, lo_half ? z : vb);
      const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
      f32x4_t b0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, wlo, zero, 0, 0, 0);
      b0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, whi, b0, 0, 0, 0);
      f32x4_t b1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, wlo, zero, 0, 0, 0);
      b1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, whi, b1, 0, 0, 0);
      const float d0 = f16_to_f32(s_d[c16 * nb + 2 * p]);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] += d0 * b0[r];
      if (2 * p + 1 < nb) {   // uniform
        const float d1 = f16_to_f32(s_d[c16 * nb + 2 * p + 1]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] += d1 * b1[r];
      }
    }
  }
  if (!staged) {   // a wave with no pairs still takes part in the staging barrier
#pragma unroll
    for (int i = 0; i < DI; ++i) {
      const uint32_t j = tid + (uint32_t)i * (WAVES * 64);
      if (j < dn) s_d[j] = dv[i];
    }
    lds_barrier();
  }
  // Lanes 0..31 hold tokens 0..7 (4 g + i for g = 0, 1).
  if (lane < 32) s_red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && lane < 32) {
    f32x4_t v = s_red[0][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      const f32x4_t o = s_red[w][lane];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] += o[r];
    }
    const uint32_t n = row0 + c16;
    if (n < rows) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t m = 4 * grp + r;
        if (m < M_rt) {
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * rows + n] = f32_to_bf16(v[r]);
          else
            static_cast<float*>(y)[(size_t)m * rows + n] = v[r];
        }
      }
    }
  }
}

// Used for M = 5..8 with K <= 2048 (launch_kind).  Measured on MI355X against
// the dot2 kernels, M = 8: 1570 vs 1113 GB/s at K x N = 2048 x 6144, 3110 vs
// 2307 for the 151936-row LM head, level at 2048 x 2048; behind at M = 4
// (the MFMA cost does not shrink with M) and at K = 6144 x N = 2048, where
// 128 row tiles leave most CUs idle (987 vs 1089 GB/s on 4 waves, 1023 on 8).
// cb4-g64 x bf16 (or f32), one token, staged through LDS (gemv_g64_m1_kernel).
// Requires 16-byte aligned activations, 16-byte pieces wholly inside or
// outside the row, and NS K steps.
template <int RPW, int WAVES, int NS, bool XBF16 = true>
hipError_t launch_g64_m1_t(const DevTensor& t, const void* x, void* y, bool y_bf16, hipStream_t s) {
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || t.cols % (XBF16 ? 8 : 4) != 0 ||
      (t.kp + kStep - 1) / kStep != (uint32_t)NS)
    return hipErrorInvalidValue;
  const uint32_t per_block = WAVES * RPW;
  hipLaunchKernelGGL((gemv_g64_m1_kernel<RPW, WAVES, NS, XBF16>), dim3((t.rows + per_block - 1) / per_block),
                     dim3(WAVES * 64), 0, s, t, x, y, (uint32_t)(y_bf16 ? 1u : 0u));
  return hipGetLastError();
}

// cb4 x bf16 / f32, one token, staged through LDS (gemv_cb4_m1_kernel).
// Requires 16-byte aligned activations, 16-byte pieces wholly inside or
// outside the row, and NS K steps.
template <int RPW, int WAVES, int NS, bool XBF16>
hipError_t launch_cb4_m1_t(const DevTensor& t, const void* x, void* y, bool y_bf16, hipStream_t s) {
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || t.cols % (XBF16 ? 8 : 4) != 0 ||
      (t.kp + kStep - 1) / kStep != (uint32_t)NS)
    return hipErrorInvalidValue;
  const uint32_t per_block = WAVES * RPW;
  hipLaunchKernelGGL((gemv_cb4_m1_kernel<RPW, WAVES, NS, XBF16>), dim3((t.rows + per_block - 1) / per_block),
                     dim3(WAVES * 64), 0, s, t, x, y, (uint32_t)(y_bf16 ? 1u : 0u));
  return hipGetLastError();
}

// The same kernel with a gated epilogue (outs = n_ff) and / or the norm
// prologue (x unused), eight waves per workgroup.
template <int RPW, int NS, bool XBF16, int EPI, bool NORM, uint32_t NP = 8>
hipError_t launch_cb4_m1_e(const DevTensor& t, const void* x, uint32_t outs, void* y, bool y_bf16, uint32_t n_ff,
                           uint32_t y_stride, const NormIn& nin, hipStream_t s) {
  constexpr int WAVES = 8;
  constexpr uint32_t per_block = WAVES * (EPI == kEpiPlain ? RPW : RPW / 2);
  hipLaunchKernelGGL((gemv_cb4_m1_kernel<RPW, WAVES, NS, XBF16, EPI, NORM, NP>),
                     dim3((outs + per_block - 1) / per_block), dim3(WAVES * 64), 0, s, t, x, y,
                     (uint32_t)(y_bf16 ? 1u : 0u), n_ff, y_stride, nin);
  return hipGetLastError();
}

// Q8 x f32 activations, one token, staged through LDS (gemv_q8_m1_kernel).
// Requires 16-byte aligned activations, cols % 4 == 0 and NS K steps.
template <int RPW, int WAVES, int NS, bool XBF16 = false, uint32_t KB = KIND_Q8>
hipError_t launch_q8_m1_t(const DevTensor& t, const void* x, void* y, bool y_bf16, hipStream_t s) {
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || t.cols % (XBF16 ? 8 : 4) != 0 ||
      (t.kp + kStep - 1) / kStep != (uint32_t)NS)
    return hipErrorInvalidValue;
  const uint32_t per_block = WAVES * RPW;
  hipLaunchKernelGGL((gemv_q8_m1_kernel<RPW, WAVES, NS, XBF16, KB>), dim3((t.rows + per_block - 1) / per_block),
                     dim3(WAVES * 64), 0, s, t, x, y, (uint32_t)(y_bf16 ? 1u : 0u));
  return hipGetLastError();
}

template <int WAVES, int DI>
hipError_t launch_q8_mfma_t(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  if (m > 8 || t.cols % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 || t.kp / 32 > kQ8MfmaMaxNb<WAVES, DI>)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemv_q8_mfma_kernel<WAVES, DI>), dim3((t.rows + 15) / 16), dim3(WAVES * 64), 0, s, t,
                     static_cast<const uint16_t*>(x), y, m, (uint32_t)(y_bf16 ? 1u : 0u));
  return hipGetLastError();
}

// Q8 x bf16 activations, 3..8 tokens, >= 65536 rows: the persistent MFMA
// kernel of gemv_q8p.hip (its own translation unit, compiled with MFMA
// results in VGPRs).  hipErrorInvalidValue when the shape does not fit it.
hipError_t launch_q8_lm(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s);

// Q8 x bf16 activations, 5..8 tokens, 8 rows per workgroup
// (gemv_q8_mfma8_kernel in gemv_q8p.hip), kp / 32 <= kQ8M8MaxNb.
constexpr uint32_t kQ8M8MaxNb = 256;
hipError_t launch_q8_m8(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s);

// Grid for the persistent kernel: enough workgroups to fill every CU at the
// occupancy the LDS footprint allows, never more than there are row blocks.
template <int MT, int RPW, int WAVES, int NS>
hipError_t launch_q8_lds_t(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s,
                           uint32_t per_cu = 0) {
  // Dynamic LDS above 64 KiB must be allowed per kernel, once.
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&gemv_q8_lds_kernel<MT, RPW, WAVES, NS>),
      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (attr != hipSuccess) return attr;
  const size_t lds = (size_t)MT * t.kp * 2;
  if (lds > 160u * 1024u || (t.kp + kStep - 1) / kStep != (uint32_t)NS) return hipErrorInvalidValue;
  const uint32_t nblocks = (t.rows + WAVES * RPW - 1) / (WAVES * RPW);
  uint32_t occ = per_cu ? per_cu : (uint32_t)std::min<size_t>(160u * 1024u / lds, 16u / WAVES * 2u);
  if (occ == 0) occ = 1;
  const uint32_t grid = std::min<uint32_t>(nblocks, 256u * occ);
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && t.cols % 8 == 0;
  hipLaunchKernelGGL((gemv_q8_lds_kernel<MT, RPW, WAVES, NS>), dim3(grid), dim3(WAVES * 64), lds, s, t,
                     static_cast<const uint16_t*>(x), y, m, (uint32_t)(y_bf16 ? 1u : 0u), x_vec);
  return hipGetLastError();
}

template <int MT, int RPW, int S>
hipError_t launch_q8_dot2_t(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  const uint32_t rows_per_block = kWaves * RPW;
  const dim3 grid((t.rows + rows_per_block - 1) / rows_per_block);
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && t.cols % 8 == 0;
  hipLaunchKernelGGL((gemv_q8_dot2_kernel<MT, RPW, S>), grid, dim3(kWaves * 64), 0, s, t,
                     static_cast<const uint16_t*>(x), y, m, (uint32_t)(y_bf16 ? 1u : 0u), x_vec);
  return hipGetLastError();
}

// Shape choices for Q8 x bf16 at M = 2..8, from measurements over the
// decode shapes (K x N in {2048, 6144} x {2048, 6144}, and the 151936-row LM
// head): the LDS-staged persistent kernel wins only when there are many more
// row blocks than CUs; otherwise the direct kernel with two rows per wave.
template <int MT>
hipError_t launch_q8_dot2_m(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (t.rows >= 65536 && nsteps == 1) {
    if constexpr (MT >= 8) return launch_q8_lds_t<MT, 1, 4, 1>(t, x, m, y, y_bf16, s);
    return launch_q8_lds_t<MT, 2, 8, 1>(t, x, m, y, y_bf16, s);
  }
  if constexpr (MT == 2) {
    if (nsteps == 3) return launch_q8_dot2_t<2, 1, 1>(t, x, m, y, y_bf16, s);
    if (nsteps >= 2) return launch_q8_dot2_t<2, 2, 2>(t, x, m, y, y_bf16, s);
    return launch_q8_dot2_t<2, 2, 1>(t, x, m, y, y_bf16, s);
  } else if constexpr (MT == 4) {
    if (nsteps >= 2) return launch_q8_dot2_t<4, 2, 2>(t, x, m, y, y_bf16, s);
    return launch_q8_dot2_t<4, 2, 1>(t, x, m, y, y_bf16, s);
  }
  return launch_q8_dot2_t<MT, 2, 1>(t, x, m, y, y_bf16, s);
}

template <uint32_t KIND, int MT, int RPW, int S, bool XBF16>
hipError_t launch_t(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  const uint32_t rows_per_block = kWaves * RPW;
  const dim3 grid((t.rows + rows_per_block - 1) / rows_per_block);
  const size_t esz = XBF16 ? 2 : 4;
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && t.cols % 8 == 0 &&
                         ((size_t)t.cols * esz) % 16 == 0;
  hipLaunchKernelGGL((gemv_kernel<KIND, MT, RPW, S, XBF16>), grid, dim3(kWaves * 64), 0, s, t, x, y, m,
                     (uint32_t)(y_bf16 ? 1u : 0u), x_vec);
  return hipGetLastError();
}

// Split K over KS waves per workgroup (rows shared, one step per wave).
template <uint32_t KIND, int MT, int RPW, bool XBF16, int KS>
hipError_t launch_ks(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  const dim3 grid((t.rows + RPW - 1) / RPW);
  const size_t esz = XBF16 ? 2 : 4;
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && t.cols % 8 == 0 &&
                         ((size_t)t.cols * esz) % 16 == 0;
  hipLaunchKernelGGL((gemv_kernel<KIND, MT, RPW, 1, XBF16, kEpiPlain, false, kNormPer, KS>), grid, dim3(KS * 64), 0,
                     s, t, x, y, m, (uint32_t)(y_bf16 ? 1u : 0u), x_vec);
  return hipGetLastError();
}

// Split K pays where a matrix has few rows for its K and at least two K
// steps: one wave per step of every row, up to 4.  Measured (M = 1, bf16 x):
// 2048 x 6144 g64 6.27 -> 5.61 us, Q8 6.20 -> 5.96; 1024 x 8192 g64 6.09 ->
// 4.18; 2048 x 4096 Q8 with f32 x 9.9 -> 9.7; at 4096 rows it was level or
// slower (and slower for Q8 with f32 x, whose one-row waves lose the
// four-row waves' reuse of x).
template <uint32_t KIND, int MT, bool XBF16>
bool try_split_k(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s,
                 hipError_t* e) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (nsteps < 2 || t.rows > 2048) return false;
  // cb4: each workgroup stages its centroid tables behind a barrier, which
  // costs more with three times the workgroups; measured slower at 2048 rows
  // (6.2 -> 7.1 us at K = 6144), faster at 1024 x 8192 (6.3 -> 4.9 us).
  if (KIND == KIND_CB4 && (t.rows > 1024 || nsteps < 4)) return false;
  if (nsteps == 2) *e = launch_ks<KIND, MT, 1, XBF16, 2>(t, x, m, y, y_bf16, s);
  else if (nsteps == 3) *e = launch_ks<KIND, MT, 1, XBF16, 3>(t, x, m, y, y_bf16, s);
  else *e = launch_ks<KIND, MT, 1, XBF16, 4>(t, x, m, y, y_bf16, s);
  return true;
}

// Steps per batch: all of K at once up to 3 steps (K <= 6144), else 2.
// VXT_GEMV_SPLIT_K=0 in the environment turns split K off (for comparisons).
inline bool split_k_enabled() {
  static const bool on = [] {
    const char* v = getenv("VXT_GEMV_SPLIT_K");
    return !(v && v[0] == '0');
  }();
  return on;
}

template <uint32_t KIND, int MT, int RPW, bool XBF16>
hipError_t launch_s(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (nsteps == 1) return launch_t<KIND, MT, RPW, 1, XBF16>(t, x, m, y, y_bf16, s);
  if (nsteps == 3 && MT <= 2) return launch_t<KIND, MT, RPW, 3, XBF16>(t, x, m, y, y_bf16, s);
  return launch_t<KIND, MT, RPW, 2, XBF16>(t, x, m, y, y_bf16, s);
}

template <uint32_t KIND, int MT, int RPW>
hipError_t launch_r(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y, bool y_bf16,
                    hipStream_t s) {
  return x_bf16 ? launch_s<KIND, MT, RPW, true>(t, x, m, y, y_bf16, s)
                : launch_s<KIND, MT, RPW, false>(t, x, m, y, y_bf16, s);
}

// 2 or 3..4 tokens of Q8 weights through the LDS-staged kernel: one row per
// wave (eight waves, four for three K steps); two rows and eight waves at
// >= 65536 rows (the LM head).
template <int MT>
hipError_t launch_q8_mt(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (t.rows >= 65536) {
    if (nsteps == 1) return launch_q8_mt_t<MT, 2, 8, 1>(t, x, m, y, y_bf16, s);
    if (nsteps == 2) return launch_q8_mt_t<MT, 2, 8, 2>(t, x, m, y, y_bf16, s);
    return launch_q8_mt_t<MT, 2, 8, 3>(t, x, m, y, y_bf16, s);
  }
  if (nsteps == 1) return launch_q8_mt_t<MT, 1, 8, 1>(t, x, m, y, y_bf16, s);
  if (nsteps == 2) return launch_q8_mt_t<MT, 1, 8, 2>(t, x, m, y, y_bf16, s);
  return launch_q8_mt_t<MT, 1, 4, 3>(t, x, m, y, y_bf16, s);
}

// One token of g64 weights through the LDS-staged kernel: one row per wave up
// to 8192 rows, two above; four waves per workgroup.
template <bool XBF16>
hipError_t launch_g64_m1(const DevTensor& t, const void* x, void* y, bool y_bf16, hipStream_t s, uint32_t nsteps) {
  if (t.rows > 8192) {
    if (nsteps == 1) return launch_g64_m1_t<2, 4, 1, XBF16>(t, x, y, y_bf16, s);
    if (nsteps == 2) return launch_g64_m1_t<2, 4, 2, XBF16>(t, x, y, y_bf16, s);
    return launch_g64_m1_t<2, 4, 3, XBF16>(t, x, y, y_bf16, s);
  }
  if (nsteps == 1) return launch_g64_m1_t<1, 4, 1, XBF16>(t, x, y, y_bf16, s);
  if (nsteps == 2) return launch_g64_m1_t<1, 4, 2, XBF16>(t, x, y, y_bf16, s);
  return launch_g64_m1_t<1, 4, 3, XBF16>(t, x, y, y_bf16, s);
}

// One token of cb4 weights through the LDS-staged kernel: one row per wave
// up to 8192 rows, two above; eight waves per workgroup.
template <bool XBF16>
hipError_t launch_cb4_m1(const DevTensor& t, const void* x, void* y, bool y_bf16, hipStream_t s) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (t.rows > 8192) {
    if (nsteps == 1) return launch_cb4_m1_t<2, 8, 1, XBF16>(t, x, y, y_bf16, s);
    if (nsteps == 2) return launch_cb4_m1_t<2, 8, 2, XBF16>(t, x, y, y_bf16, s);
    return launch_cb4_m1_t<2, 8, 3, XBF16>(t, x, y, y_bf16, s);
  }
  if (nsteps == 1) return launch_cb4_m1_t<1, 8, 1, XBF16>(t, x, y, y_bf16, s);
  if (nsteps == 2) return launch_cb4_m1_t<1, 8, 2, XBF16>(t, x, y, y_bf16, s);
  return launch_cb4_m1_t<1, 8, 3, XBF16>(t, x, y, y_bf16, s);
}

// One token of Q8 weights through the LDS-staged kernel: one row per wave and
// eight waves per workgroup, four and four at >= 65536 rows (the LM head).
template <bool XBF16, uint32_t KB = KIND_Q8>
hipError_t launch_q8_x1(const DevTensor& t, const void* x, void* y, bool y_bf16, hipStream_t s) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (t.rows >= 65536) {
    if (nsteps == 1) return launch_q8_m1_t<4, 4, 1, XBF16, KB>(t, x, y, y_bf16, s);
    if (nsteps == 2) return launch_q8_m1_t<4, 4, 2, XBF16, KB>(t, x, y, y_bf16, s);
    return launch_q8_m1_t<4, 4, 3, XBF16, KB>(t, x, y, y_bf16, s);
  }
  if (nsteps == 1) return launch_q8_m1_t<1, 8, 1, XBF16, KB>(t, x, y, y_bf16, s);
  if (nsteps == 2) return launch_q8_m1_t<1, 8, 2, XBF16, KB>(t, x, y, y_bf16, s);
  return launch_q8_m1_t<1, 8, 3, XBF16, KB>(t, x, y, y_bf16, s);
}

// Rows per wave: more rows per wave (more bytes in flight per wave) once rows
// are plentiful; one row per wave keeps narrow matrices spread over all CUs.
template <uint32_t KIND>
hipError_t launch_kind(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y, bool y_bf16,
                       hipStream_t s) {
  if constexpr (KIND == KIND_Q8) {
    // 2..8 tokens with bf16 activations: the LDS-staged kernel
    // (gemv_q8_mt_kernel) where it measured faster than the dot2 and MFMA
    // kernels (graph-timed, rotated copies; 2048 x 2048 / 6144 x 2048 /
    // 2048 x 6144 / 151936 x 2048): M = 2 3.99 / 5.97 / 6.29 / 64.5 us ->
    // 3.22 / 4.95 / 5.26 / 63.0; M = 4 4.95 / 7.82 / 8.75 / 84.6 -> 3.81 /
    // 5.92 / 6.64 / 80.1; M = 8 only at 2048 x 2048, 6.25 -> 4.98 (the MFMA
    // and persistent kernels keep the others).
    // 3..8 tokens over >= 65536 rows (the LM head): the persistent MFMA
    // kernel, one wave per SIMD (measured best of 1..3 per SIMD and of
    // 4 or 8 pairs per batch, 2 to 6 batches in flight).  151936 x 2048,
    // graph-timed: M = 4 89.4 -> 64.4 us (gemv_q8_mt_kernel before), M = 8
    // 101.4 -> 68.1 (gemv_q8_mfma_kernel); M = 2 stays on the LDS-staged
    // dot2 kernel (64.2 against 66-68).
    if (x_bf16 && m >= 3 && m <= 8 && t.rows >= 65536 && t.kp % 512 == 0 && t.kp <= 2 * kStep &&
        t.cols % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0)
      return launch_q8_lm(t, x, m, y, y_bf16, s);
    if (x_bf16 && m >= 2 && m <= 8) {
      const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
      if (nsteps <= 3 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && t.cols % 8 == 0) {
        if (m <= 4) return m == 2 ? launch_q8_mt<2>(t, x, m, y, y_bf16, s) : launch_q8_mt<4>(t, x, m, y, y_bf16, s);
        if (t.rows <= 4096 && nsteps == 1) return launch_q8_mt_t<8, 1, 4, 1>(t, x, m, y, y_bf16, s);
      }
    }
    if (x_bf16 && m >= 2) {
      if (m == 2) return launch_q8_dot2_m<2>(t, x, m, y, y_bf16, s);
      if (m > 4 && t.cols % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && t.kp / 32 <= kQ8MfmaMaxNb<4, 4>)
        return launch_q8_mfma_t<4, 4>(t, x, m, y, y_bf16, s);
      // Rows longer than two K steps at 5..8 tokens: the 8-row MFMA kernel,
      // twice the row tiles of the 16-row one.  Graph-timed against dot2, M =
      // 5 / 8, K = 6144: 2048 rows 11.3 / 11.8 -> 9.6 / 10.1 us, 1024 rows
      // 11.0 / 11.4 -> 9.2 / 9.8, 4096 rows 17.8 / 18.5 -> 14.0 / 15.5 (8
      // waves, 6 pairs per batch; 4 waves or 12 pairs per batch were slower);
      // level at K = 4096, so not taken there.
      if (m > 4 && t.cols % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && t.kp > 2 * kStep &&
          t.kp / 32 <= kQ8M8MaxNb && t.rows <= 4096)
        return launch_q8_m8(t, x, m, y, y_bf16, s);
      if (m <= 4) return launch_q8_dot2_m<4>(t, x, m, y, y_bf16, s);
      if (m <= 8) return launch_q8_dot2_m<8>(t, x, m, y, y_bf16, s);
      return hipErrorInvalidValue;
    }
  }
  if constexpr (KIND == KIND_Q8) {
    // f32 activations, one token: the LDS-staged kernel (gemv_q8_m1_kernel).
    // Measured against the generic kernel (graph-timed, rotated copies):
    // 4096 x 4096 (config 0) 8.46 -> 5.54 us, 2048 x 4096 7.30 -> 3.81,
    // 2048 x 2048 4.21 -> 2.89, 6144 x 6144 19.7 -> 9.7; one row per wave and
    // eight waves per workgroup were best up to 16384 rows, four rows per wave
    // and four waves at the 151936-row head (79.7 -> 58.8 us).
    // bf16 activations take the same kernel at one token (widened to f32 as
    // they are staged): 2048 x 2048 3.15 -> 2.87 us, 6144 x 2048 5.03 ->
    // 4.64, 2048 x 6144 (split K before) 5.75 -> 4.52, the 151936-row head
    // 60.5 -> 57.2.
    const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
    if (m == 1 && nsteps <= 3 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && t.cols % (x_bf16 ? 8 : 4) == 0)
      return x_bf16 ? launch_q8_x1<true>(t, x, y, y_bf16, s) : launch_q8_x1<false>(t, x, y, y_bf16, s);
  }
  if constexpr (KIND == KIND_Q40) {
    // One token: the LDS-staged block kernel with the nibble decode; the
    // generic kernel takes the rest (4.5 bits per weight streamed either way).
    const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
    if (m == 1 && nsteps <= 3 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && t.cols % (x_bf16 ? 8 : 4) == 0)
      return x_bf16 ? launch_q8_x1<true, KIND_Q40>(t, x, y, y_bf16, s)
                    : launch_q8_x1<false, KIND_Q40>(t, x, y, y_bf16, s);
  }
  if constexpr (KIND == KIND_CB4) {
    // One token: the LDS-staged kernel (gemv_cb4_m1_kernel).  Measured against
    // gemv_kernel (bf16 x, 0.7 % residuals, graph-timed, rotated copies):
    // 6144 x 2048 5.11 -> 4.80 us, 2048 x 2048 4.01 -> 3.42, 2048 x 6144
    // 6.20 -> 5.31 with one row per wave; 12288 x 2048 8.10 -> 7.01 with two;
    // eight waves per workgroup.
    const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
    if (m == 1 && nsteps <= 3 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && t.cols % (x_bf16 ? 8 : 4) == 0)
      return x_bf16 ? launch_cb4_m1<true>(t, x, y, y_bf16, s) : launch_cb4_m1<false>(t, x, y, y_bf16, s);
  }
  if constexpr (KIND == KIND_G64) {
    // One token: the LDS-staged kernel (gemv_g64_m1_kernel).  Measured
    // against gemv_kernel (graph-timed, rotated copies): 6144 x 2048 (config
    // 1) 4.86 -> 4.66 us, 2048 x 2048 3.15 -> 3.09, 2048 x 6144 (split K
    // before) 5.61 -> 5.33 with one row per wave; 12288 x 2048 7.71 -> 6.85,
    // 24576 x 2048 12.32 -> 11.59, 151936 x 2048 59.6 -> 52.4 with two; four
    // waves per workgroup throughout.
    // f32 activations (an attention output) take the same kernel, staged as
    // they are.
    const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
    if (m == 1 && nsteps <= 3 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && t.cols % (x_bf16 ? 8 : 4) == 0)
      return x_bf16 ? launch_g64_m1<true>(t, x, y, y_bf16, s, nsteps) : launch_g64_m1<false>(t, x, y, y_bf16, s, nsteps);
  }
  if (m == 1 && split_k_enabled()) {
    hipError_t e = hipSuccess;
    if (x_bf16 ? try_split_k<KIND, 1, true>(t, x, m, y, y_bf16, s, &e)
               : try_split_k<KIND, 1, false>(t, x, m, y, y_bf16, s, &e))
      return e;
  }
  if (m == 1) {
    // Q8 with f32 activations the LDS-staged kernel does not take (x not
    // 16-byte aligned, K > 6144): four rows per wave halve the activation
    // bytes each wave re-reads from L2 per weight byte (4096 x 4096: 8.68 ->
    // 8.24 us against two rows).
    if (t.rows >= 65536 || (KIND == KIND_Q8 && !x_bf16 && t.rows >= 4096))
      return launch_r<KIND, 1, 4>(t, x, x_bf16, m, y, y_bf16, s);
    if (t.rows >= 4096) return launch_r<KIND, 1, 2>(t, x, x_bf16, m, y, y_bf16, s);
    return launch_r<KIND, 1, 1>(t, x, x_bf16, m, y, y_bf16, s);
  }
  if (m == 2) {
    if (t.rows >= 65536) return launch_r<KIND, 2, 2>(t, x, x_bf16, m, y, y_bf16, s);
    return launch_r<KIND, 2, 1>(t, x, x_bf16, m, y, y_bf16, s);
  }
  if (m <= 4) return launch_r<KIND, 4, 1>(t, x, x_bf16, m, y, y_bf16, s);
  if (m <= 8) return launch_r<KIND, 8, 1>(t, x, x_bf16, m, y, y_bf16, s);
  return hipErrorInvalidValue;
}

// Gated gate/up GEMV: one output (a gate row and its up row) per wave, the
// generic kernel for every kind, M = 1 or 2 (the gate and up accumulators of
// four or more tokens do not fit in registers without spilling; the caller
// runs those as a plain GEMV and an element-wise activation pass).
template <uint32_t KIND, int MT, int S, bool XBF16, int EPI>
hipError_t launch_glu_t(const DevTensor& t, const void* x, uint32_t m, uint32_t n_ff, void* y, bool y_bf16,
                        uint32_t y_stride, hipStream_t s) {
  constexpr int RPW = 2;
  const dim3 grid((n_ff + kWaves - 1) / kWaves);
  const size_t esz = XBF16 ? 2 : 4;
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && t.cols % 8 == 0 &&
                         ((size_t)t.cols * esz) % 16 == 0;
  hipLaunchKernelGGL((gemv_kernel<KIND, MT, RPW, S, XBF16, EPI>), grid, dim3(kWaves * 64), 0, s, t, x, y, m,
                     (uint32_t)(y_bf16 ? 1u : 0u), x_vec, n_ff, y_stride);
  return hipGetLastError();
}

template <uint32_t KIND, int MT, bool XBF16, int EPI>
hipError_t launch_glu_s(const DevTensor& t, const void* x, uint32_t m, uint32_t n_ff, void* y, bool y_bf16,
                        uint32_t y_stride, hipStream_t s) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (nsteps == 1) return launch_glu_t<KIND, MT, 1, XBF16, EPI>(t, x, m, n_ff, y, y_bf16, y_stride, s);
  if (nsteps == 3 && MT <= 2) return launch_glu_t<KIND, MT, 3, XBF16, EPI>(t, x, m, n_ff, y, y_bf16, y_stride, s);
  return launch_glu_t<KIND, MT, 2, XBF16, EPI>(t, x, m, n_ff, y, y_bf16, y_stride, s);
}

template <uint32_t KIND, int MT, int EPI>
hipError_t launch_glu_x(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, uint32_t n_ff, void* y,
                        bool y_bf16, uint32_t y_stride, hipStream_t s) {
  return x_bf16 ? launch_glu_s<KIND, MT, true, EPI>(t, x, m, n_ff, y, y_bf16, y_stride, s)
                : launch_glu_s<KIND, MT, false, EPI>(t, x, m, n_ff, y, y_bf16, y_stride, s);
}

// cb4, one token: the LDS-staged kernel with the gated epilogue (16-byte
// aligned activations, cols a multiple of one 16-byte piece, 1..3 K steps).
template <int EPI>
bool try_glu_cb4_m1(const DevTensor& t, const void* x, bool x_bf16, uint32_t n_ff, void* y, bool y_bf16,
                    uint32_t y_stride, hipStream_t s, hipError_t* e) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (nsteps > 3 || reinterpret_cast<uintptr_t>(x) % 16 != 0 || t.cols % (x_bf16 ? 8 : 4) != 0) return false;
  const NormIn none{};
  if (x_bf16) {
    *e = nsteps == 1 ? launch_cb4_m1_e<2, 1, true, EPI, false>(t, x, n_ff, y, y_bf16, n_ff, y_stride, none, s)
       : nsteps == 2 ? launch_cb4_m1_e<2, 2, true, EPI, false>(t, x, n_ff, y, y_bf16, n_ff, y_stride, none, s)
                     : launch_cb4_m1_e<2, 3, true, EPI, false>(t, x, n_ff, y, y_bf16, n_ff, y_stride, none, s);
  } else {
    *e = nsteps == 1 ? launch_cb4_m1_e<2, 1, false, EPI, false>(t, x, n_ff, y, y_bf16, n_ff, y_stride, none, s)
       : nsteps == 2 ? launch_cb4_m1_e<2, 2, false, EPI, false>(t, x, n_ff, y, y_bf16, n_ff, y_stride, none, s)
                     : launch_cb4_m1_e<2, 3, false, EPI, false>(t, x, n_ff, y, y_bf16, n_ff, y_stride, none, s);
  }
  return true;
}

template <uint32_t KIND, int EPI>
hipError_t launch_glu_m(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, uint32_t n_ff, void* y,
                        bool y_bf16, uint32_t y_stride, hipStream_t s) {
  if constexpr (KIND == KIND_CB4) {
    hipError_t e = hipSuccess;
    if (m == 1 && try_glu_cb4_m1<EPI>(t, x, x_bf16, n_ff, y, y_bf16, y_stride, s, &e)) return e;
  }
  if (m == 1) return launch_glu_x<KIND, 1, EPI>(t, x, x_bf16, m, n_ff, y, y_bf16, y_stride, s);
  if (m == 2) return launch_glu_x<KIND, 2, EPI>(t, x, x_bf16, m, n_ff, y, y_bf16, y_stride, s);
  return hipErrorInvalidValue;
}

template <uint32_t KIND>
hipError_t launch_glu_kind(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, uint32_t n_ff, void* y,
                           bool y_bf16, uint32_t y_stride, bool gelu, hipStream_t s) {
  return gelu ? launch_glu_m<KIND, kEpiGelu>(t, x, x_bf16, m, n_ff, y, y_bf16, y_stride, s)
              : launch_glu_m<KIND, kEpiSilu>(t, x, x_bf16, m, n_ff, y, y_bf16, y_stride, s);
}

// Norm-prologue GEMV, batch 1 (plain or gated epilogue): the same row and
// step choices as the plain M = 1 launches and the gated launches.
template <uint32_t KIND, int RPW, int S, int EPI, uint32_t NP>
hipError_t launch_norm_np(const DevTensor& t, const NormIn& nin, uint32_t outs, void* y, bool y_bf16,
                          uint32_t y_stride, hipStream_t s) {
  constexpr uint32_t per_block = kWaves * (EPI == kEpiPlain ? RPW : RPW / 2);
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  const size_t lds = (size_t)nsteps * kStep * 2;
  hipLaunchKernelGGL((gemv_kernel<KIND, 1, RPW, S, true, EPI, true, NP>), dim3((outs + per_block - 1) / per_block),
                     dim3(kWaves * 64), lds, s, t, nullptr, y, 1u, (uint32_t)(y_bf16 ? 1u : 0u), 1u,
                     EPI == kEpiPlain ? 0u : outs, y_stride, nin);
  return hipGetLastError();
}

// Norm inputs held per thread: 8 up to 2048 columns, else 16.
template <uint32_t KIND, int RPW, int S, int EPI>
hipError_t launch_norm_t(const DevTensor& t, const NormIn& nin, uint32_t outs, void* y, bool y_bf16,
                         uint32_t y_stride, hipStream_t s) {
  if (t.cols <= 2048) return launch_norm_np<KIND, RPW, S, EPI, 8>(t, nin, outs, y, y_bf16, y_stride, s);
  return launch_norm_np<KIND, RPW, S, EPI, 16>(t, nin, outs, y, y_bf16, y_stride, s);
}

template <uint32_t KIND, int RPW, int EPI>
hipError_t launch_norm_s(const DevTensor& t, const NormIn& nin, uint32_t outs, void* y, bool y_bf16,
                         uint32_t y_stride, hipStream_t s) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (nsteps == 1) return launch_norm_t<KIND, RPW, 1, EPI>(t, nin, outs, y, y_bf16, y_stride, s);
  return launch_norm_t<KIND, RPW, 2, EPI>(t, nin, outs, y, y_bf16, y_stride, s);
}

// epi: kEpiPlain (y = W x, outs = rows) or a gated epilogue (outs = rows / 2).
// Requires cols <= 256 * kNormPer.
// cb4: the LDS-staged one-token kernel with the norm prologue (1..2 K steps).
template <int RPW, int NS, int EPI, uint32_t NP>
hipError_t launch_norm_cb4_m1(const DevTensor& t, const NormIn& nin, uint32_t outs, void* y, bool y_bf16,
                              uint32_t y_stride, hipStream_t s) {
  return launch_cb4_m1_e<RPW, NS, true, EPI, true, NP>(t, nullptr, outs, y, y_bf16, EPI == kEpiPlain ? 0u : outs,
                                                       y_stride, nin, s);
}

template <int RPW, int EPI>
hipError_t launch_norm_cb4_m1_s(const DevTensor& t, const NormIn& nin, uint32_t outs, void* y, bool y_bf16,
                                uint32_t y_stride, hipStream_t s) {
  const uint32_t nsteps = (t.kp + kStep - 1) / kStep;
  if (nsteps == 1) return launch_norm_cb4_m1<RPW, 1, EPI, 8>(t, nin, outs, y, y_bf16, y_stride, s);
  if (t.cols <= 2048) return launch_norm_cb4_m1<RPW, 2, EPI, 8>(t, nin, outs, y, y_bf16, y_stride, s);
  return launch_norm_cb4_m1<RPW, 2, EPI, 16>(t, nin, outs, y, y_bf16, y_stride, s);
}

template <uint32_t KIND>
hipError_t launch_norm_kind(const DevTensor& t, const NormIn& nin, int epi, void* y, bool y_bf16,
                            uint32_t y_stride, hipStream_t s) {
  if (t.cols > 256u * kNormPer) return hipErrorInvalidValue;
  if constexpr (KIND == KIND_CB4) {   // cols <= 4096: at most two K steps
    if (epi == kEpiSilu) return launch_norm_cb4_m1_s<2, kEpiSilu>(t, nin, t.rows / 2, y, y_bf16, y_stride, s);
    if (epi == kEpiGelu) return launch_norm_cb4_m1_s<2, kEpiGelu>(t, nin, t.rows / 2, y, y_bf16, y_stride, s);
    if (t.rows > 8192) return launch_norm_cb4_m1_s<2, kEpiPlain>(t, nin, t.rows, y, y_bf16, t.rows, s);
    return launch_norm_cb4_m1_s<1, kEpiPlain>(t, nin, t.rows, y, y_bf16, t.rows, s);
  }
  if (epi == kEpiSilu) return launch_norm_s<KIND, 2, kEpiSilu>(t, nin, t.rows / 2, y, y_bf16, y_stride, s);
  if (epi == kEpiGelu) return launch_norm_s<KIND, 2, kEpiGelu>(t, nin, t.rows / 2, y, y_bf16, y_stride, s);
  if (t.rows >= 65536) return launch_norm_s<KIND, 4, kEpiPlain>(t, nin, t.rows, y, y_bf16, t.rows, s);
  if (t.rows >= 4096) return launch_norm_s<KIND, 2, kEpiPlain>(t, nin, t.rows, y, y_bf16, t.rows, s);
  return launch_norm_s<KIND, 1, kEpiPlain>(t, nin, t.rows, y, y_bf16, t.rows, s);
}

}  // namespace gv

}  // namespace vxt
