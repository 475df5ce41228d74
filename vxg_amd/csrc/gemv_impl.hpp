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

// Per-wave LDS slot for the g64 codebooks of one row-step: 32 pair tables
// (32 bytes each) at a 48-byte stride.  64 lanes reading random entries of
// 32 tables conflict heavily on LDS banks at a 32- or 64-byte stride; 48 is
// the best of the strides measured (32..144).
constexpr uint32_t kPairStride = 48;
constexpr uint32_t kSlotBytes = 32 * kPairStride;

typedef __attribute__((address_space(3))) _Float16 lds_half_t;
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
    const uint32_t wd[4] = {c.q.x, c.q.y, c.q.z, c.q.w};
    const uint32_t base = slot + (lane >> 1) * kPairStride;   // 16-byte aligned, low 5 bits clear below
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const int sh = (j & 7) * 4 - 1;
      const uint32_t off = sh < 0 ? ((wd[j >> 3] << 1) & 0x1eu) : ((wd[j >> 3] >> sh) & 0x1eu);
      w[j] = (float)*(lds_half_t*)(size_t)(base + off);
    }
  }
}

// Kernel: MT tokens (MT in {1,2,4,8}; m >= M_rt are padding), RPW rows per
// wave, up to S steps per batch.
template <uint32_t KIND, int MT, int RPW, int S, bool XBF16>
__global__ __launch_bounds__(kWaves * 64) void gemv_kernel(DevTensor t, const void* __restrict__ x,
                                                          void* __restrict__ y, uint32_t M_rt,
                                                          uint32_t y_bf16, uint32_t x_vec) {
  __shared__ __attribute__((aligned(64))) float s_cent[48];
  __shared__ __attribute__((aligned(64))) uint4 s_slot[KIND == KIND_G64 ? kWaves * S * RPW * kSlotBytes / 16 : 1];

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t row0 = (blockIdx.x * kWaves + wave) * RPW;
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t nsteps = (kp + kStep - 1) / kStep;

  if constexpr (KIND == KIND_CB4) {   // before any global load is in flight
    if (threadIdx.x < 48) s_cent[threadIdx.x] = t.cent[threadIdx.x];
    __syncthreads();
  }
  const uint32_t slot = lds_addr(s_slot) + (KIND == KIND_G64 ? wave * S * RPW * kSlotBytes : 0);

  float acc[RPW][MT];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

  for (uint32_t s0 = 0; s0 < nsteps; s0 += S) {
    const uint32_t ns = nsteps - s0 < (uint32_t)S ? nsteps - s0 : (uint32_t)S;   // uniform
    // ---- issue: activations, then weights, for every step of the batch
    XChunk<XBF16> xc[S][MT];
    WChunk<KIND> wc[S][RPW];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if ((uint32_t)s < ns && x_vec) {
        const uint32_t k0 = (s0 + s) * kStep + lane * kChunk;
#pragma unroll
        for (int m = 0; m < MT; ++m) load_x<XBF16>(x, cols, (uint32_t)m < M_rt ? m : 0, k0, xc[s][m]);
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
        for (int r = 0; r < RPW; ++r) {
          const uint32_t row = row0 + r < rows ? row0 + r : rows - 1;
          load_chunk<KIND>(t, row, k0c, g < gmax ? g : gmax, lane & 1, wc[s][r]);
        }
      }
    }
    // ---- consume
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if ((uint32_t)s >= ns) break;
      const uint32_t k0 = (s0 + s) * kStep + lane * kChunk;
      const bool kin = k0 < kp;
      float xv[MT][kChunk];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (x_vec)
          unpack_x<XBF16>(xc[s][m], xv[m]);
        else
          load_x_scalar<XBF16>(x, cols, (uint32_t)m < M_rt ? m : 0, k0, xv[m]);
      }
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const uint32_t sl = slot + (s * RPW + r) * kSlotBytes;
        if constexpr (KIND == KIND_G64)   // lane l holds half (l & 1) of pair table l >> 1
          *(__attribute__((address_space(3))) u32x4*)(size_t)(sl + (lane >> 1) * kPairStride + (lane & 1) * 16) =
              u32x4{wc[s][r].lut.x, wc[s][r].lut.y, wc[s][r].lut.z, wc[s][r].lut.w};
        uint32_t cbase = 0;
        if constexpr (KIND == KIND_CB4) cbase = lds_addr(s_cent) + 64u * cent_table(t, row0 + r);
        float w[kChunk];
        dequant_chunk<KIND>(wc[s][r], cbase, sl, lane, w);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
          for (int j = 0; j < kChunk; j += 2) {
            p0 = __builtin_fmaf(w[j], xv[m][j], p0);
            p1 = __builtin_fmaf(w[j + 1], xv[m][j + 1], p1);
          }
          float p = p0 + p1;
          if constexpr (KIND == KIND_Q8) {
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
    // CSR residuals (codebook.rs:409-415): y += f16(res) * x[col].
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const uint32_t row = row0 + r;
      if (row >= rows) break;
      const uint32_t os = t.row_ptr[row], oe = t.row_ptr[row + 1];
      for (uint32_t i = os + lane; i < oe; i += 64) {
        const uint32_t pk = t.outliers[i];
        const uint32_t col = pk & 0xffffu;
        if (col >= cols) continue;
        const float val = f16_to_f32(pk >> 16);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const uint32_t mm = (uint32_t)m < M_rt ? m : 0;
          float xc;
          if constexpr (XBF16)
            xc = bf16_to_f32(static_cast<const uint16_t*>(x)[(size_t)mm * cols + col]);
          else
            xc = static_cast<const float*>(x)[(size_t)mm * cols + col];
          acc[r][m] = __builtin_fmaf(val, xc, acc[r][m]);
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

// Steps per batch: all of K at once up to 3 steps (K <= 6144), else 2.
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

// Rows per wave: more rows per wave (more bytes in flight per wave) once rows
// are plentiful; one row per wave keeps narrow matrices spread over all CUs.
template <uint32_t KIND>
hipError_t launch_kind(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y, bool y_bf16,
                       hipStream_t s) {
  if (m == 1) {
    if (t.rows >= 65536) return launch_r<KIND, 1, 4>(t, x, x_bf16, m, y, y_bf16, s);
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

}  // namespace gv

}  // namespace vxt
