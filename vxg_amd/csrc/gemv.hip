// gemv.hip -- fused dequantise + GEMV for M = 1..8 tokens (decode path).
//
// Reference behaviour: CodebookMatrix::gemv_cpu (codebook.rs:350-417), the Q8
// block-dot composition (llm_prefill.rs:45-54, :336-340) and the Metal GEMV
// kernels (vxt_gemv.metal:297-381, vxt_cb4_fast.metal:104-209).
//
// Mapping on CDNA4 (wave64):
//   * one wave owns RPW output rows; a "step" covers 2048 consecutive K
//     columns, 32 per lane, so every weight load is one contiguous 16-byte
//     load per lane (a fully coalesced 1 KiB per wave for 4-bit kinds);
//   * the activation chunk of a step is loaded once into registers and reused
//     across the wave's RPW rows (K outer, rows inner);
//   * weights are unpacked in registers; the 16-entry cb4 table (and the per-
//     lane g64 table) is read from LDS;
//   * per-lane partial sums are reduced across the wave at the end.
// Sums are fp32; the order differs from the CPU reference, so results agree
// to fp32 rounding (the parity bar is relative error, not bits).
#include "common.hpp"

namespace vxt {

constexpr int kWaves = 4;
constexpr int kChunk = 32;           // K columns per lane per step
constexpr int kStep = 64 * kChunk;   // K columns per wave per step

// x chunk loader: 32 activations of one token row, zero beyond cols.
template <bool XBF16, bool VEC>
__device__ __forceinline__ void load_x32(const void* __restrict__ xrow, uint32_t cols, uint32_t k0,
                                         float (&xv)[kChunk]) {
  if (VEC && k0 + kChunk <= cols) {
    if constexpr (XBF16) {
      const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xrow) + k0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint4 u = p[i];
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xv[i * 8 + 2 * j] = __uint_as_float(w[j] << 16);
          xv[i * 8 + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
      }
    } else {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(xrow) + k0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float4 f = p[i];
        xv[i * 4 + 0] = f.x;
        xv[i * 4 + 1] = f.y;
        xv[i * 4 + 2] = f.z;
        xv[i * 4 + 3] = f.w;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      uint32_t c = k0 + j;
      float v = 0.0f;
      if (c < cols) {
        if constexpr (XBF16)
          v = bf16_to_f32(static_cast<const uint16_t*>(xrow)[c]);
        else
          v = static_cast<const float*>(xrow)[c];
      }
      xv[j] = v;
    }
  }
}

template <bool XBF16>
__device__ __forceinline__ float load_x1(const void* __restrict__ xrow, uint32_t c) {
  if constexpr (XBF16)
    return bf16_to_f32(static_cast<const uint16_t*>(xrow)[c]);
  else
    return static_cast<const float*>(xrow)[c];
}

template <uint32_t KIND, int M, int RPW, bool XBF16, bool XVEC>
__global__ __launch_bounds__(kWaves * 64) void gemv_kernel(DevTensor t, const void* __restrict__ x,
                                                          void* __restrict__ y, uint32_t y_bf16) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint32_t row0 = (blockIdx.x * kWaves + wave) * RPW;
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;

  // cb4: shared 16-entry centroid table.  g64: one 17-float slot per lane.
  __shared__ float s_cent[16];
  __shared__ float s_lut[kWaves * 64 * 17];
  if constexpr (KIND == KIND_CB4) {
    if (threadIdx.x < 16) s_cent[threadIdx.x] = t.cent[threadIdx.x];
    __syncthreads();
  }
  float* my_lut = s_lut + threadIdx.x * 17;

  float acc[RPW][M];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  for (uint32_t k0 = lane * kChunk; k0 < kp; k0 += kStep) {
    float xv[M][kChunk];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const void* xrow = XBF16 ? (const void*)(static_cast<const uint16_t*>(x) + (size_t)m * cols)
                               : (const void*)(static_cast<const float*>(x) + (size_t)m * cols);
      load_x32<XBF16, XVEC>(xrow, cols, k0, xv[m]);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const uint32_t row = row0 + r;
      if (row >= rows) break;
      if constexpr (KIND == KIND_Q8) {
        const uint4* wp = reinterpret_cast<const uint4*>(static_cast<const int8_t*>(t.p0) +
                                                         (size_t)row * kp + k0);
        uint4 a = load_nt16(wp);
        uint4 b = load_nt16(wp + 1);
        float d = f16_to_f32(t.p1[(size_t)row * (kp / 32) + k0 / 32]);
        uint32_t wd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float p[M];
#pragma unroll
        for (int m = 0; m < M; ++m) p[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
          float w = (float)(int8_t)((wd[j >> 2] >> ((j & 3) * 8)) & 0xffu);
#pragma unroll
          for (int m = 0; m < M; ++m) p[m] = __builtin_fmaf(w, xv[m][j], p[m]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = __builtin_fmaf(d, p[m], acc[r][m]);
      } else if constexpr (KIND == KIND_CB4) {
        const uint4* wp = reinterpret_cast<const uint4*>(static_cast<const uint32_t*>(t.p0) +
                                                         (size_t)row * (kp / 8) + k0 / 8);
        uint4 u = load_nt16(wp);
        float sc = f16_to_f32(t.p1[(size_t)row * (kp / 128) + k0 / 128]);
        uint32_t wd[4] = {u.x, u.y, u.z, u.w};
        float p[M];
#pragma unroll
        for (int m = 0; m < M; ++m) p[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
          float w = s_cent[(wd[j >> 3] >> ((j & 7) * 4)) & 0xfu];
#pragma unroll
          for (int m = 0; m < M; ++m) p[m] = __builtin_fmaf(w, xv[m][j], p[m]);
        }
        // codebook.rs:384-386: a zero scale skips the group.
        if (sc != 0.0f) {
#pragma unroll
          for (int m = 0; m < M; ++m) acc[r][m] = __builtin_fmaf(sc, p[m], acc[r][m]);
        }
      } else {  // KIND_G64
        const uint4* ip = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(t.p0) +
                                                         (size_t)row * (kp / 2) + k0 / 2);
        uint4 u = load_nt16(ip);
        const uint4* lp = reinterpret_cast<const uint4*>(t.p1 + ((size_t)row * (kp / 64) + k0 / 64) * 16);
        uint4 l0 = load_nt16(lp);
        uint4 l1 = load_nt16(lp + 1);
        uint32_t lw[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          my_lut[2 * e] = f16_to_f32(lw[e] & 0xffffu);
          my_lut[2 * e + 1] = f16_to_f32(lw[e] >> 16);
        }
        uint32_t wd[4] = {u.x, u.y, u.z, u.w};
        float p[M];
#pragma unroll
        for (int m = 0; m < M; ++m) p[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
          float w = my_lut[(wd[j >> 3] >> ((j & 7) * 4)) & 0xfu];
#pragma unroll
          for (int m = 0; m < M; ++m) p[m] = __builtin_fmaf(w, xv[m][j], p[m]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] += p[m];
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
        for (int m = 0; m < M; ++m) {
          const void* xrow = XBF16 ? (const void*)(static_cast<const uint16_t*>(x) + (size_t)m * cols)
                                   : (const void*)(static_cast<const float*>(x) + (size_t)m * cols);
          acc[r][m] = __builtin_fmaf(val, load_x1<XBF16>(xrow, col), acc[r][m]);
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint32_t row = row0 + r;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float s = wave_sum(acc[r][m]);
      if (lane == 0 && row < rows) {
        if (y_bf16)
          static_cast<uint16_t*>(y)[(size_t)m * rows + row] = f32_to_bf16(s);
        else
          static_cast<float*>(y)[(size_t)m * rows + row] = s;
      }
    }
  }
}

// ---- host-side dispatch ---------------------------------------------------

template <uint32_t KIND, int M, int RPW, bool XBF16, bool XVEC>
static hipError_t launch_t(const DevTensor& t, const void* x, void* y, bool y_bf16, hipStream_t s) {
  const uint32_t rows_per_block = kWaves * RPW;
  dim3 grid((t.rows + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL((gemv_kernel<KIND, M, RPW, XBF16, XVEC>), grid, dim3(kWaves * 64), 0, s, t, x, y,
                     (uint32_t)(y_bf16 ? 1u : 0u));
  return hipGetLastError();
}

template <uint32_t KIND, int M>
static hipError_t launch_m(const DevTensor& t, const void* x, bool x_bf16, bool x_vec, void* y,
                           bool y_bf16, hipStream_t s) {
  constexpr int RPW = M <= 2 ? 2 : 1;
  if (x_bf16)
    return x_vec ? launch_t<KIND, M, RPW, true, true>(t, x, y, y_bf16, s)
                 : launch_t<KIND, M, RPW, true, false>(t, x, y, y_bf16, s);
  return x_vec ? launch_t<KIND, M, RPW, false, true>(t, x, y, y_bf16, s)
               : launch_t<KIND, M, RPW, false, false>(t, x, y, y_bf16, s);
}

template <uint32_t KIND>
static hipError_t launch_kind(const DevTensor& t, const void* x, bool x_bf16, bool x_vec,
                              uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  switch (m) {
    case 1: return launch_m<KIND, 1>(t, x, x_bf16, x_vec, y, y_bf16, s);
    case 2: return launch_m<KIND, 2>(t, x, x_bf16, x_vec, y, y_bf16, s);
    case 3: return launch_m<KIND, 3>(t, x, x_bf16, x_vec, y, y_bf16, s);
    case 4: return launch_m<KIND, 4>(t, x, x_bf16, x_vec, y, y_bf16, s);
    case 5: return launch_m<KIND, 5>(t, x, x_bf16, x_vec, y, y_bf16, s);
    case 6: return launch_m<KIND, 6>(t, x, x_bf16, x_vec, y, y_bf16, s);
    case 7: return launch_m<KIND, 7>(t, x, x_bf16, x_vec, y, y_bf16, s);
    case 8: return launch_m<KIND, 8>(t, x, x_bf16, x_vec, y, y_bf16, s);
    default: return hipErrorInvalidValue;
  }
}

// Launch the GEMV for batch_m in 1..8.  x_vec: x rows are 16-byte aligned
// (base aligned and cols * elem_size % 16 == 0), so chunk loads may be vector.
hipError_t launch_gemv(const DevTensor& t, const void* x, bool x_bf16, bool x_vec, uint32_t m,
                       void* y, bool y_bf16, hipStream_t s) {
  switch (t.kind) {
    case KIND_Q8: return launch_kind<KIND_Q8>(t, x, x_bf16, x_vec, m, y, y_bf16, s);
    case KIND_CB4: return launch_kind<KIND_CB4>(t, x, x_bf16, x_vec, m, y, y_bf16, s);
    case KIND_G64: return launch_kind<KIND_G64>(t, x, x_bf16, x_vec, m, y, y_bf16, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vxt
