// gemm.hip -- prefill dequantise + GEMM on the matrix cores (batch_m > 8).
//
// Reference behaviour: PackedTensor::gemm_cpu (llm_prefill.rs:156-255), which
// decodes 32-row weight tiles to f32 (decode_row) and runs a dense f32 tile
// GEMM; and the Metal prefill kernel vxt_cb4_gemm_nr2 (vxt_cb4_fast.metal:
// 290-375).  Here: Y[M, N] = X[M, K] * W[N, K]^T with W dequantised tile by
// tile into LDS and fed to v_mfma_f32_32x32x16_f16, fp32 accumulation.
//
// Exactness of the MFMA operands (products are then exact in fp32):
//   * X (bf16) is converted to f16 while it is staged; exact for |x| in the
//     f16 normal range [2^-14, 65504] (values below lose only bits under
//     2^-24 absolute).  f32 X is split like the weights, hi + lo in f16
//     (22 significant bits), with one more MFMA (lo * lo is dropped);
//   * g64 weights ARE f16 table entries: exact, one MFMA per step;
//   * Q8 weights q*d (<= 18 significant bits) and cb4 weights f32(sc*cent)
//     are split into hi = f16(w) and lo = f16((w - hi) * 2^11); hi + lo*2^-11
//     is exact for Q8 and within 2^-22 relative for cb4.  lo products go to a
//     second fp32 accumulator scaled by 2^-11 at the end (a second MFMA);
//   * cb4 CSR residuals are added in the epilogue as res * x[col] before the
//     output is rounded.
//
// Tiling: 128 (M) x 128 (N) x 64 (K) per 256-thread block, 2 x 2 waves each
// owning a 64 x 64 output patch (2 x 2 MFMA 32x32 tiles).  The next K tile is
// fetched into registers while the current one is multiplied from LDS.
#include "common.hpp"

namespace vxt {

namespace gemm {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDK = BK + 8;          // padded LDS row (halves) against bank conflicts
constexpr int THREADS = 256;
// lo halves are stored as f16((v - hi) * 2^11) so they stay out of the f16
// subnormal range; their products accumulate separately and are scaled back.
constexpr float kLoScale = 2048.0f;
constexpr float kLoInv = 1.0f / 2048.0f;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Per-thread staging registers for one K tile.  Thread t owns row t/2 of both
// the A tile and the B tile, K half (t%2)*32 .. +32.
struct Stage {
  uint32_t a[16];      // 32 activations as f16 pairs (hi)
  uint32_t al[16];     // 32 activations (lo) as f16 pairs (f32 inputs)
  uint32_t bh[16];     // 32 weights (hi) as f16 pairs
  uint32_t bl[16];     // 32 weights (lo) as f16 pairs (split kinds)
};

// A: X[m, k0 + h*32 .. +32] -> f16 (zero outside [0,M) x [0,K)).
template <bool XBF16>
__device__ __forceinline__ void load_a(const void* __restrict__ x, uint32_t M, uint32_t K, uint32_t m,
                                       uint32_t kb, bool vec, uint32_t (&a)[16], uint32_t (&al)[16]) {
  float v[32];
  if (m < M && vec && kb + 32 <= K) {
    if constexpr (XBF16) {
      const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + (size_t)m * K + kb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint4 u = p[i];
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[i * 8 + 2 * j] = __uint_as_float(w[j] << 16);
          v[i * 8 + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
      }
    } else {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + (size_t)m * K + kb);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float4 f = p[i];
        v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const uint32_t k = kb + j;
      float f = 0.0f;
      if (m < M && k < K) {
        if constexpr (XBF16)
          f = bf16_to_f32(static_cast<const uint16_t*>(x)[(size_t)m * K + k]);
        else
          f = static_cast<const float*>(x)[(size_t)m * K + k];
      }
      v[j] = f;
    }
  }
  if constexpr (XBF16) {
#pragma unroll
    for (int j = 0; j < 16; ++j) a[j] = pack_h2((_Float16)v[2 * j], (_Float16)v[2 * j + 1]);
  } else {
    // f32 activations: x = hi + lo with both halves f16 (22 significant bits)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const _Float16 h0 = (_Float16)v[2 * j], h1 = (_Float16)v[2 * j + 1];
      a[j] = pack_h2(h0, h1);
      al[j] = pack_h2((_Float16)((v[2 * j] - (float)h0) * kLoScale),
                      (_Float16)((v[2 * j + 1] - (float)h1) * kLoScale));
    }
  }
}

__device__ __forceinline__ void split_store(const float (&w)[32], uint32_t (&bh)[16], uint32_t (&bl)[16]) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const _Float16 h0 = (_Float16)w[2 * j], h1 = (_Float16)w[2 * j + 1];
    const _Float16 l0 = (_Float16)((w[2 * j] - (float)h0) * kLoScale);
    const _Float16 l1 = (_Float16)((w[2 * j + 1] - (float)h1) * kLoScale);
    bh[j] = pack_h2(h0, h1);
    bl[j] = pack_h2(l0, l1);
  }
}

// B: W[n, kb .. kb+32] dequantised (zero outside [0,N) x [0,K)).
template <uint32_t KIND>
__device__ __forceinline__ void load_b(const DevTensor& t, uint32_t n, uint32_t kb, const float* s_cent,
                                       _Float16* s_lut, Stage& st) {
  const bool live = n < t.rows && kb < t.cols;
  if constexpr (KIND == KIND_G64) {
    // group = kb/64 (BK == 64 so a 32-wide half never straddles groups)
    // Both threads of a row share one LDS table slot, so both load the table
    // whenever the 64-group is live, even if their own 32-column half is not.
    uint4 u = make_uint4(0, 0, 0, 0), l0 = u, l1 = u;
    if (live) u = load_nt16(static_cast<const uint8_t*>(t.p0) + (size_t)n * (t.kp / 2) + kb / 2);
    if (n < t.rows && (kb & ~63u) < t.cols) {
      const uint16_t* lp = t.p1 + ((size_t)n * (t.kp / 64) + kb / 64) * 16;
      l0 = load_nt16(lp);
      l1 = load_nt16(lp + 8);
    }
    // Table lookup through LDS: this thread's row slot receives the group's
    // 16 entries (both threads of a row write the same values), then each
    // index reads its entry.  Only this wave touches the slot.
    uint4* slot = reinterpret_cast<uint4*>(s_lut + (n & (BN - 1)) * 24);
    slot[0] = l0;
    slot[1] = l1;
    const uint16_t* tab = reinterpret_cast<const uint16_t*>(s_lut + (n & (BN - 1)) * 24);
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t c0 = 2 * j, c1 = 2 * j + 1;
      const uint32_t q0 = (wd[c0 >> 3] >> ((c0 & 7) * 4)) & 0xfu;
      const uint32_t q1 = (wd[c1 >> 3] >> ((c1 & 7) * 4)) & 0xfu;
      const uint32_t e0 = tab[q0], e1 = tab[q1];
      const bool z0 = !(kb + c0 < t.cols), z1 = !(kb + c1 < t.cols);
      st.bh[j] = (z0 ? 0u : e0) | ((z1 ? 0u : e1) << 16);
    }
  } else {
    float w[32];
    if constexpr (KIND == KIND_Q8) {
      uint4 a = make_uint4(0, 0, 0, 0), b = a;
      float d = 0.0f;
      if (live && kb < t.kp) {
        const int8_t* qp = static_cast<const int8_t*>(t.p0) + (size_t)n * t.kp + kb;
        a = load_nt16(qp);
        b = load_nt16(qp + 16);
        d = f16_to_f32(t.p1[(size_t)n * (t.kp / 32) + kb / 32]);
      }
      const uint32_t wd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const float q = (float)(int8_t)((wd[j >> 2] >> ((j & 3) * 8)) & 0xffu);
        w[j] = (kb + j < t.cols) ? q * d : 0.0f;
      }
    } else {  // KIND_CB4
      uint4 u = make_uint4(0, 0, 0, 0);
      float sc = 0.0f;
      if (live) {
        u = load_nt16(static_cast<const uint32_t*>(t.p0) + (size_t)n * (t.kp / 8) + kb / 8);
        sc = f16_to_f32(t.p1[(size_t)n * (t.kp / 128) + kb / 128]);
      }
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
      const float* tab = s_cent + 16u * cent_table(t, n);
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const float c = tab[(wd[j >> 3] >> ((j & 7) * 4)) & 0xfu];
        w[j] = (kb + j < t.cols) ? sc * c : 0.0f;
      }
    }
    split_store(w, st.bh, st.bl);
  }
}

template <uint32_t KIND, bool XBF16>
__global__ __launch_bounds__(THREADS) void gemm_kernel(DevTensor t, const void* __restrict__ x, uint32_t M,
                                                       void* __restrict__ y, uint32_t y_bf16, uint32_t x_vec) {
  constexpr bool SPLIT = KIND != KIND_G64;   // weights as hi + lo
  constexpr bool SPLIT_A = !XBF16;            // activations as hi + lo
  __shared__ __attribute__((aligned(16))) _Float16 sA[BM * LDK];
  __shared__ __attribute__((aligned(16))) _Float16 sAl[SPLIT_A ? BM * LDK : 8];
  __shared__ __attribute__((aligned(16))) _Float16 sB[BN * LDK];
  __shared__ __attribute__((aligned(16))) _Float16 sBl[SPLIT ? BN * LDK : 8];
  __shared__ float s_cent[48];
  __shared__ __attribute__((aligned(16))) _Float16 s_lut[KIND == KIND_G64 ? BN * 24 : 8];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63, wave = tid >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  const uint32_t n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const uint32_t N = t.rows, K = t.cols;

  if constexpr (KIND == KIND_CB4) {
    if (tid < 48) s_cent[tid] = t.cent[tid];
    __syncthreads();
  }

  // staging ownership: row tid/2, K half tid%2
  const uint32_t srow = tid >> 1, shalf = tid & 1;

  float16v acc[2][2], accl[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
        accl[i][j][r] = 0.0f;
      }

  Stage st;
  const uint32_t ktiles = (K + BK - 1) / BK;
  load_a<XBF16>(x, M, K, m0 + srow, shalf * 32, x_vec != 0, st.a, st.al);
  load_b<KIND>(t, n0 + srow, shalf * 32, s_cent, s_lut, st);

  for (uint32_t kt = 0; kt < ktiles; ++kt) {
    // registers -> LDS
    {
      uint4* da = reinterpret_cast<uint4*>(sA + srow * LDK + shalf * 32);
      uint4* db = reinterpret_cast<uint4*>(sB + srow * LDK + shalf * 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        da[i] = make_uint4(st.a[4 * i], st.a[4 * i + 1], st.a[4 * i + 2], st.a[4 * i + 3]);
        db[i] = make_uint4(st.bh[4 * i], st.bh[4 * i + 1], st.bh[4 * i + 2], st.bh[4 * i + 3]);
      }
      if constexpr (SPLIT_A) {
        uint4* dal = reinterpret_cast<uint4*>(sAl + srow * LDK + shalf * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dal[i] = make_uint4(st.al[4 * i], st.al[4 * i + 1], st.al[4 * i + 2], st.al[4 * i + 3]);
      }
      if constexpr (SPLIT) {
        uint4* dl = reinterpret_cast<uint4*>(sBl + srow * LDK + shalf * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dl[i] = make_uint4(st.bl[4 * i], st.bl[4 * i + 1], st.bl[4 * i + 2], st.bl[4 * i + 3]);
      }
    }
    __syncthreads();
    // prefetch the next K tile into registers while multiplying this one
    if (kt + 1 < ktiles) {
      const uint32_t kb = (kt + 1) * BK + shalf * 32;
      load_a<XBF16>(x, M, K, m0 + srow, kb, x_vec != 0, st.a, st.al);
      load_b<KIND>(t, n0 + srow, kb, s_cent, s_lut, st);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      half8 af[2], afl[2], bf[2], bfl[2];
      const uint32_t kofs = ks * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t ar = wm * 64 + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const half8*>(sA + ar * LDK + kofs);
        if constexpr (SPLIT_A) afl[i] = *reinterpret_cast<const half8*>(sAl + ar * LDK + kofs);
        const uint32_t br = wn * 64 + i * 32 + (lane & 31);
        bf[i] = *reinterpret_cast<const half8*>(sB + br * LDK + kofs);
        if constexpr (SPLIT) bfl[i] = *reinterpret_cast<const half8*>(sBl + br * LDK + kofs);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
          if constexpr (SPLIT)
            accl[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bfl[j], accl[i][j], 0, 0, 0);
          if constexpr (SPLIT_A)   // lo * lo is below 2^-22 relative and dropped
            accl[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bf[j], accl[i][j], 0, 0, 0);
        }
    }
    __syncthreads();
  }

  if constexpr (SPLIT || SPLIT_A) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(accl[i][j][r], kLoInv, acc[i][j][r]);
  }

  // epilogue: lane owns column n = n0 + wn*64 + j*32 + lane%32 of tile (i, j),
  // rows m = m0 + wm*64 + i*32 + (lane/32)*4 + 8*(r/4) + r%4.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t n = n0 + wn * 64 + j * 32 + (lane & 31);
    if constexpr (KIND == KIND_CB4) {
      if (n < N) {
        const uint32_t os = t.row_ptr[n], oe = t.row_ptr[n + 1];
        for (uint32_t o = os; o < oe; ++o) {
          const uint32_t pk = t.outliers[o];
          const uint32_t col = pk & 0xffffu;
          if (col >= K) continue;
          const float res = f16_to_f32(pk >> 16);
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const uint32_t m = m0 + wm * 64 + i * 32 + (lane >> 5) * 4 + 8 * (r >> 2) + (r & 3);
              if (m < M) {
                float xv;
                if constexpr (XBF16)
                  xv = bf16_to_f32(static_cast<const uint16_t*>(x)[(size_t)m * K + col]);
                else
                  xv = static_cast<const float*>(x)[(size_t)m * K + col];
                acc[i][j][r] = __builtin_fmaf(res, xv, acc[i][j][r]);
              }
            }
        }
      }
    }
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t m = m0 + wm * 64 + i * 32 + (lane >> 5) * 4 + 8 * (r >> 2) + (r & 3);
        if (m < M) {
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * N + n] = f32_to_bf16(acc[i][j][r]);
          else
            static_cast<float*>(y)[(size_t)m * N + n] = acc[i][j][r];
        }
      }
  }
}

}  // namespace gemm

template <uint32_t KIND>
static hipError_t launch_gemm_kind(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y,
                                   bool y_bf16, hipStream_t s) {
  dim3 grid((t.rows + gemm::BN - 1) / gemm::BN, (m + gemm::BM - 1) / gemm::BM);
  const size_t esz = x_bf16 ? 2 : 4;
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && ((size_t)t.cols * esz) % 16 == 0;
  if (x_bf16)
    hipLaunchKernelGGL((gemm::gemm_kernel<KIND, true>), grid, dim3(gemm::THREADS), 0, s, t, x, m, y,
                       (uint32_t)y_bf16, x_vec);
  else
    hipLaunchKernelGGL((gemm::gemm_kernel<KIND, false>), grid, dim3(gemm::THREADS), 0, s, t, x, m, y,
                       (uint32_t)y_bf16, x_vec);
  return hipGetLastError();
}

hipError_t launch_gemm(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y,
                       bool y_bf16, hipStream_t s) {
  if (m > 65535u * gemm::BM) return hipErrorInvalidValue;
  switch (t.kind) {
    case KIND_G64: return launch_gemm_kind<KIND_G64>(t, x, x_bf16, m, y, y_bf16, s);
    case KIND_Q8: return launch_gemm_kind<KIND_Q8>(t, x, x_bf16, m, y, y_bf16, s);
    case KIND_CB4: return launch_gemm_kind<KIND_CB4>(t, x, x_bf16, m, y, y_bf16, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vxt
