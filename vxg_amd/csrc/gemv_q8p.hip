// gemv_q8p.hip -- the persistent MFMA decode GEMV for Q8 weights at 3..8
// tokens over many rows (the LM head), in its own translation unit so that it
// alone is compiled with MFMA results in VGPRs (-amdgpu-mfma-vgpr-form, set
// in build.py): each fragment is scaled on the VALU right after its MFMAs,
// and with AGPR results every element needed a v_accvgpr_read first (96 of
// ~700 VALU instructions of the loop).
#include "gemv_impl.hpp"

namespace vxt {
namespace gv {

// Q8 x bf16 activations, 3..8 tokens, many rows (the LM head): the arithmetic
// of gemv_q8_mfma_kernel (two blocks of 16 rows x 32 columns per four
// v_mfma_f32_16x16x32_bf16, the block scales on the fragments) in a
// persistent grid.  Each workgroup stages every token's activations once in
// LDS (row stride NS * 2048 + 8 elements: the 16-byte pad puts the eight
// token rows of one fragment read in distinct bank groups), plus one row of
// zeros: the lanes whose half of a 64-column pair belongs to the other block
// (and lanes of tokens past M) read their MFMA operand from the zero row, so
// the operands need no selects.  Each wave owns whole 16-row tiles, all of
// K, tiles blockIdx.x * WAVES + wave, then + gridDim.x * WAVES.  The weights
// (16 bytes per lane per pair of blocks) and the scales (4 bytes per lane per
// pair) go in batches of PB pairs through NBUF register sets: the loads run
// NBUF - 1 batches ahead of the multiplication -- from clamped addresses,
// unconditionally -- also across tile boundaries.  Against
// gemv_q8_mfma_kernel this reads the activations from LDS rather than once
// per 16 rows from L2, and needs no barrier per tile.
// Requires kp % (64 PB) == 0, kp <= NS * 2048, cols % 8 == 0 and
// 16-byte aligned activations.

// The weights and scale pairs of pairs b * PB.. of tile `tile`, for lane
// (c16, grp): row tile * 16 + c16, columns 64 p + 16 grp .. + 15; scale pair
// i (blocks 2 p, 2 p + 1) in dp[i].
template <int PB>
__device__ __forceinline__ void q8p_load(const DevTensor& t, uint32_t tile, uint32_t b, uint32_t c16, uint32_t grp,
                                         u32x4 (&wv)[PB], uint32_t (&dp)[PB]) {
  const uint32_t nb = t.kp / 32;
  const uint32_t row = tile * 16 + c16 < t.rows ? tile * 16 + c16 : t.rows - 1;
  const uint8_t* wr = static_cast<const uint8_t*>(t.p0) + (size_t)row * t.kp + (size_t)b * (64 * PB) + 16 * grp;
#pragma unroll
  for (int i = 0; i < PB; ++i) wv[i] = *reinterpret_cast<const u32x4*>(wr + i * 64);
  const u32x4* dr = reinterpret_cast<const u32x4*>(t.p1 + (size_t)row * nb + (size_t)b * (2 * PB));
#pragma unroll
  for (int i = 0; i < PB / 4; ++i) {
    const u32x4 v = dr[i];
    dp[4 * i] = v.x;
    dp[4 * i + 1] = v.y;
    dp[4 * i + 2] = v.z;
    dp[4 * i + 3] = v.w;
  }
}

// Multiplies pairs b * PB.. into acc (token 4 grp + r, row c16).  xlo / xhi:
// LDS byte addresses of the lane's operand rows for the pair's first /
// second block (the token row + 32 grp, or the zero row).
template <int PB>
__device__ __forceinline__ void q8p_compute(uint32_t b, uint32_t xlo, uint32_t xhi, const u32x4 (&wv)[PB],
                                            const uint32_t (&dp)[PB], f32x4_t& acc) {
  typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t lo = xlo + b * (128 * PB), hi = xhi + b * (128 * PB);
#pragma unroll
  for (int i = 0; i < PB; ++i) {
    const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, *(lds_u32x4*)(size_t)(lo + 128 * i));
    const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, *(lds_u32x4*)(size_t)(lo + 128 * i + 16));
    const bf16x8_t a2 = __builtin_bit_cast(bf16x8_t, *(lds_u32x4*)(size_t)(hi + 128 * i));
    const bf16x8_t a3 = __builtin_bit_cast(bf16x8_t, *(lds_u32x4*)(size_t)(hi + 128 * i + 16));
    const bf16x8_t wlo = q8_bf16x8(wv[i].x, wv[i].y), whi = q8_bf16x8(wv[i].z, wv[i].w);
    f32x4_t b0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, wlo, zero, 0, 0, 0);
    b0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, whi, b0, 0, 0, 0);
    f32x4_t b1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, wlo, zero, 0, 0, 0);
    b1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, whi, b1, 0, 0, 0);
    const float d0 = f16_to_f32(dp[i] & 0xffffu), d1 = f16_to_f32(dp[i] >> 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] += d0 * b0[r];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] += d1 * b1[r];
  }
}

template <int WAVES, int NS, int PB, int NBUF>
__global__ __launch_bounds__(WAVES * 64) void gemv_q8_mfma_p_kernel(DevTensor t, const uint16_t* __restrict__ x,
                                                                   void* __restrict__ y, uint32_t M_rt,
                                                                   uint32_t y_bf16) {
  constexpr uint32_t kRow = NS * kStep + 8;   // LDS row stride, elements
  constexpr uint32_t kPieces = 8u * NS * (kStep / 8);
  static_assert(kPieces % (WAVES * 64) == 0, "staging pieces per thread");
  static_assert(NBUF >= 2, "at least one batch in flight while one is multiplied");
  constexpr uint32_t kPer = kPieces / (WAVES * 64);
  __shared__ __attribute__((aligned(16))) uint16_t s_x[9 * kRow];   // 8 token rows, then zeros
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rows = t.rows, cols = t.cols;
  // Every token's row once (zero past cols), then one barrier.
  u32x4 xv[kPer];
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t p = tid + WAVES * 64 * j, m = p / (NS * kStep / 8), q = p % (NS * kStep / 8);
    xv[j] = __builtin_amdgcn_raw_buffer_load_b128(x_row_rsrc(x, cols, m < M_rt ? m : 0), q * 16u, 0, 0);
  }
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t p = tid + WAVES * 64 * j, m = p / (NS * kStep / 8), q = p % (NS * kStep / 8);
    if (m < M_rt) *reinterpret_cast<u32x4*>(&s_x[m * kRow + q * 8]) = xv[j];
  }
  for (uint32_t q = tid; q < kRow / 8; q += WAVES * 64)
    *reinterpret_cast<u32x4*>(&s_x[8 * kRow + q * 8]) = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();

  const uint32_t ntiles = (rows + 15) / 16, stride = gridDim.x * WAVES;
  const uint32_t nbat = t.kp / (64 * PB);
  const uint32_t first = blockIdx.x * WAVES + wave;
  if (first >= ntiles) return;
  // The wave's batches in order: (tile, batch) = (first + stride * (i / nbat),
  // i % nbat).  The loads run NBUF - 1 batches ahead of the multiplication;
  // loads past the wave's last batch re-read its last tile (unconditional).
  const uint32_t n_mine = ((ntiles - 1 - first) / stride + 1) * nbat;
  const uint32_t c16 = lane & 15, grp = lane >> 4;
  const bool lo_half = grp < 2;
  const uint32_t xrow = lds_addr(s_x) + (c16 < M_rt ? c16 : 8u) * kRow * 2u + 32u * grp;
  const uint32_t zrow = lds_addr(s_x) + 8u * kRow * 2u + 32u * grp;
  const uint32_t xlo = lo_half ? xrow : zrow, xhi = lo_half ? zrow : xrow;
  const uint32_t last_tile = first + stride * (n_mine / nbat - 1);
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  u32x4 w[NBUF][PB];
  uint32_t d[NBUF][PB];
  uint32_t lt = first, lb = 0;   // next batch to load
#pragma unroll
  for (int j = 0; j < NBUF - 1; ++j) {
    q8p_load(t, lt <= last_tile ? lt : last_tile, lb, c16, grp, w[j], d[j]);
    if (++lb == nbat) {
      lb = 0;
      lt += stride;
    }
  }
  uint32_t ct = first, cb = 0, done = 0;   // batch to multiply, batches multiplied
  for (;;) {
#pragma unroll
    for (int j = 0; j < NBUF; ++j) {
      q8p_load(t, lt <= last_tile ? lt : last_tile, lb, c16, grp, w[(j + NBUF - 1) % NBUF], d[(j + NBUF - 1) % NBUF]);
      if (++lb == nbat) {
        lb = 0;
        lt += stride;
      }
      // the loads above stay ahead of the arithmetic (the scheduler would
      // otherwise sink them to their uses)
      __builtin_amdgcn_sched_barrier(0);
      q8p_compute(cb, xlo, xhi, w[j], d[j], acc);
      if (++cb == nbat) {
        const uint32_t n = ct * 16 + c16;
        if (n < rows) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t m = 4 * grp + r;
            if (m < M_rt) {
              if (y_bf16)
                static_cast<uint16_t*>(y)[(size_t)m * rows + n] = f32_to_bf16(acc[r]);
              else
                static_cast<float*>(y)[(size_t)m * rows + n] = acc[r];
            }
          }
        }
        acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        cb = 0;
        ct += stride;
      }
      if (++done == n_mine) break;
    }
    if (done == n_mine) break;
  }
}

// Q8 x bf16 activations, 5..8 tokens, 8 weight rows per workgroup: twice
// the row tiles of gemv_q8_mfma_kernel (16 rows), for matrices whose row
// count leaves CUs idle at 16.  One v_mfma_f32_16x16x32_bf16 multiplies
// both 32-column blocks of a 64-column pair for 8 rows: operand rows
// (tokens) 0-7 and columns (weight rows) 0-7 carry the pair's first block,
// operand rows and columns 8-15 its second, so the two diagonal 8 x 8
// quarters of the result are the two blocks' partial dot products and the
// off-diagonal quarters (blocks mixed) are dropped.  A result element's
// block scale depends only on its column, so each lane applies one scale
// per pair.  Half of each MFMA is kept, as in gemv_q8_mfma_kernel, whose
// masked operands give the same ratio.  The waves of a workgroup split the
// pairs (PB pairs of loads in flight per batch); the diagonal quarters of
// every wave are added through LDS in wave order.
// Requires cols % 8 == 0, 16-byte aligned activations and kp / 32 <=
// kQ8M8MaxNb.

template <int WAVES, int PB>
__global__ __launch_bounds__(WAVES * 64) void gemv_q8_mfma8_kernel(DevTensor t, const uint16_t* __restrict__ x,
                                                                  void* __restrict__ y, uint32_t M_rt,
                                                                  uint32_t y_bf16) {
  constexpr uint32_t kDi = (8 * kQ8M8MaxNb + WAVES * 64 - 1) / (WAVES * 64);   // scale loads per thread
  __shared__ uint16_t s_d[8 * kQ8M8MaxNb];
  __shared__ f32x4_t s_red[WAVES][64];
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rows = t.rows, cols = t.cols, kp = t.kp;
  const uint32_t nb = kp / 32, np = (nb + 1) / 2;
  const uint32_t row0 = blockIdx.x * 8;
  // Lane (c16, grp): operand row / column c16, K elements 8 grp .. 8 grp + 7
  // of its block; hi = second block of the pair.
  const uint32_t c16 = lane & 15, grp = lane >> 4, hi = c16 >> 3, r8 = c16 & 7;

  // The tile's scales (rows row0 .., contiguous in the plane), clamped loads.
  const uint32_t dn = 8 * nb;
  const size_t dlast = (size_t)rows * nb - 1;
  uint16_t dv[kDi];
#pragma unroll
  for (uint32_t i = 0; i < kDi; ++i) {
    const size_t idx = (size_t)row0 * nb + tid + i * (WAVES * 64);
    dv[i] = t.p1[idx < dlast ? idx : dlast];
  }

  const uint32_t row = row0 + r8 < rows ? row0 + r8 : rows - 1;   // rows past the matrix are never stored
  const bool tok_live = r8 < M_rt;                                  // operand row c16 is token r8
  const uint16_t* xr = x + (size_t)(tok_live ? r8 : 0) * cols;
  const uint8_t* wr = static_cast<const uint8_t*>(t.p0) + (size_t)row * kp;
  const uint32_t koff = 32 * hi + 8 * grp;   // the lane's columns inside a pair
  const uint32_t p_begin = wave * np / WAVES, p_end = (wave + 1) * np / WAVES;   // uniform per wave
  const u32x4 z = {0u, 0u, 0u, 0u};
  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t acc = zero;
  bool staged = false;
  for (uint32_t p0 = p_begin; p0 < p_end; p0 += PB) {
    uint2 wv[PB];
    u32x4 xv[PB];
#pragma unroll
    for (int i = 0; i < PB; ++i) {   // clamped, unconditional loads
      const uint32_t p = p0 + i < p_end ? p0 + i : p_end - 1;
      const uint32_t k = p * 64 + koff;
      // A second block past the row (odd nb) re-reads the first block's
      // bytes; its activations are past cols (zero) and its scale is 0.
      wv[i] = *reinterpret_cast<const uint2*>(wr + (k < kp ? k : k - 32));
      xv[i] = *reinterpret_cast<const u32x4*>(xr + (k < cols ? k : cols - 8));
    }
    if (!staged) {   // first batch only (uniform): scales to LDS behind the loads above
#pragma unroll
      for (uint32_t i = 0; i < kDi; ++i) {
        const uint32_t j = tid + i * (WAVES * 64);
        if (j < dn) s_d[j] = dv[i];
      }
      lds_barrier();
      staged = true;
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      const uint32_t p = p0 + i;
      if (p >= p_end) continue;   // uniform
      const uint32_t k = p * 64 + koff, blk = 2 * p + hi;
      const bf16x8_t a = __builtin_bit_cast(bf16x8_t, tok_live && k < cols ? xv[i] : z);
      const f32x4_t c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, q8_bf16x8(wv[i].x, wv[i].y), zero, 0, 0, 0);
      const float d = blk < nb ? f16_to_f32(s_d[r8 * nb + blk]) : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += d * c[j];
    }
  }
  if (!staged) {   // a wave with no pairs still takes part in the staging barrier
#pragma unroll
    for (uint32_t i = 0; i < kDi; ++i) {
      const uint32_t j = tid + i * (WAVES * 64);
      if (j < dn) s_d[j] = dv[i];
    }
    lds_barrier();
  }
  // Lane (c16, grp) holds result rows 4 grp .. 4 grp + 3 of column c16: the
  // first block's quarter in lanes c16 < 8, grp < 2 (tokens 4 grp + j, weight
  // row c16), the second block's in lanes c16 >= 8, grp >= 2, 40 lanes on.
  s_red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && grp < 2 && c16 < 8) {
    f32x4_t v = zero;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const f32x4_t a = s_red[w][lane], b = s_red[w][lane + 40];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] += a[j] + b[j];
    }
    const uint32_t n = row0 + c16;
    if (n < rows) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t m = 4 * grp + j;
        if (m < M_rt) {
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * rows + n] = f32_to_bf16(v[j]);
          else
            static_cast<float*>(y)[(size_t)m * rows + n] = v[j];
        }
      }
    }
  }
}

template <int WAVES, int PB>
hipError_t launch_q8_mfma8_t(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  if (m > 8 || t.cols % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 || t.kp / 32 > kQ8M8MaxNb)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemv_q8_mfma8_kernel<WAVES, PB>), dim3((t.rows + 7) / 8), dim3(WAVES * 64), 0, s, t,
                     static_cast<const uint16_t*>(x), y, m, (uint32_t)(y_bf16 ? 1u : 0u));
  return hipGetLastError();
}

hipError_t launch_q8_m8(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  return launch_q8_mfma8_t<8, 6>(t, x, m, y, y_bf16, s);
}

template <int WAVES, int NS, int PB, int NBUF>
hipError_t launch_q8_mfma_p_t(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s,
                              uint32_t per_cu) {
  if (m > 8 || t.cols % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 || t.kp % (64 * PB) != 0 ||
      t.kp > (uint32_t)NS * kStep || t.kp < (uint32_t)(NS - 1) * kStep)
    return hipErrorInvalidValue;
  // As many tiles per wave as the resident waves need, spread evenly: a wave
  // owns whole tiles, so a last round that only some waves run would leave
  // the rest of the chip idle for a whole tile.
  const uint32_t ntiles = (t.rows + 15) / 16, resident = 256u * per_cu * WAVES;
  const uint32_t rounds = (ntiles + resident - 1) / resident;
  const uint32_t waves = (ntiles + rounds - 1) / rounds;
  const uint32_t grid = (waves + WAVES - 1) / WAVES;
  hipLaunchKernelGGL((gemv_q8_mfma_p_kernel<WAVES, NS, PB, NBUF>), dim3(grid), dim3(WAVES * 64), 0, s, t,
                     static_cast<const uint16_t*>(x), y, m, (uint32_t)(y_bf16 ? 1u : 0u));
  return hipGetLastError();
}

hipError_t launch_q8_lm(const DevTensor& t, const void* x, uint32_t m, void* y, bool y_bf16, hipStream_t s) {
  return t.kp <= kStep ? launch_q8_mfma_p_t<4, 1, 8, 3>(t, x, m, y, y_bf16, s, 1)
                       : launch_q8_mfma_p_t<4, 2, 8, 3>(t, x, m, y, y_bf16, s, 1);
}

}  // namespace gv
}  // namespace vxt
