// gemm_dense.hip -- the dense phase of the two-phase prefill GEMM for large
// batches: Y = A * W^T with A the row-scaled f16 activations [M][kp] and W
// the f16 weight panel [N][kp] (gemm_panel.hip writes both), 128 x 128
// output tiles.
//
// Reference behaviour: the dense tile product of PackedTensor::gemm_cpu
// (llm_prefill.rs:156-255) over decoded weights; products are exact in the
// fp32 MFMA accumulators.
//
// Modes (the panel's weight representation, WMode in gemm_panel.hip):
//   * plain: f16 values (g64);
//   * hi/lo (cb4; Q8 with f32 activations or pinned paths): w * s = hi +
//     lo * 2^-11, two f16 planes, each product into its own accumulator,
//     combined as acc + accl * 2^-11 in the epilogue;
//   * Q8 block: int8 values as f16 and one f32 scale per (row, 32-column
//     block): each block is two 16-deep MFMAs into fresh fragments, then
//     acc += d * fragment (the lane's output column is fixed, so one scale
//     per fragment).
//
// Schedule (one workgroup = 4 waves in 2 x 2, 64 x 64 outputs per wave,
// K tiles of 64):
//   * operands are register-staged two tiles ahead into two LDS stages of
//     128 rows x 128 B per operand, 16-byte chunk c of row r stored at chunk
//     c ^ ((r >> 1) & 7): fragment reads (16 lanes = 16 rows at one chunk)
//     and row writes touch distinct banks;
//   * inside a K tile, every MFMA is followed by one slice of the other
//     work: the next step's fragment reads, one 16-byte piece of the next
//     tile's activations and weights (LDS store, then the global load of
//     the tile after that into the freed registers).  Measured on MI355X at
//     2048 x 6144 x 2048 f16, this interleave takes the kernel from 718 to
//     887 TFLOP/s against the same loop with the staging bunched at the top;
//   * no memory operation in the loop body is conditional (tile indices are
//     clamped), so the compiler counts its waits in one static order and the
//     loads of the tile after next stay in flight across the stores.
//   With gridDim.y > 1 the workgroup writes fp32 partial sums of its K
//   slice; reduce_kernel adds them in slice order and applies the scales.
#include <algorithm>
#include <type_traits>

#include "common.hpp"

#pragma clang fp contract(off)

namespace vxt {

namespace gd {

constexpr int BM = 128, BN = 128, BK = 64, NT = 256;
constexpr uint32_t kOpBytes = 128 * 128;   // one operand of one stage

enum : int { kPlain = 0, kHiLo = 1, kQBlock = 2 };

// operands per stage: A, W (and W's lo plane)
template <int MODE>
constexpr uint32_t stage_bytes() { return (MODE == kHiLo ? 3 : 2) * kOpBytes; }

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));


__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t c) { return c ^ ((row >> 1) & 7u); }

// Piece j (0..3) of a 128-row x 64-column operand tile for thread tid:
// row (tid + 256 j) / 8, chunk (tid + 256 j) % 8.
__device__ __forceinline__ u32x4 gload(const uint16_t* __restrict__ P, uint32_t r0, uint32_t rows, uint32_t kp,
                                       uint32_t kt, uint32_t tid, int j) {
  const uint32_t i = tid + NT * j;
  const uint32_t row = std::min(r0 + i / 8, rows - 1);   // rows past the end repeat the last (never stored)
  return *reinterpret_cast<const u32x4*>(P + (size_t)row * kp + kt * BK + (i % 8) * 8);
}

__device__ __forceinline__ void lstore(char* op, uint32_t tid, int j, const u32x4& v) {
  const uint32_t i = tid + NT * j;
  const uint32_t row = i / 8, c = i % 8;
  *reinterpret_cast<u32x4*>(op + row * 128 + swz(row, c) * 16) = v;
}

// hi/lo and Q8 block modes hold a second accumulator set (the lo products,
// or the block's fragments): one workgroup per CU keeps it in registers.
template <int MODE>
constexpr int occupancy() { return MODE == kPlain ? 2 : 1; }

template <int MODE>
__global__ __launch_bounds__(NT, occupancy<MODE>()) void dense2_kernel(const uint16_t* __restrict__ ah, const uint16_t* __restrict__ bh,
                                                       const uint16_t* __restrict__ bl, const float* __restrict__ dsc, const float* __restrict__ inv,
                                                       uint32_t M, uint32_t N, uint32_t kp, void* __restrict__ y,
                                                       uint32_t y_bf16, float* __restrict__ partial,
                                                       uint32_t kt_per_split, uint32_t tiles_m,
                                                       const int32_t* __restrict__ xe) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const uint32_t tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave >> 1, wn = wave & 1;
  // Tile order: blocks b, b+8, ... run on one XCD (one L2), so each XCD gets
  // a contiguous range of tiles, walked in groups of 8 tile rows.
  uint32_t tm, tn;
  {
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t bb = (G % 8u == 0u) ? (b % 8u) * (G / 8u) + b / 8u : b;
    const uint32_t tiles_n = G / tiles_m;
    constexpr uint32_t GM = 8;
    const uint32_t in_group = GM * tiles_n;
    const uint32_t first = bb / in_group * GM;
    const uint32_t gsz = std::min(tiles_m - first, GM);
    tm = first + (bb % in_group) % gsz;
    tn = (bb % in_group) / gsz;
  }
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t KTT = kp / BK;
  const uint32_t kt0 = blockIdx.y * kt_per_split;
  const uint32_t kt1 = std::min(KTT, kt0 + kt_per_split);
  const uint32_t KT = kt1 - kt0;   // >= 1
  auto ktile = [&](uint32_t i) { return std::min(kt0 + i, kt1 - 1); };
  constexpr bool LO = MODE == kHiLo;
  // The tile's row exponents are requested now, so the epilogue does not
  // wait for another round trip to memory.
  const int32_t xe_pre = xe[std::min(m0 + (tid & (BM - 1)), M - 1)];
#define SA(st) (smem + (st) * stage_bytes<MODE>())
#define SB(st) (smem + (st) * stage_bytes<MODE>() + kOpBytes)
#define SL(st) (smem + (st) * stage_bytes<MODE>() + 2 * kOpBytes)

  float16v acc[2][2], accl[LO ? 2 : 1][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
        if constexpr (LO) accl[i][j][r] = 0.0f;
      }

  // fragment (i, step s) of operand rows r0 + 32 i + l32: chunk 2 s + h
  uint32_t offA[4], offB[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t ra_ = wm * 64 + l32, rb_ = wn * 64 + l32;   // + 32 i keeps the swizzle ((32 i) >> 1 & 7 == 0)
    offA[s] = ra_ * 128 + swz(ra_, 2 * s + h) * 16;
    offB[s] = rb_ * 128 + swz(rb_, 2 * s + h) * 16;
  }
  // Q8 block scales of this lane's output columns (fragment j), blocks 2 kt, 2 kt + 1
  const uint32_t nblk = kp / 32;
  uint32_t ncl[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) ncl[j] = std::min(n0 + wn * 64 + j * 32 + l32, N - 1);
  auto dload = [&](uint32_t kt, float (&d)[2][2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float2 v = *reinterpret_cast<const float2*>(dsc + (size_t)ncl[j] * nblk + 2 * kt);
      d[j][0] = v.x;
      d[j][1] = v.y;
    }
  };

  u32x4 ra[2][4], rb[2][4], rl[LO ? 2 : 1][4];
  float dq[2][2][2];   // Q8 block mode: scales of tile i in dq[i & 1], loaded two tiles ahead
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ra[p][j] = gload(ah, m0, M, kp, ktile(p), tid, j);
      rb[p][j] = gload(bh, n0, N, kp, ktile(p), tid, j);
      if constexpr (LO) rl[p][j] = gload(bl, n0, N, kp, ktile(p), tid, j);
    }
  if constexpr (MODE == kQBlock) {
    dload(ktile(0), dq[0]);
    dload(ktile(1), dq[1]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    lstore(SA(0), tid, j, ra[0][j]);
    lstore(SB(0), tid, j, rb[0][j]);
    if constexpr (LO) lstore(SL(0), tid, j, rl[0][j]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ra[0][j] = gload(ah, m0, M, kp, ktile(2), tid, j);
    rb[0][j] = gload(bh, n0, N, kp, ktile(2), tid, j);
    if constexpr (LO) rl[0][j] = gload(bl, n0, N, kp, ktile(2), tid, j);
  }
  __syncthreads();

  // One K tile from stage `st`; when STAGE is set, piece s of the next tile
  // (registers ra/rb[slot]) goes to stage st ^ 1 during step s and the slot
  // is reloaded with tile kn.
  auto tile = [&](int st, auto staged, int slot, uint32_t kn, const float (&d)[2][2]) {
    constexpr bool STAGE = decltype(staged)::value;
    const char* a_st = SA(st);
    const char* b_st = SB(st);
    const char* l_st = SL(st);
    char* const a_nx = SA(st ^ 1);
    char* const b_nx = SB(st ^ 1);
    char* const l_nx = SL(st ^ 1);
    half8 af[2][2], bf[2][2], lf[LO ? 2 : 1][2];
    float16v tmp[MODE == kQBlock ? 2 : 1][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      af[0][i] = *reinterpret_cast<const half8*>(a_st + i * 4096 + offA[0]);
      bf[0][i] = *reinterpret_cast<const half8*>(b_st + i * 4096 + offB[0]);
      if constexpr (LO) lf[0][i] = *reinterpret_cast<const half8*>(l_st + i * 4096 + offB[0]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      auto mma = [&](int i, int j) {
        if constexpr (MODE == kQBlock)
          tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][i], bf[cur][j], (s & 1) ? tmp[i][j] : float16v{},
                                                             0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][i], bf[cur][j], acc[i][j], 0, 0, 0);
        if constexpr (LO)
          accl[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][i], lf[cur][j], accl[i][j], 0, 0, 0);
      };
      __builtin_amdgcn_sched_barrier(0);
      mma(0, 0);
      if (s < 3) {
        af[nxt][0] = *reinterpret_cast<const half8*>(a_st + offA[s + 1]);
        bf[nxt][0] = *reinterpret_cast<const half8*>(b_st + offB[s + 1]);
        if constexpr (LO) lf[nxt][0] = *reinterpret_cast<const half8*>(l_st + offB[s + 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      mma(0, 1);
      if constexpr (STAGE) {
        lstore(a_nx, tid, s, ra[slot][s]);
        ra[slot][s] = gload(ah, m0, M, kp, kn, tid, s);
      }
      __builtin_amdgcn_sched_barrier(0);
      mma(1, 0);
      if (s < 3) {
        af[nxt][1] = *reinterpret_cast<const half8*>(a_st + 4096 + offA[s + 1]);
        bf[nxt][1] = *reinterpret_cast<const half8*>(b_st + 4096 + offB[s + 1]);
        if constexpr (LO) lf[nxt][1] = *reinterpret_cast<const half8*>(l_st + 4096 + offB[s + 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      mma(1, 1);
      if constexpr (STAGE) {
        lstore(b_nx, tid, s, rb[slot][s]);
        rb[slot][s] = gload(bh, n0, N, kp, kn, tid, s);
        if constexpr (LO) {
          lstore(l_nx, tid, s, rl[slot][s]);
          rl[slot][s] = gload(bl, n0, N, kp, kn, tid, s);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (MODE == kQBlock) {
        if (s & 1) {   // block s / 2 done: acc += d * fragment
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(d[j][s >> 1], tmp[i][j][r], acc[i][j][r]);
        }
      }
    }
  };
  using T = std::true_type;
  using F = std::false_type;
  // Iteration i (P = i & 1): multiply stage P; stage tile i+1 (slot P^1)
  // into stage P^1 and reload the slot with tile i+3; reload the scales of
  // tile i with those of tile i+2.
  uint32_t i = 0;
  for (; i + 2 < KT; i += 2) {
    tile(0, T{}, 1, ktile(i + 3), dq[0]);
    if constexpr (MODE == kQBlock) dload(ktile(i + 2), dq[0]);
    __syncthreads();
    tile(1, T{}, 0, ktile(i + 4), dq[1]);
    if constexpr (MODE == kQBlock) dload(ktile(i + 3), dq[1]);
    __syncthreads();
  }
  if (i + 1 < KT) {
    tile(0, T{}, 1, ktile(i + 3), dq[0]);
    __syncthreads();
    tile(1, F{}, 0, 0, dq[1]);
  } else {
    tile(0, F{}, 0, 0, dq[0]);
  }
#undef SA
#undef SB
#undef SL

  // Lane owns column n0 + wn*64 + j*32 + l32 of fragment (i, j), rows
  // m0 + wm*64 + i*32 + 4h + 8(r/4) + r%4.  The tile's 128 row exponents go
  // through LDS (loaded in the prologue): read per output from global memory
  // they cost more than the last K tiles.  bf16 outputs of a whole tile are
  // transposed through LDS and written as 16-byte pieces of full rows (lane
  // stores of 2 bytes write half lines, which costs as much as the last
  // fifth of the K loop).
  const bool to_partial = gridDim.y > 1;
  int32_t* s_xe = reinterpret_cast<int32_t*>(smem);
  uint16_t* s_out = reinterpret_cast<uint16_t*>(smem + 1024);   // [128][128 + 8] bf16
  constexpr uint32_t LDO = BN + 8;
  const bool rows_fast = y_bf16 && !to_partial && N % 8 == 0 && n0 + BN <= N &&
                         reinterpret_cast<uintptr_t>(y) % 16 == 0;
  if (!to_partial) {
    __syncthreads();   // every wave is done with the stages
    if (tid < BM) s_xe[tid] = xe_pre;
    __syncthreads();
  }
  // this lane's 32 row exponents, 4 consecutive rows per 16-byte read
  int xs[2][16];
  if (!to_partial) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int4 e4 = *reinterpret_cast<const int4*>(s_xe + wm * 64 + ii * 32 + h * 4 + 8 * q);
        xs[ii][4 * q + 0] = e4.x;
        xs[ii][4 * q + 1] = e4.y;
        xs[ii][4 * q + 2] = e4.z;
        xs[ii][4 * q + 3] = e4.w;
      }
  }
  // One loop per output mode (a mode test per output compiles to branches
  // per output).
  auto row_of = [&](int ii, int r) { return (uint32_t)(wm * 64 + ii * 32 + h * 4 + 8 * (r >> 2) + (r & 3)); };
  auto value = [&](int ii, int j, int r) {
    float v = acc[ii][j][r];
    if constexpr (LO) v = hilo_combine(v, accl[ii][j][r]);
    return v;
  };
  if (rows_fast) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t nl = wn * 64 + j * 32 + l32;
      const float sc = inv[n0 + nl];
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s_out[row_of(ii, r) * LDO + nl] = f32_to_bf16(ldexpf(value(ii, j, r) * sc, -xs[ii][r]));
    }
  } else if (to_partial) {
    const bool full = m0 + BM <= M && n0 + BN <= N;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t n = n0 + wn * 64 + j * 32 + l32;
      float* const pp = partial + ((size_t)blockIdx.y * M + m0) * N + n;
      if (full) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int r = 0; r < 16; ++r) pp[(size_t)row_of(ii, r) * N] = value(ii, j, r);
      } else {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (m0 + row_of(ii, r) < M && n < N) pp[(size_t)row_of(ii, r) * N] = value(ii, j, r);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t n = n0 + wn * 64 + j * 32 + l32;
      const float sc = inv[std::min(n, N - 1)];
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t m = m0 + row_of(ii, r);
          if (m >= M || n >= N) continue;
          const float o = ldexpf(value(ii, j, r) * sc, -xs[ii][r]);
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * N + n] = f32_to_bf16(o);
          else
            static_cast<float*>(y)[(size_t)m * N + n] = o;
        }
    }
  }
  if (rows_fast) {   // uniform
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t idx = tid + NT * k, row = idx / 16, c = idx % 16;
      if (m0 + row >= M) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(s_out + row * LDO + c * 8);
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(y) + (size_t)(m0 + row) * N + n0 + c * 8) = v;
    }
  }
}

template <int MODE>
hipError_t launch(const uint16_t* ah, const uint16_t* bh, const uint16_t* bl, const float* dsc, const float* inv,
                  uint32_t m, uint32_t n, uint32_t kp, void* y, bool y_bf16, float* partial, uint32_t splits,
                  uint32_t kt_per_split, const int32_t* xe, hipStream_t s) {
  constexpr size_t lds = 2 * stage_bytes<MODE>();
  static_assert(lds <= 160 * 1024 && lds >= 1024 + (size_t)BM * (BN + 8) * 2, "LDS budget");
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&dense2_kernel<MODE>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  const uint32_t tiles_m = (m + BM - 1) / BM;
  hipLaunchKernelGGL((dense2_kernel<MODE>), dim3(tiles_m * ((n + BN - 1) / BN), splits), dim3(NT), lds, s, ah, bh,
                     bl, dsc, inv, m, n, kp, y, (uint32_t)y_bf16, partial, kt_per_split, tiles_m, xe);
  return hipGetLastError();
}

}  // namespace gd

// Dense phase for f16 activations without a lo plane: wmode 0 (plain f16
// panel), 1 (hi/lo panel: bh + bl * 2^-11) or 2 (Q8 int8 values + block
// scales).  kp % 64 == 0.
hipError_t launch_dense2(int wmode, const uint16_t* ah, const uint16_t* bh, const uint16_t* bl, const float* dsc,
                         const float* inv, uint32_t m, uint32_t n, uint32_t kp, void* y, bool y_bf16, float* partial,
                         uint32_t splits, uint32_t kt_per_split, const int32_t* xe, hipStream_t s) {
  if (kp % gd::BK != 0 || xe == nullptr) return hipErrorInvalidValue;
  switch (wmode) {
    case gd::kPlain:
      return gd::launch<gd::kPlain>(ah, bh, bl, dsc, inv, m, n, kp, y, y_bf16, partial, splits, kt_per_split, xe, s);
    case gd::kHiLo:
      return gd::launch<gd::kHiLo>(ah, bh, bl, dsc, inv, m, n, kp, y, y_bf16, partial, splits, kt_per_split, xe, s);
    case gd::kQBlock:
      return gd::launch<gd::kQBlock>(ah, bh, bl, dsc, inv, m, n, kp, y, y_bf16, partial, splits, kt_per_split, xe, s);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace vxt
