// gemm_dense3.hip -- large-tile dense phase of the two-phase prefill GEMM:
// Y = A * W^T with A the row-scaled f16 activations [M][kp] and W the f16
// weight panel [N][kp] (gemm_panel.hip writes both), each stored in 1 KB
// pieces of 16 rows x 32 columns: piece (r / 16, k / 32) at byte
// ((r / 16) * kp / 32 + k / 32) * 1024, row r % 16 at 64 (r % 16) inside,
// rows padded to a multiple of 16.
//
// Reference behaviour: the dense tile product of PackedTensor::gemm_cpu
// (llm_prefill.rs:156-255) over decoded weights; MFMA products are exact in
// the fp32 accumulators.
//
// Shape: a workgroup is NW = 4 or 8 waves in NW / 2 x 2; wave (wm, wn) owns
// WM x WN fragments of v_mfma_f32_32x32x16_f16 (32·WM activation rows x
// 32·WN weight rows), so the workgroup tile is 16·NW·WM x 64·WN.  The wave
// tile is the lever: every 16-deep step reads WM + WN fragments (1 KB each)
// from LDS for WM·WN MFMAs, so 4 x 4 fragments need half the LDS reads per
// MFMA of the 2 x 2 fragments of a 128 x 128 tile.  Eight waves of 2 x 2
// fragments (256 x 128) keep two waves per SIMD, as two 4-wave 128 x 128
// workgroups per CU do, with a quarter less L2 -> LDS traffic per output.
//
// Operands move global -> LDS with buffer_load_dwordx4 ... lds (no VGPR
// round trip, no ds_write).  A K tile is 32 columns (64 bytes per row); the
// hardware writes lane l's 16 bytes at LDS base + 16 l, so one instruction
// fills 16 rows from one contiguous 1 KB piece, eight whole 128-byte lines
// (from row-major planes the same instruction fetched 16 half lines at the
// row stride: a Q8 M = 2048 call took 114 us against 82 us on pieces).  The
// bank swizzle is applied on the global side: lane l fetches logical chunk
// (l % 4) ^ ((l >> 4) & 3) of row l / 4, i.e. chunk c of row r sits at
// position c ^ ((r >> 2) & 3).  Fragment reads (16 lanes = 16 consecutive
// rows at one logical chunk) then hit 16 distinct 16-byte bank groups.
//
// Pipeline: NS LDS stages (3 to 5, as many as fit), each a separate
// __shared__ array, so the compiler can tell the loads into one stage from
// the fragment reads of another and does not wait for the loads before those
// reads.  Tile t runs in two 16-deep steps:
//   step 0: its MFMAs, between them the fragment reads of its step 1;
//   wait for this wave's loads of tile t + 1, then one barrier: every wave
//     has then finished reading tile t's stage, and tile t + 1 has landed;
//   step 1: its MFMAs, between them the fragment reads of tile t + 1's step
//     0 and the loads of tile t + NS into the stage tile t just left.
// So loads run NS - 1.5 tiles ahead of their use, the barrier sits between
// two runs of MFMAs, and fragment registers are double-buffered across the
// tile boundary: the matrix pipe never waits for an LDS read it could have
// issued earlier.  Each slice (one MFMA, at most one read, at most one load)
// is fenced with sched_barrier so the compiler keeps that order.
//
// Modes (the panel's weight representation, as in gemm_dense.hip):
//   * plain: f16 values;
//   * hi/lo: w * s = hi + lo * 2^-11, each product into its own accumulator,
//     combined as acc + accl * 2^-11 in the epilogue;
//   * Q8 block: int8 values as f16 and one f32 scale per (row, 32-column
//     block).  A K tile is exactly one block: its two steps' MFMAs go into a
//     fresh fragment set, and acc += d * fragment (the lane's output column
//     is fixed, so one scale per fragment) -- for tile t in tile t + 1's
//     step 0, fragment q's sixteen FMAs just before the MFMA that restarts
//     fragment q.  Two waves per SIMD (two 4-wave workgroups per CU, or one
//     of 8 waves), so one wave's scale FMAs run in the VALU while the other
//     wave's MFMAs keep the matrix pipe busy.  The tile's scales travel with
//     it: a 4-byte-per-lane LDS load of the scales of the tile's weight rows
//     (waves 0 and 1 fetch them, the others repeat the same loads so that
//     every wave counts the same loads per tile).  The two scale register
//     sets alternate with the stage parity, so the stage count is even.
// With gridDim.y > 1 the workgroup writes fp32 partial sums of its K slice;
// reduce_kernel adds them in slice order and applies the scales.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "common.hpp"

#pragma clang fp contract(off)

namespace vxt {

namespace g3 {

constexpr int BK = 32;
enum : int { kPlain = 0, kHiLo = 1, kQBlock = 2 };

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order.
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// 4-wave workgroups of 2 x 2-fragment waves (128 x 128 tiles) run two per
// CU (the LDS budget halves); every other shape one per CU.
constexpr int occupancy(int wm, int wn, int nw) { return (nw == 4 && wm == 2 && wn == 2) ? 2 : 1; }

// NW waves per workgroup in NW / 2 x 2 (wave rows x wave columns).
template <int WM, int WN, int MODE, int NW = 4>
struct Cfg {
  static constexpr int NT = 64 * NW;
  static constexpr int BM = 32 * WM * (NW / 2), BN = 64 * WN;
  static constexpr bool LO = MODE == kHiLo, QB = MODE == kQBlock;
  static constexpr int A_BYTES = BM * 64, B_BYTES = BN * 64;   // one stage of one operand
  static constexpr int D_BYTES = QB ? BN * 4 : 16;             // Q8 block: the tile's scales
  static constexpr int STAGE = A_BYTES + B_BYTES * (LO ? 2 : 1) + (QB ? D_BYTES : 0);
  static constexpr int OCC = occupancy(WM, WN, NW);
  // Q8 block mode alternates two scale register sets by stage parity (tile t
  // uses set t & 1 from stage t mod NS), which needs an even stage count.
  static constexpr int NS0 = std::min(5, (160 * 1024 / OCC - 2048) / STAGE);
  static constexpr int NS = QB ? NS0 & ~1 : NS0;
  static constexpr int NA = BM / (16 * NW), NB = BN / (16 * NW), NL = LO ? NB : 0;   // 1 KB loads per wave per tile
  static constexpr int ND = QB ? 1 : 0;   // one 4-byte-per-lane scale load per wave per tile
  static constexpr int NLD = NA + NB + NL + ND;
  static constexpr int NR = WM + WN + (LO ? WN : 0);   // fragment reads per step
  static constexpr int NM = WM * WN * (LO ? 2 : 1);    // MFMAs per step
  static_assert(NS >= 3, "stages");
  static constexpr int LPS = (NLD + NM - 1) / NM;   // loads per MFMA slice of step 1
  static_assert(NR <= NM && LPS <= 2, "one read and at most two loads per MFMA slice");
  static_assert(NA * 16 * NW == BM && NB * 16 * NW == BN, "whole 16-row pieces per wave");
  // epilogue: a transpose region per wave, RPA per stage A array, then RPB
  // per stage W array
  static constexpr int REGION = 32 * (32 * WN + 8) * 2, RPA = A_BYTES / REGION, RPB = B_BYTES / REGION;
  static_assert(NW <= NS * (RPA + RPB), "epilogue transpose regions");
  // Q8 block: two waves per SIMD (one wave's scale FMAs beside the other's MFMAs)
  static_assert(!QB || (WM == 2 && WN == 2 && NW * OCC == 8), "Q8 block mode: 2 x 2-fragment waves, two per SIMD");
};

// 16 bytes per lane from buffer `r` at voff + soff into LDS at lds + 16 lane
// (a __device__ function, not a lambda: the LDS address-space cast must not
// appear in code the host pass compiles).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, char* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 4, voff, soff, 0, 0);
}

// Raw buffer resource over [base, base + bytes): bounds-checked by the
// hardware (every offset the kernel forms is in range; rows past the end
// are clamped to the last row).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, size_t bytes) {
  const int n = (int)std::min<size_t>(bytes, 0x7ffffff0u);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// s_waitcnt with vmcnt(V) and lgkmcnt(0) (expcnt not waited).
template <int V>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(V >= 0 && V < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | (7 << 4));
}

template <int WM, int WN, int MODE, int NW>
__global__ __launch_bounds__(64 * NW, occupancy(WM, WN, NW)) void dense3_kernel(const uint16_t* __restrict__ ah, const uint16_t* __restrict__ bh,
                                                      const uint16_t* __restrict__ bl, const float* __restrict__ dsc,
                                                      const float* __restrict__ inv,
                                                      uint32_t M, uint32_t N, uint32_t kp, void* __restrict__ y,
                                                      uint32_t y_bf16, float* __restrict__ partial,
                                                      uint32_t kt_per_split, uint32_t tiles_m,
                                                      const int32_t* __restrict__ xe) {
  using C = Cfg<WM, WN, MODE, NW>;
  constexpr int BM = C::BM, BN = C::BN, NS = C::NS;
  constexpr bool LO = C::LO, QB = C::QB;
#define VXT_STAGE(k)                                                                  \
  __shared__ __attribute__((aligned(1024))) char sA##k[k < NS ? C::A_BYTES : 16];     \
  __shared__ __attribute__((aligned(1024))) char sB##k[k < NS ? C::B_BYTES : 16];     \
  __shared__ __attribute__((aligned(1024))) char sL##k[k < NS && LO ? C::B_BYTES : 16]; \
  __shared__ __attribute__((aligned(256))) char sD##k[k < NS ? C::D_BYTES : 16];
  VXT_STAGE(0)
  VXT_STAGE(1)
  VXT_STAGE(2)
  VXT_STAGE(3)
  VXT_STAGE(4)
#undef VXT_STAGE
  __shared__ int32_t s_xe[BM];
  auto stA = [&](auto k_) -> char* {
    constexpr int k = decltype(k_)::value;
    if constexpr (k == 0) return sA0; else if constexpr (k == 1) return sA1; else if constexpr (k == 2) return sA2;
    else if constexpr (k == 3) return sA3; else return sA4;
  };
  auto stB = [&](auto k_) -> char* {
    constexpr int k = decltype(k_)::value;
    if constexpr (k == 0) return sB0; else if constexpr (k == 1) return sB1; else if constexpr (k == 2) return sB2;
    else if constexpr (k == 3) return sB3; else return sB4;
  };
  auto stL = [&](auto k_) -> char* {
    constexpr int k = decltype(k_)::value;
    if constexpr (k == 0) return sL0; else if constexpr (k == 1) return sL1; else if constexpr (k == 2) return sL2;
    else if constexpr (k == 3) return sL3; else return sL4;
  };
  auto stD = [&](auto k_) -> char* {
    constexpr int k = decltype(k_)::value;
    if constexpr (k == 0) return sD0; else if constexpr (k == 1) return sD1; else if constexpr (k == 2) return sD2;
    else if constexpr (k == 3) return sD3; else return sD4;
  };

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

  const size_t pa = (size_t)((M + 15u) & ~15u) * kp * 2, pb = (size_t)((N + 15u) & ~15u) * kp * 2;   // padded planes
  const __amdgpu_buffer_rsrc_t ra = rsrc(ah, pa);
  const __amdgpu_buffer_rsrc_t rb = rsrc(bh, pb);
  const __amdgpu_buffer_rsrc_t rl = rsrc(LO ? bl : bh, pb);
  const uint32_t nblk = kp / BK;   // Q8 block scales per weight row
  const __amdgpu_buffer_rsrc_t rd = rsrc(QB ? (const void*)dsc : (const void*)bh, QB ? (size_t)N * nblk * 4 : 16);

  // Per-lane byte offsets of the load instructions (tile 0 of the slice):
  // instruction j of this wave fills rows 16 (wave + NW j) .. + 15, one piece.
  uint32_t va[C::NA], vb[C::NB], vd = 0;
  if constexpr (QB)   // wave w loads the scales of weight rows 64 (w % 2) .. + 63 (the other waves repeat waves 0, 1)
    vd = std::min(n0 + 64 * (wave & 1) + lane, N - 1) * nblk * 4 + kt0 * 4;
  {
    const uint32_t r16 = lane >> 2, chunk = (lane & 3) ^ ((lane >> 4) & 3);
    auto off = [&](uint32_t g) { return (g >> 4) * KTT * 1024u + (g & 15u) * 64u + chunk * 16u + kt0 * 1024u; };
#pragma unroll
    for (int j = 0; j < C::NA; ++j) va[j] = off(std::min(m0 + 16 * (wave + NW * j) + r16, M - 1));
#pragma unroll
    for (int j = 0; j < C::NB; ++j) vb[j] = off(std::min(n0 + 16 * (wave + NW * j) + r16, N - 1));
  }
  // Load piece j (A pieces, then W, then W's lo plane) of slice tile t into
  // stage k.
  auto load_piece = [&](auto k_, int j, uint32_t t) {
    const uint32_t so = t * 1024u;   // the next piece of the same 16 rows
    if (QB && j == C::NLD - 1) {
      dma4(rd, stD(k_) + 256 * (wave & 1), vd, t * 4);
    } else if (j < C::NA) {
      dma16(ra, stA(k_) + 1024 * (wave + NW * j), va[j], so);
    } else if (j < C::NA + C::NB) {
      const int q = j - C::NA;
      dma16(rb, stB(k_) + 1024 * (wave + NW * q), vb[q], so);
    } else {
      const int q = j - C::NA - C::NB;
      dma16(rl, stL(k_) + 1024 * (wave + NW * q), vb[q], so);
    }
  };

  if (tid < BM) s_xe[tid] = xe[std::min(m0 + tid, M - 1)];

  float16v acc[WM][WN];
  float16v accl[LO ? WM : 1][LO ? WN : 1];
  // Q8 block mode: the block's fragments, and the scales of this lane's
  // output columns for the tile being multiplied (set t & 1) and the one
  // being scaled
  float16v tmp[QB ? WM : 1][QB ? WN : 1];
  float dreg[QB ? 2 : 1][QB ? WN : 1];
  if constexpr (QB) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) tmp[i][j][r] = 0.0f;   // "tile -1": adds 0 * 0
#pragma unroll
    for (int j = 0; j < WN; ++j) dreg[1][j] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
        if constexpr (LO) accl[i][j][r] = 0.0f;
      }

  // fragment (i, step s): operand rows base + 32 i + l32, logical chunk 2 s + h
  uint32_t offA[2], offB[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const uint32_t pos = ((2 * s + h) ^ ((l32 >> 2) & 3u)) * 16;   // + 32 i keeps the swizzle
    offA[s] = (wm * (32 * WM) + l32) * 64 + pos;
    offB[s] = (wn * (32 * WN) + l32) * 64 + pos;
  }

  half8 af[2][WM], bf[2][WN], lf[2][LO ? WN : 1];
  // fragment read q of step s from stage k into register set `set`, in the
  // order the step's MFMAs need them: A0, B0 .. B(WN-1) (each with its lo
  // plane), A1 .. A(WM-1)
  auto read = [&](auto k_, auto s_, auto set_, auto q_) {
    constexpr int s = decltype(s_)::value, set = decltype(set_)::value, q = decltype(q_)::value;
    constexpr int NBL = WN * (LO ? 2 : 1);
    if constexpr (q == 0) {
      af[set][0] = *reinterpret_cast<const half8*>(stA(k_) + offA[s]);
    } else if constexpr (q <= NBL) {
      constexpr int j = (q - 1) / (LO ? 2 : 1);
      if constexpr (LO && (q - 1) % 2 == 1)
        lf[set][j] = *reinterpret_cast<const half8*>(stL(k_) + j * 2048 + offB[s]);
      else
        bf[set][j] = *reinterpret_cast<const half8*>(stB(k_) + j * 2048 + offB[s]);
    } else {
      constexpr int i = q - NBL;
      af[set][i] = *reinterpret_cast<const half8*>(stA(k_) + i * 2048 + offA[s]);
    }
  };
  auto mma = [&](auto set_, auto q_) {
    constexpr int set = decltype(set_)::value, q = decltype(q_)::value;
    constexpr int p = LO ? q / 2 : q;
    constexpr int i = p / WN, j = p % WN;
    if constexpr (LO && q % 2 == 1)
      accl[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[set][i], lf[set][j], accl[i][j], 0, 0, 0);
    else if constexpr (QB)   // step 0 (set 0) starts the block's fragment
      tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[set][i], bf[set][j], set == 0 ? float16v{} : tmp[i][j],
                                                         0, 0, 0);
    else
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[set][i], bf[set][j], acc[i][j], 0, 0, 0);
  };
  // Q8 block: acc += d * fragment q of the previous tile (scales set par)
  auto scale = [&](auto par_, auto q_) {
    constexpr int par = decltype(par_)::value, q = decltype(q_)::value;
    constexpr int i = q / WN, j = q % WN;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(dreg[par][j], tmp[i][j][r], acc[i][j][r]);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  // prologue: tiles 0 .. NS-1 into stages 0 .. NS-1, wait for tile 0, read
  // its step-0 fragments
  static_for<NS>([&](auto k_) {
    constexpr int k = decltype(k_)::value;
#pragma unroll
    for (int j = 0; j < C::NLD; ++j) load_piece(k_, j, std::min<uint32_t>(k, KT - 1));
  });
  wait_vm_lgkm0<(NS - 1) * C::NLD>();
  __builtin_amdgcn_s_barrier();
  static_for<C::NR>([&](auto q_) { read(I0{}, I0{}, I0{}, q_); });

  // Tile t from stage k (= t mod NS).
  auto tile = [&](auto k_, uint32_t t) {
    constexpr int k = decltype(k_)::value;
    using KN = std::integral_constant<int, (k + 1) % NS>;
    using PAR = std::integral_constant<int, k & 1>;          // this tile's fragment set (Q8 block)
    using PPAR = std::integral_constant<int, (k & 1) ^ 1>;   // the previous tile's
    // step 0: MFMAs on set 0, reads of step 1 into set 1
    static_for<C::NM>([&](auto q_) {
      constexpr int q = decltype(q_)::value;
      if constexpr (QB) scale(PPAR{}, q_);   // the previous block's fragment q, before the MFMA restarts it
      mma(I0{}, q_);
      if constexpr (q < C::NR) read(k_, I1{}, I1{}, q_);
      if constexpr (QB && q < WN)   // this tile's scales, before its stage is released
        dreg[PAR::value][q] = *reinterpret_cast<const float*>(stD(k_) + 4 * (wn * (32 * WN) + q * 32 + l32));
      __builtin_amdgcn_sched_barrier(0);
    });
    // tile t + 1 landed (this wave's loads; the barrier covers the others)
    // and every wave is done reading stage k
    wait_vm_lgkm0<(NS - 2) * C::NLD>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // step 1: MFMAs on set 1, reads of tile t + 1's step 0 into set 0, loads
    // of tile t + NS into stage k
    const uint32_t tl = std::min(t + NS, KT - 1);
    static_for<C::NM>([&](auto q_) {
      constexpr int q = decltype(q_)::value;
      mma(I1{}, q_);
      if constexpr (q < C::NR) read(KN{}, I0{}, I0{}, q_);
      static_for<C::LPS>([&](auto u_) {
        constexpr int j = q * C::LPS + decltype(u_)::value;
        if constexpr (j < C::NLD) load_piece(k_, j, tl);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  uint32_t t = 0;
  for (; t + NS <= KT; t += NS) {
    static_for<NS>([&](auto k_) { tile(k_, t + decltype(k_)::value); });
  }
  {
    const uint32_t rem = KT - t;
    static_for<NS - 1>([&](auto k_) {
      if (decltype(k_)::value < rem) tile(k_, t + decltype(k_)::value);
    });
    if constexpr (QB) {   // the last tile's scaling: its scales are set (KT - 1) & 1
      if (((KT - 1) & 1) == 0)
        static_for<C::NM>([&](auto q_) { scale(I0{}, q_); });
      else
        static_for<C::NM>([&](auto q_) { scale(I1{}, q_); });
    }
  }
  __syncthreads();   // drains the clamped tail loads too: the epilogue reuses stages

  // Epilogue.  Lane owns column n0 + wn*32*WN + j*32 + l32 of fragment
  // (i, j), rows m0 + wm*32*WM + i*32 + 4h + 8(r/4) + r%4.
  const bool to_partial = gridDim.y > 1;
  auto value = [&](int i, int j, int r) {
    float v = acc[i][j][r];
    if constexpr (LO) v = hilo_combine(v, accl[i][j][r]);
    return v;
  };
  auto row_of = [&](int i, int r) { return (uint32_t)(wm * 32 * WM + i * 32 + h * 4 + 8 * (r >> 2) + (r & 3)); };
  const bool rows_fast = y_bf16 && !to_partial && N % 8 == 0 && n0 + BN <= N &&
                         reinterpret_cast<uintptr_t>(y) % 16 == 0;
  if (rows_fast) {
    // Each wave transposes its 32·WM x 32·WN block through its own LDS
    // region (the stages' A arrays first, then their W arrays), 32 rows at a
    // time, and writes whole-row 16-byte pieces.  Rows
    // r and r + 1 of a lane are converted as one pair (one v_cvt_pk_bf16_f32)
    // and stored as the pair's two halves.
    constexpr uint32_t LDO = 32 * WN + 8;   // bf16 elements per LDS row
    auto pick = [](uint32_t k, char* a0, char* a1, char* a2, char* a3, char* a4) {
      return k == 0 ? a0 : k == 1 ? a1 : k == 2 ? a2 : k == 3 ? a3 : a4;
    };
    char* rbase;
    if (C::RPA > 0 && wave < (uint32_t)(NS * C::RPA)) {
      rbase = pick(wave / C::RPA, sA0, sA1, sA2, sA3, sA4) + (wave % C::RPA) * C::REGION;
    } else {
      const uint32_t w = wave - NS * C::RPA;
      rbase = pick(w / C::RPB, sB0, sB1, sB2, sB3, sB4) + (w % C::RPB) * C::REGION;
    }
    uint16_t* reg = reinterpret_cast<uint16_t*>(rbase);
    float sc[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) sc[j] = inv[n0 + wn * 32 * WN + j * 32 + l32];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      // this lane's 16 row exponents (4 consecutive rows per 16-byte read)
      int nxe[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int4 e4 = *reinterpret_cast<const int4*>(s_xe + wm * 32 * WM + i * 32 + h * 4 + 8 * q);
        nxe[4 * q + 0] = -e4.x;
        nxe[4 * q + 1] = -e4.y;
        nxe[4 * q + 2] = -e4.z;
        nxe[4 * q + 3] = -e4.w;
      }
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const uint32_t rr = h * 4 + 8 * (r >> 2) + (r & 3);
          const uint32_t p = bf16x2_pack(ldexpf(value(i, j, r) * sc[j], nxe[r]),
                                         ldexpf(value(i, j, r + 1) * sc[j], nxe[r + 1]));
          reg[rr * LDO + j * 32 + l32] = (uint16_t)p;
          reg[(rr + 1) * LDO + j * 32 + l32] = (uint16_t)(p >> 16);
        }
      // 32 rows x 32·WN columns: 4·WN lanes per row, 16 bytes each (LDS
      // operations of one wave complete in order: no barrier needed)
      constexpr uint32_t LPR = 4 * WN, ROWS_PER = 64 / LPR;
#pragma unroll
      for (uint32_t q = 0; q < (32 + ROWS_PER - 1) / ROWS_PER; ++q) {
        const uint32_t rr = q * ROWS_PER + lane / LPR, c = lane % LPR;
        const uint32_t m = m0 + wm * 32 * WM + i * 32 + rr;
        if (rr < 32 && lane < ROWS_PER * LPR && m < M) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(reg + rr * LDO + c * 8);
          *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(y) + (size_t)m * N + n0 + wn * 32 * WN + c * 8) = v;
        }
      }
    }
  } else if (to_partial) {
    const bool full = m0 + BM <= M && n0 + BN <= N;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const uint32_t n = n0 + wn * 32 * WN + j * 32 + l32;
      float* const pp = partial + ((size_t)blockIdx.y * M + m0) * N + n;
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (full || (m0 + row_of(i, r) < M && n < N)) pp[(size_t)row_of(i, r) * N] = value(i, j, r);
    }
  } else {
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const uint32_t n = n0 + wn * 32 * WN + j * 32 + l32;
      const float sc = inv[std::min(n, N - 1)];
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t m = m0 + row_of(i, r);
          if (m >= M || n >= N) continue;
          const float o = ldexpf(value(i, j, r) * sc, -s_xe[row_of(i, r)]);
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * N + n] = f32_to_bf16(o);
          else
            static_cast<float*>(y)[(size_t)m * N + n] = o;
        }
    }
  }
}

template <int WM, int WN, int MODE, int NW = 4>
hipError_t launch(const uint16_t* ah, const uint16_t* bh, const uint16_t* bl, const float* dsc, const float* inv, uint32_t m,
                  uint32_t n, uint32_t kp, void* y, bool y_bf16, float* partial, uint32_t splits,
                  uint32_t kt_per_split, const int32_t* xe, hipStream_t s) {
  using C = Cfg<WM, WN, MODE, NW>;
  const uint32_t tiles_m = (m + C::BM - 1) / C::BM;
  hipLaunchKernelGGL((dense3_kernel<WM, WN, MODE, NW>), dim3(tiles_m * ((n + C::BN - 1) / C::BN), splits), dim3(C::NT), 0,
                     s, ah, bh, bl, dsc, inv, m, n, kp, y, (uint32_t)y_bf16, partial, kt_per_split, tiles_m, xe);
  return hipGetLastError();
}

}  // namespace g3

// Large-tile dense phase.  cfg selects the wave tile (WM x WN fragments) and
// the waves per workgroup: 0 = 4 x 4, 4 waves (workgroup tile 256 x 256),
// 1 = 4 x 3, 4 waves (256 x 192), 2 = 4 x 2, 4 waves (256 x 128), 3 = 2 x 2,
// 4 waves (128 x 128), 4 = 2 x 2, 8 waves (256 x 128).  wmode 0 = plain f16
// panel (cfg 0-3), 1 = hi/lo panel (bh + bl * 2^-11; cfg 3 and 4), 2 = Q8
// block (int8 values as f16 in bh, f32 scales dsc [n][kp / 32]; cfg 3 and 4).  ah, bh and bl are planes of 1 KB
// pieces (16 rows x 32 columns, rows padded to 16).  kt_per_split counts
// 32-column K tiles; kp % 32 == 0.
hipError_t launch_dense3(int cfg, int wmode, const uint16_t* ah, const uint16_t* bh, const uint16_t* bl,
                         const float* dsc, const float* inv, uint32_t m, uint32_t n, uint32_t kp, void* y, bool y_bf16,
                         float* partial, uint32_t splits, uint32_t kt_per_split, const int32_t* xe, hipStream_t s) {
  if (kp % g3::BK != 0 || xe == nullptr || m == 0 || n == 0 || kt_per_split == 0) return hipErrorInvalidValue;
#define VXT_D3(WM, WN, MODE, NW) \
  return g3::launch<WM, WN, MODE, NW>(ah, bh, bl, dsc, inv, m, n, kp, y, y_bf16, partial, splits, kt_per_split, xe, s)
  switch (wmode * 16 + cfg) {
    case g3::kPlain * 16 + 0: VXT_D3(4, 4, g3::kPlain, 4);
    case g3::kPlain * 16 + 1: VXT_D3(4, 3, g3::kPlain, 4);
    case g3::kPlain * 16 + 2: VXT_D3(4, 2, g3::kPlain, 4);
    case g3::kPlain * 16 + 3: VXT_D3(2, 2, g3::kPlain, 4);
    case g3::kHiLo * 16 + 3: VXT_D3(2, 2, g3::kHiLo, 4);
    case g3::kHiLo * 16 + 4: VXT_D3(2, 2, g3::kHiLo, 8);
    case g3::kQBlock * 16 + 3: VXT_D3(2, 2, g3::kQBlock, 4);
    case g3::kQBlock * 16 + 4: VXT_D3(2, 2, g3::kQBlock, 8);
    default: return hipErrorInvalidValue;
  }
#undef VXT_D3
}

}  // namespace vxt
