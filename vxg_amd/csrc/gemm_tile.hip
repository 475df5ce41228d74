// gemm_tile.hip -- prefill GEMM (batch_m > 64) for cb4-g64 weights and bf16
// activations, the weights decoded in registers inside the MFMA loop.
//
// Reference behaviour: PackedTensor::gemm_cpu (llm_prefill.rs:156-255)
// decodes weight tiles to f32 and multiplies them densely; every g64 weight
// is an f16 table entry, so an f16 MFMA operand holds it exactly, and the
// products are exact in the fp32 accumulator.
//
// Two launches (plus the split-K reduction when K is split):
//   1. xprep_kernel: per activation row, the power-of-two exponent xe[m]
//      that puts the row's largest finite magnitude in [2^14, 2^15) (0 for
//      rows with no non-zero finite entry; Inf and NaN entries stay Inf and
//      NaN), then X[m] * 2^xe[m] as f16 (exact for
//      bf16 X within 2^28 of the row's largest), padded with zeros to kp and
//      stored with each aligned group of 8 columns in the order
//      0 2 4 6 1 3 5 7 -- the order in which the weight decode below
//      produces f16 pairs.
//   2. tile_kernel: a workgroup computes 128 activation rows x 128 weight
//      rows over a K range, with KW K-ways of 4 waves (K-way g takes the
//      range's K tiles g, g + KW, ...; the ways are summed through LDS in
//      ascending order at the end).  Wave w of a way owns weight rows
//      32w..32w+31 and all 128 activation rows: four 32x32x16 MFMA fragments
//      per 16-deep step, the activation fragments read from LDS and the
//      weight fragment decoded by the lane itself.
//        * activations: register-staged, two tiles ahead, into two LDS
//          stages of 128 rows x 128 B; 16-byte chunk c of row r is stored at
//          chunk c ^ ((r >> 1) & 7) so the fragment reads of 16 lanes (rows
//          r..r+15 at one chunk) and the row writes touch distinct banks;
//        * weights: lane (w, l) loads its row's 32 nibbles of the tile (16 B,
//          columns 32h.. of the tile, h = l / 32) and half of the group's
//          16-entry table (16 B; v_permlane32_swap with the lane of the other
//          half completes it), two tiles ahead.  Lookups are v_perm_b32
//          byte selects from the table held in registers: the low and high
//          bytes of entries 0-7 and 8-15 form four 8-byte sources; a perm
//          picks four bytes by nibble & 7, a second perm takes the 8-15 half
//          where bit 3 is set, and two more interleave low and high bytes
//          into f16 pairs (columns 0,2 / 4,6 / 1,3 / 5,7 of each group of 8);
//        * the loop body has no conditional memory operation, so the
//          compiler keeps the next tile's loads in flight across the LDS
//          stores (its waits are counted per static load order).
//      Columns past K are zero in the activations, so the padding weights
//      add nothing (decode_row stops at `cols`) unless an entry they index
//      is Inf/NaN; tensors where that can happen take the panel path (the
//      upload records it), so the loop body has no branch.  With gridDim.y > 1
//      the workgroup writes fp32 partial sums of its K slice and
//      reduce_kernel adds them in slice order, then applies 2^-xe[m].
#include <algorithm>
#include <type_traits>

#include "common.hpp"

#pragma clang fp contract(off)

namespace vxt {

hipError_t launch_gemm_reduce(const float* partial, uint32_t splits, const float* inv, const int32_t* xe, uint32_t m,
                              uint32_t n, void* y, bool y_bf16, hipStream_t s);

namespace gt {

constexpr int BM = 128;   // activation rows per workgroup
constexpr int BN = 128;   // weight rows per workgroup (4 waves x 32)
constexpr int BK = 64;    // K tile = one g64 group
constexpr int NT = 256;   // threads of one K-way
constexpr uint32_t kStageBytes = BM * BK * 2;   // one activation stage

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

// ---- activation preparation --------------------------------------------------

// |v| of a finite v, 0 for Inf / NaN: a row's exponent comes from its largest
// finite magnitude, and its Inf / NaN entries stay Inf / NaN when scaled and
// converted, so they reach the products as gemm_cpu sees them.
__device__ __forceinline__ float finite_abs(float v) {
  const float a = fabsf(v);
  return a <= 3.4028234663852886e38f ? a : 0.0f;
}

__device__ __forceinline__ int row_exponent(float b) {
  return (b > 0.0f && b <= 3.4028234663852886e38f) ? 14 - ilogbf(b) : 0;
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

// One wave per activation row.  x_vec: rows are 16-byte aligned and K % 8 == 0.
// NP > 0: the row (at most NP 16-byte pieces per lane, K <= 512 NP) is read
// once into registers, all loads in flight together, and converted from
// there; NP == 0: two passes over the row (any K).
template <int NPT>
__global__ __launch_bounds__(256) void xprep_kernel(const uint16_t* __restrict__ x, uint32_t M, uint32_t K,
                                                    uint32_t kp, uint32_t x_vec, uint16_t* __restrict__ xh,
                                                    int32_t* __restrict__ xe) {
  // One workgroup (4 waves) per activation row: thread t takes the row's
  // 16-byte pieces t, t + 256, ...; the row maximum is combined through LDS
  // (the maximum does not depend on the order, so neither does xe).
  __shared__ float s_mx[4];
  const uint32_t m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* row = x + (size_t)m * K;
  const uint32_t np = kp / 8;   // 16-byte pieces of the padded row
  auto store = [&](uint32_t pc, const float (&v)[8], int e) {
    float w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = ldexpf(v[j], e);   // exact (a power of two)
    // columns 0 2 4 6 1 3 5 7 of the group
    *reinterpret_cast<uint4*>(xh + (size_t)m * kp + pc * 8) =
        make_uint4(pack2(w[0], w[2]), pack2(w[4], w[6]), pack2(w[1], w[3]), pack2(w[5], w[7]));
  };
  auto piece = [&](uint32_t pc, float (&v)[8]) {   // scalar path: columns past K are zero
    const uint32_t k = pc * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = k + j < K ? bf16_to_f32(row[k + j]) : 0.0f;
  };
  auto row_max = [&](float mx) {
    mx = lane_reduce<64, true>(mx);
    if (lane == 0) s_mx[wave] = mx;
    __syncthreads();
    return fmaxf(fmaxf(s_mx[0], s_mx[1]), fmaxf(s_mx[2], s_mx[3]));
  };
  if constexpr (NPT > 0) {
    float v[NPT][8];
    if (x_vec) {
      const uint32_t nv = K / 8;   // pieces inside the row
      uint4 u[NPT];
#pragma unroll
      for (int i = 0; i < NPT; ++i) u[i] = reinterpret_cast<const uint4*>(row)[std::min(i * 256 + tid, nv - 1)];
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const bool in = i * 256 + tid < nv;
        const uint32_t w[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[i][2 * j] = in ? __uint_as_float(w[j] << 16) : 0.0f;
          v[i][2 * j + 1] = in ? __uint_as_float(w[j] & 0xffff0000u) : 0.0f;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < NPT; ++i) piece(i * 256 + tid, v[i]);
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < NPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, finite_abs(v[i][j]));
    const int e = row_exponent(row_max(mx));
    if (tid == 0) xe[m] = e;
#pragma unroll
    for (int i = 0; i < NPT; ++i)
      if (i * 256 + tid < np) store(i * 256 + tid, v[i], e);
  } else {
    float mx = 0.0f;
    for (uint32_t pc = tid; pc < np; pc += 256) {
      float v[8];
      piece(pc, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, finite_abs(v[j]));
    }
    const int e = row_exponent(row_max(mx));
    if (tid == 0) xe[m] = e;
    for (uint32_t pc = tid; pc < np; pc += 256) {
      float v[8];
      piece(pc, v);
      store(pc, v, e);
    }
  }
}

// ---- weight decode -------------------------------------------------------------

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Byte planes of one 16-entry f16 table: L0..L3 the low bytes of entries
// 0-3, 4-7, 8-11, 12-15, H0..H3 the high bytes.
struct Planes {
  uint32_t L0, L1, L2, L3, H0, H1, H2, H3;
};

__device__ __forceinline__ Planes make_planes(const u32x4& t0, const u32x4& t1) {
  Planes p;
  p.L0 = perm(t0.y, t0.x, 0x06040200u);
  p.H0 = perm(t0.y, t0.x, 0x07050301u);
  p.L1 = perm(t0.w, t0.z, 0x06040200u);
  p.H1 = perm(t0.w, t0.z, 0x07050301u);
  p.L2 = perm(t1.y, t1.x, 0x06040200u);
  p.H2 = perm(t1.y, t1.x, 0x07050301u);
  p.L3 = perm(t1.w, t1.z, 0x06040200u);
  p.H3 = perm(t1.w, t1.z, 0x07050301u);
  return p;
}

// Four nibbles q (one per byte, high nibble of each byte zero) -> table
// entries as f16 pairs (byte 0, byte 1) and (byte 2, byte 3).
__device__ __forceinline__ void lookup4(const Planes& p, uint32_t q, uint32_t& p01, uint32_t& p23) {
  const uint32_t s = q & 0x07070707u;
  const uint32_t sel = ((q >> 1) & 0x04040404u) | 0x03020100u;   // byte i from the 8-15 half when bit 3 is set
  const uint32_t la = perm(p.L1, p.L0, s), lb = perm(p.L3, p.L2, s);
  const uint32_t ha = perm(p.H1, p.H0, s), hb = perm(p.H3, p.H2, s);
  const uint32_t l = perm(lb, la, sel), h = perm(hb, ha, sel);
  p01 = perm(h, l, 0x05010400u);
  p23 = perm(h, l, 0x07030602u);
}

// 8 nibbles (columns 0..7 of a group of 8, low nibble first) -> f16 pairs
// (0,2) (4,6) (1,3) (5,7).
__device__ __forceinline__ u32x4 decode8(const Planes& p, uint32_t w) {
  uint32_t a, b, c, d;
  lookup4(p, w & 0x0F0F0F0Fu, a, b);
  lookup4(p, (w >> 4) & 0x0F0F0F0Fu, c, d);
  return u32x4{a, b, c, d};
}

// Lanes l and l + 32 of a wave take the same weight row (the two 32-column
// halves of the tile), so each loads one 16-byte half of the row's table and
// v_permlane32_swap gives both lanes the whole of it.
struct Raw {
  u32x4 nib;   // 32 nibbles: columns 32h .. 32h + 31 of the tile
  u32x4 th;    // table entries 8h .. 8h + 7 of the group
};

__device__ __forceinline__ void bload(const DevTensor& t, uint32_t n, uint32_t kt, uint32_t h, Raw& r) {
  const uint32_t kp = t.kp;
  r.nib = *reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(t.p0) + (size_t)n * (kp / 2) + kt * 32 + 16 * h);
  r.th = reinterpret_cast<const u32x4*>(t.p1 + ((size_t)n * (kp / 64) + kt) * 16)[h];
}

__device__ __forceinline__ Planes planes_of(const Raw& r) {
  u32x4 t0, t1;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const auto v = __builtin_amdgcn_permlane32_swap(r.th[j], r.th[j], false, false);
    t0[j] = v[0];   // lanes 0-31 keep entries 0-7, lanes 32-63 receive them
    t1[j] = v[1];   // lanes 32-63 keep entries 8-15, lanes 0-31 receive them
  }
  return make_planes(t0, t1);
}

// ---- activation tiles ------------------------------------------------------------

__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t c) { return c ^ ((row >> 1) & 7u); }

// 128 rows x 64 columns of xh: 4 pieces of 16 B per thread of the K-way.
__device__ __forceinline__ void aload(const uint16_t* __restrict__ xh, uint32_t m0, uint32_t M, uint32_t kp,
                                      uint32_t kt, uint32_t tid, u32x4 (&r)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t i = tid + NT * j;
    const uint32_t row = std::min(m0 + i / 8, M - 1);   // rows past M repeat row M-1 (never stored)
    r[j] = *reinterpret_cast<const u32x4*>(xh + (size_t)row * kp + kt * BK + (i % 8) * 8);
  }
}

__device__ __forceinline__ void astore(char* stage, uint32_t tid, const u32x4 (&r)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t i = tid + NT * j;
    const uint32_t row = i / 8, c = i % 8;
    *reinterpret_cast<u32x4*>(stage + row * 128 + swz(row, c) * 16) = r[j];
  }
}

// LDS: the activation stages (reused for the K-way sums at the end), the
// tile's 128 row exponents, then the bf16 output tile [128][136].
constexpr uint32_t LDO = BN + 8;

template <int KW>
constexpr size_t xe_offset() {
  const size_t stages = (size_t)KW * 2 * kStageBytes;
  const size_t red = (size_t)(KW - 1) * 4 * 4 * 16 * 64 * 4;   // K-way sums at the end
  return stages > red ? stages : red;
}

template <int KW>
constexpr size_t out_offset() { return xe_offset<KW>() + BM * 4; }

template <int KW>
constexpr size_t lds_bytes() { return out_offset<KW>() + (size_t)BM * LDO * 2; }

// gridDim.x = tiles_m * tiles_n, gridDim.y = K slices of kt_per_split tiles.
template <int KW>
__global__ __launch_bounds__(NT * KW, KW == 1 ? 2 : 1) void tile_kernel(DevTensor t, const uint16_t* __restrict__ xh,
                                                                         uint32_t M, const int32_t* __restrict__ xe,
                                                                         void* __restrict__ y, uint32_t y_bf16,
                                                                         float* __restrict__ partial,
                                                                         uint32_t kt_per_split, uint32_t tiles_m) {
  extern __shared__ __attribute__((aligned(1024))) char smem_all[];
  const uint32_t lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const uint32_t wave = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) & 3);
  const uint32_t kg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 8);   // K-way
  const uint32_t tid = threadIdx.x & (NT - 1);
  char* const smem = smem_all + kg * (2 * kStageBytes);
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
  const uint32_t N = t.rows, kp = t.kp;
  const uint32_t KTT = kp / BK;
  const uint32_t kt0 = blockIdx.y * kt_per_split;
  const uint32_t kt1 = std::min(KTT, kt0 + kt_per_split);
  const uint32_t ntiles = kt1 - kt0;                 // >= 1 (the plan guarantees it)
  const uint32_t KT = (ntiles + KW - 1) / KW;        // iterations of every K-way
  // K-way kg's tile at iteration i (clamped to the slice; only the last
  // iteration of a way can lie past it, and is then not multiplied)
  auto ktile = [&](uint32_t i) { return std::min(kt0 + kg + KW * i, kt1 - 1); };
  const uint32_t n = std::min(n0 + wave * 32 + l32, N - 1);   // rows past N repeat row N-1 (never stored)
  // The tile's row exponents are requested now, so the epilogue does not
  // wait for another round trip to memory.
  const int32_t xe_pre = xe[std::min(m0 + (tid & (BM - 1)), M - 1)];
#define STAGE(st) (smem + (st) * kStageBytes)

  float16v acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  // fragment offsets: fragment i, step t reads row 32i + l32, chunk 4h + t
  uint32_t offA[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) offA[tt] = l32 * 128 + swz(l32, 4 * h + tt) * 16;   // + 4096 i (same swizzle)

  // Weight tile i is decoded during iteration i - 1 (into bf[i & 1]) from
  // the raw slot rb[i & 1], which was loaded two iterations before that.
  u32x4 ra[2][4];
  Raw rb[2];
  u32x4 bf[2][4];
  aload(xh, m0, M, kp, ktile(0), tid, ra[0]);
  aload(xh, m0, M, kp, ktile(1), tid, ra[1]);
  bload(t, n, ktile(0), h, rb[0]);
  bload(t, n, ktile(1), h, rb[1]);
  astore(STAGE(0), tid, ra[0]);
  aload(xh, m0, M, kp, ktile(2), tid, ra[0]);
  {
    const Planes p0 = planes_of(rb[0]);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) bf[0][tt] = decode8(p0, rb[0].nib[tt]);
  }
  bload(t, n, ktile(2), h, rb[0]);
  __syncthreads();

  // Iteration i (P = i & 1): multiply stage P by bf[P] (tile i).  Spread
  // between the 16 MFMAs: the next step's activation fragments; storing
  // activation tile i+1 (slot P^1) into stage P^1 and loading tile i+3 into
  // the slot; decoding weight tile i+1 (rb[P^1]) into bf[P^1].  Then the raw
  // slot is reloaded with tile i+3.  Every memory operation is unconditional
  // (clamped tiles), so the compiler counts its waits in one static order;
  // sched_barrier keeps the interleave.
  auto body = [&](uint32_t i, auto par) {
    constexpr int P = decltype(par)::value;
    const char* stage = STAGE(P);
    char* const next_stage = STAGE(P ^ 1);
    const uint32_t kn = ktile(i + 3);
    const Planes pl = planes_of(rb[P ^ 1]);
    half8 af[2][4];
#pragma unroll
    for (int f = 0; f < 4; ++f) af[0][f] = *reinterpret_cast<const half8*>(stage + f * 4096 + offA[0]);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int cur = tt & 1, nxt = cur ^ 1;
      const half8 b = __builtin_bit_cast(half8, bf[P][tt]);
      const uint32_t w = rb[P ^ 1].nib[tt];
      uint32_t d0, d1, d2, d3;
      __builtin_amdgcn_sched_barrier(0);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][0], b, acc[0], 0, 0, 0);
      if (tt < 3) af[nxt][0] = *reinterpret_cast<const half8*>(stage + 0 * 4096 + offA[tt + 1]);
      {
        const uint32_t pi = tid + NT * tt, row = pi / 8, c = pi % 8;
        *reinterpret_cast<u32x4*>(next_stage + row * 128 + swz(row, c) * 16) = ra[P ^ 1][tt];
        const uint32_t grow = std::min(m0 + pi / 8, M - 1);
        ra[P ^ 1][tt] = *reinterpret_cast<const u32x4*>(xh + (size_t)grow * kp + kn * BK + c * 8);
      }
      __builtin_amdgcn_sched_barrier(0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][1], b, acc[1], 0, 0, 0);
      if (tt < 3) af[nxt][1] = *reinterpret_cast<const half8*>(stage + 1 * 4096 + offA[tt + 1]);
      lookup4(pl, w & 0x0F0F0F0Fu, d0, d1);
      __builtin_amdgcn_sched_barrier(0);
      acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][2], b, acc[2], 0, 0, 0);
      if (tt < 3) af[nxt][2] = *reinterpret_cast<const half8*>(stage + 2 * 4096 + offA[tt + 1]);
      lookup4(pl, (w >> 4) & 0x0F0F0F0Fu, d2, d3);
      __builtin_amdgcn_sched_barrier(0);
      acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][3], b, acc[3], 0, 0, 0);
      if (tt < 3) af[nxt][3] = *reinterpret_cast<const half8*>(stage + 3 * 4096 + offA[tt + 1]);
      bf[P ^ 1][tt] = u32x4{d0, d1, d2, d3};
      __builtin_amdgcn_sched_barrier(0);
    }
    bload(t, n, kn, h, rb[P ^ 1]);
    __syncthreads();
  };
  auto last = [&](const char* stage, const u32x4 (&b)[4]) {
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      half8 af[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) af[f] = *reinterpret_cast<const half8*>(stage + f * 4096 + offA[tt]);
#pragma unroll
      for (int f = 0; f < 4; ++f)
        acc[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[f], __builtin_bit_cast(half8, b[tt]), acc[f], 0, 0, 0);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  uint32_t i = 0;
  for (; i + 2 < KT; i += 2) {
    body(i, I0{});
    body(i + 1, I1{});
  }
  if (i + 1 < KT) {
    body(i, I0{});
    ++i;
  }
  // last iteration: stage i&1, weights bf[i&1]; a K-way whose tiles ran out
  // (kt0 + kg + KW i >= kt1) skips it
  if (kt0 + kg + KW * i < kt1) {
    if (i & 1)
      last(STAGE(1), bf[1]);
    else
      last(STAGE(0), bf[0]);
  }
#undef STAGE

  // The tile's 128 row exponents go through LDS (loaded in the prologue by
  // the threads of K-way 0): read per output from global memory they cost
  // more than the last K tiles.  bf16 outputs of a whole tile are transposed through LDS
  // and written as 16-byte pieces of full rows (2-byte lane stores write
  // half lines).  Every wave runs every barrier; K-ways > 0 only hand over
  // their sums.
  const bool to_partial = gridDim.y > 1;
  const uint32_t N_ = N;
  const bool rows_fast = y_bf16 && !to_partial && N_ % 8 == 0 && n0 + BN <= N_ &&
                         reinterpret_cast<uintptr_t>(y) % 16 == 0;
  int32_t* s_xe = reinterpret_cast<int32_t*>(smem_all + xe_offset<KW>());
  uint16_t* s_out = reinterpret_cast<uint16_t*>(smem_all + out_offset<KW>());
  __syncthreads();   // every way is done with its stages
  if (kg == 0 && tid < BM && !to_partial) s_xe[tid] = xe_pre;
  if constexpr (KW > 1) {
    float* red = reinterpret_cast<float*>(smem_all);
    if (kg > 0) {
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[((((kg - 1) * 4 + wave) * 4 + f) * 16 + r) * 64 + lane] = acc[f][r];
    }
  }
  __syncthreads();
  if (kg == 0) {
    if constexpr (KW > 1) {
      const float* red = reinterpret_cast<const float*>(smem_all);
#pragma unroll
      for (uint32_t g = 1; g < (uint32_t)KW; ++g)
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[f][r] += red[((((g - 1) * 4 + wave) * 4 + f) * 16 + r) * 64 + lane];
    }
    // Lane owns output column n0 + 32 wave + l32 and rows
    // m0 + 32 f + 4 h + 8 (r / 4) + r % 4 of fragment f.  Each output mode
    // has a loop of its own: a mode test per output became a pair of
    // branches per output, whose cold code cost microseconds per workgroup.
    const uint32_t nl = wave * 32 + l32, ncol = n0 + nl;
    auto row_of = [&](int f, int r) { return (uint32_t)(f * 32 + h * 4 + 8 * (r >> 2) + (r & 3)); };
    // fragment f's 16 row exponents, 4 consecutive rows per 16-byte read
    auto load_xs = [&](int f, int (&xs)[16]) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int4 e4 = *reinterpret_cast<const int4*>(s_xe + f * 32 + h * 4 + 8 * q);
        xs[4 * q + 0] = e4.x;
        xs[4 * q + 1] = e4.y;
        xs[4 * q + 2] = e4.z;
        xs[4 * q + 3] = e4.w;
      }
    };
    const bool full = m0 + BM <= M && n0 + BN <= N_;
    if (rows_fast) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        int xs[16];
        load_xs(f, xs);
#pragma unroll
        for (int r = 0; r < 16; ++r) s_out[row_of(f, r) * LDO + nl] = f32_to_bf16(ldexpf(acc[f][r], -xs[r]));
      }
    } else if (to_partial) {
      float* const pp = partial + ((size_t)blockIdx.y * M + m0) * N_ + ncol;
      if (full) {
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
          for (int r = 0; r < 16; ++r) pp[(size_t)row_of(f, r) * N_] = acc[f][r];
      } else {
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (m0 + row_of(f, r) < M && ncol < N_) pp[(size_t)row_of(f, r) * N_] = acc[f][r];
      }
    } else {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        int xs[16];
        load_xs(f, xs);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t m = m0 + row_of(f, r);
          if (m >= M || ncol >= N_) continue;
          const float o = ldexpf(acc[f][r], -xs[r]);
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * N_ + ncol] = f32_to_bf16(o);
          else
            static_cast<float*>(y)[(size_t)m * N_ + ncol] = o;
        }
      }
    }
  }
  if (rows_fast) {   // uniform
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t idx = tid + NT * k, row = idx / 16, c = idx % 16;
        if (m0 + row >= M) continue;
        const u32x4 v = *reinterpret_cast<const u32x4*>(s_out + row * LDO + c * 8);
        *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(y) + (size_t)(m0 + row) * N_ + n0 + c * 8) = v;
      }
    }
  }
}

// ---- cb4 (reference layout) -------------------------------------------------------
//
// tile_cb4_kernel: the tile kernel's structure (one K-way of 4 waves, 128 x
// 128 tiles, activations from xprep_kernel staged two tiles ahead) for the
// reference cb4 layout.  decode_row (codebook.rs:285-337) forms each weight
// as w = scale * centroid in f32 and then adds the row's CSR residuals.  Here
// every weight is multiplied by the row's power-of-two exponent (fixed at
// upload, so |w| * 2^e < 2^15) and carried on f16 MFMA operands exactly:
//   * the product part p = scale * 2^e * centroid (f32, rounded as decode_row
//     rounds it) is split into two f16 planes, p = hi + lo * 2^-11, each on
//     its own MFMA into its own accumulator;
//   * a residual r (an f16 value; r * 2^e is still one) goes on a third B
//     operand that is zero except at the residual's columns, multiplied into
//     the hi accumulator.  A window of 8 columns (one 16-deep MFMA step) where
//     no lane of the wave has a residual skips those 4 MFMAs.
// The sum is p + r without decode_row's final f32 rounding of w, a difference
// of at most half an f32 ulp of the few weights that have a residual.
//
// Tables: the product part of a weight depends only on its nibble and its
// 128-column group's scale, so each lane keeps its row's 16 products, as
// (hi | lo << 16) words, in LDS (entry e of lane l of a wave at word
// 64 e + l, so the 64 lanes of a lookup hit 64 distinct banks whatever the
// nibbles) and rebuilds them when its lane's columns enter a new group.  A
// weight then costs one LDS read and half of two byte permutes.
//
// K order: the workgroup's K slice [S, S + 64 KT) is cut in two halves of
// H = 32 KT columns; in iteration i, lanes 0-31 of a wave take columns
// S + 32 i .. +31 of their row and lanes 32-63 columns S + H + 32 i .. +31
// (the activation stage holds the same two pieces of every activation row,
// and the MFMA sums over k in any order).  Every lane thus walks one
// contiguous column range of its row, so its residuals come in column order
// without gaps: the residual lists of the block's 128 rows are staged in LDS
// at the start, each lane finds its first entry by bisection and keeps its
// next entry in registers.
// cb4 packs its nibbles as g64 does (column c: nibble c % 8 of word c / 8,
// low nibble first), so 8 nibbles pair with one 8-column activation group.
constexpr uint32_t kCb4ResCap = 16384;   // residuals of one 128-row block (upload checks it)

struct RawC {
  u32x4 nib;     // 32 nibbles: columns c0 .. c0 + 31 of the lane's row
  uint32_t sc;   // the f16 scale of their 128-column group
};

__device__ __forceinline__ void bload_cb4(const DevTensor& t, uint32_t n, uint32_t c0, RawC& r) {
  const uint32_t kp = t.kp;
  r.nib = *reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(t.p0) + (size_t)n * (kp / 2) + c0 / 2);
  r.sc = t.p1[(size_t)n * (kp / 128) + c0 / 128];
}

// Activation pieces of iteration i: piece c (16 B) of row r holds columns
// S + (c / 4) H + 32 i + 8 (c % 4) .. +7.
__device__ __forceinline__ void aload_cb4(const uint16_t* __restrict__ xh, uint32_t m0, uint32_t M, uint32_t kp,
                                          uint32_t S, uint32_t H, uint32_t i, uint32_t tid, u32x4 (&r)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t q = tid + NT * j, c = q % 8;
    const uint32_t row = std::min(m0 + q / 8, M - 1);   // rows past M repeat row M-1 (never stored)
    r[j] = *reinterpret_cast<const u32x4*>(xh + (size_t)row * kp + S + (c / 4) * H + 32 * i + 8 * (c % 4));
  }
}

// LDS of tile_cb4_kernel: activation stages, residual list, centroid tables,
// row exponents, the lanes' product tables (4 waves x 16 entries x 64 lanes);
// the bf16 output tile reuses the stages (and the start of the residual
// list) after the K loop.
constexpr uint32_t kC4Res = 2 * kStageBytes;
constexpr uint32_t kC4Cent = kC4Res + kCb4ResCap * 4;
constexpr uint32_t kC4Xe = kC4Cent + 256;
constexpr uint32_t kC4Tab = (kC4Xe + BM * 4 + 4095) / 4096 * 4096;   // 4 KB aligned: table word bits 8-11 free
constexpr uint32_t kC4Bytes = kC4Tab + 4 * 16 * 64 * 4;
static_assert((size_t)BM * (BN + 8) * 2 <= kC4Cent, "output tile fits below the centroid tables");
static_assert(kC4Bytes <= 160 * 1024, "LDS budget");

typedef __attribute__((address_space(3))) uint32_t lds_u32;

// Rebuild a lane's table for the group scale sce = scale * 2^e: entry e is
// p = sce * centroid[e] split as (hi | lo << 16), p = hi + lo * 2^-11.
__device__ __forceinline__ void build_table(uint32_t tb, const float (&cvals)[16], float sce) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float p = sce * cvals[e];
    // hi and lo both from the one f16 rounding of p (its bits, converted back
    // exactly), so hi + lo * 2^-11 = p to 22 bits whichever instruction rounds
    const uint32_t hb = __builtin_bit_cast(uint16_t, (_Float16)p);
    const uint32_t lb = __builtin_bit_cast(uint16_t, (_Float16)((p - f16_to_f32(hb)) * 2048.0f));
    *(lds_u32*)(size_t)(tb + e * 256) = hb | (lb << 16);
  }
}

// Table words of 8 nibbles (columns 0..7 of a group of 8, low nibble first).
__device__ __forceinline__ void table_lookup8(uint32_t word, uint32_t tb, uint32_t (&d)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) d[j] = *(const lds_u32*)(size_t)(tb + (__builtin_amdgcn_ubfe(word, 4 * j, 4) << 8));
}

// Table words of columns 0..7 -> the hi and lo B operands: f16 pairs
// (0,2) (4,6) (1,3) (5,7), the pair order of the activations.
__device__ __forceinline__ void table_pack8(const uint32_t (&d)[8], u32x4& hi, u32x4& lo) {
  hi = u32x4{__builtin_amdgcn_perm(d[2], d[0], 0x05040100u), __builtin_amdgcn_perm(d[6], d[4], 0x05040100u),
             __builtin_amdgcn_perm(d[3], d[1], 0x05040100u), __builtin_amdgcn_perm(d[7], d[5], 0x05040100u)};
  lo = u32x4{__builtin_amdgcn_perm(d[2], d[0], 0x07060302u), __builtin_amdgcn_perm(d[6], d[4], 0x07060302u),
             __builtin_amdgcn_perm(d[3], d[1], 0x07060302u), __builtin_amdgcn_perm(d[7], d[5], 0x07060302u)};
}

// A lane's position in its row's residual list, one window ahead of the
// MFMAs: the next two entries decoded (column, and the f16 bits of value *
// 2^e; column ~0u past the lane's entries), the raw entry after them, and
// the raw entry after that (read from LDS one window earlier, so consuming an
// entry never waits for a read), which is list entry p.
struct ResWalk {
  uint32_t c0, r0, c1, r1, k2, k3, p, pe;
};

__device__ __forceinline__ uint32_t res_col(uint32_t k, uint32_t idx, uint32_t pe) {
  return idx < pe ? (k & 0xffffu) : ~0u;
}
__device__ __forceinline__ uint32_t res_val(uint32_t k, float e2) {
  return __builtin_bit_cast(uint16_t, (_Float16)(f16_to_f32(k >> 16) * e2));
}
__device__ __forceinline__ uint32_t res_read(const uint32_t* s_res, uint32_t idx) {
  return s_res[std::min(idx, kCb4ResCap - 1)];
}

// Start at list entry p0.
__device__ __forceinline__ void res_start(const uint32_t* s_res, ResWalk& w, uint32_t p0, float e2) {
  const uint32_t k0 = res_read(s_res, p0), k1 = res_read(s_res, p0 + 1);
  w.c0 = res_col(k0, p0, w.pe);
  w.r0 = res_val(k0, e2);
  w.c1 = res_col(k1, p0 + 1, w.pe);
  w.r1 = res_val(k1, e2);
  w.k2 = res_read(s_res, p0 + 2);
  w.k3 = res_read(s_res, p0 + 3);
  w.p = p0 + 3;
}

// Where `take`: drop entry 0 and move the queue up one; then read list entry
// p (unconditionally: without a take it is the entry already held).
__device__ __forceinline__ void res_shift(const uint32_t* s_res, ResWalk& w, float e2, bool take) {
  const uint32_t c2 = res_col(w.k2, w.p - 1, w.pe), r2 = res_val(w.k2, e2);
  w.c0 = take ? w.c1 : w.c0;
  w.r0 = take ? w.r1 : w.r0;
  w.c1 = take ? c2 : w.c1;
  w.r1 = take ? r2 : w.r1;
  w.k2 = take ? w.k3 : w.k2;
  w.p += take ? 1u : 0u;
  w.k3 = res_read(s_res, w.p);
}

// Residual entry (column c, f16 bits r) at its place in the B operand of
// window ws: pair order as table_pack8, c in [ws, ws + 8) when `hit`.
__device__ __forceinline__ void res_place(u32x4& R, uint32_t c, uint32_t r, uint32_t ws, bool hit) {
  const uint32_t j = c - ws;
  const uint32_t d = hit ? (((j & 1u) << 1) | ((j >> 2) & 1u)) : 4u, v = r << ((j & 2u) << 3);
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) R[k] |= d == k ? v : 0u;
}

// The residual B operand of columns ws .. ws + 7 (zero where the row has no
// residual), consuming those entries.  The lane's entries before ws are
// consumed, so c0 >= ws.  One residual per lane is placed branch-free; a
// second one in the same window takes the loop (a branch for the wave).
__device__ __forceinline__ u32x4 res_operand(const uint32_t* s_res, ResWalk& w, float e2, uint32_t ws) {
  u32x4 R = u32x4{0u, 0u, 0u, 0u};
  const bool hit = w.c0 < ws + 8u;
  res_place(R, w.c0, w.r0, ws, hit);
  res_shift(s_res, w, e2, hit);
  if (__builtin_amdgcn_ballot_w64(w.c0 < ws + 8u) != 0) {   // uniform, rare
    while (w.c0 < ws + 8u) {
      res_place(R, w.c0, w.r0, ws, true);
      res_shift(s_res, w, e2, true);
    }
  }
  return R;
}

// Keeps the computation of v in the block where this stands (the compiler
// would otherwise sink it to its use in the next iteration, away from the
// MFMAs it runs beside).
__device__ __forceinline__ void keep_here(const u32x4& v) { asm volatile("" ::"v"(v)); }

// gridDim.x = tiles_m * tiles_n, gridDim.y = K slices of kt_per_split tiles.
__global__ __launch_bounds__(NT, 1) void tile_cb4_kernel(DevTensor t, const uint16_t* __restrict__ xh, uint32_t M,
                                                         const int32_t* __restrict__ xe, void* __restrict__ y,
                                                         uint32_t y_bf16, float* __restrict__ partial,
                                                         uint32_t kt_per_split, uint32_t tiles_m) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const uint32_t tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const uint32_t N = t.rows, kp = t.kp;
  const uint32_t KTT = kp / BK;
  const uint32_t kt0 = blockIdx.y * kt_per_split;
  const uint32_t KT = std::min(KTT, kt0 + kt_per_split) - kt0;   // >= 1 (the plan guarantees it)
  const uint32_t S = kt0 * BK, H = KT * 32;
  auto it = [&](uint32_t i) { return std::min(i, KT - 1); };   // iterations past the slice repeat its last
  const uint32_t cl = S + H * h;                                // the lane's first column
  const uint32_t n = std::min(n0 + wave * 32 + l32, N - 1);   // rows past N repeat row N-1 (never stored)
  const int32_t xe_pre = xe[std::min(m0 + (tid & (BM - 1)), M - 1)];
  const int er = t.rexp[n];
  const float e2 = ldexpf(1.0f, er);
  float* const s_cent = reinterpret_cast<float*>(smem + kC4Cent);
  uint32_t* const s_res = reinterpret_cast<uint32_t*>(smem + kC4Res);
  const uint32_t tb = (uint32_t)(size_t)((__attribute__((address_space(3))) char*)(smem + kC4Tab)) + wave * 4096u +
                      lane * 4u;   // the lane's table: entry e at tb + 256 e

  // Prologue.  The first operand loads go out before the residual staging,
  // so their latencies overlap, and all loads are issued in the order the
  // loop expects (sched barriers keep it): each slot the first iteration
  // reads has at least as many younger loads as in the steady state, so the
  // waits the compiler places at the loop head (it merges both entries) stay
  // partial.
  u32x4 ra[2][4];
  RawC rb[2];
  u32x4 bh[2][4], bl[2][4];
  bload_cb4(t, n, cl + 32 * it(0), rb[0]);
  bload_cb4(t, n, cl + 32 * it(1), rb[1]);
  aload_cb4(xh, m0, M, kp, S, H, it(0), tid, ra[0]);
  aload_cb4(xh, m0, M, kp, S, H, it(1), tid, ra[1]);
  __builtin_amdgcn_sched_barrier(0);

  // Stage the centroid tables and the residual list of the block's rows.
  const uint32_t rbase = t.row_ptr[n0], rcount = t.row_ptr[std::min(n0 + BN, N)] - rbase;
  if (tid < 48) s_cent[tid] = t.cent[tid];
  // (eight loads in flight per thread, then their stores)
  for (uint32_t q0 = 0; q0 < rcount; q0 += 8 * NT) {
    uint32_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = t.outliers[rbase + std::min(q0 + u * NT + tid, rcount - 1)];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (q0 + u * NT + tid < rcount) s_res[q0 + u * NT + tid] = v[u];
  }
  ResWalk rw;
  rw.pe = t.row_ptr[n + 1] - rbase;
  uint32_t lo = t.row_ptr[n] - rbase;
  __syncthreads();
  float cvals[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) cvals[e] = s_cent[16 * cent_table(t, n) + e];
  {   // first entry of the row at or past column cl
    uint32_t hi = rw.pe;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) / 2;
      if ((s_res[mid] & 0xffffu) < cl)
        lo = mid + 1;
      else
        hi = mid;
    }
  }
  res_start(s_res, rw, lo, e2);

#define STAGE(st) (smem + (st) * kStageBytes)
  float16v acc[4], accl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      acc[i][r] = 0.0f;
      accl[i][r] = 0.0f;
    }
  uint32_t offA[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) offA[tt] = l32 * 128 + swz(l32, 4 * h + tt) * 16;
  // group of the lane's columns in iteration i
  auto group = [&](uint32_t i) { return (cl + 32 * it(i)) / 128; };

  astore(STAGE(0), tid, ra[0]);
  __builtin_amdgcn_sched_barrier(0);
  aload_cb4(xh, m0, M, kp, S, H, it(2), tid, ra[0]);
  __builtin_amdgcn_sched_barrier(0);
  build_table(tb, cvals, f16_to_f32(rb[0].sc) * e2);
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    uint32_t d[8];
    table_lookup8(rb[0].nib[tt], tb, d);
    table_pack8(d, bh[0][tt], bl[0][tt]);
  }
  __builtin_amdgcn_sched_barrier(0);
  bload_cb4(t, n, cl + 32 * it(2), rb[0]);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 rq = res_operand(s_res, rw, e2, cl);   // residual operand of the next step (here iteration 0, step 0)
  __syncthreads();

  // Iteration i (P = i & 1): multiply stage P by bh / bl[P] (iteration i)
  // and by the residual operands; stage activation pieces i+1 and load pieces
  // i+3 into the freed slot; decode the weights of iteration i+1 into
  // bh / bl[P^1] (rebuilding the table first when its group changes); reload
  // the raw slot with iteration i+3.  Step tt runs its 12 MFMAs (residual,
  // hi, lo for each of the 4 A fragments) with everything else of the step
  // between them, in program order (sched_barrier keeps it: the wave issues
  // in order, and VALU work overlaps the MFMAs only when it stands between
  // them): the packing of window tt of iteration i+1 (table words read the
  // step before), the residual operand of the next window, the table reads of
  // the next window and the A fragments of the next step.
  auto body = [&](uint32_t i, auto par) {
    constexpr int P = decltype(par)::value;
    const char* stage = STAGE(P);
    char* const next_stage = STAGE(P ^ 1);
    const uint32_t in = it(i + 3);
    if (group(i + 1) != group(i)) build_table(tb, cvals, f16_to_f32(rb[P ^ 1].sc) * e2);
    half8 af[2][4];
    uint32_t d[2][8];
#pragma unroll
    for (int f = 0; f < 4; ++f) af[0][f] = *reinterpret_cast<const half8*>(stage + f * 4096 + offA[0]);
    table_lookup8(rb[P ^ 1].nib[0], tb, d[0]);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int C = tt & 1;
      const half8 b = __builtin_bit_cast(half8, bh[P][tt]);
      const half8 c = __builtin_bit_cast(half8, bl[P][tt]);
      const half8 R = __builtin_bit_cast(half8, rq);
      const uint32_t q = tid + NT * tt, row = q / 8, cc = q % 8;
      const uint32_t(&w)[8] = d[C];
      const uint32_t wn = cl + 32 * i + 8 * (tt + 1);   // the next window
      u32x4 nh, nl;
      u32x4 Rn = u32x4{0u, 0u, 0u, 0u};
      bool hit;
      __builtin_amdgcn_sched_barrier(0);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][0], R, acc[0], 0, 0, 0);
      nh[0] = __builtin_amdgcn_perm(w[2], w[0], 0x05040100u);
      nl[0] = __builtin_amdgcn_perm(w[2], w[0], 0x07060302u);
      nh[1] = __builtin_amdgcn_perm(w[6], w[4], 0x05040100u);
      nl[1] = __builtin_amdgcn_perm(w[6], w[4], 0x07060302u);
      __builtin_amdgcn_sched_barrier(0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][1], R, acc[1], 0, 0, 0);
      hit = rw.c0 < wn + 8u;
      res_place(Rn, rw.c0, rw.r0, wn, hit);
      __builtin_amdgcn_sched_barrier(0);
      acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][2], R, acc[2], 0, 0, 0);
      nh[2] = __builtin_amdgcn_perm(w[3], w[1], 0x05040100u);
      nl[2] = __builtin_amdgcn_perm(w[3], w[1], 0x07060302u);
      nh[3] = __builtin_amdgcn_perm(w[7], w[5], 0x05040100u);
      nl[3] = __builtin_amdgcn_perm(w[7], w[5], 0x07060302u);
      *reinterpret_cast<u32x4*>(next_stage + row * 128 + swz(row, cc) * 16) = ra[P ^ 1][tt];
      __builtin_amdgcn_sched_barrier(0);
      acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][3], R, acc[3], 0, 0, 0);
      res_shift(s_res, rw, e2, hit);
      __builtin_amdgcn_sched_barrier(0);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][0], b, acc[0], 0, 0, 0);
      {
        const uint32_t grow = std::min(m0 + row, M - 1);
        ra[P ^ 1][tt] =
            *reinterpret_cast<const u32x4*>(xh + (size_t)grow * kp + S + (cc / 4) * H + 32 * in + 8 * (cc % 4));
      }
      __builtin_amdgcn_sched_barrier(0);
      accl[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][0], c, accl[0], 0, 0, 0);
      if (tt < 3) table_lookup8(rb[P ^ 1].nib[tt + 1], tb, d[C ^ 1]);
      __builtin_amdgcn_sched_barrier(0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][1], b, acc[1], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      accl[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][1], c, accl[1], 0, 0, 0);
      if (tt < 3) {
#pragma unroll
        for (int f = 0; f < 4; ++f) af[C ^ 1][f] = *reinterpret_cast<const half8*>(stage + f * 4096 + offA[tt + 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][2], b, acc[2], 0, 0, 0);
      accl[2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][2], c, accl[2], 0, 0, 0);
      acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][3], b, acc[3], 0, 0, 0);
      accl[3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[C][3], c, accl[3], 0, 0, 0);
      bh[P ^ 1][tt] = nh;
      bl[P ^ 1][tt] = nl;
      keep_here(nh);
      keep_here(nl);
      __builtin_amdgcn_sched_barrier(0);
      if (__builtin_amdgcn_ballot_w64(rw.c0 < wn + 8u) != 0) {   // uniform, rare: a second residual
        while (rw.c0 < wn + 8u) {
          res_place(Rn, rw.c0, rw.r0, wn, true);
          res_shift(s_res, rw, e2, true);
        }
      }
      rq = Rn;
    }
    bload_cb4(t, n, cl + 32 * in, rb[P ^ 1]);
    __syncthreads();
  };
  // The slice's last iteration i (operands in slot `odd`): MFMAs only.
  auto last = [&](uint32_t i, bool odd) {
    const char* stage = odd ? STAGE(1) : STAGE(0);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      half8 af[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) af[f] = *reinterpret_cast<const half8*>(stage + f * 4096 + offA[tt]);
      const half8 R = __builtin_bit_cast(half8, rq);
      const half8 b = __builtin_bit_cast(half8, odd ? bh[1][tt] : bh[0][tt]);
      const half8 c = __builtin_bit_cast(half8, odd ? bl[1][tt] : bl[0][tt]);
#pragma unroll
      for (int f = 0; f < 4; ++f) acc[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[f], R, acc[f], 0, 0, 0);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        acc[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[f], b, acc[f], 0, 0, 0);
        accl[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[f], c, accl[f], 0, 0, 0);
      }
      if (tt < 3) rq = res_operand(s_res, rw, e2, cl + 32 * i + 8 * (tt + 1));
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  uint32_t i = 0;
  for (; i + 2 < KT; i += 2) {
    body(i, I0{});
    body(i + 1, I1{});
  }
  if (i + 1 < KT) {
    body(i, I0{});
    ++i;
  }
  last(i, (i & 1) != 0);
#undef STAGE

  // Epilogue: w * 2^e = hi + lo * 2^-11, so y = (acc + accl * 2^-11) * 2^-(e + xe).
  const bool to_partial = gridDim.y > 1;
  const uint32_t N_ = N;
  const bool rows_fast = y_bf16 && !to_partial && N_ % 8 == 0 && n0 + BN <= N_ &&
                         reinterpret_cast<uintptr_t>(y) % 16 == 0;
  int32_t* s_xe = reinterpret_cast<int32_t*>(smem + kC4Xe);
  uint16_t* s_out = reinterpret_cast<uint16_t*>(smem);
  __syncthreads();   // every wave is done with the stages and the residual list
  if (tid < BM && !to_partial) s_xe[tid] = xe_pre;
  __syncthreads();
  // One loop per output mode (a mode test per output compiles to branches
  // per output).
  const uint32_t nl = wave * 32 + l32, ncol = n0 + nl;
  auto row_of = [&](int f, int r) { return (uint32_t)(f * 32 + h * 4 + 8 * (r >> 2) + (r & 3)); };
  auto value = [&](int f, int r) { return hilo_combine(acc[f][r], accl[f][r]); };
  auto load_xs = [&](int f, int (&xs)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int4 e4 = *reinterpret_cast<const int4*>(s_xe + f * 32 + h * 4 + 8 * q);
      xs[4 * q + 0] = e4.x;
      xs[4 * q + 1] = e4.y;
      xs[4 * q + 2] = e4.z;
      xs[4 * q + 3] = e4.w;
    }
  };
  if (rows_fast) {
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      int xs[16];
      load_xs(f, xs);
#pragma unroll
      for (int r = 0; r < 16; ++r) s_out[row_of(f, r) * LDO + nl] = f32_to_bf16(ldexpf(value(f, r), -(xs[r] + er)));
    }
  } else if (to_partial) {
    float* const pp = partial + ((size_t)blockIdx.y * M + m0) * N_ + ncol;
    if (m0 + BM <= M && n0 + BN <= N_) {
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) pp[(size_t)row_of(f, r) * N_] = ldexpf(value(f, r), -er);
    } else {
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (m0 + row_of(f, r) < M && ncol < N_) pp[(size_t)row_of(f, r) * N_] = ldexpf(value(f, r), -er);
    }
  } else {
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      int xs[16];
      load_xs(f, xs);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t m = m0 + row_of(f, r);
        if (m >= M || ncol >= N_) continue;
        const float o = ldexpf(value(f, r), -(xs[r] + er));
        if (y_bf16)
          static_cast<uint16_t*>(y)[(size_t)m * N_ + ncol] = f32_to_bf16(o);
        else
          static_cast<float*>(y)[(size_t)m * N_ + ncol] = o;
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
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(y) + (size_t)(m0 + row) * N_ + n0 + c * 8) = v;
    }
  }
}

struct Plan {
  uint32_t tiles_m, tiles_n, kw, splits, kps;
  size_t xe_off, xh_off, partial_off, bytes;
};

inline size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

// Grid shape.  Two workgroups of 4 waves fit a CU (512 slots): from 384
// tiles on, one K-way; below, K split across workgroups until the grid has
// about 256 workgroups, with >= 4 tiles per slice and at most 16 MB of
// partial sums, and two K-ways (8 waves, one workgroup per CU) unless that
// takes more than 4 slices.
constexpr size_t kMaxPartialBytes = (size_t)16 << 20;

inline Plan plan(const DevTensor& t, uint32_t m) {
  Plan p{};
  p.tiles_m = (m + BM - 1) / BM;
  p.tiles_n = (t.rows + BN - 1) / BN;
  const uint32_t ktt = t.kp / BK;
  const uint32_t tiles = p.tiles_m * p.tiles_n;
  p.kw = tiles >= 384 ? 1 : 2;
  uint32_t splits = 1;
  if (p.kw == 2) {
    const size_t slice_bytes = (size_t)m * t.rows * 4;
    splits = (256u + tiles - 1) / tiles;
    splits = std::min<uint32_t>(splits, std::max<uint32_t>(1u, ktt / (2 * p.kw)));
    splits = (uint32_t)std::min<size_t>(splits, std::max<size_t>(1, kMaxPartialBytes / slice_bytes));
  }
  p.kps = (ktt + splits - 1) / splits;
  p.splits = (ktt + p.kps - 1) / p.kps;
  // With more than 4 K slices each way would walk only a few tiles: one
  // K-way per workgroup is then faster (M = 128: 11.9 against 12.7 us at
  // 6144 x 2048, 12.8 against 14.2 us at 2048 x 6144).
  if (p.splits > 4) p.kw = 1;
  p.xe_off = 0;
  p.xh_off = al256((size_t)m * 4);
  p.partial_off = p.xh_off + al256((size_t)m * t.kp * 2);
  p.bytes = p.partial_off + (p.splits > 1 ? al256((size_t)p.splits * m * t.rows * 4) : 0);
  return p;
}

template <int KW>
hipError_t launch_tile(const DevTensor& t, const uint16_t* xh, uint32_t m, const int32_t* xe, void* y, bool y_bf16,
                       float* partial, const Plan& p, hipStream_t s) {
  constexpr size_t lds = lds_bytes<KW>();
  static_assert(lds <= 160 * 1024, "LDS budget");
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&tile_kernel<KW>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((tile_kernel<KW>), dim3(p.tiles_m * p.tiles_n, p.splits), dim3(NT * KW), lds, s, t, xh, m, xe, y,
                     (uint32_t)y_bf16, partial, p.kps, p.tiles_m);
  return hipGetLastError();
}

// cb4 grid: one workgroup of 4 waves per CU (registers), K split across
// workgroups until about 256 workgroups, >= 2 tiles per slice, at most 16 MB
// of partial sums.
inline Plan plan_cb4(const DevTensor& t, uint32_t m) {
  Plan p{};
  p.tiles_m = (m + BM - 1) / BM;
  p.tiles_n = (t.rows + BN - 1) / BN;
  const uint32_t ktt = t.kp / BK;
  const uint32_t tiles = p.tiles_m * p.tiles_n;
  p.kw = 1;
  const size_t slice_bytes = (size_t)m * t.rows * 4;
  uint32_t splits = (256u + tiles - 1) / tiles;
  splits = std::min<uint32_t>(splits, std::max<uint32_t>(1u, ktt / 2));
  splits = (uint32_t)std::min<size_t>(splits, std::max<size_t>(1, kMaxPartialBytes / slice_bytes));
  p.kps = (ktt + splits - 1) / splits;
  p.splits = (ktt + p.kps - 1) / p.kps;
  p.xe_off = 0;
  p.xh_off = al256((size_t)m * 4);
  p.partial_off = p.xh_off + al256((size_t)m * t.kp * 2);
  p.bytes = p.partial_off + (p.splits > 1 ? al256((size_t)p.splits * m * t.rows * 4) : 0);
  return p;
}

inline hipError_t launch_tile_cb4(const DevTensor& t, const uint16_t* xh, uint32_t m, const int32_t* xe, void* y,
                                  bool y_bf16, float* partial, const Plan& p, hipStream_t s) {
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&tile_cb4_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)kC4Bytes);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(tile_cb4_kernel, dim3(p.tiles_m * p.tiles_n, p.splits), dim3(NT), kC4Bytes, s, t, xh, m, xe, y,
                     (uint32_t)y_bf16, partial, p.kps, p.tiles_m);
  return hipGetLastError();
}

// The activation pre-pass (row exponents, row-scaled permuted f16 rows):
// one workgroup per row, up to 4 pieces of 16 bytes per thread in registers
// (rows up to 8192 columns), longer rows in two passes.
inline hipError_t launch_xprep(const uint16_t* x, uint32_t m, uint32_t cols, uint32_t kp, uint16_t* xh, int32_t* xe,
                               hipStream_t s) {
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (cols % 8 == 0);
  const dim3 xg(m), xb(256);
  const uint32_t npt = (kp / 8 + 255) / 256;   // 16-byte pieces per thread
  if (npt <= 1)
    hipLaunchKernelGGL(xprep_kernel<1>, xg, xb, 0, s, x, m, cols, kp, x_vec, xh, xe);
  else if (npt <= 2)
    hipLaunchKernelGGL(xprep_kernel<2>, xg, xb, 0, s, x, m, cols, kp, x_vec, xh, xe);
  else if (npt <= 4)
    hipLaunchKernelGGL(xprep_kernel<4>, xg, xb, 0, s, x, m, cols, kp, x_vec, xh, xe);
  else
    hipLaunchKernelGGL(xprep_kernel<0>, xg, xb, 0, s, x, m, cols, kp, x_vec, xh, xe);
  return hipGetLastError();
}

}  // namespace gt

bool gemm_tile_supported(const DevTensor& t, bool x_bf16) {
  return x_bf16 && t.kind == KIND_G64 && t.kp % 64 == 0 && !(t.cols % 64 != 0 && t.tail_nonfinite);
}

size_t gemm_tile_workspace_bytes(const DevTensor& t, uint32_t m) { return gt::plan(t, m).bytes; }

hipError_t launch_gemm_tile(const DevTensor& t, const uint16_t* x, uint32_t m, void* y, bool y_bf16, void* ws,
                            size_t ws_bytes, hipStream_t s) {
  if (!gemm_tile_supported(t, true) || m == 0) return hipErrorInvalidValue;
  const gt::Plan p = gt::plan(t, m);
  if (ws_bytes < p.bytes) return hipErrorInvalidValue;
  char* base = static_cast<char*>(ws);
  int32_t* xe = reinterpret_cast<int32_t*>(base + p.xe_off);
  uint16_t* xh = reinterpret_cast<uint16_t*>(base + p.xh_off);
  float* partial = reinterpret_cast<float*>(base + p.partial_off);
  hipError_t e = gt::launch_xprep(x, m, t.cols, t.kp, xh, xe, s);
  if (e != hipSuccess) return e;
  e = p.kw == 1 ? gt::launch_tile<1>(t, xh, m, xe, y, y_bf16, partial, p, s)
                : gt::launch_tile<2>(t, xh, m, xe, y, y_bf16, partial, p, s);
  if (e != hipSuccess || p.splits == 1) return e;
  return launch_gemm_reduce(partial, p.splits, nullptr, xe, m, t.rows, y, y_bf16, s);
}

bool gemm_tile_cb4_supported(const DevTensor& t, bool x_bf16) {
  return x_bf16 && t.kind == KIND_CB4 && t.rexp != nullptr && t.kp % 128 == 0;
}

size_t gemm_tile_cb4_workspace_bytes(const DevTensor& t, uint32_t m) { return gt::plan_cb4(t, m).bytes; }

hipError_t launch_gemm_tile_cb4(const DevTensor& t, const uint16_t* x, uint32_t m, void* y, bool y_bf16, void* ws,
                                size_t ws_bytes, hipStream_t s) {
  if (!gemm_tile_cb4_supported(t, true) || m == 0) return hipErrorInvalidValue;
  const gt::Plan p = gt::plan_cb4(t, m);
  if (ws_bytes < p.bytes) return hipErrorInvalidValue;
  char* base = static_cast<char*>(ws);
  int32_t* xe = reinterpret_cast<int32_t*>(base + p.xe_off);
  uint16_t* xh = reinterpret_cast<uint16_t*>(base + p.xh_off);
  float* partial = reinterpret_cast<float*>(base + p.partial_off);
  hipError_t e = gt::launch_xprep(x, m, t.cols, t.kp, xh, xe, s);
  if (e != hipSuccess) return e;
  e = gt::launch_tile_cb4(t, xh, m, xe, y, y_bf16, partial, p, s);
  if (e != hipSuccess || p.splits == 1) return e;
  return launch_gemm_reduce(partial, p.splits, nullptr, xe, m, t.rows, y, y_bf16, s);
}

}  // namespace vxt
