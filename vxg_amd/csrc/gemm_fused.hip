// gemm_fused.hip -- prefill GEMM (batch_m > 8) with the weights decoded inside
// the MFMA loop, for g64 and Q8_0 tensors and bf16 activations.
//
// Reference behaviour: PackedTensor::gemm_cpu (llm_prefill.rs:156-255) decodes
// weight tiles to f32 and multiplies them densely; the result must match it to
// fp32-accumulation error.  Where the two-phase path (gemm_panel.hip) writes
// the decoded weights to an f16 panel in HBM and reads them back, this kernel
// decodes them once into MFMA operand registers:
//
//   * workgroup = 4 x KW waves: 128 weight rows (4 row groups of 32) x
//     BM = 32*FI activation rows; its K range is walked in chunks of KC = 4
//     K tiles of 64 columns, and K way wk of a row group takes the chunk's
//     tiles wk, wk + KW, ...  The K ways are summed through LDS at the end
//     (ascending wk), so a workgroup holds 4 x KW waves in flight without
//     extra partial sums in HBM; more waves per SIMD is what hides the LDS
//     latency of the table decode;
//   * activations (bf16) go global -> LDS with global_load_lds, stored in
//     MFMA A-operand order (one 1 KB block per 32 rows x one MFMA step);
//     two buffers, so chunk c+1 loads while chunk c is multiplied;
//   * each lane loads its own weight row's packed bytes for its tiles of the
//     chunk before the first wait, and decodes them into B fragments:
//       g64: the f16 table entries themselves (exact), looked up in a 48-byte
//            LDS slot per row holding the group's table (two slots per row,
//            alternating); v_mfma_f32_32x32x16_f16, with the chunk's
//            activations converted to f16 once, in place, after a power-of-
//            two scale per activation row (xe, from xscale_kernel) that puts
//            the row's largest magnitude in [2^14, 2^15): exact for every
//            element within 2^28 of it, whatever the row's magnitude; the
//            epilogue (or the split-K reduction) undoes the scale;
//       Q8:  the int8 values, exact in bf16, against the bf16 activations
//            as they are (v_mfma_f32_32x32x16_bf16: the products are exact in
//            fp32); each 32-column block is two MFMA steps into a fresh
//            fragment, then acc += d * fragment;
//   * K is also split across workgroups when the tile grid is small; the
//     fp32 partial sums are added in ascending split order by reduce_kernel.
//
// Within a K tile the 64 columns are assigned to (MFMA step t, lane half h)
// as col8(t, h) .. +8; A and B use the same assignment, so the dot products
// are unchanged.  g64: col8 = 32h + 8t (a lane's 32 columns are contiguous);
// Q8: col8 = 32(t/2) + 16h + 8(t%2) (steps 2b, 2b+1 cover block b).
#include <algorithm>

#include "common.hpp"

#pragma clang fp contract(off)

namespace vxt {

namespace fz {


constexpr int BN = 128;      // weight rows per workgroup
constexpr int BK = 64;       // K tile
constexpr int KC = 4;        // K tiles per chunk
constexpr int FRAG = 1024;   // bytes of one A block: 64 lanes x 16 B
constexpr int SLOT = 48;     // g64 table slot stride (bytes)

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr;

template <uint32_t KIND>
__device__ __forceinline__ uint32_t col8(uint32_t t, uint32_t h) {
  if constexpr (KIND == KIND_Q8)
    return 32u * (t >> 1) + 16u * h + 8u * (t & 1u);
  else
    return 32u * h + 8u * t;
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left unconstrained; gfx9 encoding).
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8)); }

template <int FI>
constexpr int a_bytes() { return KC * FI * 4 * FRAG; }

template <uint32_t KIND, int KW>
constexpr size_t slot_bytes() { return KIND == KIND_G64 ? (size_t)4 * KW * 64 * SLOT : 0; }

// LDS: two activation buffers (the first reused for the K-way sums at the
// end), then the g64 table slots.
template <uint32_t KIND, int FI, int KW>
constexpr size_t lds_bytes() {
  const size_t a = 2 * (size_t)a_bytes<FI>();
  const size_t red = (size_t)(KW - 1) * 4 * FI * 16 * 64 * 4;
  return (a > red ? a : red) + slot_bytes<KIND, KW>();
}

// Activation blocks of one chunk.  Block (kl, g, t) -- K tile kl of the chunk,
// rows g*32.., MFMA step t -- sits at ((kl*FI + g)*4 + t)*FRAG; lane l holds
// row g*32 + l%32, columns col8(t, l/32) .. +8 as 8 bf16.  Wave (wn, wk) loads
// the blocks of step t = wn with kl*FI + g = wk, wk + KW, ...  Rows past M
// repeat row M-1 (never stored); columns past K are zero.
template <uint32_t KIND, int FI, int KW>
__device__ __forceinline__ void issue_a(const uint16_t* __restrict__ x, uint32_t M, uint32_t K, uint32_t x_vec,
                                        uint32_t m0, uint32_t kt0, uint32_t KT, char* abuf, uint32_t wn,
                                        uint32_t wk, uint32_t lane) {
  const uint32_t h = lane >> 5;
  // Every tile of the chunk inside the rows (uniform): all blocks by DMA,
  // with no LDS store beside them -- an LDS store after a DMA into the same
  // buffer would make the compiler wait for the DMA first, one round trip
  // per block.  The DMA targets are formed from the buffer's own pointer, so
  // the compiler can tell them from the other buffer's fragment reads.
  const uint32_t kt_last = std::min(kt0 + KC, KT) - 1;
  if (x_vec && (kt_last + 1) * BK <= K) {
#pragma unroll
    for (int j = 0; j < KC * FI / KW; ++j) {
      const uint32_t kg = wk + KW * j;   // kl * FI + g
      const uint32_t kl = kg / FI, g = kg % FI;
      const uint32_t kt = kt0 + kl;
      if (kt >= KT) continue;   // uniform
      const uint32_t col = kt * BK + col8<KIND>(wn, h);
      const uint32_t row = std::min(m0 + g * 32 + (lane & 31), M - 1);
      const uint32_t blk = (kg * 4 + wn) * FRAG;
      __builtin_amdgcn_global_load_lds(x + (size_t)row * K + col, (lds_ptr)(abuf + blk), 16, 0, 0);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < KC * FI / KW; ++j) {
    const uint32_t kg = wk + KW * j;
    const uint32_t kl = kg / FI, g = kg % FI;
    const uint32_t kt = kt0 + kl;
    if (kt >= KT) continue;   // uniform
    const uint32_t col = kt * BK + col8<KIND>(wn, h);
    const uint32_t row = std::min(m0 + g * 32 + (lane & 31), M - 1);
    const uint32_t blk = (kg * 4 + wn) * FRAG;
    // element loads from clamped (always valid) addresses, masked after
    const uint16_t* rowp = x + (size_t)row * K;
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = rowp[std::min(col + i, K - 1)];
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (col + 2 * i < K ? e[2 * i] : 0u) | ((col + 2 * i + 1 < K ? e[2 * i + 1] : 0u) << 16);
    *reinterpret_cast<u32x4*>(abuf + blk + lane * 16) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// 8 bf16 times 2^e -> 8 f16 (two per v_cvt_pk_f16_f32; the scaling is exact).
__device__ __forceinline__ u32x4 bf16x8_to_f16(u32x4 raw, int e) {
  u32x4 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float2v f = {ldexpf(__uint_as_float(raw[j] << 16), e), ldexpf(__uint_as_float(raw[j] & 0xffff0000u), e)};
    out[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2v));
  }
  return out;
}

// The chunk's activation blocks, bf16 -> f16 in place with the row scales
// 2^xe (all threads; the caller brackets it with barriers).  Piece i is lane
// i % 64 of block i / 64, which holds activation row m0 + g * 32 + lane % 32
// (g = block / 4 % FI; rows past M repeat row M - 1).
template <int FI, int KW>
__device__ __forceinline__ void convert_a(char* abuf, uint32_t tiles, uint32_t m0, uint32_t M,
                                          const int32_t* __restrict__ xe) {
  const uint32_t pieces = tiles * FI * 4 * (FRAG / 16);
  for (uint32_t i = threadIdx.x; i < pieces; i += 256 * KW) {
    const uint32_t g = (i / 64 / 4) % FI;
    const int e = xe[std::min(m0 + g * 32 + (i & 31), M - 1)];
    u32x4* p = reinterpret_cast<u32x4*>(abuf + i * 16);
    *p = bf16x8_to_f16(*p, e);
  }
}

// int8 bytes 2p, 2p+1 of w as a packed bf16 pair (exact).
__device__ __forceinline__ uint32_t i8pair_bf16(uint32_t w, int p) {
  const float f0 = (float)(int8_t)((w >> (16 * p)) & 0xffu);
  const float f1 = (float)(int8_t)((w >> (16 * p + 8)) & 0xffu);
  return (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
}

// Per-lane packed weights of one K tile.
template <uint32_t KIND>
struct BTile;

template <>
struct BTile<KIND_G64> {
  u32x4 nib;   // 32 nibbles: columns kb + 32h ..
  u32x4 lut;   // half h of the group's 16-entry f16 table
};

template <>
struct BTile<KIND_Q8> {
  u32x4 q[2];    // int8 values of block b: columns kb + 32b + 16h .. +16
  u32x4 dch;     // (tile 0 of a chunk only) the row's f16 scales of the chunk's 8 blocks
};

template <uint32_t KIND>
__device__ __forceinline__ void load_b(const DevTensor& t, uint32_t n, uint32_t kt, uint32_t h, BTile<KIND>& b) {
  const uint32_t kp = t.kp, kb = kt * BK;
  if constexpr (KIND == KIND_G64) {
    b.nib = *reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(t.p0) + (size_t)n * (kp / 2) + (kb + 32 * h) / 2);
    b.lut = *reinterpret_cast<const u32x4*>(t.p1 + ((size_t)n * (kp / 64) + kt) * 16 + h * 8);
  } else {
    // kp is a multiple of 32: the tile's second block may lie past the row;
    // it is then loaded from the first block's address (valid memory) and
    // its scale is taken as zero where it is used.  No value is combined
    // here, so every load of the chunk is in flight before the first wait.
    const int8_t* qs = static_cast<const int8_t*>(t.p0) + (size_t)n * kp;
    const uint32_t b1 = kb + 32 < kp ? kb + 32 : kb;
    b.q[0] = *reinterpret_cast<const u32x4*>(qs + kb + 16 * h);
    b.q[1] = *reinterpret_cast<const u32x4*>(qs + b1 + 16 * h);
  }
}

// Loads of one chunk for wave (wn, wk): activation blocks into the LDS buffer
// at abuf, and this lane's packed weights of tiles
// wk, wk + KW, ... into b.  Tiles past the row repeat its last one (loaded,
// never used).
template <uint32_t KIND, int FI, int KW>
__device__ __forceinline__ void issue_chunk(const DevTensor& t, const uint16_t* __restrict__ x, uint32_t M,
                                            uint32_t x_vec, uint32_t m0, uint32_t n, uint32_t kt0, uint32_t KT,
                                            char* abuf, uint32_t wn, uint32_t wk, uint32_t lane,
                                            BTile<KIND> (&b)[KC / KW]) {
  issue_a<KIND, FI, KW>(x, M, t.cols, x_vec, m0, kt0, KT, abuf, wn, wk, lane);
#pragma unroll
  for (int j = 0; j < KC / KW; ++j) load_b<KIND>(t, n, std::min(kt0 + wk + KW * j, KT - 1), lane >> 5, b[j]);
  if constexpr (KIND == KIND_Q8) {
    // The row's scales of the chunk's 2 * KC blocks, one 16-byte load: the
    // plane holds kp / 32 scales per row and chunks start at multiples of
    // 2 * KC blocks, so the load is 4-byte aligned, and the upload keeps 16
    // bytes after the plane's last scale, so it stays inside the allocation
    // (scales past the row belong to the next row or the padding; blocks
    // past the row are never applied).
    const uint32_t nb = t.kp / 32;
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(t.p1), (short)0, (int)(t.rows * nb * 2u + 16u), 0x00020000);
    b[0].dch = __builtin_amdgcn_raw_buffer_load_b128(rd, (n * nb + 2u * kt0) * 2u, 0, 0);
  }
}

// Decode and multiply this wave's tiles of one chunk (activations at abuf).
template <uint32_t KIND, int FI, int KW>
__device__ __forceinline__ void compute_chunk(const DevTensor& t, const char* abuf, char* slot,
                                              const BTile<KIND> (&b)[KC / KW], uint32_t kt0, uint32_t KT,
                                              uint32_t wk, uint32_t lane, float16v (&acc)[FI]) {
  const uint32_t h = lane >> 5, K = t.cols;
#pragma unroll
  for (int j = 0; j < KC / KW; ++j) {
    const uint32_t kl = wk + KW * j;
    const uint32_t kt = kt0 + kl;
    if (kt >= KT) break;   // uniform
    const uint32_t kb = kt * BK;
    u32x4 bf[4];   // B fragments: f16 (g64) or bf16 (Q8) pairs
    if constexpr (KIND == KIND_G64) {
      char* sl = slot + (j & 1) * 32 * SLOT;
      *reinterpret_cast<u32x4*>(sl + h * 16) = b[j].lut;
      const uint16_t* tab = reinterpret_cast<const uint16_t*>(sl);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t wd = b[j].nib[s];
#pragma unroll
        for (int e = 0; e < 8; e += 2)
          bf[s][e >> 1] = (uint32_t)tab[(wd >> (4 * e)) & 0xfu] | ((uint32_t)tab[(wd >> (4 * e + 4)) & 0xfu] << 16);
      }
      if (kb + BK > K) {   // uniform: the last tile of a ragged row; columns past K are zero
        const uint32_t valid = K > kb + 32 * h ? K - (kb + 32 * h) : 0u;   // of this lane's 32
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t c = 8 * s + 2 * i;
            bf[s][i] &= (c < valid ? 0xffffu : 0u) | (c + 1 < valid ? 0xffff0000u : 0u);
          }
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4 q = b[j].q[s >> 1];
#pragma unroll
        for (int i = 0; i < 4; ++i) bf[s][i] = i8pair_bf16(q[(s & 1) * 2 + (i >> 1)], i & 1);   // gguf.rs:223-229
      }
    }
    float16v tmp[FI];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int i = 0; i < FI; ++i) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(abuf + ((kl * FI + i) * 4 + s) * FRAG + lane * 16);
        if constexpr (KIND == KIND_G64) {
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                          __builtin_bit_cast(half8, bf[s]), acc[i], 0, 0, 0);
        } else {
          tmp[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                           __builtin_bit_cast(bf16x8, bf[s]),
                                                           (s & 1) ? tmp[i] : float16v{}, 0, 0, 0);
        }
      }
      if constexpr (KIND == KIND_Q8) {
        if (s & 1) {
          const uint32_t e = 2u * kl + (uint32_t)(s >> 1);   // block of the chunk
          const uint32_t dbits = (b[0].dch[e >> 1] >> (16u * (e & 1u))) & 0xffffu;
          const float d = (s >> 1) && !(kb + 32 < t.kp) ? 0.0f : f16_to_f32(dbits);
#pragma unroll
          for (int i = 0; i < FI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][r] = __builtin_fmaf(d, tmp[i][r], acc[i][r]);
        }
      }
    }
  }
}

// One workgroup: weight rows n0.. (4 row groups x 32), activation rows m0..
// (32*FI), chunks [c0, c1) of its K range.  Two activation buffers and two
// register sets of packed weights: chunk c+1 is loading while chunk c is
// multiplied.
template <uint32_t KIND, int FI, int KW>
__global__ __launch_bounds__(256 * KW) void fused_kernel(DevTensor t, const uint16_t* __restrict__ x, uint32_t M,
                                                         uint32_t x_vec, void* __restrict__ y, uint32_t y_bf16,
                                                         float* __restrict__ partial, uint32_t chunks_per_split,
                                                         uint32_t tiles_m, const int32_t* __restrict__ xe) {
  constexpr uint32_t BM = 32 * FI;
  constexpr uint32_t AB = a_bytes<FI>();
  constexpr int NT = KC / KW;
  // Two activation buffers and the g64 table slots, each its own array:
  // the compiler then knows that a DMA into one buffer does not write what
  // the fragment reads of the other read, and does not wait for it.
  constexpr size_t SB = slot_bytes<KIND, KW>();
  __shared__ __attribute__((aligned(1024))) char s_buf0[AB];
  __shared__ __attribute__((aligned(1024))) char s_buf1[AB];
  __shared__ __attribute__((aligned(16))) char s_slot[SB > 0 ? SB : 16];
  static_assert((size_t)(KW - 1) * 4 * FI * 16 * 64 * 4 <= AB, "K-way sums fit in one buffer");
  const uint32_t lane = threadIdx.x & 63, h = lane >> 5;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t wn = wave & 3, wk = wave >> 2;
  const uint32_t tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t N = t.rows;
  const uint32_t KT = (t.kp + BK - 1) / BK;
  const uint32_t nchunks = (KT + KC - 1) / KC;
  const uint32_t c0 = blockIdx.y * chunks_per_split;
  const uint32_t c1 = std::min(nchunks, c0 + chunks_per_split);
  const uint32_t n = std::min(n0 + wn * 32 + (lane & 31), N - 1);
  char* const buf0 = s_buf0;
  char* const buf1 = s_buf1;
  // g64: this row's two table slots in this wave's region
  char* slot = s_slot + (wave * 64 + (lane & 31)) * SLOT;

  float16v acc[FI];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;

  BTile<KIND> b0[NT], b1[NT];
  if (c0 < c1) issue_chunk<KIND, FI, KW>(t, x, M, x_vec, m0, n, c0 * KC, KT, buf0, wn, wk, lane, b0);
  for (uint32_t c = c0; c < c1; c += 2) {
    wait_vm0();        // chunk c has landed (nothing else is in flight)
    __syncthreads();   // ... for every wave; and the other buffer is free
    if constexpr (KIND == KIND_G64) {
      convert_a<FI, KW>(buf0, std::min<uint32_t>(KC, KT - c * KC), m0, M, xe);
      __syncthreads();
    }
    if (c + 1 < c1)
      issue_chunk<KIND, FI, KW>(t, x, M, x_vec, m0, n, (c + 1) * KC, KT, buf1, wn, wk, lane, b1);
    compute_chunk<KIND, FI, KW>(t, buf0, slot, b0, c * KC, KT, wk, lane, acc);
    if (c + 1 >= c1) break;
    wait_vm0();
    __syncthreads();
    if constexpr (KIND == KIND_G64) {
      convert_a<FI, KW>(buf1, std::min<uint32_t>(KC, KT - (c + 1) * KC), m0, M, xe);
      __syncthreads();
    }
    if (c + 2 < c1)
      issue_chunk<KIND, FI, KW>(t, x, M, x_vec, m0, n, (c + 2) * KC, KT, buf0, wn, wk, lane, b0);
    compute_chunk<KIND, FI, KW>(t, buf1, slot, b1, (c + 1) * KC, KT, wk, lane, acc);
  }

  // K ways 1.. hand their sums to K way 0 through LDS; added in ascending wk.
  if constexpr (KW > 1) {
    __syncthreads();   // every wave is done with the activation buffers
    float* red = reinterpret_cast<float*>(s_buf0);
    if (wk > 0) {
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[((((wk - 1) * 4 + wn) * FI + i) * 16 + r) * 64 + lane] = acc[i][r];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (uint32_t k = 1; k < (uint32_t)KW; ++k)
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] += red[((((k - 1) * 4 + wn) * FI + i) * 16 + r) * 64 + lane];
  }

  // Lane owns weight row n0 + wn*32 + lane%32 (an output column) and
  // activation rows m0 + i*32 + (lane/32)*4 + 8*(r/4) + r%4.
  const uint32_t ncol = n0 + wn * 32 + (lane & 31);
  if (ncol >= N) return;
  const bool to_partial = gridDim.y > 1;
  if constexpr (FI == 4) {
    // One loop per output mode (a mode test per output compiles to a pair
    // of branches per output); the smaller instantiations keep the shared
    // loop below, whose registers they need.
    auto row_of = [&](int i, int r) { return (uint32_t)(i * 32 + h * 4 + 8 * (r >> 2) + (r & 3)); };
    if (to_partial) {
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t m = m0 + row_of(i, r);
          if (m < M) partial[((size_t)blockIdx.y * M + m) * N + ncol] = acc[i][r];
        }
    } else {
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t m = m0 + row_of(i, r);
          if (m >= M) continue;
          float v = acc[i][r];
          if constexpr (KIND == KIND_G64) v = ldexpf(v, -xe[m]);
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * N + ncol] = f32_to_bf16(v);
          else
            static_cast<float*>(y)[(size_t)m * N + ncol] = v;
        }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint32_t m = m0 + i * 32 + h * 4 + 8 * (r >> 2) + (r & 3);
      if (m >= M) continue;
      float v = acc[i][r];
      if constexpr (KIND == KIND_G64) {
        if (!to_partial) v = ldexpf(v, -xe[m]);
      }
      if (to_partial)
        partial[((size_t)blockIdx.y * M + m) * N + ncol] = v;
      else if (y_bf16)
        static_cast<uint16_t*>(y)[(size_t)m * N + ncol] = f32_to_bf16(v);
      else
        static_cast<float*>(y)[(size_t)m * N + ncol] = v;
    }
}

struct Plan {
  int fi;
  uint32_t tiles_m, tiles_n, cps, splits;
  size_t partial_bytes;
};

inline Plan plan(const DevTensor& t, uint32_t m) {
  Plan p{};
  p.tiles_n = (t.rows + BN - 1) / BN;
  const uint32_t kt = (t.kp + BK - 1) / BK;
  const uint32_t nchunks = (kt + KC - 1) / KC;
  // Activation tiles of 32·fi rows; K split across workgroups until about
  // one workgroup per CU.
  // fit: the slice length grows until the grid is at most 256 workgroups
  // (one 8-wave workgroup per CU).
  auto shape = [&](int fi, uint32_t& tiles_m, uint32_t& cps, uint32_t& splits, bool fit) {
    tiles_m = (m + 32 * fi - 1) / (32 * fi);
    const uint32_t tiles = tiles_m * p.tiles_n;
    cps = std::max<uint32_t>(1u, (uint32_t)(((uint64_t)nchunks * tiles + 255) / 256));
    cps = std::min(cps, nchunks);
    splits = (nchunks + cps - 1) / cps;
    while (fit && tiles * splits > 256 && cps < nchunks) {
      ++cps;
      splits = (nchunks + cps - 1) / cps;
    }
    return tiles * splits;   // workgroups
  };
  p.fi = m <= 32 ? 1 : (m <= 64 ? 2 : 4);
  uint32_t tm, cps, sp;
  // Q8 at 65..128 rows: 64-row tiles (two per 128 rows, 8 waves per
  // workgroup) where 128-row tiles leave some of the CUs idle, with K slices
  // long enough that the grid fits one workgroup per CU.  Measured (whole
  // call, TFLOP/s, M = 128 / 96, 128-row vs 64-row tiles): 6144 -> 2048
  // 123 / 97 vs 142 / 111, 2048 -> 2048 59 / 49 vs 68 / 58, 2048 -> 6144
  // 116 vs 126 (two K slices; 110 in three, 288 workgroups); kept at 128
  // rows: 12288 -> 2048 (128-row tiles already fill the CUs) 191 / 155 vs
  // 182 / 144.
  const bool fi2 = t.kind == KIND_Q8 && p.fi == 4 && shape(4, tm, cps, sp, false) < 256 &&
                   shape(2, tm, cps, sp, true) <= 256;
  if (fi2) p.fi = 2;
  shape(p.fi, p.tiles_m, p.cps, p.splits, fi2);
  p.partial_bytes = p.splits > 1 ? ((size_t)p.splits * m * t.rows * 4 + 255) / 256 * 256 : 0;
  return p;
}

template <uint32_t KIND, int FI, int KW>
hipError_t launch(const DevTensor& t, const uint16_t* x, uint32_t m, uint32_t x_vec, void* y, bool y_bf16,
                  const Plan& p, float* partial, const int32_t* xe, hipStream_t s) {
  static_assert(lds_bytes<KIND, FI, KW>() <= 160 * 1024, "LDS budget");   // static arrays in the kernel
  hipLaunchKernelGGL((fused_kernel<KIND, FI, KW>), dim3(p.tiles_m * p.tiles_n, p.splits), dim3(256 * KW), 0, s,
                     t, x, m, x_vec, y, (uint32_t)y_bf16, partial, p.cps, p.tiles_m, xe);
  return hipGetLastError();
}

template <uint32_t KIND>
hipError_t launch_kind(const DevTensor& t, const uint16_t* x, uint32_t m, uint32_t x_vec, void* y, bool y_bf16,
                       const Plan& p, float* partial, const int32_t* xe, hipStream_t s) {
  if (p.fi == 1) return launch<KIND, 1, 2>(t, x, m, x_vec, y, y_bf16, p, partial, xe, s);
  if (p.fi == 2) return launch<KIND, 2, 2>(t, x, m, x_vec, y, y_bf16, p, partial, xe, s);
  // Q8 at 4 fragments holds a second accumulator set per block: one K way
  // keeps it within the registers of 2 waves per SIMD (measured equal speed).
  return launch<KIND, 4, KIND == KIND_Q8 ? 1 : 2>(t, x, m, x_vec, y, y_bf16, p, partial, xe, s);
}

}  // namespace fz

hipError_t launch_gemm_reduce(const float* partial, uint32_t splits, const float* inv, const int32_t* xe, uint32_t m,
                              uint32_t n, void* y, bool y_bf16, hipStream_t s);

bool gemm_fused_supported(const DevTensor& t, bool x_bf16) {
  return x_bf16 && (t.kind == KIND_G64 || t.kind == KIND_Q8);
}

// g64 multiplies f16 activations (row-scaled); Q8 the bf16 activations as they are.
bool gemm_fused_scales_x(const DevTensor& t) { return t.kind == KIND_G64; }

size_t gemm_fused_workspace_bytes(const DevTensor& t, uint32_t m) { return fz::plan(t, m).partial_bytes; }

hipError_t launch_gemm_fused(const DevTensor& t, const uint16_t* x, uint32_t m, void* y, bool y_bf16, void* ws,
                             size_t ws_bytes, const int32_t* xe, hipStream_t s) {
  const fz::Plan p = fz::plan(t, m);
  if (ws_bytes < p.partial_bytes) return hipErrorInvalidValue;
  float* partial = static_cast<float*>(ws);
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (t.cols % 8 == 0);
  hipError_t e;
  if (t.kind == KIND_G64)
    e = fz::launch_kind<KIND_G64>(t, x, m, x_vec, y, y_bf16, p, partial, xe, s);
  else if (t.kind == KIND_Q8)
    e = fz::launch_kind<KIND_Q8>(t, x, m, x_vec, y, y_bf16, p, partial, nullptr, s);
  else
    return hipErrorInvalidValue;
  if (e != hipSuccess || p.splits == 1) return e;
  return launch_gemm_reduce(partial, p.splits, nullptr, t.kind == KIND_G64 ? xe : nullptr, m, t.rows, y, y_bf16, s);
}

}  // namespace vxt

