// gemm_panel.hip -- prefill GEMM (batch_m > 8) in two phases on one stream.
//
// Reference behaviour: PackedTensor::gemm_cpu (llm_prefill.rs:156-255) decodes
// 32-row weight tiles to f32 with CodebookMatrix::decode_row and multiplies
// them densely.  The same split, laid out for CDNA4:
//
//   1. panel_kernel: every weight row is decoded bit-exactly (the values
//      decode_row / the Q8_0 and g64 rules produce, cb4 CSR residuals applied
//      in CSR order) and written once to an f16 panel in HBM, K-contiguous
//      rows padded to a multiple of 64 with zeros:
//        * g64: the f16 table entry itself (exact), one plane;
//        * Q8 and cb4: w * s = hi + lo * 2^-11 with hi = f16(w s),
//          lo = f16((w s - hi) * 2^11), where s = 2^e per row keeps the
//          row's largest magnitude in [2^14, 2^15) (no f16 overflow, lo out
//          of the subnormal range).  hi + lo carries 22 significant bits:
//          exact for Q8 (q * d has <= 18), within 2^-22 relative for cb4.
//   2. dense phase: Y = X * W^T on v_mfma_f32_32x32x16_f16 from LDS tiles,
//      fp32 accumulation -- the interleaved 128 x 128 kernel of
//      gemm_dense.hip for bf16 X from M = 256, dense_kernel below (64 x 64
//      tiles below M = 256, and for f32 X); lo products go to a second
//      accumulator folded in as acc + accl * 2^-11, then scaled by 1/s.
//      Activations get a
//      power-of-two scale per row too (xscale_kernel: the row's largest
//      magnitude in [2^14, 2^15)), undone in the epilogue, so X of any
//      magnitude converts to f16 without overflow: bf16 X exactly (8
//      significant bits) for elements within 2^28 of the row's largest; f32
//      X is split into hi + lo like the weights, with one more MFMA (lo * lo
//      dropped).
//      Small M*N grids split K across workgroups; reduce_kernel then adds the
//      partial sums in a fixed order (results do not depend on timing).
//      Only when a caller pins kGemmLibrary does the dense phase run on
//      hipBLASLt (library_dense below, gemm_blas.cpp), with reduce_kernel as
//      the 1/s + bf16 epilogue -- a comparison, never the automatic path.
//
// g64 weights with bf16 activations take the tile kernel of gemm_tile.hip
// (M > 64) or the fused kernel of gemm_fused.hip (M <= 64); Q8_0 with bf16
// activations takes the fused kernel up to M = 256 (launch_gemm chooses).
//
// The panel costs one pass over the packed weights plus one f16 (or 2 x f16)
// write; the fused alternative re-decodes every weight tile once per M tile
// and adds cb4 residuals from scattered activation reads per output.
#include <algorithm>

#include "common.hpp"

#pragma clang fp contract(off)

namespace vxt {

hipError_t launch_gemm_reduce(const float* partial, uint32_t splits, const float* inv, const int32_t* xe, uint32_t m,
                              uint32_t n, void* y, bool y_bf16, hipStream_t s);
hipError_t blas_gemm_f16_tn(const uint16_t* A, uint32_t lda, const uint16_t* B, uint32_t ldb, uint32_t M, uint32_t N,
                            uint32_t K, uint32_t batch, float alpha, float beta, float* D, hipStream_t s);
hipError_t launch_dense2(int wmode, const uint16_t* ah, const uint16_t* bh, const uint16_t* bl, const float* dsc,
                         const float* inv, uint32_t m, uint32_t n, uint32_t kp, void* y, bool y_bf16, float* partial,
                         uint32_t splits, uint32_t kt_per_split, const int32_t* xe, hipStream_t s);
hipError_t launch_dense3(int cfg, int wmode, const uint16_t* ah, const uint16_t* bh, const uint16_t* bl,
                         const float* dsc, const float* inv, uint32_t m, uint32_t n, uint32_t kp, void* y, bool y_bf16,
                         float* partial, uint32_t splits, uint32_t kt_per_split, const int32_t* xe, hipStream_t s);

namespace gp {

constexpr int BK = 64;
constexpr int LDK = BK + 8;   // padded LDS row (halves): conflict-light fragment reads
constexpr int THREADS = 256;
constexpr float kLoScale = 2048.0f;

// The lo half (v - hi) * 2^11 of a hi/lo split; 0 for Inf / NaN v, whose hi
// half carries it whole (Inf - Inf would turn an Inf product into NaN).
__device__ __forceinline__ float lo_part(float v, float hi) {
  return fabsf(v) <= 3.4028234663852886e38f ? (v - hi) * kLoScale : 0.0f;
}
constexpr float kLoInv = 1.0f / 2048.0f;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

struct Panel {
  uint16_t* hi;     // [N][kp] f16
  uint16_t* lo;     // [N][kp] f16 (hi/lo mode)
  float* inv;       // [N] 1 / s
  float* dsc;       // [N][kp/32] block scales (Q8 block mode)
  uint32_t kp;      // K rounded up to BK
  uint32_t tiled;   // hi / lo in 1 KB pieces (plane_off), else row-major
};

// How a panel represents the weights.
enum WMode : int {
  kWPlain = 0,    // f16 values (g64)
  kWHiLo = 1,     // w*s = hi + lo*2^-11 (cb4; Q8 with f32 activations)
  kWQBlock = 2,   // f16 int8 values + f32 scale per 32-column block (Q8, bf16 activations)
};

__host__ __device__ inline size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

// Element offset of (row, col) in an f16 plane of kp columns: row-major, or
// (tiled) in 1 KB pieces of 16 rows x 32 columns, piece (row / 16, col / 32)
// at element ((row / 16) * kp / 32 + col / 32) * 512 and row row % 16 at
// 32 (row % 16) inside it.  The large-tile dense kernel (gemm_dense3.hip)
// loads one whole piece per wave instruction; a tiled plane holds its rows
// rounded up to 16.  8 columns from a multiple of 8 stay contiguous.
__device__ __forceinline__ size_t plane_off(uint32_t row, uint32_t col, uint32_t kp, uint32_t tiled) {
  return tiled ? ((size_t)(row >> 4) * (kp >> 5) + (col >> 5)) * 512u + (row & 15u) * 32u + (col & 31u)
               : (size_t)row * kp + col;
}

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// s = 2^e with bound * s in [2^14, 2^15); 1 for zero or non-finite bounds.
__device__ __forceinline__ float row_scale(float bound) {
  if (!(bound > 0.0f) || !(bound < 3.0e38f)) return 1.0f;
  const int e = 14 - ilogbf(bound);
  return ldexpf(1.0f, e);
}

__device__ __forceinline__ void split_write(float w, float s, uint16_t* hi, uint16_t* lo, size_t i) {
  const float ws = w * s;                              // exact: s is a power of two
  const _Float16 h = (_Float16)ws;
  hi[i] = __builtin_bit_cast(uint16_t, h);
  lo[i] = __builtin_bit_cast(uint16_t, (_Float16)lo_part(ws, (float)h));
}

// ---- phase 1: activations and panel -----------------------------------------

// Activation conversion, run by the first `blocks` workgroups of the panel
// launch, one activation row per workgroup at a time: the row's largest
// finite magnitude first (its exponent xe[m] puts it in [2^14, 2^15): 0 for
// a row with none; Inf / NaN entries pass as they are), then X[m] * 2^xe[m]
// -> A [M][kp] f16,
// zero for k >= K; f32 X also gets the lo plane (x - hi) * 2^11.  One thread
// per 8 columns.
struct XConv {
  const void* x;
  uint16_t* ah;
  uint16_t* al;
  int32_t* xe;   // per-row exponent, written here
  uint32_t m, cols, x_bf16, x_vec, blocks;
  uint32_t tiled;   // A (and its lo plane) in the panel's piece layout (plane_off)
};

// 8 activations at column k of row m (zero past K).
template <bool XBF16>
__device__ __forceinline__ void load8(const void* __restrict__ x, uint32_t K, uint32_t x_vec, uint32_t m, uint32_t k,
                                      float (&v)[8]) {
  if (x_vec && k + 8 <= K) {
    if constexpr (XBF16) {
      const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + (size_t)m * K + k);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __uint_as_float(w[j] << 16);
        v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    } else {
      const float4* f = reinterpret_cast<const float4*>(static_cast<const float*>(x) + (size_t)m * K + k);
      const float4 f0 = f[0], f1 = f[1];
      v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
      v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float f = 0.0f;
      if (k + j < K) {
        if constexpr (XBF16)
          f = bf16_to_f32(static_cast<const uint16_t*>(x)[(size_t)m * K + k + j]);
        else
          f = static_cast<const float*>(x)[(size_t)m * K + k + j];
      }
      v[j] = f;
    }
  }
}

// Exponent that puts `b` (a row's largest finite magnitude) in [2^14, 2^15),
// or 0 when the row has no non-zero finite entry.
__device__ __forceinline__ int row_exponent(float b) {
  return (b > 0.0f && b <= 3.4028234663852886e38f) ? 14 - ilogbf(b) : 0;
}

// |v| of a finite v, 0 for Inf / NaN: a row's exponent comes from its largest
// finite magnitude, and its Inf / NaN entries stay Inf / NaN when scaled and
// converted, so they reach the products as gemm_cpu sees them.
__device__ __forceinline__ float finite_abs(float v) {
  const float a = fabsf(v);
  return a <= 3.4028234663852886e38f ? a : 0.0f;
}

template <bool XBF16>
__device__ __forceinline__ void xconv_blocks(const XConv& c, uint32_t kp) {
  __shared__ float s_max[THREADS / 64];
  const void* __restrict__ x = c.x;
  uint16_t* __restrict__ ah = c.ah;
  uint16_t* __restrict__ al = c.al;
  const uint32_t K = c.cols, x_vec = c.x_vec;
  for (uint32_t m = blockIdx.x; m < c.m; m += c.blocks) {
    float mx = 0.0f;
    for (uint32_t k = threadIdx.x * 8; k < K; k += THREADS * 8) {
      float v[8];
      load8<XBF16>(x, K, x_vec, m, k, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, finite_abs(v[j]));
    }
    mx = lane_reduce<64, true>(mx);
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = mx;
    __syncthreads();
    float b = s_max[0];
#pragma unroll
    for (int w = 1; w < THREADS / 64; ++w) b = fmaxf(b, s_max[w]);
    const int e = row_exponent(b);
    if (threadIdx.x == 0) c.xe[m] = e;
    __syncthreads();   // s_max is reused by the next row
    for (uint32_t k = threadIdx.x * 8; k < kp; k += THREADS * 8) {
      float v[8];
      load8<XBF16>(x, K, x_vec, m, k, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = ldexpf(v[j], e);   // exact (a power of two)
      uint32_t h[4], l[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const _Float16 h0 = (_Float16)v[2 * j], h1 = (_Float16)v[2 * j + 1];
        h[j] = pack_h2(h0, h1);
        if constexpr (!XBF16)
          l[j] = pack_h2((_Float16)lo_part(v[2 * j], (float)h0), (_Float16)lo_part(v[2 * j + 1], (float)h1));
      }
      const size_t o = plane_off(m, k, kp, c.tiled);
      *reinterpret_cast<uint4*>(ah + o) = make_uint4(h[0], h[1], h[2], h[3]);
      if constexpr (!XBF16) *reinterpret_cast<uint4*>(al + o) = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }
}

// bf16 rows of 16-byte aligned pieces (x_vec) up to NPT * THREADS * 8
// columns: each row is read once into registers (NPT pieces of 8 columns per
// thread, all loads in flight together, unconditional from clamped
// addresses), its maximum combined through LDS, then converted from the
// registers.  xconv_blocks reads every row twice; this halves the activation
// reads and takes one memory round trip per row off the launch's tail.
template <int NPT>
__device__ __forceinline__ void xconv_rows_bf16(const XConv& c, uint32_t kp) {
  __shared__ float s_max[THREADS / 64];
  const uint32_t K = c.cols, np = K / 8, npk = kp / 8, tid = threadIdx.x;
  for (uint32_t m = blockIdx.x; m < c.m; m += c.blocks) {
    const uint4* row = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(c.x) + (size_t)m * K);
    uint4 u[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) u[i] = row[std::min(i * THREADS + tid, np - 1)];
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      if (i * THREADS + tid >= np) continue;
      const uint32_t w[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        mx = fmaxf(mx, finite_abs(__uint_as_float(w[j] << 16)));
        mx = fmaxf(mx, finite_abs(__uint_as_float(w[j] & 0xffff0000u)));
      }
    }
    mx = lane_reduce<64, true>(mx);
    if ((tid & 63) == 0) s_max[tid >> 6] = mx;
    __syncthreads();
    float b = s_max[0];
#pragma unroll
    for (int w = 1; w < THREADS / 64; ++w) b = fmaxf(b, s_max[w]);
    const int e = row_exponent(b);
    if (tid == 0) c.xe[m] = e;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const uint32_t pc = i * THREADS + tid;
      if (pc >= npk) continue;
      const bool in = pc < np;   // pieces past K are zero
      const uint32_t w[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = in ? ldexpf(__uint_as_float(w[j] << 16), e) : 0.0f;   // exact (a power of two)
        const float bb = in ? ldexpf(__uint_as_float(w[j] & 0xffff0000u), e) : 0.0f;
        h[j] = pack_h2((_Float16)a, (_Float16)bb);
      }
      *reinterpret_cast<uint4*>(c.ah + plane_off(m, pc * 8, kp, c.tiled)) = make_uint4(h[0], h[1], h[2], h[3]);
    }
    __syncthreads();   // s_max is reused by the next row
  }
}

__device__ __forceinline__ float wave_max(float v) { return lane_reduce<64, true>(v); }
__device__ __forceinline__ float wave_add(float v) { return lane_reduce<64>(v); }

// Per activation row m: xe[m] such that the row's largest finite magnitude
// times 2^xe[m] lies in [2^14, 2^15), so the f16 operands neither overflow
// nor (for bf16 X) round; 0 for a row with no non-zero finite entry.  Inf and
// NaN entries stay Inf and NaN and propagate as in the reference's f32
// arithmetic.  One wave per row.
template <bool XBF16>
__global__ __launch_bounds__(THREADS) void xscale_kernel(const void* __restrict__ x, uint32_t M, uint32_t K,
                                                         uint32_t x_vec, int32_t* __restrict__ xe) {
  const uint32_t m = blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (m >= M) return;
  float mx = 0.0f;
  // four 8-column pieces per lane in flight before any is used (a round
  // covers 2048 columns, one round trip); the loads are unconditional from
  // clamped addresses and columns past K are masked after them
  if (x_vec) {   // uniform: 16-byte rows pieces (K % 8 == 0 for bf16, % 4 for f32)
    constexpr uint32_t EPP = XBF16 ? 8 : 4;   // elements per 16-byte piece
    const uint32_t np = K / EPP;
    const uint4* row = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + (size_t)m * K * (XBF16 ? 2 : 4));
    for (uint32_t p0 = 0; p0 < np; p0 += 4 * 64) {
      uint4 u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] = row[std::min(p0 + i * 64 + lane, np - 1)];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (p0 + i * 64 + lane >= np) continue;
        const uint32_t w[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (XBF16) {
            mx = fmaxf(mx, finite_abs(__uint_as_float(w[j] << 16)));
            mx = fmaxf(mx, finite_abs(__uint_as_float(w[j] & 0xffff0000u)));
          } else {
            mx = fmaxf(mx, finite_abs(__uint_as_float(w[j])));
          }
        }
      }
    }
  } else {
    for (uint32_t k = lane; k < K; k += 64) {
      const float v = XBF16 ? bf16_to_f32(static_cast<const uint16_t*>(x)[(size_t)m * K + k])
                            : static_cast<const float*>(x)[(size_t)m * K + k];
      mx = fmaxf(mx, finite_abs(v));
    }
  }
  mx = lane_reduce<64, true>(mx);
  if (lane == 0) xe[m] = row_exponent(mx);
}

// 8 consecutive f32 weights -> hi (and lo) f16 pieces at element offset c.
template <bool SPLIT>
__device__ __forceinline__ void store8(const float (&w)[8], float s, uint16_t* hi, uint16_t* lo, size_t c) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = w[2 * j] * s, b = w[2 * j + 1] * s;   // exact: s is a power of two
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    h[j] = pack_h2(ha, hb);
    if constexpr (SPLIT) l[j] = pack_h2((_Float16)lo_part(a, (float)ha), (_Float16)lo_part(b, (float)hb));
  }
  *reinterpret_cast<uint4*>(hi + c) = make_uint4(h[0], h[1], h[2], h[3]);
  if constexpr (SPLIT) *reinterpret_cast<uint4*>(lo + c) = make_uint4(l[0], l[1], l[2], l[3]);
}

// One wave per (weight row, 2048-column segment).  Lane l decodes the four
// 8-column pieces seg + 512 i + 8 l (i = 0..3), so each of its loads and each
// 16-byte store instruction covers a contiguous stretch of the row across the
// wave (1 KB of f16 per store).  Rows that need a power-of-two scale (hi/lo
// modes) derive it in every segment's wave from the row's scales and
// residuals, requested together with the segment's own weights, so no wave
// walks a row serially.  cb4 residuals are applied by the wave owning the
// column's segment, after its dense stores, in CSR order.
template <uint32_t KIND>
__global__ __launch_bounds__(THREADS) void panel_kernel(DevTensor t, Panel p, uint32_t qblock, uint32_t nseg, XConv xc) {
  constexpr uint32_t kTab = 32;   // g64 table bytes per 64-column group
  __shared__ __attribute__((aligned(64))) uint32_t s_tab[KIND == KIND_G64 ? 4 * 32 * kTab / 4 : 1];
  __shared__ __attribute__((aligned(64))) float s_cent[48];
  if (blockIdx.x < xc.blocks) {   // uniform per workgroup: the activation conversion's share
    const uint32_t npt = (p.kp / 8 + THREADS - 1) / THREADS;   // 8-column pieces per thread
    if (xc.x_bf16 && xc.x_vec && npt <= 1)
      xconv_rows_bf16<1>(xc, p.kp);
    else if (xc.x_bf16 && xc.x_vec && npt <= 2)
      xconv_rows_bf16<2>(xc, p.kp);
    else if (xc.x_bf16 && xc.x_vec && npt <= 4)
      xconv_rows_bf16<4>(xc, p.kp);
    else if (xc.x_bf16)
      xconv_blocks<true>(xc, p.kp);
    else
      xconv_blocks<false>(xc, p.kp);
    return;
  }
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t N = t.rows, K = t.cols, kp = t.kp, KP = p.kp;
  if constexpr (KIND == KIND_CB4) {
    if (threadIdx.x < 48) s_cent[threadIdx.x] = t.cent[threadIdx.x];
    __syncthreads();
  }
  const uint32_t unit = (blockIdx.x - xc.blocks) * 4 + wave;
  if (unit >= N * nseg) return;
  const uint32_t n = unit / nseg, seg = (unit % nseg) * (64 * 32);
  // Piece i starts at column c0 + 512 i; KP % 64 == 0, so a piece is wholly
  // inside or outside the panel row.
  const uint32_t c0 = seg + 8 * lane;
  uint16_t* hi = p.hi;
  uint16_t* lo = p.lo;
  auto at = [&](uint32_t c) { return plane_off(n, c, KP, p.tiled); };   // column c of row n
  float s = 1.0f;
  if constexpr (KIND == KIND_G64) {
    // KP <= kp here (kp is a multiple of 64 and at least K).  The segment's
    // 32 tables go to the wave's LDS slot, lane l holding half of table l / 2;
    // groups past the row's last are clamped (their columns are >= K).
    const uint32_t ng = kp / 64;
    const uint32_t g = std::min(seg / 64 + lane / 2, ng - 1);
    const uint4 lt = *reinterpret_cast<const uint4*>(t.p1 + ((size_t)n * ng + g) * 16 + (lane & 1) * 8);
    const uint8_t* qr = static_cast<const uint8_t*>(t.p0) + (size_t)n * (kp / 2);
    uint32_t wd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = c0 + 512 * i;
      wd[i] = *reinterpret_cast<const uint32_t*>(qr + (c < KP ? c : 0) / 2);
    }
    char* slot = reinterpret_cast<char*>(s_tab) + wave * 32 * kTab;
    *reinterpret_cast<uint4*>(slot + lane * 16) = lt;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = c0 + 512 * i;
      if (c >= KP) continue;
      const uint16_t* tab = reinterpret_cast<const uint16_t*>(slot + (8 * i + lane / 8) * kTab);
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t e0 = c + 2 * j < K ? tab[(wd[i] >> (8 * j)) & 0xfu] : 0u;
        const uint32_t e1 = c + 2 * j + 1 < K ? tab[(wd[i] >> (8 * j + 4)) & 0xfu] : 0u;
        h[j] = e0 | (e1 << 16);
      }
      *reinterpret_cast<uint4*>(hi + at(c)) = make_uint4(h[0], h[1], h[2], h[3]);
    }
  } else if constexpr (KIND == KIND_Q8 || KIND == KIND_Q40) {
    // kp may be 32 short of KP: pieces past kp read the row's last 8 bytes
    // (their columns are >= K and come out zero).
    const uint16_t* dp = t.p1 + (size_t)n * (kp / 32);
    uint2 q[4];
    if constexpr (KIND == KIND_Q8) {
      const int8_t* qr = static_cast<const int8_t*>(t.p0) + (size_t)n * kp;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t c = c0 + 512 * i;
        q[i] = *reinterpret_cast<const uint2*>(qr + (c < kp ? c : kp - 8));
      }
    } else {
      // Q4_0: columns c .. c + 7 of a block are the low (c % 32 < 16) or high
      // nibbles of bytes c % 16 .. + 7; each is widened to the int8 q - 8
      // (q4_0.rs:89-93), so the rest is the Q8 decode.
      const uint8_t* qr = static_cast<const uint8_t*>(t.p0) + (size_t)n * (kp / 2);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t c = c0 + 512 * i, cc = c < kp ? c : kp - 8;
        const uint2 raw = *reinterpret_cast<const uint2*>(qr + (cc / 32) * 16 + cc % 16);
        const uint32_t sh = (cc % 32) < 16 ? 0u : 4u;
        q[i].x = ((((raw.x >> sh) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        q[i].y = ((((raw.y >> sh) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
      }
    }
    float d[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (qblock) {   // block scales as f32; blocks past the weights' own are zero
      const uint32_t b0 = seg / 32 + lane;
      if (b0 < KP / 32)
        p.dsc[(size_t)n * (KP / 32) + b0] = b0 < kp / 32 ? f16_to_f32_exact(dp[b0]) : 0.0f;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t c = c0 + 512 * i;
        d[i] = f16_to_f32_exact(dp[(c < kp ? c : kp - 8) / 32]);
      }
      float dm = 0.0f;
      for (uint32_t g = lane; g < kp / 32; g += 64) dm = fmaxf(dm, fabsf(f16_to_f32_exact(dp[g])));
      s = row_scale((KIND == KIND_Q8 ? 127.0f : 8.0f) * wave_max(dm));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = c0 + 512 * i;
      if (c >= KP) continue;
      const uint32_t wd[2] = {q[i].x, q[i].y};
      float w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)   // gguf.rs:223-229
        w[j] = c + j < K ? (float)(int8_t)((wd[j >> 2] >> ((j & 3) * 8)) & 0xffu) * d[i] : 0.0f;
      if (qblock)   // the int8 value itself, exact in f16
        store8<false>(w, 1.0f, hi, lo, at(c));
      else
        store8<true>(w, s, hi, lo, at(c));
    }
  } else {
    // KP <= kp here (kp is a multiple of 128 and at least K).
    const uint32_t* pw = static_cast<const uint32_t*>(t.p0) + (size_t)n * (kp / 8);
    const uint16_t* sp = t.p1 + (size_t)n * (kp / 128);
    uint32_t wd[4];
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = c0 + 512 * i, cc = c < KP ? c : 0;
      wd[i] = pw[cc / 8];
      sc[i] = f16_to_f32_exact(sp[cc / 128]);
    }
    const uint32_t os = t.row_ptr[n], oe = t.row_ptr[n + 1];
    const float* cent = s_cent + 16u * cent_table(t, n);
    float sm = 0.0f, rs = 0.0f, cm = 0.0f;
    for (uint32_t g = lane; g < kp / 128; g += 64) sm = fmaxf(sm, fabsf(f16_to_f32_exact(sp[g])));
    for (uint32_t o = os + lane; o < oe; o += 64) rs += fabsf(f16_to_f32_exact(t.outliers[o] >> 16));
#pragma unroll
    for (int i = 0; i < 16; ++i) cm = fmaxf(cm, fabsf(cent[i]));
    s = row_scale(wave_max(sm) * cm + wave_add(rs));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = c0 + 512 * i;
      if (c >= KP) continue;
      float w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = c + j < K ? sc[i] * cent[(wd[i] >> (4 * j)) & 0xfu] : 0.0f;
      store8<true>(w, s, hi, lo, at(c));
    }
    // CSR residuals of this segment's columns (codebook.rs:316-333): the lane
    // holding a column's first entry rebuilds the column from sc * cent[q] and
    // adds its residuals in CSR order, over the halves stored above.  A row
    // whose columns strictly increase (what the reference's encoders emit,
    // codebook.rs:228-250 and cb4_opt.rs) has one entry per column, proved by
    // one parallel comparison with the previous entry; only other rows scan
    // the row for earlier and later entries of the same column.
    if (oe > os) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");   // the dense stores above land first
      const uint32_t c_end = seg + 64 * 32;
      bool inc = true;
      for (uint32_t i = os + 1 + lane; i < oe; i += 64)
        inc = inc && (t.outliers[i] & 0xffffu) > (t.outliers[i - 1] & 0xffffu);
      const bool unique = __all(inc);
      for (uint32_t i = os + lane; i < oe; i += 64) {
        const uint32_t pk0 = t.outliers[i];
        const uint32_t c = pk0 & 0xffffu;
        bool first = c < K && c >= seg && c < c_end;
        if (!unique)
          for (uint32_t j = os; j < i && first; ++j) first = (t.outliers[j] & 0xffffu) != c;
        if (!first) continue;
        const uint32_t cw = static_cast<const uint32_t*>(t.p0)[(size_t)n * (kp / 8) + c / 8];
        float v = f16_to_f32_exact(sp[c / 128]) * cent[(cw >> ((c % 8) * 4)) & 0xfu];
        if (unique) {
          v += f16_to_f32_exact(pk0 >> 16);
        } else {
          for (uint32_t j = i; j < oe; ++j) {
            const uint32_t pk = t.outliers[j];
            if ((pk & 0xffffu) == c) v += f16_to_f32_exact(pk >> 16);
          }
        }
        split_write(v, s, hi, lo, at(c));
      }
    }
  }
  if (lane == 0 && seg == 0) p.inv[n] = 1.0f / s;
}

// ---- phase 2: dense GEMM -----------------------------------------------------

// 16-byte pieces of one operand tile: piece p of the thread covers row
// r0 + p/8 (clamped to the last row: rows past the end are never stored),
// columns kb + (p%8)*8 .. +8.
template <int NP, bool LO>
__device__ __forceinline__ void fetch_tile(const uint16_t* __restrict__ hi, const uint16_t* __restrict__ lo,
                                           uint32_t r0, uint32_t rows, uint32_t kp, uint32_t kb, u32x4 (&h)[NP],
                                           u32x4 (&l)[LO ? NP : 1]) {
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const uint32_t piece = threadIdx.x + THREADS * i;
    const uint32_t r = std::min(r0 + piece / 8, rows - 1);
    const size_t off = (size_t)r * kp + kb + (piece % 8) * 8;
    h[i] = *reinterpret_cast<const u32x4*>(hi + off);
    if constexpr (LO) l[i] = *reinterpret_cast<const u32x4*>(lo + off);
  }
}

template <int NP, bool LO>
__device__ __forceinline__ void commit_tile(_Float16* sh, _Float16* sl, uint32_t st, uint32_t stage_halves,
                                            const u32x4 (&h)[NP], const u32x4 (&l)[LO ? NP : 1]) {
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const uint32_t piece = threadIdx.x + THREADS * i;
    const uint32_t o = st * stage_halves + (piece / 8) * LDK + (piece % 8) * 8;
    *reinterpret_cast<u32x4*>(sh + o) = h[i];
    if constexpr (LO) *reinterpret_cast<u32x4*>(sl + o) = l[i];
  }
}

// Block tile BM x BN, 2 x 2 waves of (BM/2) x (BN/2) with 32x32x16 f16 MFMA
// fragments.  Operands are f16 rows of length kp (A: activations, B: panel);
// LDS holds two stages, so one barrier per K tile: tile k+1 is fetched into
// registers while tile k is multiplied, then written to the other stage.
// blockIdx.y selects a K range; with gridDim.y > 1 the block writes fp32
// partial sums (hi + lo combined, unscaled) to `partial` [z][M][N].
template <int BM, int BN, int WMODE, bool SPLIT_A>
__global__ __launch_bounds__(THREADS) void dense_kernel(Panel p, const uint16_t* __restrict__ ah,
                                                        const uint16_t* __restrict__ al, uint32_t M, uint32_t N,
                                                        void* __restrict__ y, uint32_t y_bf16,
                                                        float* __restrict__ partial, uint32_t kt_per_split,
                                                        uint32_t tiles_m, const int32_t* __restrict__ xe) {
  constexpr bool SPLIT = WMODE == kWHiLo;
  constexpr bool QBLK = WMODE == kWQBlock;
  static_assert(!(QBLK && SPLIT_A), "block-scaled weights take f16 activations");
  constexpr int FI = BM / 64, FJ = BN / 64;
  constexpr int PA = BM * 8 / THREADS, PB = BN * 8 / THREADS;   // 16-byte pieces per thread
  constexpr int SA = BM * LDK, SB = BN * LDK;                   // halves per stage
  extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
  _Float16* sA = smem;
  _Float16* sB = sA + 2 * SA;
  _Float16* sAl = sB + 2 * SB;
  _Float16* sBl = sAl + (SPLIT_A ? 2 * SA : 0);
  // Q8 block mode: scales of the tile's two 32-column blocks, [stage][row][2]
  float* sD = reinterpret_cast<float*>(sBl + (SPLIT ? 2 * SB : 0));
  const uint32_t nblk = p.kp / 32;

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  // Tile order: blocks b, b+8, b+16, ... run on one XCD (one L2), so each XCD
  // gets a contiguous range of tiles, walked in groups of 8 tile rows: the
  // blocks an XCD runs together share A rows and B columns in its L2.
  // (10 % at M = 2048 over row-major order with round-robin XCDs.)
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
  const uint32_t kp = p.kp, ktiles = kp / BK;
  const uint32_t kt0 = blockIdx.y * kt_per_split;
  const uint32_t kt1 = std::min(ktiles, kt0 + kt_per_split);

  float16v acc[FI][FJ], accl[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
        accl[i][j][r] = 0.0f;
      }

  u32x4 ra[PA], ral[SPLIT_A ? PA : 1], rb[PB], rbl[SPLIT ? PB : 1];
  float rd = 0.0f;   // Q8 block mode: this thread's block scale (row tid/2, block tid%2)
  const uint32_t drow = std::min(n0 + (tid >> 1), N - 1);

  if (kt0 < kt1) {
    fetch_tile<PA, SPLIT_A>(ah, al, m0, M, kp, kt0 * BK, ra, ral);
    fetch_tile<PB, SPLIT>(p.hi, p.lo, n0, N, kp, kt0 * BK, rb, rbl);
    if constexpr (QBLK) {
      if (tid < 2 * BN) rd = p.dsc[(size_t)drow * nblk + kt0 * 2 + (tid & 1)];
    }
    commit_tile<PA, SPLIT_A>(sA, sAl, 0, SA, ra, ral);
    commit_tile<PB, SPLIT>(sB, sBl, 0, SB, rb, rbl);
    if constexpr (QBLK) {
      if (tid < 2 * BN) sD[tid] = rd;
    }
  }
  __syncthreads();
  for (uint32_t kt = kt0; kt < kt1; ++kt) {
    const uint32_t st = (kt - kt0) & 1;
    if (kt + 1 < kt1) {
      fetch_tile<PA, SPLIT_A>(ah, al, m0, M, kp, (kt + 1) * BK, ra, ral);
      fetch_tile<PB, SPLIT>(p.hi, p.lo, n0, N, kp, (kt + 1) * BK, rb, rbl);
      if constexpr (QBLK) {
        if (tid < 2 * BN) rd = p.dsc[(size_t)drow * nblk + (kt + 1) * 2 + (tid & 1)];
      }
    }
    const _Float16* a_st = sA + st * SA;
    const _Float16* b_st = sB + st * SB;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      half8 af[FI], afl[SPLIT_A ? FI : 1], bf[FJ], bfl[SPLIT ? FJ : 1];
      const uint32_t kofs = ks * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < FI; ++i) {
        const uint32_t ar = (wm * (BM / 2) + i * 32 + (lane & 31)) * LDK + kofs;
        af[i] = *reinterpret_cast<const half8*>(a_st + ar);
        if constexpr (SPLIT_A) afl[i] = *reinterpret_cast<const half8*>(sAl + st * SA + ar);
      }
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        const uint32_t br = (wn * (BN / 2) + j * 32 + (lane & 31)) * LDK + kofs;
        bf[j] = *reinterpret_cast<const half8*>(b_st + br);
        if constexpr (SPLIT) bfl[j] = *reinterpret_cast<const half8*>(sBl + st * SB + br);
      }
      if constexpr (QBLK) {
        // one 32-column block = two 16-deep MFMAs into a fresh fragment, then
        // acc += d[n, block] * fragment (the lane's column n is fixed)
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
          for (int j = 0; j < FJ; ++j)
            accl[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], (ks & 1) ? accl[i][j] : float16v{},
                                                                0, 0, 0);
        if (ks & 1) {
#pragma unroll
          for (int j = 0; j < FJ; ++j) {
            const float d = sD[st * 2 * BN + (wn * (BN / 2) + j * 32 + (lane & 31)) * 2 + (ks >> 1)];
#pragma unroll
            for (int i = 0; i < FI; ++i)
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(d, accl[i][j][r], acc[i][j][r]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
          for (int j = 0; j < FJ; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            if constexpr (SPLIT)
              accl[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bfl[j], accl[i][j], 0, 0, 0);
            if constexpr (SPLIT_A)   // lo * lo is below 2^-22 relative and dropped
              accl[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bf[j], accl[i][j], 0, 0, 0);
          }
      }
    }
    if (kt + 1 < kt1) {
      commit_tile<PA, SPLIT_A>(sA, sAl, st ^ 1u, SA, ra, ral);
      commit_tile<PB, SPLIT>(sB, sBl, st ^ 1u, SB, rb, rbl);
      if constexpr (QBLK) {
        if (tid < 2 * BN) sD[(st ^ 1u) * 2 * BN + tid] = rd;
      }
    }
    __syncthreads();
  }

  // Lane owns column n = n0 + wn*(BN/2) + j*32 + lane%32 of fragment (i, j),
  // rows m = m0 + wm*(BM/2) + i*32 + (lane/32)*4 + 8*(r/4) + r%4.
  const bool to_partial = gridDim.y > 1;
#pragma unroll
  for (int j = 0; j < FJ; ++j) {
    const uint32_t n = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
    if (n >= N) continue;
    const float inv = p.inv[n];
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t m = m0 + wm * (BM / 2) + i * 32 + (lane >> 5) * 4 + 8 * (r >> 2) + (r & 3);
        if (m >= M) continue;
        float v = acc[i][j][r];
        if constexpr (SPLIT || SPLIT_A) v = hilo_combine(v, accl[i][j][r]);   // not in block mode
        if (to_partial) {
          partial[((size_t)blockIdx.y * M + m) * N + n] = v;
        } else {
          v = ldexpf(v * inv, -xe[m]);
          if (y_bf16)
            static_cast<uint16_t*>(y)[(size_t)m * N + n] = f32_to_bf16(v);
          else
            static_cast<float*>(y)[(size_t)m * N + n] = v;
        }
      }
  }
}

// Y[m, n] = (sum_z partial[z, m, n], z ascending) / s[n] * 2^-xe[m] (no
// weight scaling when inv is null, no activation scaling when xe is null);
// four outputs per thread when N % 4 == 0.
// sum_z p[z * stride], z = 0 .. splits-1 added in ascending order, with up to
// 8 loads in flight: the loads of a group of 8 slices (the last group's past
// `splits` clamped to a valid slice and not added) are issued before any of
// them is added, so a thread waits for one memory latency per group rather
// than one per slice.
template <typename V>
__device__ __forceinline__ V sum_slices(const V* __restrict__ p, size_t stride, uint32_t splits) {
  V v{};
  for (uint32_t z = 0; z < splits; z += 8) {
    V a[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) a[j] = p[(size_t)std::min(z + j, splits - 1) * stride];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j)
      if (z + j < splits) v = v + a[j];
  }
  return v;
}

__device__ __forceinline__ float4 operator+(const float4& a, const float4& b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__global__ __launch_bounds__(THREADS) void reduce_kernel(const float* __restrict__ partial, uint32_t splits,
                                                         const float* __restrict__ inv,
                                                         const int32_t* __restrict__ xe, uint32_t M, uint32_t N,
                                                         void* __restrict__ y, uint32_t y_bf16) {
  const size_t total = (size_t)M * N;
  if (N % 4u == 0u) {
    const size_t i = ((size_t)blockIdx.x * THREADS + threadIdx.x) * 4;
    if (i >= total) return;
    float4 v = sum_slices(reinterpret_cast<const float4*>(partial + i), total / 4, splits);
    if (inv) {
      const float4 iv = *reinterpret_cast<const float4*>(inv + i % N);
      v.x *= iv.x; v.y *= iv.y; v.z *= iv.z; v.w *= iv.w;
    }
    if (xe) {   // the four outputs share a row (N % 4 == 0)
      const int e = -xe[i / N];
      v.x = ldexpf(v.x, e); v.y = ldexpf(v.y, e); v.z = ldexpf(v.z, e); v.w = ldexpf(v.w, e);
    }
    if (y_bf16) {
      const uint32_t lo = f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16);
      const uint32_t hi = f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + i) = make_uint2(lo, hi);
    } else {
      *reinterpret_cast<float4*>(static_cast<float*>(y) + i) = v;
    }
    return;
  }
  const size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x;
  if (i >= total) return;
  float v = sum_slices(partial + i, total, splits);
  if (inv) v *= inv[i % N];
  if (xe) v = ldexpf(v, -xe[i / N]);
  if (y_bf16)
    static_cast<uint16_t*>(y)[i] = f32_to_bf16(v);
  else
    static_cast<float*>(y)[i] = v;
}

// ---- planning ------------------------------------------------------------------

struct Plan {
  int bm, bn, wmode;
  bool lib;   // dense phase on the vendor library (gemm_blas.cpp)
  uint32_t kp, splits, kt_per_split;
  uint32_t lib_splits;   // K slices of the library call (one strided batch)
  int d3cfg;             // >= 0: the dense phase on dense3_kernel (gemm_dense3.hip) in this shape (launch_dense3)
  int d3mode;            // its weight mode (0 plain, 1 hi/lo, 2 Q8 block)
  size_t panel_plane, dsc_bytes, panel_bytes, a_plane, a_bytes, partial_bytes;
};

inline Plan plan(const DevTensor& t, uint32_t m, bool x_bf16, bool lib) {
  Plan pl{};
  pl.lib = lib;
  // The library multiplies plain f16 operands: Q8 then takes the hi/lo panel
  // (exact for q * d) instead of int8 values with block scales.
  pl.wmode = t.kind == KIND_G64 ? kWPlain
                                : ((t.kind == KIND_Q8 || t.kind == KIND_Q40) && x_bf16 && !lib ? kWQBlock : kWHiLo);
  pl.kp = (t.cols + BK - 1) / BK * BK;
  const uint32_t ktiles = pl.kp / BK;
  pl.bm = m >= 256 ? 128 : 64;
  pl.bn = pl.bm;
  const uint32_t tiles = ((m + pl.bm - 1) / pl.bm) * ((t.rows + pl.bn - 1) / pl.bn);
  // Split K until the grid covers the 256 CUs (>= 4 K tiles per split), and
  // on to two blocks per CU while the K ranges stay long (>= 16 K tiles):
  // measured, the partial sums cost less than a half-empty second round.
  uint32_t splits = 1;
  while (tiles * splits < 256 && ktiles / (splits * 2) >= 4) splits *= 2;
  while (tiles * splits < 512 && ktiles / (splits * 2) >= 16) splits *= 2;
  pl.kt_per_split = (ktiles + splits - 1) / splits;
  pl.splits = (ktiles + pl.kt_per_split - 1) / pl.kt_per_split;
  // bf16 activations from 96 output tiles of 128 x 128: the large-tile
  // kernel (gemm_dense3.hip) on the piece-layout planes.  Wave tile and K
  // slices as measured best (whole call, graph-timed, TFLOP/s; lab sweeps of
  // every tile and 1-4 slices, K x N = 2048 x 6144 / 6144 x 2048):
  //   * plain (g64): 256 x 192 from 192 such tiles (M = 1536: 640 vs 580 /
  //     591 for 256 x 128 / 128 x 128; M = 2048: 781 vs 697 / 705), else
  //     256 x 128 from 256 tiles (M = 4096 x 6144 -> 2048: 858 vs 815), else
  //     128 x 128 (M = 768: 457; M = 2048 x 6144 -> 2048: 675 vs 600 for
  //     256 x 128);
  //   * Q8 block and hi/lo (cb4) panels: waves of 2 x 2 fragments, two per
  //     SIMD (one wave's scale FMAs beside the other's MFMAs), as 256 x 128
  //     tiles of 8 waves where those number 192-256 or >= 512 (Q8 / cb4
  //     M = 1024 x 2048 -> 6144: 429 / 354 vs 404 / 338; M = 4096: 683 / 529
  //     and 654 / 529 vs 594 / 520 and 568 / 511), else 128 x 128 tiles of 4
  //     waves, two workgroups per CU (M = 2048 x 2048 -> 6144, 384 of the
  //     larger tiles: cb4 456 vs 429; fewer than 192: Q8 M = 2048 x 6144 ->
  //     2048 502 vs 391);
  //   * K slices: 128 x 128 tiles take two below 192 tiles and one from 192
  //     (g64 M = 2048 x 6144 -> 2048, 256 tiles: 675 vs 606 in two; Q8 /
  //     cb4 M = 1024 x 6144 -> 2048, 128 tiles: 363 / 324 vs 292 / 296 in
  //     one and 313 / 288 on dense2_kernel); the 256-row tiles split while
  //     the grid stays within one workgroup per CU and a slice keeps >= 8
  //     K tiles (cb4 M = 2048 x 6144 -> 2048 on 256 x 128: 411 vs 372).
  // Below 96 tiles dense2_kernel: at Q8 / cb4 M = 512 x 6144 -> 2048 (64
  // tiles) the slices the large-tile grid needs cost as much as they give
  // (258 / 221 vs 259 / 227 in four).
  pl.d3cfg = -1;
  pl.d3mode = 0;
  const uint32_t t128 = ((m + 127) / 128) * ((t.rows + 127) / 128);
  // The large-tile kernel reads each plane through a buffer resource of at
  // most 2^31 - 16 bytes (and 32-bit lane offsets): larger planes take
  // dense2_kernel, whose addresses are 64-bit.
  const size_t kRsrcMax = 0x7ffffff0u;
  const bool fits = (size_t)((m + 15u) & ~15u) * pl.kp * 2 <= kRsrcMax &&
                    (size_t)((t.rows + 15u) & ~15u) * pl.kp * 2 <= kRsrcMax;
  if (x_bf16 && !lib && t128 >= 96 && fits) {
    pl.d3mode = pl.wmode == kWPlain ? 0 : pl.wmode == kWHiLo ? 1 : 2;
    const uint32_t m256 = (m + 255) / 256, t256 = m256 * ((t.rows + 127) / 128);
    if (pl.wmode == kWPlain && t.rows % 192 == 0 && m256 * (t.rows / 192) >= 192)
      pl.d3cfg = 1;
    else if (pl.wmode == kWPlain && t256 >= 256)
      pl.d3cfg = 2;
    else if (pl.wmode != kWPlain && t256 >= 192 && (t256 <= 256 || t256 >= 512))
      pl.d3cfg = 4;
    else
      pl.d3cfg = 3;
  }
  if (pl.d3cfg >= 0) {
    const uint32_t bm = pl.d3cfg == 3 ? 128 : 256, bn = pl.d3cfg == 1 ? 192 : 128;
    const uint32_t tiles3 = ((m + bm - 1) / bm) * ((t.rows + bn - 1) / bn);
    const uint32_t kt32 = pl.kp / 32;
    uint32_t sp = 1;
    if (pl.d3cfg == 3)
      sp = tiles3 < 192 && kt32 >= 16 ? 2 : 1;
    else
      while (tiles3 * sp * 2 <= 256 && kt32 / (sp * 2) >= 8) sp *= 2;
    pl.kt_per_split = (kt32 + sp - 1) / sp;
    pl.splits = (kt32 + pl.kt_per_split - 1) / pl.kt_per_split;
  }
  // The large-tile kernel reads both planes in 1 KB pieces (plane_off):
  // rows rounded up to 16.
  const bool tiled = pl.d3cfg >= 0;
  const size_t prow = tiled ? (t.rows + 15u) & ~15u : t.rows, arow = tiled ? (m + 15u) & ~15u : m;
  pl.panel_plane = al256(prow * pl.kp * 2);
  pl.dsc_bytes = pl.wmode == kWQBlock ? al256((size_t)t.rows * (pl.kp / 32) * 4) : 0;
  pl.panel_bytes = pl.panel_plane * (pl.wmode == kWHiLo ? 2 : 1) + pl.dsc_bytes + al256((size_t)t.rows * 4);
  pl.a_plane = al256(arow * pl.kp * 2);
  pl.a_bytes = pl.a_plane * (x_bf16 ? 1 : 2);
  pl.partial_bytes = pl.splits > 1 ? al256((size_t)pl.splits * m * t.rows * 4) : 0;
  // Library: for products of fewer than 128 output tiles of 128 x 128, K
  // slices until ~256 tiles are in flight, each slice at least 1024 columns
  // and a whole number of K tiles (at 512 x 6144 outputs, 192 tiles, two
  // slices measured slower than none); fp32 D
  // [lib_splits][M][N] (also room for the own kernel's partial sums, its
  // fallback when the library offers no algorithm for a shape).
  pl.lib_splits = 1;
  if (lib) {
    const uint32_t tiles128 = ((m + 127) / 128) * ((t.rows + 127) / 128);
    while (tiles128 < 128 && tiles128 * pl.lib_splits < 256 && pl.kp / (pl.lib_splits * 2) >= 1024 &&
           pl.kp % (pl.lib_splits * 2 * BK) == 0)
      pl.lib_splits *= 2;
    pl.partial_bytes = std::max(pl.partial_bytes, al256((size_t)pl.lib_splits * m * t.rows * 4));
  }
  return pl;
}

template <int BM, int BN, int WMODE, bool SPLIT_A>
hipError_t launch_dense(const Panel& p, const uint16_t* ah, const uint16_t* al, uint32_t m, uint32_t n, void* y,
                        bool y_bf16, const Plan& pl, float* partial, const int32_t* xe, hipStream_t s) {
  constexpr size_t lds = (size_t)(2 * BM * LDK + 2 * BN * LDK + (SPLIT_A ? 2 * BM * LDK : 0) +
                                  (WMODE == kWHiLo ? 2 * BN * LDK : 0)) * 2 +
                         (WMODE == kWQBlock ? 2 * 2 * BN * 4 : 0);
  static_assert(lds <= 160 * 1024, "LDS budget");
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&dense_kernel<BM, BN, WMODE, SPLIT_A>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  const uint32_t tiles_m = (m + BM - 1) / BM;
  const dim3 grid(tiles_m * ((n + BN - 1) / BN), pl.splits);
  hipLaunchKernelGGL((dense_kernel<BM, BN, WMODE, SPLIT_A>), grid, dim3(THREADS), lds, s, p, ah, al, m, n, y,
                     (uint32_t)y_bf16, partial, pl.kt_per_split, tiles_m, xe);
  return hipGetLastError();
}

template <int BM, int WMODE>
hipError_t launch_dense_x(const Panel& p, const uint16_t* ah, const uint16_t* al, bool x_bf16, uint32_t m,
                          uint32_t n, void* y, bool y_bf16, const Plan& pl, float* partial, const int32_t* xe,
                          hipStream_t s) {
  if (x_bf16) return launch_dense<BM, BM, WMODE, false>(p, ah, al, m, n, y, y_bf16, pl, partial, xe, s);
  if constexpr (WMODE == kWQBlock) {
    return hipErrorInvalidValue;   // f32 activations use the hi/lo panel
  } else {
    return launch_dense<BM, BM, WMODE, true>(p, ah, al, m, n, y, y_bf16, pl, partial, xe, s);
  }
}

template <int WMODE>
hipError_t launch_dense_m(const Panel& p, const uint16_t* ah, const uint16_t* al, bool x_bf16, uint32_t m,
                          uint32_t n, void* y, bool y_bf16, const Plan& pl, float* partial, const int32_t* xe,
                          hipStream_t s) {
  if (pl.bm == 128) return launch_dense_x<128, WMODE>(p, ah, al, x_bf16, m, n, y, y_bf16, pl, partial, xe, s);
  return launch_dense_x<64, WMODE>(p, ah, al, x_bf16, m, n, y, y_bf16, pl, partial, xe, s);
}

// The dense phase on the vendor library: D = sum of f16 GEMMs over the
// hi/lo planes present (lo terms scaled by 2^-11; lo x lo dropped, as in
// dense_kernel), each as one strided batch over `splits` K slices, then
// Y = (sum of the slices' D) / s through reduce_kernel (slices added in
// ascending order).  hipErrorNotSupported when the library has no
// algorithm for the shape.
hipError_t library_dense(const Panel& p, const uint16_t* ah, const uint16_t* al, bool split_a, int wmode, uint32_t m,
                         uint32_t n, uint32_t splits, void* y, bool y_bf16, float* d, const int32_t* xe,
                         hipStream_t s) {
  struct Term { const uint16_t* a; const uint16_t* b; float alpha; };
  Term terms[3];
  int nt = 0;
  terms[nt++] = {ah, p.hi, 1.0f};
  if (wmode == kWHiLo) terms[nt++] = {ah, p.lo, kLoInv};
  if (split_a) terms[nt++] = {al, p.hi, kLoInv};
  for (int i = 0; i < nt; ++i) {
    const hipError_t e = blas_gemm_f16_tn(terms[i].a, p.kp, terms[i].b, p.kp, m, n, p.kp / splits, splits,
                                          terms[i].alpha, i == 0 ? 0.0f : 1.0f, d, s);
    if (e != hipSuccess) return e;
  }
  return launch_gemm_reduce(d, splits, p.inv, xe, m, n, y, y_bf16, s);
}

template <uint32_t KIND>
hipError_t run(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y, bool y_bf16, void* ws,
               size_t ws_bytes, const int32_t* xe, hipStream_t s, bool lib) {
  const Plan pl = plan(t, m, x_bf16, lib);
  if (ws_bytes < pl.panel_bytes + pl.a_bytes + pl.partial_bytes) return hipErrorInvalidValue;
  char* base = static_cast<char*>(ws);
  const bool hilo = pl.wmode == kWHiLo;
  Panel p;
  p.hi = reinterpret_cast<uint16_t*>(base);
  p.lo = reinterpret_cast<uint16_t*>(base + (hilo ? pl.panel_plane : 0));
  p.dsc = reinterpret_cast<float*>(base + pl.panel_plane * (hilo ? 2 : 1));
  p.inv = reinterpret_cast<float*>(base + pl.panel_plane * (hilo ? 2 : 1) + pl.dsc_bytes);
  p.kp = pl.kp;
  p.tiled = pl.d3cfg >= 0;
  uint16_t* ah = reinterpret_cast<uint16_t*>(base + pl.panel_bytes);
  uint16_t* al = reinterpret_cast<uint16_t*>(base + pl.panel_bytes + (x_bf16 ? 0 : pl.a_plane));
  float* partial = reinterpret_cast<float*>(base + pl.panel_bytes + pl.a_bytes);

  const size_t esz = x_bf16 ? 2 : 4;
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && ((size_t)t.cols * esz) % 16 == 0;
  // One launch: the activation conversion's workgroups first, then one
  // wave per (weight row, 2048-column segment) of the panel decode.
  // The register-resident conversion takes one row per workgroup (up to
  // 4096 workgroups); the two-pass one walks rows over at most 1024.
  const bool xreg = x_bf16 && x_vec && p.kp <= 4u * THREADS * 8u;
  XConv xc{x, ah, al, const_cast<int32_t*>(xe), m, t.cols, (uint32_t)x_bf16, x_vec,
           std::min<uint32_t>(m, xreg ? 4096u : 1024u), p.tiled};
  const uint32_t nseg = (p.kp + 64 * 32 - 1) / (64 * 32);
  const uint32_t pgrid = (uint32_t)(((size_t)t.rows * nseg + 3) / 4);
  hipLaunchKernelGGL((panel_kernel<KIND>), dim3(xc.blocks + pgrid), dim3(THREADS), 0, s, t, p,
                     (uint32_t)(pl.wmode == kWQBlock ? 1u : 0u), nseg, xc);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (pl.lib) {
    e = library_dense(p, ah, al, !x_bf16, pl.wmode, m, t.rows, pl.lib_splits, y, y_bf16, partial, xe, s);
    if (e != hipErrorNotSupported) return e;
    (void)hipGetLastError();   // no algorithm for this shape: the own dense kernel on the same panel
  }
  if (pl.d3cfg >= 0) {
    e = launch_dense3(pl.d3cfg, pl.d3mode, ah, p.hi, p.lo, p.dsc, p.inv, m, t.rows, pl.kp, y, y_bf16, partial, pl.splits,
                      pl.kt_per_split, xe, s);
  } else if (x_bf16 && pl.bm == 128) {
    // 128 x 128 tiles with bf16 (exact f16) activations: the interleaved
    // dense kernel (gemm_dense.hip), any weight mode
    e = launch_dense2(pl.wmode, ah, p.hi, p.lo, p.dsc, p.inv, m, t.rows, pl.kp, y, y_bf16, partial, pl.splits,
                      pl.kt_per_split, xe, s);
  } else if constexpr (KIND == KIND_G64) {
    e = launch_dense_m<kWPlain>(p, ah, al, x_bf16, m, t.rows, y, y_bf16, pl, partial, xe, s);
  } else if constexpr (KIND == KIND_Q8 || KIND == KIND_Q40) {
    if (pl.wmode == kWQBlock)
      e = launch_dense_m<kWQBlock>(p, ah, al, x_bf16, m, t.rows, y, y_bf16, pl, partial, xe, s);
    else
      e = launch_dense_m<kWHiLo>(p, ah, al, x_bf16, m, t.rows, y, y_bf16, pl, partial, xe, s);
  } else {
    e = launch_dense_m<kWHiLo>(p, ah, al, x_bf16, m, t.rows, y, y_bf16, pl, partial, xe, s);
  }
  if (e != hipSuccess || pl.splits == 1) return e;
  return launch_gemm_reduce(partial, pl.splits, p.inv, xe, m, t.rows, y, y_bf16, s);
}

}  // namespace gp

hipError_t launch_gemm_reduce(const float* partial, uint32_t splits, const float* inv, const int32_t* xe, uint32_t m,
                              uint32_t n, void* y, bool y_bf16, hipStream_t s) {
  const size_t total = (size_t)m * n;
  const size_t threads = n % 4u == 0u ? total / 4 : total;
  hipLaunchKernelGGL(gp::reduce_kernel, dim3((uint32_t)((threads + gp::THREADS - 1) / gp::THREADS)),
                     dim3(gp::THREADS), 0, s, partial, splits, inv, xe, m, n, y, (uint32_t)y_bf16);
  return hipGetLastError();
}

// Per-row activation exponents (xscale_kernel) into xe[m].
hipError_t launch_xscale(const void* x, bool x_bf16, uint32_t m, uint32_t k, int32_t* xe, hipStream_t s) {
  const size_t esz = x_bf16 ? 2 : 4;
  const uint32_t x_vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && ((size_t)k * esz) % 16 == 0 && k > 0;
  const dim3 grid((m + gp::THREADS / 64 - 1) / (gp::THREADS / 64));
  if (x_bf16)
    hipLaunchKernelGGL(gp::xscale_kernel<true>, grid, dim3(gp::THREADS), 0, s, x, m, k, x_vec, xe);
  else
    hipLaunchKernelGGL(gp::xscale_kernel<false>, grid, dim3(gp::THREADS), 0, s, x, m, k, x_vec, xe);
  return hipGetLastError();
}

bool gemm_fused_supported(const DevTensor& t, bool x_bf16);
bool gemm_fused_scales_x(const DevTensor& t);
size_t gemm_fused_workspace_bytes(const DevTensor& t, uint32_t m);
hipError_t launch_gemm_fused(const DevTensor& t, const uint16_t* x, uint32_t m, void* y, bool y_bf16, void* ws,
                             size_t ws_bytes, const int32_t* xe, hipStream_t s);

bool gemm_tile_supported(const DevTensor& t, bool x_bf16);
size_t gemm_tile_workspace_bytes(const DevTensor& t, uint32_t m);
hipError_t launch_gemm_tile(const DevTensor& t, const uint16_t* x, uint32_t m, void* y, bool y_bf16, void* ws,
                            size_t ws_bytes, hipStream_t s);
bool gemm_tile_cb4_supported(const DevTensor& t, bool x_bf16);
size_t gemm_tile_cb4_workspace_bytes(const DevTensor& t, uint32_t m);
hipError_t launch_gemm_tile_cb4(const DevTensor& t, const uint16_t* x, uint32_t m, void* y, bool y_bf16, void* ws,
                                size_t ws_bytes, hipStream_t s);

// Path choice, unless the caller pins one (every path runs every kind):
//   * g64 weights, bf16 activations: the fused kernel up to batch 64; the
//     decode-in-registers tile kernel (gemm_tile.hip) from batch 128 to 767
//     (to 1023 when K > N); the two-phase path otherwise;
//   * cb4 weights, bf16 activations, within the tile kernel's limits
//     (gemm_tile_cb4_supported): its decode-in-loop tile kernel from batch
//     128 to 511, to 255 when K < N (M = 128 / 256: 96 / 84 and 137 / 145
//     TFLOP/s against the two-phase path's 81 / 77 and 121 / 131; at M = 64
//     and 512 the two-phase path is ahead; with the two-phase planes in 1 KB
//     pieces, at 2048 -> 6144 M = 256 / 384: 133 / 146 against 149 / 172,
//     at 6144 -> 2048 148 / 169 against 143 / 160);
//   * Q8 weights, bf16 activations: the fused kernel up to batch 128, and
//     up to 511 when K >= N (M = 256 / 384: 196 / 212 TFLOP/s against
//     171 / 182 two-phase at 6144 -> 2048, 91 / 126 against 81 / 106 at
//     2048 -> 2048; level at 512; behind at 2048 -> 6144, 154 / 177 against
//     179 / 195);
//   * everything else: the two-phase path with the own dense kernel.
// The vendor dense GEMM runs only when pinned (kGemmLibrary), as a
// comparison.  Measured on MI355X (whole call, graph of 100 calls, TFLOP/s,
// K x N = 2048 x 6144 / 6144 x 2048):
//   g64 M = 64: fused 73 / 61, two-phase 68 / 61; M = 96: tile 82, two-phase
//   89 (2048 x 6144); M = 128: tile 134 / 118, two-phase 115 / 107; M = 512:
//   tile 407 / 350, two-phase 300 / 325; with the two-phase planes in 1 KB
//   pieces: M = 512: tile 409 / 358, two-phase 418 / 321; M = 768: tile
//   378 / 396, two-phase 457 / 384; M = 1024: tile 484 / 463, two-phase
//   554 / 465; M = 1536: tile 513 / 517, two-phase 640 / 555; M = 4096: tile
//   693 (6144 x 2048), two-phase 858;
//   Q8 M = 64: fused 81 / 71, two-phase 61 / 54; M = 256: fused 125 / 161,
//   two-phase 132 / 163.
constexpr uint32_t kFusedMaxM = 128;
constexpr uint32_t kQ8FusedMaxMTall = 512;   // exclusive, K >= N
constexpr uint32_t kG64FusedMaxM = 64;
constexpr uint32_t kTileMinM = 128;
constexpr uint32_t kTileMaxM = 768;        // exclusive
constexpr uint32_t kTileMaxMTall = 1024;   // exclusive, K > N
constexpr uint32_t kCb4TileMaxM = 512;      // exclusive
constexpr uint32_t kCb4TileMaxMWide = 256;  // exclusive, K < N

enum class Path { Fused, Tile, TileCb4, Panel };

static Path choose_path(const DevTensor& t, uint32_t m, bool x_bf16, int mode) {
  if (mode == kGemmPanel || mode == kGemmLibrary) return Path::Panel;
  const bool tile_ok = gemm_tile_supported(t, x_bf16);
  const bool fused_ok = gemm_fused_supported(t, x_bf16);
  if (mode == kGemmFused) {   // decode inside the MFMA loop wherever it applies
    if (gemm_tile_cb4_supported(t, x_bf16)) return Path::TileCb4;
    if (tile_ok && m > kG64FusedMaxM) return Path::Tile;
    return fused_ok ? Path::Fused : Path::Panel;
  }
  if (t.kind == KIND_CB4 && m >= kTileMinM && m < (t.cols < t.rows ? kCb4TileMaxMWide : kCb4TileMaxM) &&
      gemm_tile_cb4_supported(t, x_bf16))
    return Path::TileCb4;
  if (t.kind == KIND_G64 && x_bf16) {
    if (fused_ok && m <= kG64FusedMaxM) return Path::Fused;
    if (tile_ok && m >= kTileMinM && m < (t.cols > t.rows ? kTileMaxMTall : kTileMaxM)) return Path::Tile;
    return Path::Panel;
  }
  if (fused_ok && (m <= kFusedMaxM || (t.kind == KIND_Q8 && t.cols >= t.rows && m < kQ8FusedMaxMTall)))
    return Path::Fused;
  return Path::Panel;
}

static bool library_path(int mode) { return mode == kGemmLibrary; }

// Workspace: the per-row activation exponents first, then the path's own
// (the tile path keeps its exponents in its own block).
static size_t xe_bytes(uint32_t m) { return gp::al256((size_t)m * 4); }

size_t gemm_workspace_bytes(const DevTensor& t, uint32_t m, bool x_bf16, int mode) {
  switch (choose_path(t, m, x_bf16, mode)) {
    case Path::Tile: return gemm_tile_workspace_bytes(t, m);
    case Path::TileCb4: return gemm_tile_cb4_workspace_bytes(t, m);
    case Path::Fused: return xe_bytes(m) + gemm_fused_workspace_bytes(t, m);
    default: break;
  }
  const gp::Plan pl = gp::plan(t, m, x_bf16, library_path(mode));
  return xe_bytes(m) + pl.panel_bytes + pl.a_bytes + pl.partial_bytes;
}

hipError_t launch_gemm(const DevTensor& t, const void* x, bool x_bf16, uint32_t m, void* y, bool y_bf16, void* ws,
                       size_t ws_bytes, hipStream_t s, int mode) {
  if (m == 0 || (size_t)m * t.rows > (size_t)1 << 40) return hipErrorInvalidValue;
  const Path path = choose_path(t, m, x_bf16, mode);
  if (path == Path::Tile)
    return launch_gemm_tile(t, static_cast<const uint16_t*>(x), m, y, y_bf16, ws, ws_bytes, s);
  if (path == Path::TileCb4)
    return launch_gemm_tile_cb4(t, static_cast<const uint16_t*>(x), m, y, y_bf16, ws, ws_bytes, s);
  if (ws_bytes < xe_bytes(m)) return hipErrorInvalidValue;
  int32_t* xe = static_cast<int32_t*>(ws);
  void* rest = static_cast<char*>(ws) + xe_bytes(m);
  const size_t rest_bytes = ws_bytes - xe_bytes(m);
  if (path == Path::Fused) {
    // f16 operands need the activations' row scales: the fused g64 kernel
    // takes them from this pre-pass (the fused Q8 kernel multiplies bf16
    // activations as they are; the two-phase path's activation conversion
    // finds them itself).
    if (gemm_fused_scales_x(t)) {
      const hipError_t e = launch_xscale(x, x_bf16, m, t.cols, xe, s);
      if (e != hipSuccess) return e;
    }
    return launch_gemm_fused(t, static_cast<const uint16_t*>(x), m, y, y_bf16, rest, rest_bytes, xe, s);
  }
  const bool lib = library_path(mode);
  switch (t.kind) {
    case KIND_G64: return gp::run<KIND_G64>(t, x, x_bf16, m, y, y_bf16, rest, rest_bytes, xe, s, lib);
    case KIND_Q8: return gp::run<KIND_Q8>(t, x, x_bf16, m, y, y_bf16, rest, rest_bytes, xe, s, lib);
    case KIND_Q40: return gp::run<KIND_Q40>(t, x, x_bf16, m, y, y_bf16, rest, rest_bytes, xe, s, lib);
    case KIND_CB4: return gp::run<KIND_CB4>(t, x, x_bf16, m, y, y_bf16, rest, rest_bytes, xe, s, lib);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vxt
