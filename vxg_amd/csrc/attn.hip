// attn.hip -- Q8_0 KV cache for decode and prefill: prepare a step's q and
// k, append positions, attend over the cache.
//
// Reference: KvQ8Block (llm_prefill.rs:17-63), step_full_gqa_q8
// (llm_prefill.rs:259-367) and apply_rope (llm_ops.rs:81-99); the Metal
// runner's batched prep (vxt_cb4_gqa_prep_batch, vxt_cb4_fast_gqa.metal:
// 455-541).
//
// Device layout (the caller's VxtKvQ8Cache; row t holds position t):
//   k_qs, v_qs  int8 [max_seq][n_kv * hd]        (16-byte aligned rows)
//   k_d,  v_d   f16  [max_seq][n_kv * hd / 32]   (one scale per 32 values)
// -- the KvQ8Block's two fields as separate planes, so a position's values
// load as aligned 16-byte pieces.  The bits of every value and scale are
// those KvQ8Block::quantize produces.
//
// Append: one lane per value, a 32-lane group per block: amax of |x| (NaN
// ignored, as f32::max does), d = f16(amax / 127) rounded to nearest even,
// q = round_ties_even(x / f32(d)) clamped to +-127 (NaN -> 0).
//
// Prep: one wave per (head, token) splits a gated q, applies the per-head
// RMSNorm and RoPE to q and k and quantises K and V into the token's row.
//
// Attention (split sequence): workgroup (kv head, chunk of positions, token)
// serves the query heads that share the kv head.  Each position is read once
// per token: a position's K and V rows are split across hd / 16 lanes (16
// values each), all requested up front; the dot with every head's q (staged
// in LDS) is reduced over those lanes and scaled by 1 / sqrt(hd); the chunk's
// scores stay in LDS; the chunk's max m, the sum l of exp(s - m) and
// sum exp(s - m) V go to a partials buffer.  A second kernel merges the
// chunks per head (exp(m_c - m) rescaling), divides by the total and applies
// the optional sigmoid gate.  Token z of a batch attends to positions
// [0, seq0 + z) (causal prefill).  The sums run in a different order from the
// CPU loop (fp32, parity by tolerance).
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace vxt {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kMaxGroup = 8;   // query heads per kv head

// f32 -> f16 bits, round to nearest even, subnormals kept (fp16.rs:33-77).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float val) {
  const uint32_t b = __float_as_uint(val);
  const uint32_t sign = (b >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((b >> 23) & 0xffu);
  const uint32_t mant = b & 0x007fffffu;
  if (exp == 255) return mant ? (sign | 0x7e00u | (mant >> 13)) : (sign | 0x7c00u);
  const int32_t unb = exp - 127;
  if (unb > 15) return sign | 0x7c00u;
  if (unb < -25) return sign;
  if (unb < -14) {
    const uint32_t shift = (uint32_t)(-14 - unb);
    const uint32_t full = mant | 0x00800000u;
    const uint32_t rs = 13u + shift;
    const uint32_t half = 1u << (rs - 1), rem = full & ((1u << rs) - 1u);
    uint32_t m16 = full >> rs;
    if (rem > half || (rem == half && (m16 & 1u))) m16 += 1;
    return sign | m16;
  }
  const uint32_t e16 = (uint32_t)(unb + 15) << 10;
  const uint32_t rem = mant & 0x1fffu;
  uint32_t m16 = mant >> 13;
  if (rem > 0x1000u || (rem == 0x1000u && (m16 & 1u))) {
    m16 += 1;
    if (m16 == 0x0400u) return sign | (e16 + 0x0400u);
  }
  return sign | e16 | m16;
}

// KvQ8Block::quantize of one value per lane, each aligned 32-lane group
// holding one block (every lane of the wave must call it): amax of |x| with
// NaN ignored, dh = f16 bits of amax / 127, q = round_ties_even(x / f32(dh))
// clamped to +-127, NaN -> 0.
__device__ __forceinline__ int q8_lane(float x, uint32_t& dh) {
#pragma clang fp contract(off)
  const float a = fabsf(x);
  float amax = a == a ? a : 0.0f;
  amax = lane_reduce<32, true>(amax);
  dh = f32_to_f16_bits(amax / 127.0f);
  const float df = f16_to_f32_exact(dh);
  const float inv = df > 0.0f ? 1.0f / df : 0.0f;
  const float r = rintf(x * inv);
  return r != r ? 0 : (int)fminf(fmaxf(r, -127.0f), 127.0f);
}

__global__ __launch_bounds__(kThreads) void kv_append_kernel(KvQ8Dev c, const float* __restrict__ k,
                                                            const float* __restrict__ v, uint32_t pos) {
  const uint32_t per = c.n_kv * c.hd;
  const uint32_t e = blockIdx.x * kThreads + threadIdx.x;   // per % 32 == 0: a 32-group never straddles K/V
  const bool live = e < 2u * per;
  const bool is_v = e >= per;
  const uint32_t i = is_v ? e - per : e;
  const float x = live ? (is_v ? v[i] : k[i]) : 0.0f;
  uint32_t dh;
  const int q = q8_lane(x, dh);
  if (!live) return;
  int8_t* qs = is_v ? c.v_qs : c.k_qs;
  uint16_t* ds = is_v ? c.v_d : c.k_d;
  qs[(size_t)pos * per + i] = (int8_t)q;
  if ((i & 31u) == 0) ds[(size_t)pos * (per / 32) + i / 32] = (uint16_t)dh;
}

// ---- the step's q / k preparation (llm_prefill.rs:284-313) ----------------
// One wave per (head, token): blockIdx.x < n_head is query head x, the rest
// are kv heads; blockIdx.y is the token.  A lane holds the values d = lane +
// 64 j of its head.  Query head: q_raw slice (+ bias), the gate half copied
// out, RMSNorm with q_norm (sum of squares over the wave, then x * scale * w
// as two roundings), RoPE, q_out.  Kv head: V (+ bias) quantised into the
// cache; K (+ bias), RMSNorm with k_norm, RoPE, quantised.  RoPE angles are
// (float)(rope_pos + token) * freq[i] with freq[i] = powf(base, -2i / rdim)
// evaluated on the host (the same call as the reference's), sine and cosine
// of the f32 angle evaluated in double and rounded once; both rotation
// products round separately.
struct RopeFreq {
  float f[128];
};

template <int HD>
__global__ __launch_bounds__(64) void gqa_prep_kernel(KvQ8Dev c, GqaPrep a, RopeFreq rf) {
#pragma clang fp contract(off)
  constexpr int J = HD >= 64 ? HD / 64 : 1;
  __shared__ float s_x[HD];
  const uint32_t lane = threadIdx.x, idx = blockIdx.x, m = blockIdx.y;
  const bool is_q = idx < a.n_head;
  const uint32_t kvh = is_q ? 0u : idx - a.n_head;
  const uint32_t per = c.n_kv * HD;
  const size_t row = (size_t)a.pos + m;
  const uint32_t qoff = idx * (a.gated ? 2u : 1u) * HD;
  const float* src = is_q ? a.q_raw + (size_t)m * a.q_stride + qoff : a.k_cur + (size_t)m * a.kv_stride + kvh * HD;
  const float* bias = is_q ? (a.q_bias ? a.q_bias + qoff : nullptr) : (a.k_bias ? a.k_bias + kvh * HD : nullptr);
  const float* nw = is_q ? a.q_norm : a.k_norm;

  float x[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t d = lane + 64u * j;
    x[j] = 0.0f;
    if (d < HD) {
      x[j] = src[d];
      if (bias) x[j] = x[j] + bias[d];
    }
  }
  if (is_q && a.gated) {
    float* g = a.gate_out + (size_t)m * a.n_head * HD + (size_t)idx * HD;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t d = lane + 64u * j;
      if (d < HD) g[d] = bias ? src[HD + d] + bias[HD + d] : src[HD + d];
    }
  }
  if (!is_q) {
    const float* vs = a.v_cur + (size_t)m * a.kv_stride + kvh * HD;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t d = lane + 64u * j;
      float vv = 0.0f;
      if (d < HD) {
        vv = vs[d];
        if (a.v_bias) vv = vv + a.v_bias[kvh * HD + d];
      }
      uint32_t dh;
      const int q = q8_lane(vv, dh);
      if (d < HD) {
        c.v_qs[row * per + kvh * HD + d] = (int8_t)q;
        if ((d & 31u) == 0) c.v_d[row * (per / 32) + (kvh * HD + d) / 32] = (uint16_t)dh;
      }
    }
  }
  if (nw) {
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) sq = __builtin_fmaf(x[j], x[j], sq);
    sq = lane_reduce<64>(sq);
    const float scale = 1.0f / sqrtf(sq / (float)HD + a.eps);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t d = lane + 64u * j;
      if (d < HD) x[j] = x[j] * scale * nw[d];
    }
  }
  if (a.half) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t d = lane + 64u * j;
      if (d < HD) s_x[d] = x[j];
    }
    __syncthreads();
    const float p = (float)(a.rope_pos + m);
    for (uint32_t i = lane; i < a.half; i += 64u) {
      const float theta = p * rf.f[i];
      const float sn = (float)sin((double)theta), cs = (float)cos((double)theta);
      const uint32_t i0 = a.neox ? i : 2u * i, i1 = a.neox ? i + a.half : 2u * i + 1u;
      const float x0 = s_x[i0], x1 = s_x[i1];
      s_x[i0] = x0 * cs - x1 * sn;
      s_x[i1] = x0 * sn + x1 * cs;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t d = lane + 64u * j;
      if (d < HD) x[j] = s_x[d];
    }
  }
  if (is_q) {
    float* qo = a.q_out + (size_t)m * a.n_head * HD + (size_t)idx * HD;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t d = lane + 64u * j;
      if (d < HD) qo[d] = x[j];
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t d = lane + 64u * j;
    uint32_t dh;
    const int q = q8_lane(x[j], dh);
    if (d < HD) {
      c.k_qs[row * per + kvh * HD + d] = (int8_t)q;
      if ((d & 31u) == 0) c.k_d[row * (per / 32) + (kvh * HD + d) / 32] = (uint16_t)dh;
    }
  }
}

// 16 int8 -> f32
__device__ __forceinline__ void unpack16(const u32x4 w, float (&f)[16]) {
  const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 16; ++j) f[j] = (float)(int8_t)((a[j >> 2] >> ((j & 3) * 8)) & 0xffu);
}

// LPT lanes per position (hd = 16 * LPT).  A chunk is 4 passes of the
// 4 * TPW positions the workgroup covers at once, so every lane requests its
// 4 K pieces and 4 V pieces (16 bytes each, plus scales) before any wait:
// one trip to memory per workgroup.
template <int LPT>
__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(KvQ8Dev c, const float* __restrict__ q, uint32_t group,
                                                             uint32_t seq0, uint32_t n_chunks,
                                                             float* __restrict__ part) {
  constexpr uint32_t HD = LPT * 16, TPW = 64 / LPT, PASSES = 4, CH = PASSES * 4 * TPW;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* s_q = smem;                       // [group][HD]
  float* s_p = smem + group * HD;          // [group][CH] scores, then exp(s - m)
  float* s_red = s_p + group * CH;         // [4 waves][4 heads][HD] reduction space
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t slot = lane / LPT, sub = lane % LPT;
  const uint32_t kvh = blockIdx.x, ck = blockIdx.y;
  const uint32_t seq_len = seq0 + blockIdx.z;             // token z sees positions [0, seq0 + z)
  const uint32_t t0 = ck * CH;
  if (t0 >= seq_len) return;                              // a chunk past this token's positions
  const uint32_t n = min(seq_len - t0, CH);
  q += (size_t)blockIdx.z * c.n_kv * group * HD;
  part += (size_t)blockIdx.z * c.n_kv * group * n_chunks * (HD + 2);
  const uint32_t row_q = c.n_kv * HD, row_d = c.n_kv * (HD / 32);
  const float scale = 1.0f / sqrtf((float)HD);

  // q first (small, cached), then every K and V piece of the chunk.
  float qv[kMaxGroup * HD / kThreads + 1];
  const uint32_t nq = group * HD;
#pragma unroll
  for (uint32_t r = 0; r < kMaxGroup * HD / kThreads + 1; ++r) {
    const uint32_t i = tid + r * kThreads;
    qv[r] = i < nq ? q[(size_t)kvh * nq + i] : 0.0f;
  }
  // Raw scale bits: converting them here would wait for the load (and, the
  // memory counter draining in order, for every load issued before it).
  u32x4 kw[PASSES], vw[PASSES];
  uint32_t kdb[PASSES], vdb[PASSES];
  uint32_t tl[PASSES];
#pragma unroll
  for (uint32_t p = 0; p < PASSES; ++p) {
    tl[p] = (p * 4u + wave) * TPW + slot;
    const uint32_t tc = t0 + (tl[p] < n ? tl[p] : n - 1);
    const size_t qo = (size_t)tc * row_q + kvh * HD + sub * 16u;
    const size_t dof = (size_t)tc * row_d + kvh * (HD / 32) + sub / 2u;
    kw[p] = *reinterpret_cast<const u32x4*>(c.k_qs + qo);
    vw[p] = *reinterpret_cast<const u32x4*>(c.v_qs + qo);
    kdb[p] = c.k_d[dof];
    vdb[p] = c.v_d[dof];
  }
#pragma unroll
  for (uint32_t r = 0; r < kMaxGroup * HD / kThreads + 1; ++r) {
    const uint32_t i = tid + r * kThreads;
    if (i < nq) s_q[i] = qv[r];
  }
  __syncthreads();

  // ---- scores
#pragma unroll
  for (uint32_t p = 0; p < PASSES; ++p) {
    float kf[16];
    unpack16(kw[p], kf);
    for (uint32_t g = 0; g < group; ++g) {
      const float* qg = s_q + g * HD + sub * 16u;
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = __builtin_fmaf(qg[j], kf[j], acc);
      acc *= f16_to_f32_exact(kdb[p]);
      acc = lane_reduce<LPT>(acc);
      if (sub == 0 && tl[p] < n) s_p[g * CH + tl[p]] = acc * scale;
    }
  }
  __syncthreads();

  // ---- chunk softmax pieces: one wave per head
  for (uint32_t g = wave; g < group; g += 4u) {
    float m = -__builtin_inff();
    for (uint32_t t = lane; t < n; t += 64u) m = fmaxf(m, s_p[g * CH + t]);
    m = lane_reduce<64, true>(m);
    float l = 0.0f;
    for (uint32_t t = lane; t < n; t += 64u) {
      const float e = expf(s_p[g * CH + t] - m);
      s_p[g * CH + t] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      float* pp = part + ((size_t)(kvh * group + g) * n_chunks + ck) * (HD + 2);
      pp[0] = m;
      pp[1] = l;
    }
  }
  __syncthreads();

  // ---- sum exp(s - m) V from the registers, four heads at a time
  float vf[PASSES][16];
#pragma unroll
  for (uint32_t p = 0; p < PASSES; ++p) {
    unpack16(vw[p], vf[p]);
    const float vd = f16_to_f32_exact(vdb[p]);
#pragma unroll
    for (int j = 0; j < 16; ++j) vf[p][j] *= vd;
  }
  for (uint32_t g0 = 0; g0 < group; g0 += 4u) {
    const uint32_t gn = min(4u, group - g0);
    float acc[4][16];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][j] = 0.0f;
#pragma unroll
    for (uint32_t p = 0; p < PASSES; ++p) {
      const bool ok = tl[p] < n;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float w = (ok && (uint32_t)a < gn) ? s_p[(g0 + a) * CH + tl[p]] : 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[a][j] = __builtin_fmaf(w, vf[p][j], acc[a][j]);
      }
    }
    // reduce over the slots of the wave (lanes with the same sub), then over
    // waves; only the heads present
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      if ((uint32_t)a >= gn) break;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        acc[a][j] = stride_sum<LPT>(acc[a][j]);
      if (slot == 0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) s_red[(wave * 4u + a) * HD + sub * 16u + j] = acc[a][j];
      }
    }
    __syncthreads();
    for (uint32_t i = tid; i < gn * HD; i += kThreads) {
      const uint32_t a = i / HD, d = i % HD;
      const float sum = (s_red[(0 * 4u + a) * HD + d] + s_red[(1 * 4u + a) * HD + d]) +
                        (s_red[(2 * 4u + a) * HD + d] + s_red[(3 * 4u + a) * HD + d]);
      part[((size_t)(kvh * group + g0 + a) * n_chunks + ck) * (HD + 2) + 2 + d] = sum;
    }
    __syncthreads();
  }
}

// Merge: workgroup (head, 64 dimensions) of kMergeWaves waves.  The chunks'
// maximum first, then wave w sums chunks w, w + kMergeWaves, ... (sixteen
// at a time in flight), then the waves' sums are added in wave order.
constexpr uint32_t kMergeWaves = 16;

__global__ __launch_bounds__(kMergeWaves * 64) void attn_merge_kernel(const float* __restrict__ part, uint32_t hd,
                                                                     uint32_t chunk_stride, uint32_t chunk,
                                                                     uint32_t seq0, const float* __restrict__ gate,
                                                                     float* __restrict__ out) {
#pragma clang fp contract(off)
  constexpr uint32_t W = kMergeWaves;
  __shared__ float s_m[W], s_acc[W][64], s_l[W];
  const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t d = blockIdx.y * 64u + lane;
  const uint32_t z = blockIdx.z, n_head = gridDim.x;
  const uint32_t n_chunks = (seq0 + z + chunk - 1u) / chunk;   // token z's chunks
  const size_t stride = hd + 2;
  const float* ph = part + ((size_t)z * n_head + h) * chunk_stride * stride;
  if (gate) gate += (size_t)z * n_head * hd;
  out += (size_t)z * n_head * hd;
  float m = -__builtin_inff();
  for (uint32_t c = tid; c < n_chunks; c += W * 64u) m = fmaxf(m, ph[c * stride]);
  m = lane_reduce<64, true>(m);
  if (lane == 0) s_m[wave] = m;
  __syncthreads();
  m = s_m[0];
#pragma unroll
  for (uint32_t w = 1; w < W; ++w) m = fmaxf(m, s_m[w]);
  const uint32_t dc = d < hd ? d : hd - 1;
  float acc = 0.0f, l = 0.0f;
  uint32_t c = wave;
  constexpr int U = 16;   // chunks in flight per lane
  for (; c + W * (U - 1) < n_chunks; c += W * U) {
    float mc[U], lc[U], ac[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float* pc = ph + (size_t)(c + W * u) * stride;
      mc[u] = pc[0];
      lc[u] = pc[1];
      ac[u] = pc[2 + dc];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float e = expf(mc[u] - m);
      l += lc[u] * e;
      acc += ac[u] * e;
    }
  }
  for (; c < n_chunks; c += W) {
    const float* pc = ph + (size_t)c * stride;
    const float e = expf(pc[0] - m);
    l += pc[1] * e;
    acc += pc[2 + dc] * e;
  }
  s_acc[wave][lane] = acc;
  if (lane == 0) s_l[wave] = l;
  __syncthreads();
  if (wave != 0 || d >= hd) return;
  float tot = s_l[0], o = s_acc[0][lane];
#pragma unroll
  for (uint32_t w = 1; w < W; ++w) {
    tot += s_l[w];
    o += s_acc[w][lane];
  }
  o = o / tot;
  if (gate) o *= 1.0f / (1.0f + expf(-gate[(size_t)h * hd + d]));
  out[(size_t)h * hd + d] = o;
}

template <int LPT>
hipError_t launch_chunks(const KvQ8Dev& c, const float* q, uint32_t group, uint32_t seq0, uint32_t n_chunks,
                         uint32_t batch, float* part, hipStream_t s) {
  constexpr uint32_t HD = LPT * 16, CH = 16u * (64u / LPT);
  const size_t lds = ((size_t)group * HD + (size_t)group * CH + 16u * HD) * 4u;
  hipLaunchKernelGGL(attn_chunk_kernel<LPT>, dim3(c.n_kv, n_chunks, batch), dim3(kThreads), lds, s, c, q, group,
                     seq0, n_chunks, part);
  return hipGetLastError();
}

// Positions per chunk: 4 passes of 4 waves x 64 / (hd / 16) positions.
uint32_t chunk_of(uint32_t hd) { return 16u * (64u / (hd / 16u)); }

template <int HD>
void launch_prep(const KvQ8Dev& c, const GqaPrep& a, const RopeFreq& rf, uint32_t batch, hipStream_t s) {
  hipLaunchKernelGGL(gqa_prep_kernel<HD>, dim3(a.n_head + c.n_kv, batch), dim3(64), 0, s, c, a, rf);
}

}  // namespace

hipError_t launch_kv_append(const KvQ8Dev& c, const float* k, const float* v, uint32_t pos, hipStream_t s) {
  const uint32_t n = 2u * c.n_kv * c.hd;
  hipLaunchKernelGGL(kv_append_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s, c, k, v, pos);
  return hipGetLastError();
}

// The rotation frequencies are a function of (freq_base, rdim) only; the last
// table is kept per host thread.
hipError_t launch_gqa_prep(const KvQ8Dev& c, GqaPrep a, uint32_t rope_dim, float freq_base, uint32_t batch,
                           hipStream_t s) {
  thread_local RopeFreq tab{};
  thread_local uint32_t tab_rdim = 0;
  thread_local float tab_base = 0.0f;
  const uint32_t rdim = std::min(rope_dim, c.hd);
  a.half = rdim / 2u;
  if (a.half && (tab_rdim != rdim || std::memcmp(&tab_base, &freq_base, sizeof(float)) != 0)) {
    for (uint32_t i = 0; i < a.half; ++i) tab.f[i] = powf(freq_base, -(2.0f * (float)i) / (float)rdim);
    tab_rdim = rdim;
    tab_base = freq_base;
  }
  switch (c.hd) {
    case 32: launch_prep<32>(c, a, tab, batch, s); break;
    case 64: launch_prep<64>(c, a, tab, batch, s); break;
    case 128: launch_prep<128>(c, a, tab, batch, s); break;
    case 256: launch_prep<256>(c, a, tab, batch, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Partials of a batch: batch x n_head x chunks of the longest token x (hd + 2).
size_t attn_workspace_bytes(uint32_t n_head, uint32_t seq_len, uint32_t n_kv, uint32_t hd, uint32_t batch) {
  (void)n_kv;
  const uint32_t chunk = chunk_of(hd);
  const size_t n_chunks = ((size_t)seq_len + batch - 1 + chunk - 1) / chunk;
  return (size_t)batch * n_head * n_chunks * (hd + 2) * sizeof(float);
}

// batch tokens; token z has q at q + z * n_head * hd and attends to positions
// [0, seq0 + z).  Requires hd in {32, 64, 128, 256}, n_head % n_kv == 0,
// n_head / n_kv <= 8, 1 <= seq0, seq0 + batch - 1 <= max_seq; ws holds
// attn_workspace_bytes(n_head, seq0, n_kv, hd, batch).
hipError_t launch_attn(const KvQ8Dev& c, const float* q, uint32_t n_head, uint32_t seq0, uint32_t batch,
                       const float* gate, float* out, void* ws, hipStream_t s) {
  const uint32_t group = n_head / c.n_kv;
  if (group == 0 || group > kMaxGroup || batch == 0 || batch > 65535u) return hipErrorInvalidValue;
  const uint32_t chunk = chunk_of(c.hd);
  const uint32_t n_chunks = (uint32_t)(((size_t)seq0 + batch - 1 + chunk - 1) / chunk);
  if (n_chunks > 65535u) return hipErrorInvalidValue;
  float* part = static_cast<float*>(ws);
  hipError_t e;
  switch (c.hd) {
    case 32: e = launch_chunks<2>(c, q, group, seq0, n_chunks, batch, part, s); break;
    case 64: e = launch_chunks<4>(c, q, group, seq0, n_chunks, batch, part, s); break;
    case 128: e = launch_chunks<8>(c, q, group, seq0, n_chunks, batch, part, s); break;
    case 256: e = launch_chunks<16>(c, q, group, seq0, n_chunks, batch, part, s); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attn_merge_kernel, dim3(n_head, (c.hd + 63) / 64, batch), dim3(kMergeWaves * 64), 0, s, part,
                     c.hd, n_chunks, chunk, seq0, gate, out);
  return hipGetLastError();
}

}  // namespace vxt
