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
//
// Prefill (16 tokens or more): a flash-attention kernel on bf16 MFMA with
// split operands, 128 query rows per workgroup, position segments merged by
// a small kernel (see attn_prefill_bf16_kernel).
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace vxt {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kMaxGroup = 8;   // query heads per kv head

typedef float float16v __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr uint32_t kSegTiles = 16;   // prefill: 32-position tiles per position segment

// f32 -> f16 bits, round to nearest even with f16 subnormals kept and
// overflow to infinity: what fp16.rs:33-77 computes with integer steps, here
// v_cvt_f16_f32 (default round-to-nearest-even mode, f16 denormals on).
// Inputs are never NaN (the callers pass a maximum of magnitudes that skips
// NaN).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float val) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)val);
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
// One workgroup per token; its four waves take the heads in turn (query
// heads, then kv heads), after the token's rotation angles are tabulated in
// LDS once.  A lane holds the values d = lane + 64 j of its head.  Query head: q_raw slice (+ bias), the gate half copied
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
__global__ __launch_bounds__(256) void gqa_prep_kernel(KvQ8Dev c, GqaPrep a, RopeFreq rf) {
#pragma clang fp contract(off)
  constexpr int J = HD >= 64 ? HD / 64 : 1;
  __shared__ float s_x[4][HD];          // a wave's head during the rotation
  __shared__ float s_cs[HD];            // sin, cos of pair i at 2 i, 2 i + 1
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, m = blockIdx.x;
  const uint32_t per = c.n_kv * HD, n_units = a.n_head + c.n_kv;
  const size_t row = (size_t)a.pos + m;
  // the token's rotation angles, once for all its heads
  if (tid < a.half) {
    const float theta = (float)(a.rope_pos + m) * rf.f[tid];
    double sd, cd;
    sincos((double)theta, &sd, &cd);
    s_cs[2u * tid] = (float)sd;
    s_cs[2u * tid + 1u] = (float)cd;
  }
  __syncthreads();
  // wave w takes heads w, w + 4, ... (query heads, then kv heads); every
  // wave runs the same number of rounds so the barriers line up
  for (uint32_t base = 0; base < n_units; base += 4u) {
    const uint32_t idx = base + wave;
    const bool active = idx < n_units;
    const uint32_t idc = active ? idx : 0u;
    const bool is_q = idc < a.n_head;
    const uint32_t kvh = is_q ? 0u : idc - a.n_head;
    const uint32_t qoff = idc * (a.gated ? 2u : 1u) * HD;
    const float* src = is_q ? a.q_raw + (size_t)m * a.q_stride + qoff : a.k_cur + (size_t)m * a.kv_stride + kvh * HD;
    const float* bias = is_q ? (a.q_bias ? a.q_bias + qoff : nullptr) : (a.k_bias ? a.k_bias + kvh * HD : nullptr);
    const float* nw = is_q ? a.q_norm : a.k_norm;
    float* sx = s_x[wave];

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
    if (active && is_q && a.gated) {
      float* gt = a.gate_out + (size_t)m * a.n_head * HD + (size_t)idc * HD;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const uint32_t d = lane + 64u * j;
        if (d < HD) gt[d] = bias ? src[HD + d] + bias[HD + d] : src[HD + d];
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
        const int qq = q8_lane(vv, dh);
        if (active && d < HD) {
          c.v_qs[row * per + kvh * HD + d] = (int8_t)qq;
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
        if (d < HD) sx[d] = x[j];
      }
      lds_barrier();
      for (uint32_t i = lane; i < a.half; i += 64u) {
        const float sn = s_cs[2u * i], cs = s_cs[2u * i + 1u];
        const uint32_t i0 = a.neox ? i : 2u * i, i1 = a.neox ? i + a.half : 2u * i + 1u;
        const float x0 = sx[i0], x1 = sx[i1];
        sx[i0] = x0 * cs - x1 * sn;
        sx[i1] = x0 * sn + x1 * cs;
      }
      lds_barrier();
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const uint32_t d = lane + 64u * j;
        if (d < HD) x[j] = sx[d];
      }
      lds_barrier();   // the next round writes sx again
    }
    if (is_q) {
      if (active) {
        float* qo = a.q_out + (size_t)m * a.n_head * HD + (size_t)idc * HD;
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const uint32_t d = lane + 64u * j;
          if (d < HD) qo[d] = x[j];
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const uint32_t d = lane + 64u * j;
        uint32_t dh;
        const int qq = q8_lane(x[j], dh);
        if (active && d < HD) {
          c.k_qs[row * per + kvh * HD + d] = (int8_t)qq;
          if ((d & 31u) == 0) c.k_d[row * (per / 32) + (kvh * HD + d) / 32] = (uint16_t)dh;
        }
      }
    }
  }
}

// 16 int8 -> f32
__device__ __forceinline__ void unpack16(const u32x4 w, float (&f)[16]) {
  const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 16; ++j) f[j] = (float)(int8_t)((a[j >> 2] >> ((j & 3) * 8)) & 0xffu);
}

// The prep of a decode step inside the chunk kernel (PREP): every
// workgroup builds its heads' q from q_raw (bias, RMSNorm, RoPE) in LDS,
// and the workgroup whose chunk holds the current position (the last one)
// also prepares that position's K and V, writes them to the cache row and
// uses them in place of the row it loaded before writing it.  Values are
// those of gqa_prep_kernel (same operations, same order).
//
// Normalise heads [0, nh) of buf (HD floats each) with the weight values
// w[j] = weight[lane + 64 j] (loaded beforehand): one wave per head, wave
// (g + first) % 4 taking head g.
template <int HD, int J>
__device__ __forceinline__ void norm_heads(float* buf, uint32_t nh, uint32_t first, const float (&w)[J], float eps,
                                           uint32_t wave, uint32_t lane) {
#pragma clang fp contract(off)
  for (uint32_t g = (wave + 4u - first % 4u) % 4u; g < nh; g += 4u) {
    float x[J];
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t d = lane + 64u * j;
      x[j] = d < HD ? buf[g * HD + d] : 0.0f;
      sq = __builtin_fmaf(x[j], x[j], sq);
    }
    sq = lane_reduce<64>(sq);
    const float scale = 1.0f / sqrtf(sq / (float)HD + eps);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t d = lane + 64u * j;
      if (d < HD) buf[g * HD + d] = x[j] * scale * w[j];
    }
  }
}

// LPT lanes per position (hd = 16 * LPT).  A chunk is 4 passes of the
// 4 * TPW positions the workgroup covers at once, so every lane requests its
// 4 K pieces and 4 V pieces (16 bytes each, plus scales) before any wait:
// one trip to memory per workgroup.
template <int LPT, bool PREP>
__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(KvQ8Dev c, const float* __restrict__ q, uint32_t group,
                                                             uint32_t seq0, uint32_t n_chunks,
                                                             float* __restrict__ part, GqaPrep pp, RopeFreq rf) {
  constexpr uint32_t HD = LPT * 16, TPW = 64 / LPT, PASSES = 4, CH = PASSES * 4 * TPW;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* s_q = smem;                       // [group][HD]
  float* s_p = smem + group * HD;          // [group][CH] scores, then exp(s - m)
  float* s_red = s_p + group * CH;         // [4 waves][4 heads][HD] reduction space
  // PREP only: [HD / 2][2] sin, cos; [HD] current k; [2][HD] int8 K, V; [2][HD / 32] scale bits
  float* s_cs = s_red + 16u * HD;
  float* s_k = s_cs + HD;
  int8_t* s_q8 = reinterpret_cast<int8_t*>(s_k + HD);
  uint16_t* s_d8 = reinterpret_cast<uint16_t*>(s_q8 + 2u * HD);
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t slot = lane / LPT, sub = lane % LPT;
  const uint32_t kvh = blockIdx.x, ck = blockIdx.y;
  if constexpr (PREP) {
    if (pp.dpos) seq0 = min(pp.dpos[0], c.max_seq - 1u) + 1u;   // device position (one token)
  }
  const uint32_t seq_len = seq0 + blockIdx.z;             // token z sees positions [0, seq0 + z)
  const uint32_t t0 = ck * CH;
  if (t0 >= seq_len) return;                              // a chunk past this token's positions
  const uint32_t n = min(seq_len - t0, CH);
  if constexpr (!PREP) q += (size_t)blockIdx.z * c.n_kv * group * HD;
  part += (size_t)blockIdx.z * c.n_kv * group * n_chunks * (HD + 2);
  const uint32_t row_q = c.n_kv * HD, row_d = c.n_kv * (HD / 32);
  const float scale = 1.0f / sqrtf((float)HD);

  // q first (small, cached), then every K and V piece of the chunk.  Every
  // early load is unconditional (clamped index) and combined only where it is
  // used: the memory counter drains in order, so a load that has to be waited
  // for inside a branch, or one issued after the cache rows, makes the wave
  // wait for everything issued before it.
  constexpr uint32_t R = kMaxGroup * HD / kThreads + 1;
  const uint32_t nq = group * HD;
  float qv[R], qb[R];
#pragma unroll
  for (uint32_t r = 0; r < R; ++r) {
    const uint32_t i = min(tid + r * kThreads, nq - 1u);
    if constexpr (PREP) {
      const uint32_t off = (kvh * group + i / HD) * (pp.gated ? 2u : 1u) * HD + i % HD;
      qv[r] = pp.q_raw[off];
      qb[r] = (pp.q_bias ? pp.q_bias : pp.q_raw)[off];
    } else {
      qv[r] = q[(size_t)kvh * nq + i];
    }
  }
  // PREP: the current position's k and v (and biases), and this lane's
  // rotation frequency, loaded by every workgroup before the cache rows.
  constexpr int JP = PREP ? (HD >= 64 ? HD / 64 : 1) : 1;
  float kc[JP], vc[JP], kbs[JP], vbs[JP], wq[JP], wk[JP];
  float fr = 0.0f;
  if constexpr (PREP) {
    const size_t base = (size_t)kvh * HD;
    const float* kb = pp.k_bias ? pp.k_bias : pp.k_cur;
    const float* vb = pp.v_bias ? pp.v_bias : pp.v_cur;
    const float* qn = pp.q_norm ? pp.q_norm : pp.k_cur;
    const float* kn = pp.k_norm ? pp.k_norm : pp.k_cur;
#pragma unroll
    for (int j = 0; j < JP; ++j) {
      const uint32_t d = min(lane + 64u * j, HD - 1u);
      kc[j] = pp.k_cur[base + d];
      vc[j] = pp.v_cur[base + d];
      kbs[j] = kb[base + d];
      vbs[j] = vb[base + d];
      wq[j] = qn[d];
      wk[j] = kn[d];
    }
    fr = rf.f[(tid - 64u) & 127u];
    asm volatile("" ::: "memory");   // keep the loads above ahead of the cache rows
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
  for (uint32_t r = 0; r < R; ++r) {
    const uint32_t i = tid + r * kThreads;
    if (i < nq) s_q[i] = PREP && pp.q_bias ? qv[r] + qb[r] : qv[r];
  }
  if constexpr (PREP) {
#pragma clang fp contract(off)
    constexpr int J = HD >= 64 ? HD / 64 : 1;
    const uint32_t pos = seq_len - 1u;
    const bool cur = pos - t0 < CH;                       // this chunk holds the current position
    if (cur && wave == 0) {                               // the current position's k, raw
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const uint32_t d = lane + 64u * j;
        if (d < HD) s_k[d] = pp.k_bias ? kc[j] + kbs[j] : kc[j];
      }
    }
    lds_barrier();
    // sine and cosine of pair i by thread 64 + i (waves 1 and 2), beside the
    // norms and the V quantisation
    if (tid >= 64u && tid - 64u < pp.half) {
      const float th = (float)(pp.dpos ? pp.dpos[1] : pp.rope_pos) * fr;
      double sd, cd;
      sincos((double)th, &sd, &cd);
      s_cs[2u * (tid - 64u)] = (float)sd;
      s_cs[2u * (tid - 64u) + 1u] = (float)cd;
    }
    if (pp.q_norm) norm_heads<HD>(s_q, group, 0, wq, pp.eps, wave, lane);
    if (cur && pp.k_norm) norm_heads<HD>(s_k, 1, group, wk, pp.eps, wave, lane);
    if (cur) {
      // V quantised as it is, alongside the norms: wave 3 - j takes values
      // lane + 64 j
#pragma unroll
      for (int j = 0; j < J; ++j) {
        if (wave != 3u - (uint32_t)j) continue;
        const uint32_t d = lane + 64u * j;
        const float vv = d < HD ? (pp.v_bias ? vc[j] + vbs[j] : vc[j]) : 0.0f;
        uint32_t dh;
        const int qq = q8_lane(vv, dh);
        if (d < HD) {
          s_q8[HD + d] = (int8_t)qq;
          if ((d & 31u) == 0) s_d8[HD / 32 + d / 32] = (uint16_t)dh;
        }
      }
    }
    lds_barrier();
    if (pp.half) {
      const uint32_t nh = group + (cur ? 1u : 0u);
      for (uint32_t idx = tid; idx < nh * pp.half; idx += kThreads) {
        const uint32_t g = idx / pp.half, i = idx - g * pp.half;
        float* v = g < group ? s_q + g * HD : s_k;
        const uint32_t i0 = pp.neox ? i : 2u * i, i1 = pp.neox ? i + pp.half : 2u * i + 1u;
        const float sn = s_cs[2u * i], cs = s_cs[2u * i + 1u];
        const float x0 = v[i0], x1 = v[i1];
        v[i0] = x0 * cs - x1 * sn;
        v[i1] = x0 * sn + x1 * cs;
      }
      lds_barrier();
    }
    if (cur) {
      // K quantised: wave j takes values lane + 64 j
#pragma unroll
      for (int j = 0; j < J; ++j) {
        if (wave != (uint32_t)j) continue;
        const uint32_t d = lane + 64u * j;
        uint32_t dh;
        const int qq = q8_lane(d < HD ? s_k[d] : 0.0f, dh);
        if (d < HD) {
          s_q8[d] = (int8_t)qq;
          if ((d & 31u) == 0) s_d8[d / 32] = (uint16_t)dh;
        }
      }
      lds_barrier();
    }
  } else {
    __syncthreads();
  }
  // PREP: the current row's K / V pieces of this lane, taken in place of the
  // loaded ones (stale: the row is written at the end) by the lanes whose
  // (clamped) position is the current one, at each use.
  u32x4 fk{}, fv{};
  uint32_t fkd = 0, fvd = 0;
  bool here[PASSES];
#pragma unroll
  for (uint32_t p = 0; p < PASSES; ++p) here[p] = false;
  if constexpr (PREP) {
    fk = *reinterpret_cast<const u32x4*>(s_q8 + sub * 16u);
    fv = *reinterpret_cast<const u32x4*>(s_q8 + HD + sub * 16u);
    fkd = s_d8[sub / 2u];
    fvd = s_d8[HD / 32 + sub / 2u];
    const uint32_t pos = seq_len - 1u;
#pragma unroll
    for (uint32_t p = 0; p < PASSES; ++p) here[p] = t0 + (tl[p] < n ? tl[p] : n - 1) == pos;
  }

  // ---- scores
#pragma unroll
  for (uint32_t p = 0; p < PASSES; ++p) {
    float kf[16];
    unpack16(here[p] ? fk : kw[p], kf);
    for (uint32_t g = 0; g < group; ++g) {
      const float* qg = s_q + g * HD + sub * 16u;
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = __builtin_fmaf(qg[j], kf[j], acc);
      acc *= f16_to_f32_exact(here[p] ? fkd : kdb[p]);
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
    unpack16(here[p] ? fv : vw[p], vf[p]);
    const float vd = f16_to_f32_exact(here[p] ? fvd : vdb[p]);
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
  if constexpr (PREP) {
    // the current position's K and V rows, from LDS, once nothing waits on them
    const uint32_t pos = seq_len - 1u;
    if (pos - t0 < CH && wave == 0) {
      const size_t vo = (size_t)pos * row_q + (size_t)kvh * HD, so = (size_t)pos * row_d + kvh * (HD / 32);
      for (uint32_t w = lane; w < HD / 2u; w += 64u) {      // 4 bytes a lane: K words, then V words
        const bool is_v = w >= HD / 4u;
        const uint32_t o = (is_v ? w - HD / 4u : w) * 4u;
        *reinterpret_cast<uint32_t*>((is_v ? c.v_qs : c.k_qs) + vo + o) =
            *reinterpret_cast<const uint32_t*>(s_q8 + (is_v ? HD : 0u) + o);
      }
      if (lane < HD / 16u) {
        const bool is_v = lane >= HD / 32u;
        const uint32_t b = is_v ? lane - HD / 32u : lane;
        (is_v ? c.v_d : c.k_d)[so + b] = s_d8[(is_v ? HD / 32u : 0u) + b];
      }
    }
  }
}

// Merge: workgroup (head, 64 dimensions, token) of W waves.  The chunks'
// maximum first, then wave w sums chunks w, w + W, ... (sixteen at a time in
// flight), then the waves' sums are added in wave order.  W = 16 for a long
// decode sequence; a prefill token has few chunks, and fewer waves serve it.
template <uint32_t W>
__global__ __launch_bounds__(W * 64) void attn_merge_kernel(const float* __restrict__ part, uint32_t hd,
                                                            uint32_t chunk_stride, uint32_t chunk, uint32_t seq0,
                                                            const float* __restrict__ gate, uint32_t gate_stride,
                                                            const float* __restrict__ gate_bias,
                                                            float* __restrict__ out,
                                                            const uint32_t* __restrict__ dpos) {
#pragma clang fp contract(off)
  __shared__ float s_m[W], s_acc[W][64], s_l[W];
  const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t d = blockIdx.y * 64u + lane;
  const uint32_t z = blockIdx.z, n_head = gridDim.x;
  if (dpos) seq0 = dpos[0] + 1u;   // device position (one token); clamped below like the chunks
  const uint32_t n_chunks = min((seq0 + z + chunk - 1u) / chunk, chunk_stride);   // token z's chunks
  const size_t stride = hd + 2;
  const float* ph = part + ((size_t)z * n_head + h) * chunk_stride * stride;
  if (gate) gate += (size_t)z * n_head * gate_stride;
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
  constexpr int U = 16;   // chunks in flight per lane
  uint32_t c0 = wave;
  for (; c0 + W * (U - 1) < n_chunks; c0 += W * U) {
    float mc[U], lc[U], ac[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float* pc = ph + (size_t)(c0 + W * u) * stride;
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
  if (c0 < n_chunks) {
    // the last, partial batch: loads from clamped indices, all in flight
    // together, only the valid ones used
    float mc[U], lc[U], ac[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float* pc = ph + (size_t)min(c0 + W * u, n_chunks - 1u) * stride;
      mc[u] = pc[0];
      lc[u] = pc[1];
      ac[u] = pc[2 + dc];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + W * u < n_chunks) {   // uniform across the wave; the valid chunks are a prefix
        const float e = expf(mc[u] - m);
        l += lc[u] * e;
        acc += ac[u] * e;
      }
    }
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
  if (gate) {
    float g = gate[(size_t)h * gate_stride + d];
    if (gate_bias) g = g + gate_bias[(size_t)h * gate_stride + d];
    o *= 1.0f / (1.0f + expf(-g));
  }
  out[(size_t)h * hd + d] = o;
}

// ---- prefill: causal attention of a batch of prepared queries on MFMA ------
// Workgroup (kv head, block of tq tokens, position segment): 4 waves, 32
// query rows each; row r is token tb + r / group, query head kvh * group +
// r % group.  Positions are walked in tiles of 32 up to the block's last
// token (or the segment's end); K and V of a tile are dequantised into LDS,
// the next tile's bytes already in flight.  Per wave and tile:
//   S^T (32 positions x 32 rows) = K Q^T;
//   online softmax: each lane owns one row (lane % 32) and 16 of the tile's
//     positions, its partner lane ^ 32 the other 16; scores in base 2, the
//     weights taken against a reference that moves only when the row's max
//     passes it by more than 8, so O^T and l are rescaled on few tiles;
//   O^T (hd x 32 rows) += V^T P^T, step s taking the positions the lanes hold
//     in accumulator registers 8 s .. 8 s + 7.
// Every row keeps its own running sums, so a rescale is one factor per lane;
// positions after a row's token are masked to -inf.  The products run on
// v_mfma_f32_32x32x16_bf16 with split operands:
//   S^T: A = K's int8 values (exact in bf16), B = Q^T as three bf16 terms
//     (hi + mid + lo represent an f32 exactly), one fresh accumulator per
//     32-dim block, then S += d_k[position][block] * T in f32 -- the scores
//     carry fp32 accuracy;
//   O^T: A = V dequantised (int8 x f16 scale) as two bf16 terms, B = the
//     weights as two bf16 terms, hi*hi + hi*lo + lo*hi (relative error
//     about 2^-17 per product).
// K tile in LDS as bf16 [position][hd + 8]; V^T hi and lo as bf16
// [dim][32 + 8] with the positions of each 16 stored in the order the
// weights sit in the accumulator (bits 2 and 3 of the position swapped), so
// one 16-byte read gives a lane its 8 operands.  A thread dequantises two
// adjacent positions x 8 dims of the tile.
template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_bf16_kernel(KvQ8Dev c, const float* __restrict__ q,
                                                                const float* __restrict__ gate,
                                                                float* __restrict__ out, float* __restrict__ part,
                                                                uint32_t n_head, uint32_t group, uint32_t tq,
                                                                uint32_t pos0, uint32_t batch) {
  constexpr uint32_t TP = 32, NST = HD / 16, NB = HD / 32;
  constexpr uint32_t KST = HD + 8, VST = TP + 8;        // bf16 strides
  constexpr uint32_t NPC = (TP / 2) * (HD / 8);         // pieces: 2 positions x 8 dims
  constexpr uint32_t PER = (NPC + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint16_t s_kb[TP * KST];
  __shared__ __attribute__((aligned(16))) float s_kd[NB * TP];
  __shared__ __attribute__((aligned(16))) uint16_t s_vh[HD * VST];
  __shared__ __attribute__((aligned(16))) uint16_t s_vl[HD * VST];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, h = lane >> 5, col = lane & 31u;
  const uint32_t kvh = blockIdx.x, tb = blockIdx.y * tq;
  const uint32_t t_end = min(batch, tb + tq);
  const uint32_t r = wave * 32u + col;
  const uint32_t tk = tb + r / group, g = r % group;
  const bool live = r < tq * group && tk < batch;
  const uint32_t tkc = live ? tk : tb;                  // spare rows shadow the block's first token
  const uint32_t my_pos = pos0 + tkc;
  const uint32_t head = kvh * group + g;
  const uint32_t last = pos0 + t_end - 1u;
  const uint32_t tile0 = blockIdx.z * kSegTiles;
  if (tile0 * TP > last) return;
  const uint32_t n_tiles = gridDim.z == 1 ? last / TP + 1u : min(last / TP + 1u, tile0 + kSegTiles);
  const uint32_t row_q = c.n_kv * HD, row_d = c.n_kv * (HD / 32);
  const float scale2 = 1.4426950408889634f / sqrtf((float)HD);

  // Q^T operand: lane holds row col's dims 16 st + 8 h .. + 7, three terms
  bf16x8 q0[NST], q1[NST], q2[NST];
  {
    const float* qr = q + ((size_t)tkc * n_head + head) * HD + 8u * h;
#pragma unroll
    for (uint32_t st = 0; st < NST; ++st) {
      const float4 a = *reinterpret_cast<const float4*>(qr + 16u * st);
      const float4 b = *reinterpret_cast<const float4*>(qr + 16u * st + 4u);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const __bf16 t0 = (__bf16)v[j];
        const float r1 = v[j] - (float)t0;
        const __bf16 t1 = (__bf16)r1;
        q0[st][j] = t0;
        q1[st][j] = t1;
        q2[st][j] = (__bf16)(r1 - (float)t1);
      }
    }
  }
  float16v o[NB];
#pragma unroll
  for (uint32_t b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[b][i] = 0.0f;
  float m_run = -__builtin_inff(), l_run = 0.0f;

  // piece ch: positions 2 (ch % 16) + {0, 1}, dims 8 (ch / 16) .. + 7
  uint2 kq[PER][2], vq[PER][2];
  uint32_t kdb[PER][2], vdb[PER][2];
  auto fetch = [&](uint32_t p0) {
#pragma unroll
    for (uint32_t u = 0; u < PER; ++u) {
      const uint32_t ch = min(tid + 256u * u, NPC - 1u);
      const uint32_t dg = ch / 16u;
#pragma unroll
      for (uint32_t e = 0; e < 2; ++e) {
        const uint32_t p = min(p0 + 2u * (ch % 16u) + e, last);
        const size_t qo = (size_t)p * row_q + kvh * HD + 8u * dg, dof = (size_t)p * row_d + kvh * (HD / 32) + dg / 4u;
        kq[u][e] = *reinterpret_cast<const uint2*>(c.k_qs + qo);
        vq[u][e] = *reinterpret_cast<const uint2*>(c.v_qs + qo);
        kdb[u][e] = c.k_d[dof];
        vdb[u][e] = c.v_d[dof];
      }
    }
  };
  fetch(tile0 * TP);

  for (uint32_t T = tile0; T < n_tiles; ++T) {
    const uint32_t p0 = T * TP;
#pragma unroll
    for (uint32_t u = 0; u < PER; ++u) {
      const uint32_t ch = tid + 256u * u;
      if (ch < NPC) {
        const uint32_t pq = ch % 16u, dg = ch / 16u;
        // slot of position 2 pq within its 16: bits 2 and 3 swapped
        const uint32_t rr = (2u * pq) & 15u;
        const uint32_t slot = (2u * pq & ~15u) | ((rr & 4u) << 1) | ((rr & 8u) >> 1) | (rr & 3u);
        uint32_t vh_w[8], vl_w[8];
#pragma unroll
        for (uint32_t e = 0; e < 2; ++e) {
          const uint32_t pp = 2u * pq + e;
          const uint32_t w2[2] = {kq[u][e].x, kq[u][e].y};
          uint32_t kb4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float f0 = (float)(int8_t)((w2[j >> 1] >> (16 * (j & 1))) & 0xffu);
            const float f1 = (float)(int8_t)((w2[j >> 1] >> (16 * (j & 1) + 8)) & 0xffu);
            kb4[j] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);   // exact
          }
          *reinterpret_cast<u32x4*>(s_kb + pp * KST + 8u * dg) = u32x4{kb4[0], kb4[1], kb4[2], kb4[3]};
          if ((dg & 3u) == 0) s_kd[(dg / 4u) * TP + pp] = f16_to_f32_exact(kdb[u][e]);
          const float vd = f16_to_f32_exact(vdb[u][e]);
          const uint32_t v2[2] = {vq[u][e].x, vq[u][e].y};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float v = (float)(int8_t)((v2[j >> 2] >> (8 * (j & 3))) & 0xffu) * vd;
            const __bf16 hi = (__bf16)v;
            const __bf16 lo = (__bf16)(v - (float)hi);
            const uint32_t hb = __builtin_bit_cast(uint16_t, hi), lb = __builtin_bit_cast(uint16_t, lo);
            vh_w[j] = e ? (vh_w[j] | (hb << 16)) : hb;
            vl_w[j] = e ? (vl_w[j] | (lb << 16)) : lb;
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          *reinterpret_cast<uint32_t*>(s_vh + (8u * dg + j) * VST + slot) = vh_w[j];
          *reinterpret_cast<uint32_t*>(s_vl + (8u * dg + j) * VST + slot) = vl_w[j];
        }
      }
    }
    if (T + 1u < n_tiles) fetch(p0 + TP);
    lds_barrier();

    // S^T = sum over 32-dim blocks of d_k * (K Q^T over the block)
    float16v sacc;
#pragma unroll
    for (int i = 0; i < 16; ++i) sacc[i] = 0.0f;
#pragma unroll
    for (uint32_t b = 0; b < NB; ++b) {
      float16v tacc;
#pragma unroll
      for (int i = 0; i < 16; ++i) tacc[i] = 0.0f;
#pragma unroll
      for (uint32_t t = 0; t < 2; ++t) {
        const uint32_t st = 2u * b + t;
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(s_kb + col * KST + 16u * st + 8u * h);
        tacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, q0[st], tacc, 0, 0, 0);
        tacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, q1[st], tacc, 0, 0, 0);
        tacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, q2[st], tacc, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 dk = *reinterpret_cast<const float4*>(s_kd + b * TP + 8u * j + 4u * h);
        sacc[4 * j] = __builtin_fmaf(dk.x, tacc[4 * j], sacc[4 * j]);
        sacc[4 * j + 1] = __builtin_fmaf(dk.y, tacc[4 * j + 1], sacc[4 * j + 1]);
        sacc[4 * j + 2] = __builtin_fmaf(dk.z, tacc[4 * j + 2], sacc[4 * j + 2]);
        sacc[4 * j + 3] = __builtin_fmaf(dk.w, tacc[4 * j + 3], sacc[4 * j + 3]);
      }
    }

    // online softmax (as the fp32 kernel): base 2, lazy reference
    float pm = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t pos = p0 + 8u * (i >> 2) + 4u * h + (i & 3);
      const float sv = pos <= my_pos ? sacc[i] * scale2 : -__builtin_inff();
      sacc[i] = sv;
      pm = fmaxf(pm, sv);
    }
    pm = xor32_pair(pm, true);
    const bool move = pm > m_run + 8.0f;
    const float m_new = move ? pm : m_run;
    const float alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    const bool none = m_new == -__builtin_inff();
    float ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e = none ? 0.0f : __builtin_amdgcn_exp2f(sacc[i] - m_new);
      sacc[i] = e;
      ps += e;
    }
    ps = xor32_pair(ps, false);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    const bool rescale = __builtin_amdgcn_ballot_w64(move) != 0;

    // weights as two bf16 terms; step s takes accumulator registers 8 s .. + 7
    bf16x8 ph[2], pl[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const __bf16 hi = (__bf16)sacc[i];
      ph[i >> 3][i & 7] = hi;
      pl[i >> 3][i & 7] = (__bf16)(sacc[i] - (float)hi);
    }
#pragma unroll
    for (uint32_t b = 0; b < NB; ++b) {
      if (rescale) {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[b][i] *= alpha;
      }
#pragma unroll
      for (uint32_t t = 0; t < 2; ++t) {
        const uint32_t off = (32u * b + col) * VST + 16u * t + 8u * h;
        const bf16x8 ah = *reinterpret_cast<const bf16x8*>(s_vh + off);
        const bf16x8 al = *reinterpret_cast<const bf16x8*>(s_vl + off);
        o[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, ph[t], o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, pl[t], o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, ph[t], o[b], 0, 0, 0);
      }
    }
    lds_barrier();
  }

  if (!live) return;
  if (gridDim.z > 1) {
    float* pr = part + (((size_t)tk * n_head + head) * gridDim.z + blockIdx.z) * (HD + 2);
    if (h == 0) {
      pr[0] = m_run;
      pr[1] = l_run;
    }
#pragma unroll
    for (uint32_t b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) pr[2 + 32u * b + 8u * (i >> 2) + 4u * h + (i & 3)] = o[b][i];
    return;
  }
  const float inv = 1.0f / l_run;
  const size_t base = ((size_t)tk * n_head + head) * HD;
  float gv[NB * 16];
  const float* gp = gate ? gate + base : q;
#pragma unroll
  for (uint32_t b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 16; ++i) gv[b * 16 + i] = gp[32u * b + 8u * (i >> 2) + 4u * h + (i & 3)];
#pragma unroll
  for (uint32_t b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v = o[b][i] * inv;
      if (gate) v *= 1.0f / (1.0f + expf(-gv[b * 16 + i]));
      out[base + 32u * b + 8u * (i >> 2) + 4u * h + (i & 3)] = v;
    }
}

// Merge of the prefill's position segments: one wave per (token, head);
// segments in ascending order, exp2(m_s - m) rescaling (the segments' scores
// and references are base 2), divide, gate.
__global__ __launch_bounds__(256) void attn_prefill_merge_kernel(const float* __restrict__ part, uint32_t hd,
                                                                 uint32_t n_head, uint32_t n_seg, uint32_t seg_len,
                                                                 uint32_t pos0, uint32_t batch,
                                                                 const float* __restrict__ gate,
                                                                 float* __restrict__ out) {
#pragma clang fp contract(off)
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);   // token * n_head + head
  if (row >= batch * n_head) return;
  const uint32_t tk = row / n_head;
  const uint32_t ns = min(n_seg, (pos0 + tk) / seg_len + 1u);   // segments holding positions <= the token's
  const float* pr = part + (size_t)row * n_seg * (hd + 2);
  float m = -__builtin_inff();
  for (uint32_t sg = 0; sg < ns; ++sg) m = fmaxf(m, pr[(size_t)sg * (hd + 2)]);
  for (uint32_t d = lane; d < hd; d += 64u) {
    float l = 0.0f, acc = 0.0f;
    for (uint32_t sg = 0; sg < ns; ++sg) {
      const float* ps = pr + (size_t)sg * (hd + 2);
      const float e = ps[0] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(ps[0] - m);   // base-2 references
      l += ps[1] * e;
      acc += ps[2 + d] * e;
    }
    float v = acc / l;
    if (gate) v *= 1.0f / (1.0f + expf(-gate[(size_t)row * hd + d]));
    out[(size_t)row * hd + d] = v;
  }
}

template <int LPT, bool PREP>
hipError_t launch_chunks(const KvQ8Dev& c, const float* q, uint32_t group, uint32_t seq0, uint32_t n_chunks,
                         uint32_t batch, float* part, const GqaPrep& pp, const RopeFreq& rf, hipStream_t s) {
  constexpr uint32_t HD = LPT * 16, CH = 16u * (64u / LPT);
  size_t lds = ((size_t)group * HD + (size_t)group * CH + 16u * HD) * 4u;
  if (PREP) lds += 2u * HD * 4u + 2u * HD + 2u * (HD / 32u) * 2u;
  hipLaunchKernelGGL((attn_chunk_kernel<LPT, PREP>), dim3(c.n_kv, n_chunks, batch), dim3(kThreads), lds, s, c, q,
                     group, seq0, n_chunks, part, pp, rf);
  return hipGetLastError();
}

template <bool PREP>
hipError_t launch_chunks_hd(const KvQ8Dev& c, const float* q, uint32_t group, uint32_t seq0, uint32_t n_chunks,
                            uint32_t batch, float* part, const GqaPrep& pp, const RopeFreq& rf, hipStream_t s) {
  switch (c.hd) {
    case 32: return launch_chunks<2, PREP>(c, q, group, seq0, n_chunks, batch, part, pp, rf, s);
    case 64: return launch_chunks<4, PREP>(c, q, group, seq0, n_chunks, batch, part, pp, rf, s);
    case 128: return launch_chunks<8, PREP>(c, q, group, seq0, n_chunks, batch, part, pp, rf, s);
    case 256: return launch_chunks<16, PREP>(c, q, group, seq0, n_chunks, batch, part, pp, rf, s);
    default: return hipErrorInvalidValue;
  }
}

// The rotation frequencies powf(base, -2i / rdim), i < rdim / 2, with rdim =
// min(rope_dim, hd): a function of (freq_base, rdim) only, so the last table
// is kept per host thread.
const RopeFreq& rope_table(uint32_t rope_dim, float freq_base, uint32_t hd, uint32_t* half) {
  thread_local RopeFreq tab{};
  thread_local uint32_t tab_rdim = 0;
  thread_local float tab_base = 0.0f;
  const uint32_t rdim = std::min(rope_dim, hd);
  *half = rdim / 2u;
  if (*half && (tab_rdim != rdim || std::memcmp(&tab_base, &freq_base, sizeof(float)) != 0)) {
    for (uint32_t i = 0; i < *half; ++i) tab.f[i] = powf(freq_base, -(2.0f * (float)i) / (float)rdim);
    tab_rdim = rdim;
    tab_base = freq_base;
  }
  return tab;
}

// The merge: 16 waves per workgroup when there are few workgroups (a decode
// step: the chunks of one token spread over the waves), fewer when a batch
// already gives every CU workgroups (prefill: a token has few chunks).
hipError_t launch_merge(const float* part, uint32_t hd, uint32_t n_head, uint32_t batch, uint32_t n_chunks,
                        uint32_t chunk, uint32_t seq0, const float* gate, uint32_t gate_stride,
                        const float* gate_bias, float* out, hipStream_t s, const uint32_t* dpos = nullptr) {
  const dim3 grid(n_head, (hd + 63) / 64, batch);
  if ((size_t)grid.x * grid.y * grid.z < 512u)
    hipLaunchKernelGGL(attn_merge_kernel<16>, grid, dim3(16 * 64), 0, s, part, hd, n_chunks, chunk, seq0, gate,
                       gate_stride, gate_bias, out, dpos);
  else if (n_chunks >= 8)
    hipLaunchKernelGGL(attn_merge_kernel<4>, grid, dim3(4 * 64), 0, s, part, hd, n_chunks, chunk, seq0, gate,
                       gate_stride, gate_bias, out, dpos);
  else
    hipLaunchKernelGGL(attn_merge_kernel<1>, grid, dim3(64), 0, s, part, hd, n_chunks, chunk, seq0, gate,
                       gate_stride, gate_bias, out, dpos);
  return hipGetLastError();
}

// Positions per chunk: 4 passes of 4 waves x 64 / (hd / 16) positions.
uint32_t chunk_of(uint32_t hd) { return 16u * (64u / (hd / 16u)); }

template <int HD>
void launch_prep(const KvQ8Dev& c, const GqaPrep& a, const RopeFreq& rf, uint32_t batch, hipStream_t s) {
  hipLaunchKernelGGL(gqa_prep_kernel<HD>, dim3(batch), dim3(256), 0, s, c, a, rf);
}

}  // namespace

hipError_t launch_kv_append(const KvQ8Dev& c, const float* k, const float* v, uint32_t pos, hipStream_t s) {
  const uint32_t n = 2u * c.n_kv * c.hd;
  hipLaunchKernelGGL(kv_append_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s, c, k, v, pos);
  return hipGetLastError();
}

hipError_t launch_gqa_prep(const KvQ8Dev& c, GqaPrep a, uint32_t rope_dim, float freq_base, uint32_t batch,
                           hipStream_t s) {
  const RopeFreq& tab = rope_table(rope_dim, freq_base, c.hd, &a.half);
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
  hipError_t e = launch_chunks_hd<false>(c, q, group, seq0, n_chunks, batch, part, GqaPrep{}, RopeFreq{}, s);
  if (e != hipSuccess) return e;
  return launch_merge(part, c.hd, n_head, batch, n_chunks, chunk, seq0, gate, c.hd, nullptr, out, s);
}

// Causal attention of batch prepared queries (q, gate: [batch][n_head][hd])
// on MFMA: tokens at positions pos0 .. pos0 + batch - 1, every cache row up to
// the last written.  hd <= 128.  Positions are cut into segments of
// kSegTiles * 32 when there are more than one; ws then holds
// attn_prefill_workspace_bytes(...) of partial sums.
uint32_t prefill_segments(uint32_t pos0, uint32_t batch) {
  return (pos0 + batch - 1u) / (kSegTiles * 32u) + 1u;
}

size_t attn_prefill_workspace_bytes(uint32_t n_head, uint32_t hd, uint32_t pos0, uint32_t batch) {
  const uint32_t ns = prefill_segments(pos0, batch);
  return ns > 1 ? (size_t)batch * n_head * ns * (hd + 2) * sizeof(float) : 0;
}

hipError_t launch_attn_prefill(const KvQ8Dev& c, const float* q, const float* gate, float* out, uint32_t n_head,
                               uint32_t pos0, uint32_t batch, void* ws, hipStream_t s) {
  const uint32_t group = n_head / c.n_kv;
  if (group == 0 || group > kMaxGroup || batch == 0) return hipErrorInvalidValue;
  const uint32_t tq = 128u / group;
  const uint32_t blocks = (batch + tq - 1) / tq;
  const uint32_t ns = prefill_segments(pos0, batch);
  if (blocks > 65535u || ns > 65535u) return hipErrorInvalidValue;
  float* part = static_cast<float*>(ws);
  const dim3 grid(c.n_kv, blocks, ns);
  switch (c.hd) {
    case 32: hipLaunchKernelGGL(attn_prefill_bf16_kernel<32>, grid, dim3(256), 0, s, c, q, gate, out, part, n_head,
                                group, tq, pos0, batch); break;
    case 64: hipLaunchKernelGGL(attn_prefill_bf16_kernel<64>, grid, dim3(256), 0, s, c, q, gate, out, part, n_head,
                                group, tq, pos0, batch); break;
    case 128: hipLaunchKernelGGL(attn_prefill_bf16_kernel<128>, grid, dim3(256), 0, s, c, q, gate, out, part, n_head,
                                 group, tq, pos0, batch); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || ns == 1) return e;
  const uint32_t rows = batch * n_head;
  hipLaunchKernelGGL(attn_prefill_merge_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, part, c.hd, n_head, ns,
                     kSegTiles * 32u, pos0, batch, gate, out);
  return hipGetLastError();
}

// One decode step (a single token at row pp.pos, rope position pp.rope_pos)
// in two launches: the chunk kernel with the prep folded in, then the merge
// (the gate read from q_raw's gate halves).  ws holds
// attn_workspace_bytes(n_head, pp.pos + 1, n_kv, hd, 1).  With pp.dpos the
// position is read on the device: the grids cover the whole cache (chunks
// past the position return at once) and ws holds
// attn_workspace_bytes(n_head, max_seq, n_kv, hd, 1).
hipError_t launch_attn_step(const KvQ8Dev& c, GqaPrep pp, uint32_t rope_dim, float freq_base, float* out, void* ws,
                            hipStream_t s) {
  const uint32_t group = pp.n_head / c.n_kv;
  if (group == 0 || group > kMaxGroup) return hipErrorInvalidValue;
  const RopeFreq& tab = rope_table(rope_dim, freq_base, c.hd, &pp.half);
  const uint32_t chunk = chunk_of(c.hd), seq0 = pp.dpos ? c.max_seq : pp.pos + 1u;
  const uint32_t n_chunks = (seq0 + chunk - 1) / chunk;
  if (n_chunks > 65535u) return hipErrorInvalidValue;
  float* part = static_cast<float*>(ws);
  hipError_t e = launch_chunks_hd<true>(c, nullptr, group, seq0, n_chunks, 1, part, pp, tab, s);
  if (e != hipSuccess) return e;
  const float* gate = pp.gated ? pp.q_raw + c.hd : nullptr;
  const float* gate_bias = pp.gated && pp.q_bias ? pp.q_bias + c.hd : nullptr;
  return launch_merge(part, c.hd, pp.n_head, 1, n_chunks, chunk, seq0, gate, 2u * c.hd, gate_bias, out, s,
                      pp.dpos);
}

}  // namespace vxt
