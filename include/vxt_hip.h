/*
 * vxt_hip.h -- C ABI of the MI355X (gfx950) compressed-weight matmul engine.
 *
 * Drop-in for vxg-tensor's GPU matmul boundary: the same create / upload /
 * run / free life cycle, opaque handles, caller-provided error buffers and
 * synchronous semantics as the reference's Metal bridge
 * (crates/vxg-tensor/src/metal_ffi.rs:27-49, native/metal_gemv.mm:258-475),
 * with a HIP engine behind it.  Plain pointers and sizes only.
 *
 * Conventions (kept from the reference):
 *   - constructors return an opaque pointer, NULL on failure, with a
 *     NUL-terminated message in (err, err_cap) (metal_gemv.mm:49-52);
 *   - every other call returns VXT_OK (0) or a negative VXT_E_* code and
 *     writes a message; no C++ exception crosses this boundary;
 *   - uploads COPY the host planes (host memory is not retained after return);
 *     device memory is released by vxt_hip_free_tensor / vxt_hip_destroy;
 *   - host-pointer entry points are synchronous: outputs are in host memory
 *     when they return (metal_gemv.mm:444-472);
 *   - one context is used by one thread at a time (metal_ffi.rs:96); tensors
 *     may be shared between threads.
 *
 * Layout conventions: rows = N (output features), cols = K (reduction axis),
 * batch_m = M (tokens).  y[m*rows + r] = sum_c W[r,c] * x[m*cols + c].
 */
#ifndef VXT_HIP_H
#define VXT_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define VXT_API __attribute__((visibility("default")))
#else
#define VXT_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define VXT_OK 0
#define VXT_E_ARG (-1)         /* null handle or pointer, bad enum value      */
#define VXT_E_SHAPE (-2)       /* sizes do not match the tensor / each other  */
#define VXT_E_FORMAT (-3)      /* corrupt planes (lengths, CSR indices)       */
#define VXT_E_DEVICE (-4)      /* HIP runtime error (message carries it)      */
#define VXT_E_UNSUPPORTED (-5) /* valid request this build does not support   */

/* ---- element types for activations / outputs --------------------------- */
#define VXT_DTYPE_F32 0u
#define VXT_DTYPE_BF16 1u

/* FFN activations (llm_cpu.rs:457-464) */
#define VXT_ACT_SILU 0u       /* silu(g) * u, llm_ops.rs:39-41                  */
#define VXT_ACT_GELU_TANH 1u  /* gelu_tanh_f32(g) * u, llm_prefill.rs:66-71     */

/* vxt_hip_norm_matmul_dev modes */
#define VXT_NORM_PLAIN 0u          /* y = W x                                   */
#define VXT_NORM_GLU_SILU 1u       /* y = silu(gate . x) * (up . x)             */
#define VXT_NORM_GLU_GELU_TANH 2u  /* y = gelu_tanh(gate . x) * (up . x)        */

/* ---- tensor kinds (kind 2 = codebook, as VxtMetalOp.kind in
 *      native/metal_internal.h:14) ---------------------------------------- */
#define VXT_KIND_CB4 2u     /* CodebookMatrix, bits = 4 (codebook.rs:9-24)   */
#define VXT_KIND_Q4_0 4u    /* Q4_0Matrix blocks of 32 (q4_0.rs:7-14)        */
#define VXT_KIND_Q8_0 8u    /* GGUF Q8_0 / KvQ8Block rows (llm_prefill.rs:17) */
#define VXT_KIND_CB4_G64 9u /* cb4 with a per-64-group fp16 codebook         */

/* Borrowed view of a CodebookMatrix (codebook.rs:9-24), bits = 4.
 * Mirrors the sub-matrix descriptor the reference passes to its device packer
 * (metal_cb4_fast_ffi.rs:38-85).  Plane lengths are validated as the archive
 * reader does (format.rs:423-440, :565-574). */
typedef struct VxtCb4View {
    uint32_t bits;         /* must be 4                                     */
    uint32_t rows;
    uint32_t cols;
    uint32_t padded_cols;  /* multiple of 128, >= cols                      */
    const float* centroids;          /* [16]                                */
    const uint16_t* scales_f16;      /* [rows * padded_cols/128]            */
    size_t n_scales;
    const uint32_t* packed_words;    /* [rows * padded_cols/8]              */
    size_t n_words;
    const uint32_t* outlier_row_ptr; /* [rows + 1]                          */
    size_t n_row_ptr;
    const uint32_t* outliers_packed; /* [n_outliers], col | f16 << 16       */
    size_t n_outliers;
} VxtCb4View;

/* Borrowed view of a cb4-g64 matrix: idx[r*padded_cols/2 + c/2] >> 4*(c%2)
 * is column c's index, lut_f16[(r*padded_cols/64 + c/64)*16 + q] its value. */
typedef struct VxtCb4G64View {
    uint32_t rows;
    uint32_t cols;
    uint32_t padded_cols;  /* multiple of 64, >= cols                       */
    uint32_t reserved;
    const uint8_t* idx;              /* [rows * padded_cols/2]              */
    size_t n_idx;
    const uint16_t* lut_f16;         /* [rows * padded_cols/64 * 16]        */
    size_t n_lut;
} VxtCb4G64View;

/* One GEMV job of vxt_hip_run_multi: a tensor and its host output
 * (the (&GpuPackedTensor, &mut [f32]) pairs of metal.rs:466-481). */
typedef struct VxtHipJob {
    void* tensor;
    float* y;              /* host, [rows]                                  */
} VxtHipJob;

/* ---- context ------------------------------------------------------------ */

/* Replaces vxt_metal_create (metal_ffi.rs:28-33).  device < 0 selects the
 * current HIP device.  Writes the device name into dev_name. */
VXT_API void* vxt_hip_create(int32_t device, char* dev_name, size_t dev_name_cap, char* err,
                     size_t err_cap);

/* Replaces vxt_metal_destroy (metal_ffi.rs:34).  Frees every tensor the
 * context still owns. NULL is a no-op. */
VXT_API void vxt_hip_destroy(void* ctx);

/* ---- weights: upload with device-residency re-layout -------------------- */

/* Replaces GpuPackedInner::upload_codebook (metal.rs:162-177) over
 * vxt_metal_upload (metal_ffi.rs:35). Returns a tensor handle or NULL. */
VXT_API void* vxt_hip_upload_cb4(void* ctx, const VxtCb4View* view, char* err, size_t err_cap);

/* Row-concatenation of 1..3 CodebookMatrix parts with equal cols into one
 * tensor ([q;k;v], [gate;up]); each part keeps its own centroid table and the
 * CSR row pointers are rebased.  Replaces VxtCb4FastConcatMat::from_subs and
 * the arena packer it feeds (metal_cb4_fast_ffi.rs:89-104,
 * metal_cb4_fast.mm:6-44,140-171). */
VXT_API void* vxt_hip_upload_cb4_concat(void* ctx, const VxtCb4View* subs, uint32_t n_subs, char* err,
                                size_t err_cap);

/* cb4-g64 upload (no reference counterpart: the decode-benchmark layout). */
VXT_API void* vxt_hip_upload_cb4_g64(void* ctx, const VxtCb4G64View* view, char* err,
                             size_t err_cap);

/* Raw GGUF Q8_0 bytes as GgufView::tensor_bytes returns them
 * (gguf.rs:160-172): rows * ceil(cols/32) blocks of 34 bytes.  Replaces the
 * reference's load-time f32 expansion (gguf.rs:223-229, llm.rs:164). */
VXT_API void* vxt_hip_upload_q8_0(void* ctx, uint32_t rows, uint32_t cols, const uint8_t* blocks,
                          size_t n_bytes, char* err, size_t err_cap);

/* Q4_0Matrix planes (q4_0.rs:7-14): padded_cols = ceil(cols/32)*32,
 * scales_f16[rows * padded_cols/32], qs_words[rows * padded_cols/32 * 4]
 * (byte j of a block: column j low nibble, column j + 16 high nibble).
 * Replaces upload_q4_0 (metal.rs:179-187); plane rules as format.rs:453-462.
 * The device holds both planes as given (4.5 bits per weight, kind
 * VXT_KIND_Q4_0 in vxt_hip_tensor_info): the GEMV streams the nibbles
 * (the reference's vxt_gemv_q4_0, vxt_gemv.metal:461-520), prefill
 * decodes them into the GEMM's weight panel; dequant bit-exact with
 * decode_row (q4_0.rs:77-97). */
VXT_API void* vxt_hip_upload_q4_0(void* ctx, uint32_t rows, uint32_t cols, uint32_t padded_cols,
                                  const uint16_t* scales_f16, size_t n_scales, const uint32_t* qs_words,
                                  size_t n_words, char* err, size_t err_cap);

/* Device-to-device copy of an uploaded tensor (same layout, new memory). */
VXT_API void* vxt_hip_clone_tensor(void* tensor, char* err, size_t err_cap);

/* Replaces vxt_metal_free_buffer (metal_ffi.rs:36). NULL is a no-op. */
VXT_API void vxt_hip_free_tensor(void* tensor);

/* kind (VXT_KIND_*), rows, cols, and device bytes of the resident layout. */
VXT_API int vxt_hip_tensor_info(void* tensor, uint32_t* kind, uint32_t* rows, uint32_t* cols,
                        uint64_t* device_bytes);

/* ---- host-pointer entry points (synchronous) ---------------------------- */

/* Replaces vxt_metal_run_multi (metal_ffi.rs:38-48): every job's GEMV over the
 * same f32 x (x_elems >= every job's cols; extra elements are ignored), run
 * `iters` times; gpu_ms (may be NULL) receives the summed kernel time.  Used by
 * MetalEngine::run_multi_same_x (metal.rs:466) and run_gemv (metal.rs:535). */
VXT_API int vxt_hip_run_multi(void* ctx, const float* x, uint32_t x_elems, const VxtHipJob* jobs,
                      uint32_t n_jobs, uint32_t iters, double* gpu_ms, char* err,
                      size_t err_cap);

/* Replaces PackedTensor::gemm_cpu (llm_prefill.rs:160): y_batch[batch_m*rows]
 * = x_batch[batch_m*cols] times W^T, f32 in and out; batch_m == 1 is the
 * GEMV (llm_prefill.rs:168-171). */
VXT_API int vxt_hip_gemm(void* ctx, void* tensor, const float* x_batch, uint32_t batch_m,
                 float* y_batch, double* gpu_ms, char* err, size_t err_cap);

/* Bit-exact dequantised rows [row0, row0+nrows) x cols, f32, host output.
 * Same values as CodebookMatrix::decode_row (codebook.rs:285-337), the Q8_0
 * expansion (gguf.rs:223-229), and the g64 table lookup. */
VXT_API int vxt_hip_dequant_rows(void* ctx, void* tensor, uint32_t row0, uint32_t nrows, float* out,
                         char* err, size_t err_cap);

/* ---- device-pointer entry points (asynchronous on `stream`) ------------- */
/* x, y, out are device pointers; stream is a hipStream_t (NULL = default).
 * Nothing is copied to or from the host.  These are what the decode loop and
 * the benchmarks call with activations already resident in HBM. */

/* y[batch_m * rows] (y_dtype) = W x for x[batch_m * cols] (x_dtype).
 * batch_m 1..8 runs the GEMV kernels; larger batch_m the GEMM kernels, which
 * use the context's workspace (activation row scales, weight panel,
 * converted activations, split-K partial sums).  The workspace grows only
 * outside any stream capture: inside one, a shape that needs more than an
 * earlier eager call allocated fails with VXT_E_ARG.  A workspace that is
 * replaced by a larger one stays allocated until vxt_hip_destroy, so graphs
 * captured earlier keep replaying.  GEMMs of one context share it; callers
 * order GEMMs they put on different streams. */
VXT_API int vxt_hip_matmul_dev(void* ctx, void* tensor, const void* x, uint32_t x_dtype,
                       uint32_t batch_m, void* y, uint32_t y_dtype, void* stream, char* err,
                       size_t err_cap);

/* Allocation-free form of vxt_hip_matmul_dev (same arguments, same kernels,
 * same results).  No counterpart in the reference: it is for callers that
 * cannot allocate device memory -- code under stream capture whose first
 * call would otherwise size the workspace, tight serving loops, harnesses
 * that forbid hipMalloc.  It never calls hipMalloc, hipFree or the vendor
 * library (a GEMM the context would send to the library's dense phase runs
 * the own dense kernel instead); its GEMM workspace is a fixed 32 MiB array
 * in device memory, one per GPU, allocated when the library's code is
 * loaded on that GPU and held until the process ends.  A GEMM that needs
 * more (e.g. the two-phase path at batch_m >= 512 on 6144 x 2048) fails
 * with VXT_E_SHAPE.  Every call on one GPU shares that array: calls that can
 * overlap on one GPU (different streams, or different contexts on the same
 * device) race and must be ordered by the caller.  batch_m 1..8 uses no
 * workspace at all. */
VXT_API int vxt_hip_matmul_noalloc_dev(void* ctx, void* tensor, const void* x, uint32_t x_dtype,
                                       uint32_t batch_m, void* y, uint32_t y_dtype, void* stream, char* err,
                                       size_t err_cap);

/* Several tensors sharing one x (forward_multi, llm_cpu.rs:51-71): tensors[i]
 * writes ys[i].  All tensors must have the same cols. */
VXT_API int vxt_hip_matmul_multi_dev(void* ctx, void* const* tensors, uint32_t n, const void* x,
                             uint32_t x_dtype, uint32_t batch_m, void* const* ys,
                             uint32_t y_dtype, void* stream, char* err, size_t err_cap);

/* Device-side bit-exact dequant of rows [row0, row0+nrows) into out (f32). */
VXT_API int vxt_hip_dequant_rows_dev(void* ctx, void* tensor, uint32_t row0, uint32_t nrows,
                             float* out, void* stream, char* err, size_t err_cap);

/* Gated FFN projection: tensor is the row-concatenated [gate; up] matrix
 * (rows = 2 * n_ff, e.g. from vxt_hip_upload_cb4_concat); act[m * act_stride
 * + i] = act(g_i) * u_i for i < n_ff with g = gate . x, u = up . x (fp32
 * sums), and 0 for n_ff <= i < act_stride.  activation is VXT_ACT_SILU or
 * VXT_ACT_GELU_TANH.  Replaces the runner's fused gate/up + SwiGLU GEMV
 * (vxt_cb4_ffn_gu_nr2_m1, vxt_cb4_fast.metal:212-287) and, for batches, its
 * GEMM + vxt_cb4_swiglu_batch (vxt_cb4_fast_ops.metal:236-262); the CPU
 * step is forward_multi + the activation loop (llm_cpu.rs:448-464).
 * batch_m 1..2 is one fused launch; larger batches stage g and u (f32) in
 * the context workspace, with the workspace rules of vxt_hip_matmul_dev. */
VXT_API int vxt_hip_ffn_glu_dev(void* ctx, void* tensor, const void* x, uint32_t x_dtype, uint32_t batch_m,
                                void* act, uint32_t act_dtype, uint32_t act_stride, uint32_t activation,
                                void* stream, char* err, size_t err_cap);

/* Residual add + RMSNorm over batch_m rows of `stride` floats:
 *   if delta: cur[i] += delta[i] (written back);
 *   out[i] = cur[i] * scale * weight[i], scale = 1 / sqrt(sum cur^2 / dim + eps)
 *   for i < dim, 0 for dim <= i < stride (out_dtype f32 or bf16).
 * rms_norm of llm_ops.rs:48-57 after the residual add of llm_cpu.rs:443-446;
 * the runner's vxt_cb4_add_rms_norm_batch / vxt_cb4_rms_norm_batch
 * (vxt_cb4_fast_ops.metal:160-234).  out may alias cur (f32 only), not delta.
 * Device pointers; no tensor involved. */
VXT_API int vxt_hip_rms_norm_dev(void* ctx, float* cur, const float* delta, const float* weight, void* out,
                                 uint32_t out_dtype, uint32_t dim, uint32_t stride, uint32_t batch_m, float eps,
                                 void* stream, char* err, size_t err_cap);

/* Batch-1 projection of a normalised residual stream, one launch:
 *   v = delta ? cur + delta : cur;  x = bf16(rms_norm(v) * norm_w)  (as
 *   vxt_hip_rms_norm_dev with a bf16 output, bit for bit);
 *   y = W x (VXT_NORM_PLAIN), or the gated activation of [gate; up] as in
 *   vxt_hip_ffn_glu_dev (VXT_NORM_GLU_*; y_stride >= rows / 2, zero padded);
 *   with delta, cur_out (a buffer other than cur and delta) receives v.
 * The pair it replaces is the runner's add-RMSNorm kernel and the GEMV that
 * reads its output (metal_cb4_fast_run.mm:81-92, 355-387); here every
 * workgroup builds x itself from cur, delta and norm_w, so the pair costs
 * one launch.  cols <= 4096 (VXT_E_UNSUPPORTED otherwise: use the two calls). */
VXT_API int vxt_hip_norm_matmul_dev(void* ctx, void* tensor, const float* cur, const float* delta,
                                    const float* norm_w, float eps, float* cur_out, uint32_t mode, void* y,
                                    uint32_t y_dtype, uint32_t y_stride, void* stream, char* err,
                                    size_t err_cap);

/* ---- Q8_0 KV cache (decode attention) --------------------------------------
 * The cache of one layer, device memory the caller allocates: position t's
 * values at k_qs[t * n_kv * head_dim ...] (int8, 16-byte aligned plane) and
 * their scales at k_d[t * n_kv * head_dim / 32 ...] (f16 bits), likewise for
 * V.  Every value and scale has the bits of KvQ8Block::quantize
 * (llm_prefill.rs:27-42); the block's two fields are kept as two planes. */
typedef struct VxtKvQ8Cache {
    void* k_qs;        /* int8 [max_seq][n_kv * head_dim]                     */
    void* k_d;         /* f16  [max_seq][n_kv * head_dim / 32]                */
    void* v_qs;
    void* v_d;
    uint32_t max_seq, n_kv, head_dim, reserved;   /* head_dim 32/64/128/256 */
} VxtKvQ8Cache;

/* Quantise one position's K and V ([n_kv * head_dim] f32 each, already
 * normed and rotated) into row pos: the cache writes of step_full_gqa_q8
 * (llm_prefill.rs:300-313). */
VXT_API int vxt_hip_kv_q8_append_dev(void* ctx, const VxtKvQ8Cache* cache, const float* k, const float* v,
                                     uint32_t pos, void* stream, char* err, size_t err_cap);

/* Attention of one decode step over positions [0, seq_len): q [n_head *
 * head_dim] (normed, rotated), head h reads kv head h / (n_head / n_kv);
 * scores q.K / sqrt(head_dim), softmax, sum of weights times V; gate (NULL
 * or [n_head * head_dim]) multiplies by 1 / (1 + exp(-g)); out [n_head *
 * head_dim] f32.  The scoring, softmax and accumulation of step_full_gqa_q8
 * (llm_prefill.rs:315-367) with KvQ8Block::dot_f32 / axpy_f32, computed over
 * chunks of positions in parallel (fp32; the order of the sums differs).
 * Uses the context workspace (rules of vxt_hip_matmul_dev).  n_head / n_kv
 * <= 8. */
VXT_API int vxt_hip_attn_q8_dev(void* ctx, const VxtKvQ8Cache* cache, const float* q, uint32_t n_head,
                                uint32_t seq_len, const float* gate, float* out, void* stream, char* err,
                                size_t err_cap);

/* The scalar arguments of step_full_gqa_q8 (llm_prefill.rs:259-278) plus the
 * optional biases the Metal runner's prep adds (vxt_cb4_gqa_prep_batch,
 * vxt_cb4_fast_gqa.metal:455-541); the cache supplies n_kv and head_dim.
 * Pointers are device memory or NULL. */
typedef struct VxtGqaParams {
    const float* q_norm;   /* NULL or [head_dim]: RMSNorm weight of every q head   */
    const float* k_norm;   /* NULL or [head_dim]                                   */
    const float* q_bias;   /* NULL or [q_rows], added to q_raw before anything else */
    const float* k_bias;   /* NULL or [n_kv * head_dim]                            */
    const float* v_bias;   /* NULL or [n_kv * head_dim]                            */
    uint32_t n_head;
    uint32_t gated_q;      /* 1: q_raw holds [q | gate] per head, q_rows = 2 * n_head * head_dim;
                              0: q_rows = n_head * head_dim                         */
    uint32_t rope_dim;     /* rotated values per head (clamped to head_dim); 0: none */
    uint32_t rope_neox;    /* 1: pairs (i, i + r / 2); 0: pairs (2i, 2i + 1)        */
    float rope_freq_base;
    float eps;             /* of the q / k RMSNorm                                  */
} VxtGqaParams;

/* The q / k preparation of step_full_gqa_q8 (llm_prefill.rs:284-313) for
 * batch_m tokens: token m reads q_raw + m * q_stride, k_cur + m * kv_stride,
 * v_cur + m * kv_stride (strides ignored for batch_m 1), and is at cache row
 * pos + m and rope position rope_pos + m.  Per query head: the q half (and,
 * gated, the gate half -> gate_out), rms_norm with q_norm (llm_ops.rs:48-57),
 * apply_rope (llm_ops.rs:81-99) -> q_out [batch_m][n_head * head_dim].  Per kv
 * head: K normed with k_norm and rotated, then K and V quantised into the
 * token's cache row (KvQ8Block::quantize bits).  k_cur is read, not
 * rewritten (the reference rotates it in place).  fp32; the norm's sum of
 * squares runs in another order than the reference loop, the rotation's
 * frequencies are the reference's powf values. */
VXT_API int vxt_hip_attn_prep_q8_dev(void* ctx, const VxtKvQ8Cache* cache, const VxtGqaParams* params,
                                     const float* q_raw, uint32_t q_stride, const float* k_cur, const float* v_cur,
                                     uint32_t kv_stride, uint32_t batch_m, uint32_t pos, uint32_t rope_pos,
                                     float* q_out, float* gate_out, void* stream, char* err, size_t err_cap);

/* step_full_gqa_q8 (llm_prefill.rs:259-367) whole, for batch_m tokens at
 * positions pos .. pos + batch_m - 1: the prep above, then token m's
 * attention over cache rows [0, pos + m] with its gate -> out + m * n_head *
 * head_dim.  batch_m 1 is the decode step (llm_cpu.rs:395-412); a batch is the
 * per-token loop of the tiled prefill (llm_prefill.rs:505-517), causal.
 * Uses the context workspace (rules of vxt_hip_matmul_dev).  n_head / n_kv
 * <= 8. */
VXT_API int vxt_hip_attn_step_q8_dev(void* ctx, const VxtKvQ8Cache* cache, const VxtGqaParams* params,
                                     const float* q_raw, uint32_t q_stride, const float* k_cur, const float* v_cur,
                                     uint32_t kv_stride, uint32_t batch_m, uint32_t pos, uint32_t rope_pos,
                                     float* out, void* stream, char* err, size_t err_cap);

/* ---- Decode-step runner ----------------------------------------------------
 * A whole forward pass of a decoder with full (grouped-query) attention over
 * a Q8_0 KV cache, held on the device: the host side of the reference's
 * device runner, vxt_metal_cb4_fast_{create, state_create, step_batch,
 * enqueue_async, wait_cmd, destroy} (metal_cb4_fast_ffi.rs:134-206; the pass
 * itself metal_cb4_fast_run.mm:94-434), for models whose layers are all
 * full-attention layers (the reference's recurrent DeltaNet layers are not
 * part of this library).  Per layer, as the CPU step (llm_cpu.rs:395-482):
 *   normed = rms_norm(cur [+= delta], attn_norm)          (bf16)
 *   qkv    = w_in . normed                                 (f32: [q | gate per head]; k; v)
 *   attn   = step_full_gqa_q8(qkv, cache, pos)             (vxt_hip_attn_step_q8_dev)
 *   delta  = w_out . attn                                  (f32)
 *   normed = rms_norm(cur += delta, post_attn_norm)        (bf16)
 *   act    = act(gate . normed) * (up . normed)            (vxt_hip_ffn_glu_dev, bf16)
 *   delta  = w_ffn_dn . act                                (f32)
 * then normed = rms_norm(cur += delta, output_norm), logits = lm_head .
 * normed (f32), and for generation the greedy id (vxt_hip_greedy_dev) whose
 * embedding row (vxt_hip_embed_dev, times embed_scale) starts the next step.
 * Every piece is the entry point named beside it; the runner adds the
 * buffers, one KV cache per layer (max_seq rows) and, for single tokens, one
 * captured HIP graph whose attention reads the position from device memory,
 * so a decode step is one graph launch with no per-token host work. */
typedef struct VxtRunnerLayer {
    void* w_in;                   /* (q_rows + 2 * n_kv * head_dim) x hidden */
    void* w_out;                  /* hidden x (n_head * head_dim)            */
    void* w_ffn_gu;               /* (2 * ffn) x hidden, [gate; up]          */
    void* w_ffn_dn;               /* hidden x ffn                            */
    const float* attn_norm;       /* device [hidden]                         */
    const float* post_attn_norm;  /* device [hidden]                         */
    const float* q_norm;          /* device [head_dim] or NULL               */
    const float* k_norm;          /* device [head_dim] or NULL               */
} VxtRunnerLayer;

/* q_rows = n_head * head_dim * (gated_q ? 2 : 1); the rope and norm fields
 * as in VxtGqaParams; activation VXT_ACT_*; embed_scale as in
 * vxt_hip_embed_dev.  max_batch bounds the tokens of one vxt_hip_runner_step. */
typedef struct VxtRunnerConfig {
    uint32_t n_layers, hidden, n_head, n_kv, head_dim, ffn, vocab;
    uint32_t gated_q, rope_dim, rope_neox, activation;
    uint32_t max_seq, max_batch;
    float rope_freq_base, eps, embed_scale;
} VxtRunnerConfig;

/* Checks every shape against the config (tensors of this context, norms
 * non-null), allocates the buffers and the KV caches, and captures the
 * single-token step.  The tensors and norm buffers must outlive the runner;
 * vxt_hip_destroy of the context also releases it. */
VXT_API void* vxt_hip_runner_create(void* ctx, const VxtRunnerConfig* cfg, const VxtRunnerLayer* layers,
                                    const float* output_norm, void* lm_head, void* embed, char* err,
                                    size_t err_cap);

/* vxt_metal_cb4_fast_step_batch (metal_cb4_fast_run.mm:440-481): batch_m
 * tokens (host ids, each < vocab) at positions pos_base .. pos_base +
 * batch_m - 1 (rope positions the same), causal over the cache rows below;
 * their K and V enter the cache.  logits_out (NULL or [vocab]) receives the
 * last token's logits.  batch_m 1 replays the captured step; larger batches
 * run the batched GEMM path.  Synchronous. */
VXT_API int vxt_hip_runner_step(void* runner, const uint32_t* tok_ids, uint32_t batch_m, uint32_t pos_base,
                                float* logits_out, char* err, size_t err_cap);

/* Greedy generation on the device, the reference's ring of enqueue_async /
 * wait_cmd (metal_cb4_fast_ffi.rs:191-206): starting from `token` at
 * pos_base, n_steps single-token steps, each feeding the greedy id of the
 * previous one; tokens_out[i] is the id chosen after step i and flags_out
 * (NULL or [n_steps]) is 1 where that step's logits held NaN or +-inf.
 * n_steps graph launches, one copy back.  Synchronous. */
VXT_API int vxt_hip_runner_generate(void* runner, uint32_t token, uint32_t pos_base, uint32_t n_steps,
                                    uint32_t* tokens_out, uint32_t* flags_out, char* err, size_t err_cap);

VXT_API void vxt_hip_runner_destroy(void* runner);

/* ---- Weight containers ----------------------------------------------------
 * Readers over bytes the caller holds (e.g. a mapped file); they keep no
 * pointer after returning.  Offsets below are byte offsets into those bytes. */

/* One tensor section of a .vxt (VXT1) archive (format.rs:178-294 layout).
 * The plane fields are filled for kind 2 (KIND_CODEBOOK) and, for kind 3
 * (KIND_Q4_0), scales_off / n_scales and words_off / n_words. */
typedef struct VxtArchiveEntry {
    uint64_t name_off, name_len;    /* UTF-8 name                            */
    uint32_t kind, sub;             /* kind 2 = codebook, sub = bits         */
    uint64_t rows, cols, padded_cols;
    uint64_t section_off, section_len;
    uint64_t centroids_off;         /* 16 f32                                */
    uint64_t scales_off, n_scales;  /* u16 [rows * padded_cols / 128]        */
    uint64_t words_off, n_words;    /* u32 [rows * padded_cols / 128 * 4 * bits] */
    uint64_t row_ptr_off, n_row_ptr;/* u32 [rows + 1]                        */
    uint64_t outliers_off, n_outliers; /* u32 col | f16 << 16                */
} VxtArchiveEntry;

/* Parse and verify a .vxt archive (read_vxt_model, format.rs:301-451): the
 * archive and per-section FNV-1a64 tags, the codebook header and plane
 * rules (bits 3 or 4, padded_cols = ceil(cols/256)*256, plane lengths), the
 * outlier CSR rules (format.rs:565-574) and the Q4_0 header and plane rules
 * (padded_cols = ceil(cols/32)*32, plane lengths; format.rs:453-462).  Call with entries = NULL to
 * get *count, then with an array of `cap` >= *count.  *meta_count receives
 * the metadata entry count (values are stepped over).  Sections of kind 7
 * (entropy-coded TurboWht) stop the walk with VXT_E_UNSUPPORTED. */
VXT_API int vxt_hip_vxt_parse(const uint8_t* bytes, size_t len, VxtArchiveEntry* entries, uint32_t cap,
                              uint32_t* count, uint32_t* meta_count, char* err, size_t err_cap);

/* Upload a parsed 4-bit codebook or Q4_0 entry of the same bytes to the
 * device (the paths upload_packed takes for PackedTensor::Codebook and
 * PackedTensor::Q4_0, metal.rs:162-187). */
VXT_API void* vxt_hip_upload_vxt_entry(void* ctx, const uint8_t* bytes, size_t len, const VxtArchiveEntry* e,
                                       char* err, size_t err_cap);

/* One tensor of a GGUF v2/v3 file (GgufTensorMeta, gguf.rs:52-73). */
typedef struct VxtGgufTensor {
    uint64_t name_off, name_len;
    uint32_t ggml_type, n_dims;     /* ggml type id (8 = Q8_0)               */
    uint64_t ne[8];                 /* ne[0] = contiguous cols               */
    uint64_t data_off, data_len;    /* absolute; data_len 0 if unsupported   */
    uint32_t supported, reserved;   /* type with a known byte size (gguf.rs:32-41) */
} VxtGgufTensor;

/* Parse a GGUF file's header, metadata (general.alignment honoured, the rest
 * stepped over by type) and tensor table (GgufView::parse, gguf.rs:83-158);
 * every supported tensor's bytes are checked to lie inside the file
 * (tensor_bytes, gguf.rs:160-172).  Two-call pattern as vxt_hip_vxt_parse. */
VXT_API int vxt_hip_gguf_parse(const uint8_t* bytes, size_t len, VxtGgufTensor* tensors, uint32_t cap,
                               uint32_t* count, uint32_t* version, uint64_t* alignment, char* err,
                               size_t err_cap);

/* Upload a Q8_0 GGUF matrix (rows = ne[1] * ne[2] ..., cols = ne[0]) from
 * its bytes as they lie in the file, with no f32 expansion on the host
 * (llm.rs:164 expands; this keeps the blocks). */
VXT_API void* vxt_hip_upload_gguf_q8_0(void* ctx, const uint8_t* bytes, size_t len, const VxtGgufTensor* t,
                                       char* err, size_t err_cap);

/* Embedding rows for batch_m token ids held in device memory (tokens[m]):
 * out[m * out_stride + c] = decode_row(tokens[m])[c] for c < cols, bit-exact,
 * multiplied by embed_scale when |embed_scale - 1| > 1e-7 (llm_cpu.rs:
 * 224-229), and 0 for cols <= c < out_stride.  An id >= rows reads the last
 * row, as the device runner's gather does (vxt_cb4_embed_exact_batch,
 * vxt_cb4_fast_ops.metal:89-113, which reads the id the greedy step left in
 * device memory); the CPU path rejects such ids (llm_cpu.rs:219-221), so
 * callers that need the error check ids on the host.  Any kind. */
VXT_API int vxt_hip_embed_dev(void* ctx, void* tensor, const uint32_t* tokens, uint32_t batch_m,
                              float embed_scale, float* out, uint32_t out_stride, void* stream, char* err,
                              size_t err_cap);

/* Greedy token selection over n f32 logits (device memory): out[0] = the
 * lowest index holding the largest non-NaN logit, or 0 when no logit is
 * above -inf (n == 0, all -inf, all NaN); out[1] = 1 if any logit is NaN or
 * +-inf, else 0.  -0 and +0 are equal.  Replaces the runner's greedy step
 * (vxt_greedy_exact, vxt_llm_ops.metal:569-600, read back at
 * metal_llm.mm:659-663; its test probe vxt_metal_llm_greedy_probe,
 * metal_llm_tests.rs:17-26) and agrees with the CPU sampler's greedy branch
 * (llm_ops.rs:318-327).  One launch, no allocation, no memset: capturable.
 * Calls of one context share a small state block, so calls on different
 * streams must not overlap in time. */
VXT_API int vxt_hip_greedy_dev(void* ctx, const float* logits, uint32_t n, uint32_t* out, void* stream,
                               char* err, size_t err_cap);

/* Measurement only, no counterpart in the reference: reads [p, p + bytes)
 * (device memory, bytes a multiple of 16) once with the decode GEMV's access
 * pattern and no arithmetic -- the HBM floor of a single launch that size.
 * Each lane folds its words by xor; `key` must be a value no lane's fold of
 * the buffer gives (e.g. 1 for a buffer of one repeated 32-bit word, whose
 * folds are 0). */
VXT_API int vxt_hip_read_probe_dev(void* ctx, const void* p, size_t bytes, uint32_t key, void* stream, char* err,
                                   size_t err_cap);

/* ---- device memory, stream and graphs ---------------------------------- */
/* What a host without another GPU runtime (the Rust engine, C callers) needs
 * to keep activations resident and to replay a decode loop without per-launch
 * CPU overhead.  No reference counterpart: the Metal bridge keeps x and y in
 * unified memory (metal_gemv.mm:350-351) and records one command buffer per
 * call (metal_gemv.mm:369-445). */

/* hipMalloc'd device buffer owned by the context (freed by destroy). */
VXT_API void* vxt_hip_device_alloc(void* ctx, size_t bytes, char* err, size_t err_cap);
VXT_API void vxt_hip_device_free(void* ctx, void* dev_ptr);

/* Synchronous copy on the context stream; kind: 0 host->device,
 * 1 device->host, 2 device->device. */
VXT_API int vxt_hip_memcpy(void* ctx, void* dst, const void* src, size_t bytes, uint32_t kind,
                           char* err, size_t err_cap);

/* The context's hipStream_t, for the *_dev entry points. */
VXT_API void* vxt_hip_stream(void* ctx);

/* Wait for all work queued on the context stream. */
VXT_API int vxt_hip_synchronize(void* ctx, char* err, size_t err_cap);

/* Start capturing the context stream into a HIP graph; enqueue *_dev calls
 * with stream = vxt_hip_stream(ctx); vxt_hip_capture_end returns the
 * instantiated graph (NULL on failure). */
VXT_API int vxt_hip_capture_begin(void* ctx, char* err, size_t err_cap);
VXT_API void* vxt_hip_capture_end(void* ctx, char* err, size_t err_cap);

/* Launch a captured graph `replays` times back to back on the context
 * stream, wait, and report the GPU time of all replays (hipEvent pair). */
VXT_API int vxt_hip_graph_launch(void* ctx, void* graph, uint32_t replays, double* gpu_ms,
                                 char* err, size_t err_cap);
VXT_API void vxt_hip_graph_free(void* graph);

/* Kernel time of the last synchronous call, in ms (hipEvent pair). */
VXT_API int vxt_hip_last_kernel_ms(void* ctx, double* ms);

/* Prefill GEMM path (batch_m > 8) of this context's later calls.  Every path
 * runs this library's own kernels except LIBRARY.  AUTO (the default), by
 * measured speed: g64 weights with bf16 activations decode inside the MFMA
 * loop -- the fused kernel up to batch_m 64, the 128 x 128 tile kernel from
 * 128 to 2047 (and beyond when cols > rows); cb4 weights with bf16
 * activations take the cb4 tile kernel described under FUSED from batch_m 128
 * to 511 when the tensor is eligible for it; Q8_0 (and Q4_0) weights with
 * bf16 activations and batch_m <= 128 take the fused kernel; every other call
 * takes the two-phase path (a decoded f16 weight panel, then the dense MFMA
 * kernel).  PANEL pins the two-phase path.  FUSED takes the decode-in-loop
 * kernels wherever they apply: for cb4 weights with bf16 activations the cb4
 * tile kernel (scale x centroid tables and the CSR residuals decoded inside
 * the MFMA loop, no weight panel), when the upload found the tensor eligible
 * (every plane finite, each row's residual columns strictly increasing, at
 * most 16384 residuals per block of 128 rows); for g64 the tile kernel above
 * batch_m 64 and the fused kernel below; for Q8_0 / Q4_0 the fused kernel;
 * the two-phase path otherwise.  LIBRARY pins the two-phase path with its
 * dense phase on hipBLASLt, a comparison only (falling back to the own
 * kernel for a shape the library has no algorithm for).  A tuning and test
 * control with no counterpart in the reference, whose gemm_cpu
 * (llm_prefill.rs:156-255) has a single path.  Returns VXT_E_ARG for an
 * unknown path. */
#define VXT_GEMM_AUTO 0u
#define VXT_GEMM_PANEL 1u
#define VXT_GEMM_FUSED 2u
#define VXT_GEMM_LIBRARY 3u
VXT_API int vxt_hip_set_gemm_path(void* ctx, uint32_t path);

#ifdef __cplusplus
}
#endif

#endif /* VXT_HIP_H */
