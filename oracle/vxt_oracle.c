/*
 * vxt_oracle.c -- CPU restatement of vxg-tensor's compressed-weight matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the CPU
 * baseline: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product library (vxg_amd/libvxt_hip.so) never links
 * or calls it.
 *
 * Every function restates one reference function (Rust, crates/vxg-tensor),
 * keeping its loop order, accumulator interleave and summation order.  Rust
 * never contracts a*b+c, and `mul_add` is a single-rounding fused multiply-add,
 * so this file is compiled with -ffp-contract=off and every reference
 * `mul_add` is written as fmaf().
 *
 * Pinning (how each function is checked independently of its own formula)
 * lives in tests/test_oracle_*.py; the header of each function names the
 * reference lines it follows.
 *
 * Layout conventions (reference `rows x cols`, benchmark notation `N x K`):
 *   rows = N (output features), cols = K (reduction), batch_m = M (tokens).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define VXO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------- */
/* fp16 / bf16 conversions                                                    */
/* ------------------------------------------------------------------------- */

static inline float bits_to_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* fp16.rs:6-29 f16_to_f32: exact widening, subnormals normalised. */
VXO_API float vxo_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)(bits & 0x8000u)) << 16;
    uint32_t exp = (bits >> 10) & 0x1fu;
    uint32_t mant = bits & 0x03ffu;
    if (exp == 0) {
        if (mant == 0) return bits_to_f32(sign);
        uint32_t m = mant, e = 127u - 14u;
        while ((m & 0x0400u) == 0) { m <<= 1; e -= 1; }
        m &= 0x03ffu;
        return bits_to_f32(sign | (e << 23) | (m << 13));
    } else if (exp == 31) {
        return bits_to_f32(sign | 0x7f800000u | (mant << 13));
    }
    return bits_to_f32(sign | ((exp + 112u) << 23) | (mant << 13));
}

/* fp16.rs:33-77 f32_to_f16: round-to-nearest-even including subnormals. */
VXO_API uint16_t vxo_f32_to_f16(float val) {
    uint32_t b = f32_to_bits(val);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t exp = (int32_t)((b >> 23) & 0xffu);
    uint32_t mant = b & 0x007fffffu;
    if (exp == 255) {
        if (mant != 0) return (uint16_t)(sign | 0x7e00u | (uint16_t)(mant >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int32_t unbiased = exp - 127;
    if (unbiased > 15) return (uint16_t)(sign | 0x7c00u);
    if (unbiased < -25) return sign;
    if (unbiased < -14) {
        uint32_t shift = (uint32_t)(-14 - unbiased);
        uint32_t full_mant = mant | 0x00800000u;
        uint32_t round_shift = 13u + shift;
        uint32_t half = 1u << (round_shift - 1);
        uint32_t mask = (1u << round_shift) - 1u;
        uint32_t rem = full_mant & mask;
        uint16_t m16 = (uint16_t)(full_mant >> round_shift);
        if (rem > half || (rem == half && (m16 & 1u) != 0)) m16 += 1;
        return (uint16_t)(sign | m16);
    }
    uint16_t e16 = (uint16_t)(((uint32_t)(unbiased + 15)) << 10);
    uint32_t rem = mant & 0x1fffu;
    uint16_t m16 = (uint16_t)(mant >> 13);
    if (rem > 0x1000u || (rem == 0x1000u && (m16 & 1u) != 0)) {
        m16 += 1;
        if (m16 == 0x0400u) return (uint16_t)(sign | (uint16_t)(e16 + 0x0400u));
    }
    return (uint16_t)(sign | e16 | m16);
}

/* fp16.rs:81-83 bf16_to_f32. */
VXO_API float vxo_bf16_to_f32(uint16_t bits) { return bits_to_f32(((uint32_t)bits) << 16); }

/* fp16.rs:113-120 f32_to_bf16: RNE via 0x7fff + lsb bias; NaN keeps a quiet bit. */
VXO_API uint16_t vxo_f32_to_bf16(float val) {
    uint32_t b = f32_to_bits(val);
    if ((b & 0x7f800000u) == 0x7f800000u && (b & 0x007fffffu) != 0)
        return (uint16_t)((b >> 16) | 0x0040u);
    uint32_t lsb = (b >> 16) & 1u;
    uint32_t bias = 0x7fffu + lsb;
    return (uint16_t)((b + bias) >> 16);
}

/* Bulk wrappers so the Python side can check all 65,536 patterns at once. */
VXO_API void vxo_f16_to_f32_n(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = vxo_f16_to_f32(src[i]);
}
VXO_API void vxo_f32_to_f16_n(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = vxo_f32_to_f16(src[i]);
}
VXO_API void vxo_bf16_to_f32_n(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = vxo_bf16_to_f32(src[i]);
}
VXO_API void vxo_f32_to_bf16_n(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = vxo_f32_to_bf16(src[i]);
}

/* ------------------------------------------------------------------------- */
/* Row-parallel driver shared by the GEMVs                                    */
/* ------------------------------------------------------------------------- */

typedef void (*vxo_rows_fn)(const void* mat, const float* x_pad, float* y, size_t r0, size_t r1);

typedef struct {
    vxo_rows_fn fn;
    const void* mat;
    const float* x_pad;
    float* y;
    size_t r0, r1;
} vxo_rows_job;

static void* vxo_rows_thread(void* p) {
    vxo_rows_job* j = (vxo_rows_job*)p;
    j->fn(j->mat, j->x_pad, j->y, j->r0, j->r1);
    return NULL;
}

/* codebook.rs:357-369: workers = clamp(threads,1,256).min(rows.max(1)); one
 * thread when workers <= 1 or rows < 16; otherwise contiguous chunks of
 * ceil(rows/workers) rows, threads spawned per call. */
static void vxo_run_rows(vxo_rows_fn fn, const void* mat, const float* x_pad, float* y,
                         size_t rows, int threads) {
    size_t t = threads < 1 ? 1 : (threads > 256 ? 256 : (size_t)threads);
    size_t workers = t < (rows > 0 ? rows : 1) ? t : (rows > 0 ? rows : 1);
    if (workers <= 1 || rows < 16) {
        fn(mat, x_pad, y, 0, rows);
        return;
    }
    size_t chunk = (rows + workers - 1) / workers;
    size_t n = (rows + chunk - 1) / chunk;
    pthread_t* tid = (pthread_t*)calloc(n, sizeof(pthread_t));
    vxo_rows_job* jobs = (vxo_rows_job*)calloc(n, sizeof(vxo_rows_job));
    for (size_t i = 0; i < n; ++i) {
        jobs[i].fn = fn; jobs[i].mat = mat; jobs[i].x_pad = x_pad; jobs[i].y = y;
        jobs[i].r0 = i * chunk;
        jobs[i].r1 = (i + 1) * chunk < rows ? (i + 1) * chunk : rows;
        pthread_create(&tid[i], NULL, vxo_rows_thread, &jobs[i]);
    }
    for (size_t i = 0; i < n; ++i) pthread_join(tid[i], NULL);
    free(tid);
    free(jobs);
}

/* ------------------------------------------------------------------------- */
/* cb4 reference layout: CodebookMatrix with bits = 4 (codebook.rs:9-24)      */
/* ------------------------------------------------------------------------- */

typedef struct {
    uint32_t rows, cols, padded_cols;   /* padded_cols % 128 == 0, >= cols */
    const float* centroids;             /* [16] */
    const uint16_t* scales_f16;         /* [rows * padded_cols/128] */
    const uint32_t* packed_words;       /* [rows * padded_cols/8], nibble c%8 of word c/8 */
    const uint32_t* outlier_row_ptr;    /* [rows + 1] */
    const uint32_t* outliers_packed;    /* col | f16_residual << 16 */
} vxo_cb4;

/* codebook.rs:285-306 + :329-336 decode_row (4-bit branch): dst[c] = sc*cent[q]
 * (one f32 rounding), then CSR residuals added in order for col < cols. */
VXO_API void vxo_cb4_decode_row(const vxo_cb4* m, size_t r, float* dst) {
    size_t gpr = m->padded_cols / 128;
    for (size_t g = 0; g < gpr; ++g) {
        size_t g_idx = r * gpr + g;
        float sc = vxo_f16_to_f32(m->scales_f16[g_idx]);
        for (size_t sub = 0; sub < 4; ++sub) {
            size_t col_base = g * 128 + sub * 32;
            if (col_base >= m->cols) break;
            size_t valid = m->cols - col_base < 32 ? m->cols - col_base : 32;
            const uint32_t* cw = m->packed_words + (g_idx * 4 + sub) * 4;
            for (size_t l = 0; l < valid; ++l) {
                uint32_t q = (cw[l / 8] >> ((l % 8) * 4)) & 0x0fu;
                dst[col_base + l] = sc * m->centroids[q];
            }
        }
    }
    uint32_t os = m->outlier_row_ptr[r], oe = m->outlier_row_ptr[r + 1];
    for (uint32_t i = os; i < oe; ++i) {
        uint32_t packed = m->outliers_packed[i];
        uint32_t col = packed & 0xffffu;
        if (col < m->cols) dst[col] += vxo_f16_to_f32((uint16_t)(packed >> 16));
    }
}

/* codebook.rs:372-417 gemv_rows_range (4-bit branch). */
static void vxo_cb4_rows(const void* mp, const float* x_pad, float* y, size_t r0, size_t r1) {
    const vxo_cb4* m = (const vxo_cb4*)mp;
    size_t gpr = m->padded_cols / 128;
    for (size_t r = r0; r < r1; ++r) {
        float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
        for (size_t g = 0; g < gpr; ++g) {
            size_t g_idx = r * gpr + g;
            float sc = vxo_f16_to_f32(m->scales_f16[g_idx]);
            if (sc == 0.0f) continue;
            float slut[16];
            for (int k = 0; k < 16; ++k) slut[k] = sc * m->centroids[k];
            for (size_t sub = 0; sub < 4; ++sub) {
                const uint32_t* cw = m->packed_words + (g_idx * 4 + sub) * 4;
                size_t base_x = g * 128 + sub * 32;
                for (size_t w = 0; w < 4; ++w) {
                    uint32_t word = cw[w];
                    const float* xv = x_pad + base_x + w * 8;
                    acc0 = fmaf(slut[word & 0x0f], xv[0], acc0);
                    acc1 = fmaf(slut[(word >> 4) & 0x0f], xv[1], acc1);
                    acc2 = fmaf(slut[(word >> 8) & 0x0f], xv[2], acc2);
                    acc3 = fmaf(slut[(word >> 12) & 0x0f], xv[3], acc3);
                    acc0 = fmaf(slut[(word >> 16) & 0x0f], xv[4], acc0);
                    acc1 = fmaf(slut[(word >> 20) & 0x0f], xv[5], acc1);
                    acc2 = fmaf(slut[(word >> 24) & 0x0f], xv[6], acc2);
                    acc3 = fmaf(slut[(word >> 28) & 0x0f], xv[7], acc3);
                }
            }
        }
        float sum = (acc0 + acc1) + (acc2 + acc3);
        uint32_t os = m->outlier_row_ptr[r], oe = m->outlier_row_ptr[r + 1];
        for (uint32_t i = os; i < oe; ++i) {
            uint32_t packed = m->outliers_packed[i];
            float val = vxo_f16_to_f32((uint16_t)(packed >> 16));
            sum = fmaf(val, x_pad[packed & 0xffffu], sum);
        }
        y[r] = sum;
    }
}

/* codebook.rs:350-370 gemv_cpu: x zero-padded to padded_cols, row-parallel. */
VXO_API void vxo_cb4_gemv(const vxo_cb4* m, const float* x, float* y, int threads) {
    float* x_pad = (float*)calloc(m->padded_cols ? m->padded_cols : 1, sizeof(float));
    memcpy(x_pad, x, (size_t)m->cols * sizeof(float));
    vxo_run_rows(vxo_cb4_rows, m, x_pad, y, m->rows, threads);
    free(x_pad);
}

/* ------------------------------------------------------------------------- */
/* cb4-g64: the benchmark's decode layout (groups of 64 along K, one 16-entry */
/* fp16 codebook per group, no scale, no outliers).  Not a reference type;    */
/* its GEMV follows the reference cb4 kernel's loop shape (codebook.rs:376-417)*/
/* with the per-group table in place of sc*centroid.                          */
/* ------------------------------------------------------------------------- */

typedef struct {
    uint32_t rows, cols, padded_cols;   /* padded_cols = roundup(cols, 64) */
    const uint8_t* idx;                 /* [rows * padded_cols/2], low nibble = even col */
    const uint16_t* lut_f16;            /* [rows * padded_cols/64 * 16] */
} vxo_g64;

VXO_API void vxo_g64_decode_row(const vxo_g64* m, size_t r, float* dst) {
    size_t gpr = m->padded_cols / 64;
    const uint8_t* row = m->idx + r * (m->padded_cols / 2);
    for (size_t c = 0; c < m->cols; ++c) {
        uint32_t q = (row[c / 2] >> ((c & 1) * 4)) & 0x0fu;
        dst[c] = vxo_f16_to_f32(m->lut_f16[(r * gpr + c / 64) * 16 + q]);
    }
}

static void vxo_g64_rows(const void* mp, const float* x_pad, float* y, size_t r0, size_t r1) {
    const vxo_g64* m = (const vxo_g64*)mp;
    size_t gpr = m->padded_cols / 64;
    for (size_t r = r0; r < r1; ++r) {
        float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
        const uint8_t* row = m->idx + r * (m->padded_cols / 2);
        for (size_t g = 0; g < gpr; ++g) {
            float lut[16];
            for (int k = 0; k < 16; ++k) lut[k] = vxo_f16_to_f32(m->lut_f16[(r * gpr + g) * 16 + k]);
            for (size_t w = 0; w < 8; ++w) {
                uint32_t word;
                memcpy(&word, row + g * 32 + w * 4, 4);
                const float* xv = x_pad + g * 64 + w * 8;
                acc0 = fmaf(lut[word & 0x0f], xv[0], acc0);
                acc1 = fmaf(lut[(word >> 4) & 0x0f], xv[1], acc1);
                acc2 = fmaf(lut[(word >> 8) & 0x0f], xv[2], acc2);
                acc3 = fmaf(lut[(word >> 12) & 0x0f], xv[3], acc3);
                acc0 = fmaf(lut[(word >> 16) & 0x0f], xv[4], acc0);
                acc1 = fmaf(lut[(word >> 20) & 0x0f], xv[5], acc1);
                acc2 = fmaf(lut[(word >> 24) & 0x0f], xv[6], acc2);
                acc3 = fmaf(lut[(word >> 28) & 0x0f], xv[7], acc3);
            }
        }
        y[r] = (acc0 + acc1) + (acc2 + acc3);
    }
}

VXO_API void vxo_g64_gemv(const vxo_g64* m, const float* x, float* y, int threads) {
    float* x_pad = (float*)calloc(m->padded_cols ? m->padded_cols : 1, sizeof(float));
    memcpy(x_pad, x, (size_t)m->cols * sizeof(float));
    vxo_run_rows(vxo_g64_rows, m, x_pad, y, m->rows, threads);
    free(x_pad);
}

/* ------------------------------------------------------------------------- */
/* Q8: the 34-byte {f16 d; i8 qs[32]} block (llm_prefill.rs:17-24, identical   */
/* to GGUF Q8_0 bytes at gguf.rs:224-228).  A Q8 weight matrix is rows x       */
/* ceil(cols/32) such blocks, row-major, as GgufView::tensor_bytes returns.   */
/* ------------------------------------------------------------------------- */

static inline uint16_t load_u16le(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* llm_prefill.rs:28-42 KvQ8Block::quantize. */
VXO_API void vxo_q8_quantize(const float* src, uint8_t* blk) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        float a = fabsf(src[i]);
        /* Rust f32::max ignores a NaN operand. */
        if (!isnan(a) && (isnan(amax) || a > amax)) amax = a;
    }
    uint16_t dh = vxo_f32_to_f16(amax / 127.0f);
    float df = vxo_f16_to_f32(dh);
    float inv = df > 0.0f ? 1.0f / df : 0.0f;
    blk[0] = (uint8_t)(dh & 0xff);
    blk[1] = (uint8_t)(dh >> 8);
    for (int i = 0; i < 32; ++i) {
        float v = rintf(src[i] * inv);            /* round_ties_even (default FE mode) */
        int8_t q;
        if (isnan(v)) q = 0;                       /* `as i8` maps NaN to 0 */
        else if (v < -127.0f) q = -127;
        else if (v > 127.0f) q = 127;
        else q = (int8_t)v;
        blk[2 + i] = (uint8_t)q;
    }
}

/* llm_prefill.rs:45-54 KvQ8Block::dot_f32: two interleaved FMA chains, then *d. */
VXO_API float vxo_q8_dot_f32(const uint8_t* blk, const float* q) {
    float sc = vxo_f16_to_f32(load_u16le(blk));
    const int8_t* qs = (const int8_t*)(blk + 2);
    float s0 = 0.0f, s1 = 0.0f;
    for (int i = 0; i < 16; ++i) {
        s0 = fmaf((float)qs[2 * i], q[2 * i], s0);
        s1 = fmaf((float)qs[2 * i + 1], q[2 * i + 1], s1);
    }
    return (s0 + s1) * sc;
}

/* llm_prefill.rs:56-62 KvQ8Block::axpy_f32. */
VXO_API void vxo_q8_axpy_f32(const uint8_t* blk, float weight, float* out) {
    float ws = weight * vxo_f16_to_f32(load_u16le(blk));
    const int8_t* qs = (const int8_t*)(blk + 2);
    for (int i = 0; i < 32; ++i) out[i] = fmaf((float)qs[i], ws, out[i]);
}

/* gguf.rs:223-229 Q8_0 dequant: w = (q as i8 as f32) * f16_to_f32(d) (exact). */
VXO_API void vxo_q8_dequant(const uint8_t* blocks, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* blk = blocks + b * 34;
        float d = vxo_f16_to_f32(load_u16le(blk));
        for (int i = 0; i < 32; ++i) out[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
    }
}

typedef struct {
    uint32_t rows, cols;                /* blocks per row = ceil(cols/32) */
    const uint8_t* blocks;              /* [rows * ceil(cols/32) * 34] */
} vxo_q8;

/* Q8 row dequant: gguf.rs:223-229 applied to one row, truncated to cols. */
VXO_API void vxo_q8_decode_row(const vxo_q8* m, size_t r, float* dst) {
    size_t kb = ((size_t)m->cols + 31) / 32;
    const uint8_t* row = m->blocks + r * kb * 34;
    for (size_t b = 0; b < kb; ++b) {
        float d = vxo_f16_to_f32(load_u16le(row + b * 34));
        for (size_t i = 0; i < 32 && b * 32 + i < m->cols; ++i)
            dst[b * 32 + i] = (float)(int8_t)row[b * 34 + 2 + i] * d;
    }
}

/* Q8 GEMV = the reference's block-dot composition (llm_prefill.rs:336-340:
 * `dot += kb[b].dot_f32(..)`, starting from 0.0, blocks in order). */
static void vxo_q8_rows(const void* mp, const float* x_pad, float* y, size_t r0, size_t r1) {
    const vxo_q8* m = (const vxo_q8*)mp;
    size_t kb = ((size_t)m->cols + 31) / 32;
    for (size_t r = r0; r < r1; ++r) {
        const uint8_t* row = m->blocks + r * kb * 34;
        float dot = 0.0f;
        for (size_t b = 0; b < kb; ++b) dot += vxo_q8_dot_f32(row + b * 34, x_pad + b * 32);
        y[r] = dot;
    }
}

VXO_API void vxo_q8_gemv(const vxo_q8* m, const float* x, float* y, int threads) {
    size_t kp = ((size_t)m->cols + 31) / 32 * 32;
    float* x_pad = (float*)calloc(kp ? kp : 1, sizeof(float));
    memcpy(x_pad, x, (size_t)m->cols * sizeof(float));
    vxo_run_rows(vxo_q8_rows, m, x_pad, y, m->rows, threads);
    free(x_pad);
}

/* ------------------------------------------------------------------------- */
/* Q4_0: Q4_0Matrix (q4_0.rs:7-14) -- blocks of 32 columns, one f16 scale and */
/* 16 bytes per block (4 little-endian u32 words); byte j holds column j in   */
/* its low nibble and column j + 16 in its high nibble; value (q - 8) * d.    */
/* ------------------------------------------------------------------------- */

typedef struct {
    uint32_t rows, cols, padded_cols;   /* padded_cols = roundup(cols, 32) */
    const uint16_t* scales_f16;         /* [rows * padded_cols/32] */
    const uint32_t* qs_words;           /* [rows * padded_cols/32 * 4] */
} vxo_q40;

/* Rust `f as i32`: saturating, NaN -> 0. */
static int32_t vxo_f32_as_i32(float f) {
    if (isnan(f)) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f < -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

/* q4_0.rs:17-64 Q4_0Matrix::encode: per block amax (NaN never compares
 * greater), d = f16(amax / 7), id = 1 / f32(d) (0 when d is 0), q =
 * clamp(floor(v * id + 8.5) as i32, 0, 15); columns past `cols` count as 0. */
VXO_API void vxo_q40_encode(uint32_t rows, uint32_t cols, const float* w, uint16_t* scales_f16,
                            uint32_t* qs_words) {
    const size_t bpr = ((size_t)cols + 31) / 32;
    for (size_t r = 0; r < rows; ++r) {
        const float* row_w = w + r * cols;
        for (size_t b = 0; b < bpr; ++b) {
            const size_t blk = r * bpr + b, c0 = b * 32;
            float amax = 0.0f, vals[32];
            for (size_t l = 0; l < 32; ++l) {
                vals[l] = 0.0f;
                if (c0 + l < cols) {
                    const float v = row_w[c0 + l];
                    vals[l] = v;
                    if (fabsf(v) > amax) amax = fabsf(v);
                }
            }
            const float d = amax / 7.0f;
            const uint16_t df16 = vxo_f32_to_f16(d);
            scales_f16[blk] = df16;
            const float d_eff = vxo_f16_to_f32(df16);
            const float id = d_eff != 0.0f ? 1.0f / d_eff : 0.0f;
            uint8_t bytes[16];
            for (int j = 0; j < 16; ++j) {
                int32_t q0 = vxo_f32_as_i32(floorf(vals[j] * id + 8.5f));
                int32_t q1 = vxo_f32_as_i32(floorf(vals[j + 16] * id + 8.5f));
                q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
                q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
                bytes[j] = (uint8_t)(q0 | (q1 << 4));
            }
            for (int wd = 0; wd < 4; ++wd)
                qs_words[blk * 4 + wd] = (uint32_t)bytes[wd * 4] | ((uint32_t)bytes[wd * 4 + 1] << 8) |
                                         ((uint32_t)bytes[wd * 4 + 2] << 16) | ((uint32_t)bytes[wd * 4 + 3] << 24);
        }
    }
}

/* q4_0.rs:77-97 Q4_0Matrix::decode_row: ((nibble as i32) - 8) as f32 * d. */
VXO_API void vxo_q40_decode_row(const vxo_q40* m, size_t r, float* dst) {
    const size_t bpr = m->padded_cols / 32;
    for (size_t b = 0; b < bpr; ++b) {
        const size_t bi = r * bpr + b, c0 = b * 32;
        const float d = vxo_f16_to_f32(m->scales_f16[bi]);
        for (size_t wd = 0; wd < 4; ++wd) {
            const uint32_t word = m->qs_words[bi * 4 + wd];
            for (size_t k = 0; k < 4; ++k) {
                const uint32_t byte = (word >> (8 * k)) & 0xffu;
                const size_t j = wd * 4 + k;
                if (c0 + j < m->cols) dst[c0 + j] = (float)((int32_t)(byte & 0x0fu) - 8) * d;
                if (c0 + j + 16 < m->cols) dst[c0 + j + 16] = (float)((int32_t)(byte >> 4) - 8) * d;
            }
        }
    }
}

/* q4_0.rs:109-145 Q4_0Matrix::gemv_cpu, per row: blk_acc is one FMA chain
 * over the block in the order (j, j + 16) for j = 0..15, then
 * sum = fma(d, blk_acc, sum), blocks in order; x is zero-padded. */
static void vxo_q40_rows(const void* mp, const float* x_pad, float* y, size_t r0, size_t r1) {
    const vxo_q40* m = (const vxo_q40*)mp;
    const size_t bpr = m->padded_cols / 32;
    for (size_t r = r0; r < r1; ++r) {
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; ++b) {
            const size_t bi = r * bpr + b;
            const float d = vxo_f16_to_f32(m->scales_f16[bi]);
            const float* xv = x_pad + b * 32;
            float blk_acc = 0.0f;
            for (size_t wd = 0; wd < 4; ++wd) {
                const uint32_t word = m->qs_words[bi * 4 + wd];
                const size_t j = wd * 4;
                for (size_t k = 0; k < 4; ++k) {
                    const uint32_t byte = (word >> (8 * k)) & 0xffu;
                    const float q0 = (float)((int32_t)(byte & 0x0fu) - 8);
                    const float q1 = (float)((int32_t)(byte >> 4) - 8);
                    blk_acc = fmaf(q0, xv[j + k], blk_acc);
                    blk_acc = fmaf(q1, xv[j + k + 16], blk_acc);
                }
            }
            sum = fmaf(d, blk_acc, sum);
        }
        y[r] = sum;
    }
}

VXO_API void vxo_q40_gemv(const vxo_q40* m, const float* x, float* y, int threads) {
    float* x_pad = (float*)calloc(m->padded_cols ? m->padded_cols : 1, sizeof(float));
    memcpy(x_pad, x, (size_t)m->cols * sizeof(float));
    vxo_run_rows(vxo_q40_rows, m, x_pad, y, m->rows, threads);
    free(x_pad);
}

/* ------------------------------------------------------------------------- */
/* Prefill GEMM: PackedTensor::gemm_cpu (llm_prefill.rs:156-255) with the      */
/* scalar dense_tile_gemm (llm_prefill.rs:139-153).                           */
/* ------------------------------------------------------------------------- */

enum { VXO_KIND_CB4 = 1, VXO_KIND_G64 = 2, VXO_KIND_Q8 = 3, VXO_KIND_Q40 = 4 };

static void vxo_decode_row_any(int kind, const void* m, size_t r, float* dst) {
    if (kind == VXO_KIND_CB4) vxo_cb4_decode_row((const vxo_cb4*)m, r, dst);
    else if (kind == VXO_KIND_G64) vxo_g64_decode_row((const vxo_g64*)m, r, dst);
    else if (kind == VXO_KIND_Q40) vxo_q40_decode_row((const vxo_q40*)m, r, dst);
    else vxo_q8_decode_row((const vxo_q8*)m, r, dst);
}

static void vxo_dims(int kind, const void* m, size_t* rows, size_t* cols) {
    if (kind == VXO_KIND_CB4) { *rows = ((const vxo_cb4*)m)->rows; *cols = ((const vxo_cb4*)m)->cols; }
    else if (kind == VXO_KIND_G64) { *rows = ((const vxo_g64*)m)->rows; *cols = ((const vxo_g64*)m)->cols; }
    else if (kind == VXO_KIND_Q40) { *rows = ((const vxo_q40*)m)->rows; *cols = ((const vxo_q40*)m)->cols; }
    else { *rows = ((const vxo_q8*)m)->rows; *cols = ((const vxo_q8*)m)->cols; }
}

/* llm_prefill.rs:139-153 (non-mac branch): y[m*ldc + r_off + r] = FMA chain. */
static void vxo_dense_tile_gemm(const float* x_batch, size_t batch_m, size_t cols,
                                const float* w_tile, size_t br, float* y_dst, size_t ldc,
                                size_t r_off) {
    for (size_t m = 0; m < batch_m; ++m) {
        const float* xm = x_batch + m * cols;
        float* ym = y_dst + m * ldc + r_off;
        for (size_t r = 0; r < br; ++r) {
            const float* wr = w_tile + r * cols;
            float s = 0.0f;
            for (size_t c = 0; c < cols; ++c) s = fmaf(wr[c], xm[c], s);
            ym[r] = s;
        }
    }
}

typedef struct {
    int kind;
    const void* m;
    const float* x_batch;
    size_t batch_m, cols, r_beg, w_rows;
    float* part_y;
} vxo_gemm_job;

#define VXO_TILE_R 32

static void* vxo_gemm_thread(void* p) {
    vxo_gemm_job* j = (vxo_gemm_job*)p;
    size_t tile_rows = j->w_rows < VXO_TILE_R ? j->w_rows : VXO_TILE_R;
    float* w_tile = (float*)malloc((tile_rows ? tile_rows : 1) * j->cols * sizeof(float));
    for (size_t loc_r = 0; loc_r < j->w_rows;) {
        size_t br = j->w_rows - loc_r < VXO_TILE_R ? j->w_rows - loc_r : VXO_TILE_R;
        for (size_t dr = 0; dr < br; ++dr)
            vxo_decode_row_any(j->kind, j->m, j->r_beg + loc_r + dr, w_tile + dr * j->cols);
        vxo_dense_tile_gemm(j->x_batch, j->batch_m, j->cols, w_tile, br, j->part_y, j->w_rows,
                            loc_r);
        loc_r += br;
    }
    free(w_tile);
    return NULL;
}

/* gemm_cpu for batch_m >= 2 (batch_m == 1 dispatches to the GEMV, :168-171,
 * which is the caller's job here).  workers = clamp(threads,1,16) capped at the
 * number of 32-row tiles; each worker decodes its tiles and writes a private
 * [batch_m x w_rows] block that is copied into y_batch afterwards (:202-254). */
VXO_API void vxo_gemm(int kind, const void* m, const float* x_batch, size_t batch_m,
                      float* y_batch, int threads) {
    size_t rows, cols;
    vxo_dims(kind, m, &rows, &cols);
    if (batch_m == 0 || rows == 0) return;
    size_t t = threads < 1 ? 1 : (threads > 16 ? 16 : (size_t)threads);
    size_t tiles_total = (rows + VXO_TILE_R - 1) / VXO_TILE_R;
    size_t workers = t < tiles_total ? t : tiles_total;
    if (workers < 1) workers = 1;
    size_t tiles_per_worker = (tiles_total + workers - 1) / workers;
    size_t rows_per_worker = tiles_per_worker * VXO_TILE_R;
    size_t n = 0;
    vxo_gemm_job* jobs = (vxo_gemm_job*)calloc(workers, sizeof(vxo_gemm_job));
    pthread_t* tid = (pthread_t*)calloc(workers, sizeof(pthread_t));
    for (size_t wi = 0; wi < workers; ++wi) {
        size_t r_beg = wi * rows_per_worker;
        if (r_beg >= rows) break;
        size_t w_rows = rows - r_beg < rows_per_worker ? rows - r_beg : rows_per_worker;
        jobs[n].kind = kind; jobs[n].m = m; jobs[n].x_batch = x_batch;
        jobs[n].batch_m = batch_m; jobs[n].cols = cols; jobs[n].r_beg = r_beg;
        jobs[n].w_rows = w_rows;
        jobs[n].part_y = (float*)calloc(batch_m * w_rows, sizeof(float));
        ++n;
    }
    if (n == 1) {
        vxo_gemm_thread(&jobs[0]);
    } else {
        for (size_t i = 0; i < n; ++i) pthread_create(&tid[i], NULL, vxo_gemm_thread, &jobs[i]);
        for (size_t i = 0; i < n; ++i) pthread_join(tid[i], NULL);
    }
    for (size_t i = 0; i < n; ++i) {
        for (size_t mm = 0; mm < batch_m; ++mm)
            memcpy(y_batch + mm * rows + jobs[i].r_beg, jobs[i].part_y + mm * jobs[i].w_rows,
                   jobs[i].w_rows * sizeof(float));
        free(jobs[i].part_y);
    }
    free(jobs);
    free(tid);
}

/* The GEMV entry used by gemm_cpu's batch_m == 1 branch, for any kind. */
VXO_API void vxo_gemv_any(int kind, const void* m, const float* x, float* y, int threads) {
    if (kind == VXO_KIND_CB4) vxo_cb4_gemv((const vxo_cb4*)m, x, y, threads);
    else if (kind == VXO_KIND_G64) vxo_g64_gemv((const vxo_g64*)m, x, y, threads);
    else if (kind == VXO_KIND_Q40) vxo_q40_gemv((const vxo_q40*)m, x, y, threads);
    else vxo_q8_gemv((const vxo_q8*)m, x, y, threads);
}

/* llm_ops.rs:39-41: silu(x) = x / (1 + exp(-x)) in f32 (Rust's f32::exp is
 * the platform libm expf on Linux, which this calls). */
VXO_API float vxo_silu(float x) { return x / (1.0f + expf(-x)); }

/* llm_prefill.rs:66-71, each operation rounded in source order. */
VXO_API float vxo_gelu_tanh(float g) {
    const float z = 0.7978846f * (g + 0.044715f * g * g * g);
    const float e2 = expf(-2.0f * fabsf(z));
    const float th = copysignf((1.0f - e2) / (1.0f + e2), z);
    return 0.5f * g * (1.0f + th);
}

/* llm_cpu.rs:457-464: out[i] = act(g[i]) * u[i]. */
VXO_API void vxo_glu(const float* g, const float* u, size_t n, int gelu, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = (gelu ? vxo_gelu_tanh(g[i]) : vxo_silu(g[i])) * u[i];
}

/* llm_ops.rs:48-57: sq = sequential f32 fma chain; scale = 1 / sqrt(sq / n +
 * eps); out[i] = x[i] * scale * w[i] (two roundings, left to right). */
VXO_API void vxo_rms_norm(const float* x, const float* w, size_t n, float eps, float* out) {
    float sq = 0.0f;
    for (size_t i = 0; i < n; ++i) sq = fmaf(x[i], x[i], sq);
    const float scale = 1.0f / sqrtf(sq / (float)n + eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

/* llm_prefill.rs:317-367: the attention of one decode step over a Q8 KV
 * cache, after q and k are normed and rotated and the step's K/V blocks are
 * in the cache.  q: [n_head * hd]; k_blocks / v_blocks: 34-byte KvQ8Block
 * rows laid out [t][kv_head][hd / 32] for t < seq_len; gate: NULL or
 * [n_head * hd]; out: [n_head * hd].  Scores are block dots summed in block
 * order, scaled by 1 / sqrt(hd); softmax subtracts the running max; the
 * output accumulates axpy_f32 of every position in order; a gate multiplies
 * by 1 / (1 + exp(-g)). */
VXO_API void vxo_attn_q8(const float* q, const uint8_t* k_blocks, const uint8_t* v_blocks, size_t seq_len,
                         uint32_t n_head, uint32_t n_kv, uint32_t hd, const float* gate, float* out) {
    const size_t bph = hd / 32, stride = (size_t)n_kv * bph;
    const uint32_t gqa = n_head / n_kv;
    const float scale = 1.0f / sqrtf((float)hd);
    float* scores = (float*)malloc((seq_len ? seq_len : 1) * sizeof(float));
    for (uint32_t h = 0; h < n_head; ++h) {
        const uint32_t kv_h = h / gqa;
        const float* qh = q + (size_t)h * hd;
        float max_s = -INFINITY;
        for (size_t t = 0; t < seq_len; ++t) {
            const uint8_t* kb = k_blocks + (t * stride + (size_t)kv_h * bph) * 34;
            float dot = 0.0f;
            for (size_t b = 0; b < bph; ++b) dot += vxo_q8_dot_f32(kb + b * 34, qh + b * 32);
            const float sc = dot * scale;
            scores[t] = sc;
            if (sc > max_s) max_s = sc;
        }
        float sum_exp = 0.0f;
        for (size_t t = 0; t < seq_len; ++t) {
            const float e = expf(scores[t] - max_s);
            scores[t] = e;
            sum_exp += e;
        }
        const float inv_sum = 1.0f / sum_exp;
        float* oh = out + (size_t)h * hd;
        for (uint32_t i = 0; i < hd; ++i) oh[i] = 0.0f;
        for (size_t t = 0; t < seq_len; ++t) {
            const float w = scores[t] * inv_sum;
            const uint8_t* vb = v_blocks + (t * stride + (size_t)kv_h * bph) * 34;
            for (size_t b = 0; b < bph; ++b) vxo_q8_axpy_f32(vb + b * 34, w, oh + b * 32);
        }
        if (gate) {
            const float* gh = gate + (size_t)h * hd;
            for (uint32_t i = 0; i < hd; ++i) oh[i] *= 1.0f / (1.0f + expf(-gh[i]));
        }
    }
    free(scores);
}

/* llm_ops.rs:81-99 apply_rope: rotate pairs of vec[0 .. min(rope_dim, len))
 * by theta_i = pos * freq_base^(-2i / rdim), i < rdim / 2 (f32 powf, the
 * product pos * freq in f32, sinf / cosf); neox pairs (i, i + rdim / 2),
 * otherwise (2i, 2i + 1).  x0' = x0 c - x1 s, x1' = x0 s + x1 c, each
 * product rounded on its own. */
VXO_API void vxo_apply_rope(float* vec, size_t len, size_t pos, size_t rope_dim, float freq_base, int neox) {
    const size_t rdim = rope_dim < len ? rope_dim : len;
    const size_t half = rdim / 2;
    for (size_t i = 0; i < half; ++i) {
        const float freq = powf(freq_base, -(2.0f * (float)i) / (float)rdim);
        const float theta = (float)pos * freq;
        const float sin_t = sinf(theta), cos_t = cosf(theta);
        const size_t i0 = neox ? i : 2 * i, i1 = neox ? i + half : 2 * i + 1;
        const float x0 = vec[i0], x1 = vec[i1];
        vec[i0] = x0 * cos_t - x1 * sin_t;
        vec[i1] = x0 * sin_t + x1 * cos_t;
    }
}

/* llm_prefill.rs:284-313: the part of step_full_gqa_q8 before the scores.
 * Per query head h: q_raw's head slice (gated: [q | gate], 2 hd values;
 * else hd), q_norm'd (rms_norm, llm_ops.rs:48-57) when q_norm is given,
 * rotated at rope_pos -> q_heads[h * hd ..], the gate half -> q_gates.  Per kv
 * head: k_cur's slice k_norm'd and rotated in place, then K and V quantised
 * (KvQ8Block::quantize) into row pos of the [t][kv head][hd / 32] block
 * arrays. */
VXO_API void vxo_gqa_prep_q8(const float* q_raw, float* k_cur, const float* v_cur, const float* q_norm,
                             const float* k_norm, int gated, uint32_t n_head, uint32_t n_kv, uint32_t hd, size_t pos,
                             size_t rope_pos, size_t rope_dim, float freq_base, int neox, float eps,
                             uint8_t* k_blocks, uint8_t* v_blocks, float* q_heads, float* q_gates) {
    float* tmp = (float*)malloc(hd * sizeof(float));
    for (uint32_t h = 0; h < n_head; ++h) {
        float* q_dst = q_heads + (size_t)h * hd;
        const float* src = q_raw + (size_t)h * (gated ? 2u : 1u) * hd;
        memcpy(q_dst, src, hd * sizeof(float));
        if (gated) memcpy(q_gates + (size_t)h * hd, src + hd, hd * sizeof(float));
        if (q_norm) {
            memcpy(tmp, q_dst, hd * sizeof(float));
            vxo_rms_norm(tmp, q_norm, hd, eps, q_dst);
        }
        vxo_apply_rope(q_dst, hd, rope_pos, rope_dim, freq_base, neox);
    }
    for (uint32_t kh = 0; kh < n_kv; ++kh) {
        float* ks = k_cur + (size_t)kh * hd;
        if (k_norm) {
            memcpy(tmp, ks, hd * sizeof(float));
            vxo_rms_norm(tmp, k_norm, hd, eps, ks);
        }
        vxo_apply_rope(ks, hd, rope_pos, rope_dim, freq_base, neox);
    }
    const size_t bph = hd / 32, stride = (size_t)n_kv * bph;
    for (uint32_t kh = 0; kh < n_kv; ++kh) {
        for (size_t b = 0; b < bph; ++b) {
            const size_t off = (size_t)kh * hd + b * 32, blk = pos * stride + (size_t)kh * bph + b;
            vxo_q8_quantize(k_cur + off, k_blocks + blk * 34);
            vxo_q8_quantize(v_cur + off, v_blocks + blk * 34);
        }
    }
    free(tmp);
}

/* llm_prefill.rs:259-367 step_full_gqa_q8, whole: the prep above, then the
 * attention of the query heads over positions [0, pos] (vxo_attn_q8) with the
 * gate of a gated q.  out: [n_head * hd]. */
VXO_API void vxo_gqa_step_q8(const float* q_raw, float* k_cur, const float* v_cur, const float* q_norm,
                             const float* k_norm, int gated, uint32_t n_head, uint32_t n_kv, uint32_t hd, size_t pos,
                             size_t rope_pos, size_t rope_dim, float freq_base, int neox, float eps,
                             uint8_t* k_blocks, uint8_t* v_blocks, float* out) {
    float* qh = (float*)malloc((size_t)n_head * hd * sizeof(float));
    float* qg = gated ? (float*)malloc((size_t)n_head * hd * sizeof(float)) : NULL;
    vxo_gqa_prep_q8(q_raw, k_cur, v_cur, q_norm, k_norm, gated, n_head, n_kv, hd, pos, rope_pos, rope_dim, freq_base,
                    neox, eps, k_blocks, v_blocks, qh, qg);
    vxo_attn_q8(qh, k_blocks, v_blocks, pos + 1, n_head, n_kv, hd, qg, out);
    free(qg);
    free(qh);
}

/* Greedy selection.  The index follows the greedy branch of
 * sample_logits_top_k_p (llm_ops.rs:307-327): an empty input gives 0; else a
 * forward scan from (best_v = -inf, best_i = 0) that takes index i only when
 * logits[i] > best_v, so the first of equal maxima wins, NaN never wins and
 * nothing above -inf leaves 0.  *nonfinite is the flag vxt_greedy_exact adds
 * (vxt_llm_ops.metal:569-600): 1 when any logit is NaN or +-inf. */
VXO_API uint32_t vxo_greedy(const float* logits, size_t n, uint32_t* nonfinite) {
    uint32_t best_i = 0, nf = 0;
    float best_v = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        const float v = logits[i];
        if (!isfinite(v)) nf = 1;
        if (v > best_v) { best_v = v; best_i = (uint32_t)i; }
    }
    if (nonfinite) *nonfinite = nf;
    return best_i;
}

VXO_API int vxo_hardware_threads(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}
