/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of gguf-runner's attention hot path, used as the parity
 * checker for the HIP kernels and as the CPU baseline leg of bench.py.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may load it; the
 * product library (libgr_attn.so) never links or calls anything here.
 *
 * Each function follows the x86_64 branch of the cited Rust function in
 * /root/reference (gguf-runner v0.7.0).  The reference cannot be built here
 * (no Rust toolchain), so this file is the oracle; tests/test_oracle_*.py pin
 * it against the reference's own unit-test constants and against closed forms.
 *
 * Arithmetic fidelity notes:
 *  - Built with -ffp-contract=off: the reference's scalar loops are compiled by
 *    rustc/LLVM without FMA contraction, so a*b+c stays two roundings.
 *  - axpy_inplace (quant.rs:1069-1080) dispatches to the AVX2-FMA kernel on
 *    x86 (quant.rs:1023-1047, 1049-1067); it is restated with fmaf().
 *  - libm expf/powf/cosf/sinf/sqrtf are the host glibc ones, like Rust's
 *    f32::{exp,powf,cos,sin,sqrt} on linux-x86_64.
 *  - Parallel-over-heads (rayon, inference.rs:2002-2007) is restated with
 *    OpenMP; every head is computed by one thread in the same order as the
 *    serial branch, so results do not depend on the thread count.
 *
 * Parity pinning status is recorded per function in the comment above it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 2
#define ORC_Q8 3  /* int8 rows, one f32 scale per kv_dim row */
#define ORC_Q8B 4 /* int8 rows, one f32 scale per 32 elements (GGUF_Q8_BLOCK_SCALES) */
#define ORC_Q8_BLOCK 32 /* Q4_BLOCK_SIZE */

/* ---------------------------------------------------------------- dtypes */

/* IEEE binary16 -> f32 (exact).  Same semantics as fp16_to_fp32,
 * src/engine/io/gguf.rs:27-61. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while ((man & 0x400u) == 0);
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* bfloat16 -> f32 (exact), gguf.rs:63-70. */
float orc_bf16_to_f32(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float load_kv(const void* base, size_t idx, int fmt) {
    switch (fmt) {
        case ORC_F16: return orc_f16_to_f32(((const uint16_t*)base)[idx]);
        case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)base)[idx]);
        case ORC_Q8:
        case ORC_Q8B: return (float)((const int8_t*)base)[idx];
        default: return ((const float*)base)[idx];
    }
}

/* ---------------------------------------------------------------- RoPE */

/* Frequency table, inference.rs:1590-1609:
 *   freq_i = 1 / theta^((2i) as f32 / rope_dim as f32)
 * Pinned by: tests/test_oracle_rope.py (reference constants 4098-4118 with
 * unit frequencies; closed form against float64). */
void orc_rope_freqs(float theta, int rope_dim, float* freqs) {
    int half = rope_dim / 2;
    for (int i = 0; i < half; i++) {
        freqs[i] = 1.0f / powf(theta, (float)(i * 2) / (float)rope_dim);
    }
}

/* rebuild_rope_cache, inference.rs:1485-1523, text positions (the position
 * plan is [pos;3] for text, 1498-1501):
 *   val = (pos as f32 * freq) * frequency_scale;  cos = val.cos(); sin = val.sin()
 * Pinned by: reference test inference.rs:4098-4118 (cos 8/sin 8/cos 1/sin 1). */
void orc_rope_cache(const float* freqs, int half, int64_t pos, float scale, float* cos_out,
                    float* sin_out) {
    for (int i = 0; i < half; i++) {
        float val = ((float)pos * freqs[i]) * scale;
        cos_out[i] = cosf(val);
        sin_out[i] = sinf(val);
    }
}

/* apply_rope_qk, inference.rs:1817-1874.
 * neox != 0: half-split pairs (i, i+rope_half) per head, 1829-1852
 *            (Gemma3 / Qwen2 / Qwen3 / Qwen3VL / Qwen3MoE / Qwen3Next);
 * neox == 0: adjacent pairs over the flat q vector, k rotated while i < kv_dim,
 *            1853-1869 (Llama).
 * gemma_q_scale != 0: q *= attn_scale afterwards, 1871-1873.
 * Pinned by: reference tests 4098-4118 and 4133-4182 (pairing, partial tail),
 * pair-norm invariant, pos 0 identity. */
void orc_apply_rope_qk(float* q, float* k, int n_heads, int n_kv_heads, int head_size, int rope_half,
                       const float* cos_t, const float* sin_t, int neox, int gemma_q_scale,
                       float attn_scale) {
    int q_dim = n_heads * head_size;
    int kv_dim = n_kv_heads * head_size;
    if (neox) {
        int pair_offset = rope_half;
        for (int h = 0; h < n_heads; h++) {
            int hs = h * head_size;
            for (int i = 0; i < rope_half; i++) {
                float fcr = cos_t[i], fci = sin_t[i];
                float v0 = q[hs + i], v1 = q[hs + i + pair_offset];
                q[hs + i] = v0 * fcr - v1 * fci;
                q[hs + i + pair_offset] = v0 * fci + v1 * fcr;
            }
        }
        for (int h = 0; h < n_kv_heads; h++) {
            int hs = h * head_size;
            for (int i = 0; i < rope_half; i++) {
                float fcr = cos_t[i], fci = sin_t[i];
                float v0 = k[hs + i], v1 = k[hs + i + pair_offset];
                k[hs + i] = v0 * fcr - v1 * fci;
                k[hs + i + pair_offset] = v0 * fci + v1 * fcr;
            }
        }
    } else {
        for (int i = 0; i < q_dim; i += 2) {
            int head_dim_idx = (i % head_size) / 2;
            float fcr = cos_t[head_dim_idx], fci = sin_t[head_dim_idx];
            int rotn = i < kv_dim ? 2 : 1;
            for (int v = 0; v < rotn; v++) {
                float* vec = v == 0 ? q : k;
                float v0 = vec[i], v1 = vec[i + 1];
                vec[i] = v0 * fcr - v1 * fci;
                vec[i + 1] = v0 * fci + v1 * fcr;
            }
        }
    }
    if (gemma_q_scale) {
        for (int i = 0; i < q_dim; i++) q[i] *= attn_scale;
    }
}

/* rmsnorm_per_head_gemma_inplace, math.rs:164-184 (QK-norm, applied by
 * qkv_bias_and_norm, inference.rs:2535-2572):
 *   ss = sum(x^2)/d + eps;  x_j = w_j * ((1/sqrt(ss)) * x_j)
 * Pinned by: closed form (unit RMS with w = 1) in tests/test_oracle_misc.py. */
void orc_rmsnorm_per_head(float* x, const float* weight, int n_heads, int head_size, float eps) {
    for (int h = 0; h < n_heads; h++) {
        int hs = h * head_size;
        float ss = 0.0f;
        for (int j = 0; j < head_size; j++) ss += x[hs + j] * x[hs + j];
        ss /= (float)head_size;
        ss += eps;
        float inv = 1.0f / sqrtf(ss);
        for (int j = 0; j < head_size; j++) x[hs + j] = weight[j] * (inv * x[hs + j]);
    }
}

/* ---------------------------------------------------------------- Q8 KV codec */

/* quantize_row_q8, x86 branch, inference.rs:249-268.  Rust f32::round is
 * half-away-from-zero == C roundf.  Pinned by closed form + tie cases. */
void orc_quantize_row_q8(const float* src, int n, int8_t* dst, float* scale_out) {
    float max_abs = 0.0f;
    for (int i = 0; i < n; i++) max_abs = fmaxf(max_abs, fabsf(src[i]));
    if (max_abs == 0.0f) {
        *scale_out = 1.0f;
        memset(dst, 0, (size_t)n);
        return;
    }
    float inv = 127.0f / max_abs;
    *scale_out = max_abs / 127.0f;
    for (int i = 0; i < n; i++) {
        float r = roundf(src[i] * inv);
        if (r < -127.0f) r = -127.0f;
        if (r > 127.0f) r = 127.0f;
        dst[i] = (int8_t)r;
    }
}

/* kv_write_token's Q8 branch, inference.rs:1886-1917, for one K or V row of
 * kv_dim elements: block mode (GGUF_Q8_BLOCK_SCALES) quantises each 32-element
 * block with quantize_row_q8 and writes kv_dim/32 scales; row mode quantises the
 * whole row with one scale.  Pinned through orc_quantize_row_q8 and the
 * per-block closed form in tests/test_oracle_rope_norm.py. */
void orc_kv_quantize_row(const float* src, int kv_dim, int block, int8_t* dst, float* scales) {
    if (block) {
        for (int b = 0; b < kv_dim / ORC_Q8_BLOCK; b++)
            orc_quantize_row_q8(src + b * ORC_Q8_BLOCK, ORC_Q8_BLOCK, dst + b * ORC_Q8_BLOCK,
                                scales + b);
    } else {
        orc_quantize_row_q8(src, kv_dim, dst, scales);
    }
}

/* ---------------------------------------------------------------- softmax */

/* softmax, x86 branch, math.rs:263-280. */
void orc_softmax(float* x, int size) {
    float max_val = x[0];
    for (int i = 1; i < size; i++)
        if (x[i] > max_val) max_val = x[i];
    float sum = 0.0f;
    for (int i = 0; i < size; i++) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    float inv_sum = 1.0f / sum;
    for (int i = 0; i < size; i++) x[i] *= inv_sum;
}

/* ---------------------------------------------------------------- attention */

/* Row dot / axpy.  Q8: dot_q8_row / axpy_q8_row scalar x86 branches,
 * inference.rs:1337-1366:  acc += q * (c * scale);  scaled = a*scale; d += scaled*c.
 * Raw storage (f32/f16/bf16): the same loops with the exact dequantiser
 * (scale == 1 removed): acc += q * c;  d += a * c. */
static inline float row_dot(const float* q, const void* cache, size_t off, int n, int fmt,
                            float scale) {
    float acc = 0.0f;
    if (fmt == ORC_Q8) {
        const int8_t* c = (const int8_t*)cache + off;
        for (int i = 0; i < n; i++) acc += q[i] * ((float)c[i] * scale);
    } else {
        for (int i = 0; i < n; i++) acc += q[i] * load_kv(cache, off + (size_t)i, fmt);
    }
    return acc;
}

static inline void row_axpy(float* dst, float a, const void* cache, size_t off, int n, int fmt,
                            float scale) {
    if (fmt == ORC_Q8) {
        const int8_t* c = (const int8_t*)cache + off;
        float scaled = a * scale;
        for (int i = 0; i < n; i++) dst[i] += scaled * (float)c[i];
    } else {
        for (int i = 0; i < n; i++) dst[i] += a * load_kv(cache, off + (size_t)i, fmt);
    }
}

/* dot_q8_row_blocks_ptr / axpy_q8_row_blocks_ptr, inference.rs:1368-1483:
 * one dot_q8_row / axpy_q8_row per 32-element block with that block's scale,
 * block dots added to the accumulator in block order (the 4-way unrolled loop
 * keeps that order). */
static inline float row_dot_blocks(const float* q, const int8_t* cache, size_t off, int n,
                                   const float* scales) {
    float acc = 0.0f;
    for (int b = 0; b * ORC_Q8_BLOCK < n; b++) {
        float part = 0.0f;
        const int8_t* c = cache + off + (size_t)b * ORC_Q8_BLOCK;
        const float* qb = q + b * ORC_Q8_BLOCK;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) part += qb[i] * ((float)c[i] * scales[b]);
        acc += part;
    }
    return acc;
}

static inline void row_axpy_blocks(float* dst, float a, const int8_t* cache, size_t off, int n,
                                   const float* scales) {
    for (int b = 0; b * ORC_Q8_BLOCK < n; b++) {
        float scaled = a * scales[b];
        const int8_t* c = cache + off + (size_t)b * ORC_Q8_BLOCK;
        float* d = dst + b * ORC_Q8_BLOCK;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) d[i] += scaled * (float)c[i];
    }
}

/* Score and value update of key row t_row for one head, any storage format.
 * Q8B scales of (row, kv head) start at t_row*kv_dim/32 + kv_head_offset/32
 * (inference.rs:2021-2027 with sb = t_row*n_blocks_per_row). */
static inline float key_dot(const float* q_head, const void* key_cache, size_t row_offset,
                            int head_size, int fmt, const float* key_scale, size_t t_row,
                            size_t kv_dim, size_t kv_head_offset) {
    if (fmt == ORC_Q8B)
        return row_dot_blocks(q_head, (const int8_t*)key_cache, row_offset, head_size,
                              key_scale + t_row * (kv_dim / ORC_Q8_BLOCK) +
                                  kv_head_offset / ORC_Q8_BLOCK);
    return row_dot(q_head, key_cache, row_offset, head_size, fmt,
                   fmt == ORC_Q8 ? key_scale[t_row] : 1.0f);
}

static inline void value_axpy(float* xb_head, float w, const void* value_cache, size_t row_offset,
                              int head_size, int fmt, const float* value_scale, size_t t_row,
                              size_t kv_dim, size_t kv_head_offset) {
    if (fmt == ORC_Q8B) {
        row_axpy_blocks(xb_head, w, (const int8_t*)value_cache, row_offset, head_size,
                        value_scale + t_row * (kv_dim / ORC_Q8_BLOCK) +
                            kv_head_offset / ORC_Q8_BLOCK);
        return;
    }
    row_axpy(xb_head, w, value_cache, row_offset, head_size, fmt,
             fmt == ORC_Q8 ? value_scale[t_row] : 1.0f);
}

/* One query head of attention_token, inference.rs:2008-2284 (the per-head
 * closure; the serial branch 2290-2528 computes the same thing).
 *   online == 0: two-pass: scores -> softmax (math.rs:263-280) -> axpy (2175-2283)
 *   online == 1: online-softmax fusion used iff online_attn_fusion (2048-2174):
 *                running max from -inf, rescale exp(m_old - m_new) applied to acc
 *                and sum only when sum > 0, final *(1/sum) when sum > 0. */
static void attention_head(const float* q_head, float* xb_head, float* att_head, int head_size,
                           const void* key_cache, const void* value_cache, int fmt,
                           const float* key_scale, const float* value_scale, size_t layer_row_base,
                           size_t kv_dim, size_t kv_head_offset, size_t vis_start, size_t vis_end,
                           float attn_scale, int apply_attn_scale, int online) {
    if (online) {
        for (int i = 0; i < head_size; i++) xb_head[i] = 0.0f;
        float max_score = -INFINITY;
        float score_sum = 0.0f;
        for (size_t t = vis_start; t < vis_end; t++) {
            size_t t_row = layer_row_base + t;
            size_t row_offset = t_row * kv_dim + kv_head_offset;
            float score = key_dot(q_head, key_cache, row_offset, head_size, fmt, key_scale, t_row,
                                  kv_dim, kv_head_offset);
            if (apply_attn_scale) score *= attn_scale;
            if (score > max_score) {
                if (score_sum > 0.0f) {
                    float rescale = expf(max_score - score);
                    for (int i = 0; i < head_size; i++) xb_head[i] *= rescale;
                    score_sum *= rescale;
                }
                max_score = score;
            }
            float weight = expf(score - max_score);
            score_sum += weight;
            value_axpy(xb_head, weight, value_cache, row_offset, head_size, fmt, value_scale, t_row,
                       kv_dim, kv_head_offset);
        }
        if (score_sum > 0.0f) {
            float inv = 1.0f / score_sum;
            for (int i = 0; i < head_size; i++) xb_head[i] *= inv;
        }
    } else {
        size_t n = vis_end - vis_start;
        for (size_t t = vis_start; t < vis_end; t++) {
            size_t t_row = layer_row_base + t;
            size_t row_offset = t_row * kv_dim + kv_head_offset;
            float score = key_dot(q_head, key_cache, row_offset, head_size, fmt, key_scale, t_row,
                                  kv_dim, kv_head_offset);
            if (apply_attn_scale) score *= attn_scale;
            att_head[t - vis_start] = score;
        }
        orc_softmax(att_head, (int)n);
        for (int i = 0; i < head_size; i++) xb_head[i] = 0.0f;
        for (size_t t = vis_start; t < vis_end; t++) {
            size_t t_row = layer_row_base + t;
            size_t row_offset = t_row * kv_dim + kv_head_offset;
            value_axpy(xb_head, att_head[t - vis_start], value_cache, row_offset, head_size, fmt,
                       value_scale, t_row, kv_dim, kv_head_offset);
        }
    }
}

/* attention_token, inference.rs:1970-2530, for one (layer, pos).
 * The KV cache is indexed like RunState's: element (row t_row, kv head g, i) at
 * t_row*kv_dim + g*head_size + i with t_row = layer_row_base + t (1880-1882).
 * GQA: kv_head = h / kv_mul (2019).  Visible keys [vis_start, vis_end) come from
 * LanguageAttentionPolicy::visible_keys (attention.rs:74-96).
 * att must hold n_heads * att_stride floats (att_stride >= vis_end - vis_start).
 * n_threads > 1 parallelises over heads like the rayon branch (2002-2007).
 * Pinned by: fp64 closed form + special cases in tests/test_oracle_attention.py. */
void orc_attention_token(const float* q, float* xb, float* att, size_t att_stride, int n_heads,
                         int n_kv_heads, int head_size, const void* key_cache,
                         const void* value_cache, int fmt, const float* key_scale,
                         const float* value_scale, size_t layer_row_base, size_t vis_start,
                         size_t vis_end, float attn_scale, int apply_attn_scale, int online,
                         int n_threads) {
    int kv_mul = n_heads / n_kv_heads;
    size_t kv_dim = (size_t)n_kv_heads * (size_t)head_size;
#pragma omp parallel for schedule(static) num_threads(n_threads > 0 ? n_threads : 1) if (n_threads > 1)
    for (int h = 0; h < n_heads; h++) {
        int kv_head = h / kv_mul;
        attention_head(q + (size_t)h * head_size, xb + (size_t)h * head_size,
                       att + (size_t)h * att_stride, head_size, key_cache, value_cache, fmt,
                       key_scale, value_scale, layer_row_base, kv_dim,
                       (size_t)kv_head * head_size, vis_start, vis_end, attn_scale,
                       apply_attn_scale, online);
    }
}

/* LanguageAttentionPolicy::visible_keys, attention.rs:74-96 (text tokens):
 * end = query + 1; start = window ? end.saturating_sub(window) : 0.
 * window == 0 encodes "None" (global layer).  Pinned by attention.rs:171-172
 * and the window semantics comment types.rs:614-616. */
void orc_visible_keys(int64_t window, int64_t query, int64_t* start, int64_t* end) {
    int64_t e = query + 1;
    int64_t s = 0;
    if (window > 0) s = e > window ? e - window : 0;
    *start = s;
    *end = e;
}

/* ---------------------------------------------------------------- per-token layer driver */

/* Round one f32 to the raw storage format (the raw-mode "kv_write_token"):
 * f16 / bf16 use IEEE round-to-nearest-even like fp32_to_fp16 / fp32_to_bf16,
 * src/engine/io/gguf.rs:72-117. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf, or NaN keeping its top payload bits, quieted (gguf.rs:78-84) */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (((ax & 0x7fffffu) >> 13) | 0x200u) : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (ax < 0x38800000u) {                                   /* subnormal / zero in f16 */
        if (ax < 0x33000000u) return (uint16_t)sign;          /* < half the smallest subnormal */
        uint32_t man = (ax & 0x7fffffu) | 0x800000u;
        int e = (int)(ax >> 23);
        int shift = 126 - e; /* 113 - e + 13 */
        uint32_t r = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax - 0x38000000u) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

/* Array forms of the four conversions (element-wise, for the pinning tests). */
void orc_f32_to_f16_n(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(x[i]);
}
void orc_f32_to_bf16_n(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(x[i]);
}
void orc_f16_to_f32_n(const uint16_t* h, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(h[i]);
}
void orc_bf16_to_f32_n(const uint16_t* h, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(h[i]);
}

static void store_kv(void* base, size_t idx, int fmt, float v) {
    switch (fmt) {
        case ORC_F16: ((uint16_t*)base)[idx] = orc_f32_to_f16(v); break;
        case ORC_BF16: ((uint16_t*)base)[idx] = orc_f32_to_bf16(v); break;
        default: ((float*)base)[idx] = v; break;
    }
}

/* The serial prefill loop of transformer_prefill_batch, inference.rs:2981-3017,
 * for the attention part of one layer and one sequence:
 *   per token i (pos = base_pos + i):  qkv_bias_and_norm (QK-norm only, 2535-2572)
 *   -> apply_rope_qk (1817-1874) -> kv_write_token (1877-1965: raw storage, or Q8
 *   rows + scales for fmt ORC_Q8 / ORC_Q8B into key_scale / value_scale)
 *   -> attention_token (1970-2530) -> xb row.
 * Inputs q [m][n_heads*d], k/v [m][n_kv_heads*d] are f32 (already upcast from the
 * test's f16/bf16 buffers).  key/value_cache are [seq_len][kv_dim] of `fmt`.
 * rope_freqs has rope_dim/2 entries for the layer (local or global table);
 * rope_scale is the layer's frequency scale.  window 0 = global.
 * q_norm/k_norm may be NULL (no QK-norm).  Pinned through the functions it calls
 * plus tests/test_oracle_attention.py (fp64 closed form on the whole layer). */
void orc_prefill_layer(const float* q_in, const float* k_in, const float* v_in, float* xb_out,
                       int m, int64_t base_pos, int n_heads, int n_kv_heads, int head_size,
                       void* key_cache, void* value_cache, int fmt, int rope_dim, int neox,
                       const float* rope_freqs, float rope_scale, int is_gemma3, int online,
                       int64_t window, const float* q_norm, const float* k_norm, float eps,
                       float* key_scale, float* value_scale, int n_threads,
                       const uint8_t* attend, int block) {
    int q_dim = n_heads * head_size;
    int kv_dim = n_kv_heads * head_size;
    int half = rope_dim / 2;
    float attn_scale = 1.0f / sqrtf((float)head_size);
    float* q = (float*)malloc(sizeof(float) * (size_t)q_dim);
    float* k = (float*)malloc(sizeof(float) * (size_t)kv_dim);
    float* cs = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    float* sn = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    size_t att_stride = (size_t)(base_pos + m);
    float* att = (float*)malloc(sizeof(float) * (size_t)n_heads * att_stride);
    /* block: the m rows are one bidirectional image block
     * (transformer_prefill_image_block, media_prefill.rs:84-121): every row is
     * staged (norm, RoPE, KV write) first, its q kept, then each row attends to
     * [min(start, base_pos), base_pos + m) (attention.rs:87-94) */
    float* q_rows = block ? (float*)malloc(sizeof(float) * (size_t)m * q_dim) : NULL;
    for (int i = 0; i < m; i++) {
        int64_t pos = base_pos + i;
        memcpy(q, q_in + (size_t)i * q_dim, sizeof(float) * (size_t)q_dim);
        memcpy(k, k_in + (size_t)i * kv_dim, sizeof(float) * (size_t)kv_dim);
        if (q_norm && k_norm) {
            orc_rmsnorm_per_head(q, q_norm, n_heads, head_size, eps);
            orc_rmsnorm_per_head(k, k_norm, n_kv_heads, head_size, eps);
        }
        if (half > 0) {
            orc_rope_cache(rope_freqs, half, pos, rope_scale, cs, sn);
            orc_apply_rope_qk(q, k, n_heads, n_kv_heads, head_size, half, cs, sn, neox, is_gemma3,
                              attn_scale);
        } else if (is_gemma3) {
            for (int j = 0; j < q_dim; j++) q[j] *= attn_scale;
        }
        if (fmt == ORC_Q8 || fmt == ORC_Q8B) {
            const int blk = fmt == ORC_Q8B;
            const size_t so = (size_t)pos * (blk ? (size_t)kv_dim / ORC_Q8_BLOCK : 1);
            orc_kv_quantize_row(k, kv_dim, blk, (int8_t*)key_cache + (size_t)pos * kv_dim,
                                key_scale + so);
            orc_kv_quantize_row(v_in + (size_t)i * kv_dim, kv_dim, blk,
                                (int8_t*)value_cache + (size_t)pos * kv_dim, value_scale + so);
        } else {
            for (int j = 0; j < kv_dim; j++) {
                store_kv(key_cache, (size_t)pos * kv_dim + j, fmt, k[j]);
                store_kv(value_cache, (size_t)pos * kv_dim + j, fmt, v_in[(size_t)i * kv_dim + j]);
            }
        }
        if (block) {
            memcpy(q_rows + (size_t)i * q_dim, q, sizeof(float) * (size_t)q_dim);
            continue;
        }
        /* attend == NULL: every row; else only rows i with attend[i] != 0 (each
         * row's attention reads the cache rows written so far and nothing else,
         * so skipping one changes no other row) */
        if (attend && !attend[i]) continue;
        int64_t s, e;
        orc_visible_keys(window, pos, &s, &e);
        orc_attention_token(q, xb_out + (size_t)i * q_dim, att, att_stride, n_heads, n_kv_heads,
                            head_size, key_cache, value_cache, fmt, key_scale, value_scale, 0, (size_t)s,
                            (size_t)e, attn_scale, !is_gemma3, online, n_threads);
    }
    for (int i = 0; block && i < m; i++) {
        if (attend && !attend[i]) continue;
        int64_t s, e;
        orc_visible_keys(window, base_pos + i, &s, &e);
        if (s > base_pos) s = base_pos;
        e = base_pos + m;
        orc_attention_token(q_rows + (size_t)i * q_dim, xb_out + (size_t)i * q_dim, att, att_stride, n_heads,
                            n_kv_heads, head_size, key_cache, value_cache, fmt, key_scale, value_scale, 0,
                            (size_t)s, (size_t)e, attn_scale, !is_gemma3, online, n_threads);
    }
    free(q_rows);
    free(q);
    free(k);
    free(cs);
    free(sn);
    free(att);
}

/* ---------------------------------------------------------------- Turbo KV codec */

/* KvCacheFormat::Turbo, inference.rs:346-1334 (x86 scalar branches).  Per KV
 * head of a row: rotate (sign flips, normalised FWHT, sign flips), 2-bit
 * Lloyd-Max code of rotated/sigma with sigma = |rotated|/sqrt(n), then a 1-bit
 * sign sketch of the residual after a second rotation, with its norm gamma.
 * Pinned by the reference's own tests (inference.rs:4534-4566: q2 packing,
 * self-inverse transform), the SplitMix64 known answers, the Hadamard closed
 * form and the fp64 attention closed form (tests/test_oracle_turbo.py). */
static const float TQ_CENTROIDS[4] = {-1.510417f, -0.45278f, 0.45278f, 1.510417f}; /* 349 */
#define TQ_THRESHOLD 0.9815985f                                                      /* 350-351 */
static const uint64_t TQ_SALTS[4] = {0x9E3779B97F4A7C15ull, 0xC2B2AE3D27D4EB4Full,   /* 352-355 */
                                     0x165667B19E3779F9ull, 0xD6E8FEB86659FD93ull};
enum { TQ_ROT_PRE = 0, TQ_ROT_POST = 1, TQ_RES_PRE = 2, TQ_RES_POST = 3 };         /* 357-360 */

/* splitmix64, inference.rs:674-679. */
uint64_t orc_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

/* turboquant_build_sign_table, inference.rs:370-395: layout
 * [slot][layer][kv_head][ceil(head_size/8)], bit i set = multiply element i by -1. */
void orc_turbo_sign_table(int n_layers, int n_kv_heads, int head_size, uint8_t* table) {
    const size_t bytes = (size_t)(head_size + 7) / 8;
    const size_t stride = (size_t)n_layers * n_kv_heads * bytes;
    memset(table, 0, 4 * stride);
    for (int slot = 0; slot < 4; slot++)
        for (int l = 0; l < n_layers; l++)
            for (int g = 0; g < n_kv_heads; g++) {
                const uint64_t seed = orc_splitmix64(((uint64_t)l << 32) ^ (uint64_t)g ^ TQ_SALTS[slot]);
                uint8_t* bits = table + slot * stride + ((size_t)l * n_kv_heads + g) * bytes;
                for (int i = 0; i < head_size; i++)
                    if (orc_splitmix64(seed ^ (uint64_t)i) & 1) bits[i / 8] |= (uint8_t)(1u << (i & 7));
            }
}

static const uint8_t* tq_slot(const uint8_t* table, int slot, int layer, int kv_head, int n_layers,
                              int n_kv_heads, int head_size) {
    const size_t bytes = (size_t)(head_size + 7) / 8;
    return table + (size_t)slot * n_layers * n_kv_heads * bytes + ((size_t)layer * n_kv_heads + kv_head) * bytes;
}

/* turboquant_apply_signs_bits (scalar tail), inference.rs:430-436. */
static void tq_apply_signs(float* v, int n, const uint8_t* bits) {
    for (int i = 0; i < n; i++)
        if ((bits[i / 8] >> (i & 7)) & 1) v[i] = -v[i];
}

/* turboquant_fwht_inplace_scalar, inference.rs:681-701; no-op unless n is a power of two (799). */
static void tq_fwht(float* v, int n) {
    if (n <= 0 || (n & (n - 1))) return;
    for (int width = 1; width < n; width *= 2)
        for (int base = 0; base < n; base += 2 * width)
            for (int i = 0; i < width; i++) {
                const float a = v[base + i], b = v[base + i + width];
                v[base + i] = a + b;
                v[base + i + width] = a - b;
            }
    const float scale = 1.0f / sqrtf((float)n);
    for (int i = 0; i < n; i++) v[i] *= scale;
}

/* turboquant_transform_with_bits, inference.rs:596-605 (x86 path). */
void orc_turbo_transform(float* v, int n, const uint8_t* first_bits, const uint8_t* second_bits) {
    tq_apply_signs(v, n, first_bits);
    tq_fwht(v, n);
    tq_apply_signs(v, n, second_bits);
}

/* l2_norm, math.rs:467-473. */
static float tq_l2(const float* x, int n) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    return sqrtf(ss);
}

/* turboquant_quantize_code, inference.rs:805-816. */
static int tq_code(float x) {
    if (x < -TQ_THRESHOLD) return 0;
    if (x < 0.0f) return 1;
    if (x < TQ_THRESHOLD) return 2;
    return 3;
}

/* quantize_turboquant_head, inference.rs:855-925, for one head of n elements
 * starting at element `elem_offset` of the packed base (4 codes per byte, low
 * bits first) and sign (8 bits per byte, bit set = residual >= 0) arrays. */
void orc_turbo_quantize_head(const float* src, int n, const uint8_t* table, int layer, int kv_head,
                             int n_layers, int n_kv_heads, uint8_t* base, uint8_t* sign,
                             size_t elem_offset, float* scale_out, float* residual_norm_out) {
    float* rot = (float*)malloc(sizeof(float) * (size_t)n);
    float* res = (float*)malloc(sizeof(float) * (size_t)n);
    memcpy(rot, src, sizeof(float) * (size_t)n);
    orc_turbo_transform(rot, n, tq_slot(table, TQ_ROT_PRE, layer, kv_head, n_layers, n_kv_heads, n),
                        tq_slot(table, TQ_ROT_POST, layer, kv_head, n_layers, n_kv_heads, n));
    const float sigma = tq_l2(rot, n) / sqrtf((float)n);
    *scale_out = sigma;
    if (sigma == 0.0f) {
        *residual_norm_out = 0.0f;
        for (int i = 0; i < (n + 3) / 4; i++) base[elem_offset / 4 + i] = 0;
        for (int i = 0; i < n; i++) sign[(elem_offset + i) / 8] |= (uint8_t)(1u << ((elem_offset + i) & 7));
        free(rot);
        free(res);
        return;
    }
    const float inv_sigma = 1.0f / sigma;
    for (int i = 0; i < n; i += 4) {
        uint8_t packed = 0;
        for (int k = 0; k < 4 && i + k < n; k++) {
            const float value = rot[i + k];
            const int code = tq_code(value * inv_sigma);
            res[i + k] = value - TQ_CENTROIDS[code] * sigma;
            packed |= (uint8_t)(code << (k * 2));
        }
        base[elem_offset / 4 + i / 4] = packed;
    }
    const float gamma = tq_l2(res, n);
    *residual_norm_out = gamma;
    if (gamma == 0.0f) {
        for (int i = 0; i < n; i++) sign[(elem_offset + i) / 8] |= (uint8_t)(1u << ((elem_offset + i) & 7));
        free(rot);
        free(res);
        return;
    }
    for (int i = 0; i < n; i++) res[i] /= gamma;
    orc_turbo_transform(res, n, tq_slot(table, TQ_RES_PRE, layer, kv_head, n_layers, n_kv_heads, n),
                        tq_slot(table, TQ_RES_POST, layer, kv_head, n_layers, n_kv_heads, n));
    for (int i = 0; i < n; i++) {
        const size_t e = elem_offset + (size_t)i;
        if (res[i] >= 0.0f) sign[e / 8] |= (uint8_t)(1u << (e & 7));
        else sign[e / 8] &= (uint8_t)~(1u << (e & 7));
    }
    free(rot);
    free(res);
}

/* kv_write_token's Turbo branch, inference.rs:1918-1963: both rows of one token,
 * aux index row_index*n_kv_heads + kv_head (turboquant_aux_index, 669-672). */
void orc_kv_write_turbo(const float* k, const float* v, int n_kv_heads, int head_size,
                        const uint8_t* table, int layer, int n_layers, size_t row_index,
                        uint8_t* kbase, uint8_t* ksign, float* kscale, float* kres, uint8_t* vbase,
                        uint8_t* vsign, float* vscale, float* vres) {
    const size_t kv_dim = (size_t)n_kv_heads * head_size;
    for (int g = 0; g < n_kv_heads; g++) {
        const size_t off = row_index * kv_dim + (size_t)g * head_size;
        const size_t aux = row_index * n_kv_heads + g;
        orc_turbo_quantize_head(k + (size_t)g * head_size, head_size, table, layer, g, n_layers,
                                n_kv_heads, kbase, ksign, off, kscale + aux, kres + aux);
        orc_turbo_quantize_head(v + (size_t)g * head_size, head_size, table, layer, g, n_layers,
                                n_kv_heads, vbase, vsign, off, vscale + aux, vres + aux);
    }
}

/* turboquant_residual_scale, inference.rs:947-954. */
static float tq_residual_scale(int n, float residual_norm) {
    return residual_norm == 0.0f ? 0.0f : residual_norm * sqrtf(1.5707964f / (float)n);
}

/* dot_turboquant_head_scalar, inference.rs:1246-1272. */
static float tq_dot(const float* q_rot, const float* q_proj, int n, const uint8_t* base,
                    const uint8_t* sign, size_t off, float scale, float residual_norm) {
    float acc = 0.0f;
    if (scale != 0.0f)
        for (int i = 0; i < n; i++) {
            const int code = (base[(off + i) / 4] >> (((off + i) & 3) * 2)) & 3;
            acc += q_rot[i] * (TQ_CENTROIDS[code] * scale);
        }
    const float rs = tq_residual_scale(n, residual_norm);
    if (rs != 0.0f)
        for (int i = 0; i < n; i++)
            acc += ((sign[(off + i) / 8] >> ((off + i) & 7)) & 1) ? rs * q_proj[i] : -rs * q_proj[i];
    return acc;
}

/* axpy_turboquant_head_scalar, inference.rs:1286-1310. */
static void tq_axpy(float* base_acc, float* res_acc, float a, int n, const uint8_t* base,
                    const uint8_t* sign, size_t off, float scale, float residual_norm) {
    if (scale != 0.0f)
        for (int i = 0; i < n; i++) {
            const int code = (base[(off + i) / 4] >> (((off + i) & 3) * 2)) & 3;
            base_acc[i] += a * TQ_CENTROIDS[code] * scale;
        }
    const float rs = a * tq_residual_scale(n, residual_norm);
    if (rs != 0.0f)
        for (int i = 0; i < n; i++)
            res_acc[i] += ((sign[(off + i) / 8] >> ((off + i) & 7)) & 1) ? rs : -rs;
}

/* attention_token over a Turbo cache (inference.rs:2008-2290, Turbo arms) for one
 * (layer, pos): turboquant_prepare_query (954-968) per head, scores with
 * tq_dot, softmax (two-pass) or online accumulation with the residual
 * accumulator rescaled alongside, then finalize_turboquant_value_head
 * (1323-1334): inverse residual rotation, accum (= add), inverse rotation. */
void orc_attention_token_turbo(const float* q, float* xb, float* att, size_t att_stride, int n_heads,
                               int n_kv_heads, int head_size, const uint8_t* kbase,
                               const uint8_t* ksign, const float* kscale, const float* kres,
                               const uint8_t* vbase, const uint8_t* vsign, const float* vscale,
                               const float* vres, const uint8_t* table, int layer, int n_layers,
                               size_t layer_row_base, size_t vis_start, size_t vis_end,
                               float attn_scale, int apply_attn_scale, int online, int n_threads) {
    const int kv_mul = n_heads / n_kv_heads;
    const size_t kv_dim = (size_t)n_kv_heads * head_size;
    const int n = head_size;
#pragma omp parallel for schedule(static) num_threads(n_threads > 0 ? n_threads : 1) if (n_threads > 1)
    for (int h = 0; h < n_heads; h++) {
        const int g = h / kv_mul;
        float* qr = (float*)malloc(sizeof(float) * (size_t)n);
        float* qp = (float*)malloc(sizeof(float) * (size_t)n);
        float* racc = (float*)calloc((size_t)n, sizeof(float));
        float* out = xb + (size_t)h * n;
        float* ah = att + (size_t)h * att_stride;
        const uint8_t* rot_pre = tq_slot(table, TQ_ROT_PRE, layer, g, n_layers, n_kv_heads, n);
        const uint8_t* rot_post = tq_slot(table, TQ_ROT_POST, layer, g, n_layers, n_kv_heads, n);
        const uint8_t* res_pre = tq_slot(table, TQ_RES_PRE, layer, g, n_layers, n_kv_heads, n);
        const uint8_t* res_post = tq_slot(table, TQ_RES_POST, layer, g, n_layers, n_kv_heads, n);
        memcpy(qr, q + (size_t)h * n, sizeof(float) * (size_t)n);
        orc_turbo_transform(qr, n, rot_pre, rot_post);
        memcpy(qp, qr, sizeof(float) * (size_t)n);
        orc_turbo_transform(qp, n, res_pre, res_post);
        for (int i = 0; i < n; i++) out[i] = 0.0f;
        if (online) {
            float max_score = -INFINITY, score_sum = 0.0f;
            for (size_t t = vis_start; t < vis_end; t++) {
                const size_t t_row = layer_row_base + t;
                const size_t off = t_row * kv_dim + (size_t)g * n;
                const size_t aux = t_row * n_kv_heads + g;
                float score = tq_dot(qr, qp, n, kbase, ksign, off, kscale[aux], kres[aux]);
                if (apply_attn_scale) score *= attn_scale;
                if (score > max_score) {
                    if (score_sum > 0.0f) {
                        const float rescale = expf(max_score - score);
                        for (int i = 0; i < n; i++) out[i] *= rescale;
                        for (int i = 0; i < n; i++) racc[i] *= rescale;
                        score_sum *= rescale;
                    }
                    max_score = score;
                }
                const float w = expf(score - max_score);
                score_sum += w;
                tq_axpy(out, racc, w, n, vbase, vsign, off, vscale[aux], vres[aux]);
            }
            if (score_sum > 0.0f) {
                const float inv = 1.0f / score_sum;
                for (int i = 0; i < n; i++) out[i] *= inv;
                for (int i = 0; i < n; i++) racc[i] *= inv;
            }
        } else {
            const size_t cnt = vis_end - vis_start;
            for (size_t t = vis_start; t < vis_end; t++) {
                const size_t t_row = layer_row_base + t;
                const size_t off = t_row * kv_dim + (size_t)g * n;
                const size_t aux = t_row * n_kv_heads + g;
                float score = tq_dot(qr, qp, n, kbase, ksign, off, kscale[aux], kres[aux]);
                if (apply_attn_scale) score *= attn_scale;
                ah[t - vis_start] = score;
            }
            orc_softmax(ah, (int)cnt);
            for (size_t t = vis_start; t < vis_end; t++) {
                const size_t t_row = layer_row_base + t;
                const size_t off = t_row * kv_dim + (size_t)g * n;
                const size_t aux = t_row * n_kv_heads + g;
                tq_axpy(out, racc, ah[t - vis_start], n, vbase, vsign, off, vscale[aux], vres[aux]);
            }
        }
        orc_turbo_transform(racc, n, res_post, res_pre);
        for (int i = 0; i < n; i++) out[i] += racc[i];
        orc_turbo_transform(out, n, rot_post, rot_pre);
        free(qr);
        free(qp);
        free(racc);
    }
}

/* ---------------------------------------------------------------- gated DeltaNet */

/* axpy_inplace on x86 with AVX2+FMA, quant.rs:1023-1047 + 1069-1080:
 * elements in 8/16-wide blocks use fused multiply-add; a tail (n % 8) uses
 * dst += a*src with two roundings. */
static inline void axpy_inplace(float* dst, float a, const float* src, int n) {
    int n_fma = n - n % 8;
    int i = 0;
    for (; i < n_fma; i++) dst[i] = fmaf(src[i], a, dst[i]);
    for (; i < n; i++) dst[i] += a * src[i];
}

static inline float finite_or_zero(float x) { return isfinite(x) ? x : 0.0f; }

/* qwen3next_state_head_step, math.rs:492-546 (gated delta rule, one head).
 * state_h is [d][d] row-major, S[j][i] (j = key dim row, i = value dim col).
 * Pinned by: delta-rule retrieval invariant, beta=0 pure decay, fp64 brute force
 * (tests/test_oracle_deltanet.py). */
void orc_deltanet_head_step(float* state_h, float* out_h, const float* q, const float* k,
                            const float* v, float g, float beta, int d) {
    float* kv_mem = (float*)malloc(sizeof(float) * (size_t)d);
    float* delta = (float*)malloc(sizeof(float) * (size_t)d);
    for (int x = 0; x < d * d; x++) state_h[x] *= g; /* scale_slice_inplace */
    for (int i = 0; i < d; i++) kv_mem[i] = 0.0f;
    for (int j = 0; j < d; j++) {
        if (k[j] == 0.0f) continue;
        axpy_inplace(kv_mem, k[j], state_h + (size_t)j * d, d);
    }
    for (int i = 0; i < d; i++) {
        kv_mem[i] = finite_or_zero(kv_mem[i]);
        delta[i] = finite_or_zero((v[i] - kv_mem[i]) * beta);
    }
    for (int j = 0; j < d; j++) {
        if (k[j] == 0.0f) continue;
        axpy_inplace(state_h + (size_t)j * d, k[j], delta, d);
    }
    for (int i = 0; i < d; i++) out_h[i] = 0.0f;
    for (int j = 0; j < d; j++) {
        if (q[j] == 0.0f) continue;
        axpy_inplace(out_h, q[j], state_h + (size_t)j * d, d);
    }
    for (int i = 0; i < d; i++)
        if (!isfinite(out_h[i])) out_h[i] = 0.0f; /* sanitize_finite_inplace */
    free(kv_mem);
    free(delta);
}

/* The per-head L2 normalisation of qwen3next_linear_attention_projected_state,
 * math.rs:833-846: q_dst = q * (1/sqrt(sum q^2 + eps)) * (1/sqrt(d)),
 * k_dst = k * (1/sqrt(sum k^2 + eps)).  (Written as (x*inv)*scale like 844.) */
void orc_deltanet_l2norm(float* q, float* k, int d, float eps) {
    float q_ss = 0.0f, k_ss = 0.0f;
    for (int i = 0; i < d; i++) {
        q_ss += q[i] * q[i];
        k_ss += k[i] * k[i];
    }
    float q_inv = 1.0f / sqrtf(q_ss + eps);
    float k_inv = 1.0f / sqrtf(k_ss + eps);
    float inv_scale_q = 1.0f / sqrtf((float)d);
    for (int i = 0; i < d; i++) {
        q[i] = finite_or_zero(q[i] * q_inv * inv_scale_q);
        k[i] = finite_or_zero(k[i] * k_inv);
    }
}

/* sigmoidf / siluf / softplusf, math.rs:406-424. */
static float orc_sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }
static float orc_siluf(float x) { return x * orc_sigmoidf(x); }
static float orc_softplusf(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return expf(x);
    return logf(1.0f + expf(x));
}

/* qwen3next_linear_attention_projected_state, math.rs:766-953, for one token
 * of one layer (what qwen3next_linear_attention_step_from_projections,
 * math.rs:715-764, runs per token in the serial prefill loop,
 * inference.rs:2866-2885):
 *   causal depthwise conv1d over [history (K-1 rows), qkv] with SiLU (800-817),
 *   history shift (819-825), per value head h the q/k of key head h % n_k
 *   (periodic tiling, 826) L2-normalised (q also / sqrt(d)) and v (827-846),
 *   beta = sigmoid(b), g = exp(softplus(a + dt_bias) A) from the fused [b | a]
 *   projection (group-major, 853-864) or the split ones (866-870),
 *   the gated delta rule per head (492-546), then the gated RMSNorm with
 *   SiLU(z) (478-488).
 * gate_b == NULL selects the fused layout: gate_a holds 2*n_v values.
 * conv_w is [conv_dim][K]; conv_hist [(K-1)][conv_dim] and state [n_v][d][d]
 * are updated in place; out is [n_v*d] (ssm_proj).  Pinned by the float64
 * stage-by-stage closed form in tests/test_oracle_deltanet.py. */
void orc_qwen3next_ssm_token(const float* qkv, const float* z, const float* gate_a, const float* gate_b,
                             int n_k_heads, int n_v_heads, int head_dim, int conv_kernel,
                             const float* conv_w, const float* dt_bias, const float* ssm_a,
                             const float* ssm_norm, float eps, float* conv_hist, float* state,
                             float* out) {
    const int d = head_dim;
    const int d_inner = n_v_heads * d;
    const int conv_dim = d_inner + 2 * n_k_heads * d;
    const int hist = conv_kernel - 1;
    float* conv = (float*)malloc(sizeof(float) * (size_t)conv_dim);
    float* q = (float*)malloc(sizeof(float) * (size_t)d_inner);
    float* k = (float*)malloc(sizeof(float) * (size_t)d_inner);
    float* v = (float*)malloc(sizeof(float) * (size_t)d_inner);
    for (int c = 0; c < conv_dim; c++) {
        float acc = qkv[c] * conv_w[c * conv_kernel + hist];
        for (int t = 0; t < hist; t++) acc += conv_hist[t * conv_dim + c] * conv_w[c * conv_kernel + t];
        if (!isfinite(acc)) acc = 0.0f;
        conv[c] = orc_siluf(acc);
    }
    if (hist > 0) {
        if (hist > 1) memmove(conv_hist, conv_hist + conv_dim, sizeof(float) * (size_t)(hist - 1) * conv_dim);
        memcpy(conv_hist + (size_t)(hist - 1) * conv_dim, qkv, sizeof(float) * (size_t)conv_dim);
    }
    const int k_off = n_k_heads * d, v_off = 2 * n_k_heads * d;
    const float inv_scale_q = 1.0f / sqrtf((float)d);
    for (int h = 0; h < n_v_heads; h++) {
        const int src_h = h % n_k_heads;
        const float* qs = conv + src_h * d;
        const float* ks = conv + k_off + src_h * d;
        const float* vs = conv + v_off + h * d;
        float q_ss = 0.0f, k_ss = 0.0f;
        for (int i = 0; i < d; i++) {
            q_ss += qs[i] * qs[i];
            k_ss += ks[i] * ks[i];
        }
        const float q_inv = 1.0f / sqrtf(q_ss + eps), k_inv = 1.0f / sqrtf(k_ss + eps);
        for (int i = 0; i < d; i++) {
            q[h * d + i] = finite_or_zero(qs[i] * q_inv * inv_scale_q);
            k[h * d + i] = finite_or_zero(ks[i] * k_inv);
            v[h * d + i] = finite_or_zero(vs[i]);
        }
    }
    const int hpg = n_v_heads / n_k_heads;
    for (int h = 0; h < n_v_heads; h++) {
        float beta, alpha;
        if (!gate_b) {
            const int group = h / hpg, idx = h % hpg, base = group * 2 * hpg;
            beta = orc_sigmoidf(gate_a[base + idx]);
            alpha = gate_a[base + hpg + idx] + dt_bias[h];
        } else {
            beta = orc_sigmoidf(gate_b[h]);
            alpha = gate_a[h] + dt_bias[h];
        }
        float gate = orc_softplusf(alpha) * ssm_a[h];
        if (!isfinite(gate)) gate = 0.0f;
        const float g = finite_or_zero(expf(gate));
        orc_deltanet_head_step(state + (size_t)h * d * d, out + h * d, q + h * d, k + h * d, v + h * d, g,
                               finite_or_zero(beta), d);
    }
    for (int h = 0; h < n_v_heads; h++) {
        float* o = out + h * d;
        const float* zh = z + h * d;
        float ss = 0.0f;
        for (int i = 0; i < d; i++) ss += o[i] * o[i];
        const float inv = 1.0f / sqrtf(ss / (float)d + eps);
        for (int i = 0; i < d; i++) o[i] = finite_or_zero(ssm_norm[i] * (o[i] * inv) * orc_siluf(zh[i]));
    }
    free(conv);
    free(q);
    free(k);
    free(v);
}

/* Token-serial recurrence over T tokens for n_heads heads, as the reference's
 * prefill runs it (inference.rs:2866-2885 -> math.rs:890-934 per token).
 * q,k,v are [T][H][d] f32 (raw, pre-normalisation when l2norm != 0),
 * gate is [T][H] log-decay (g = exp(gate), math.rs:869-874), beta [T][H]
 * (post-sigmoid).  state [H][d][d] is updated in place; out [T][H][d]. */
void orc_deltanet_scan(const float* q, const float* k, const float* v, const float* gate,
                       const float* beta, float* state, float* out, int T, int n_heads, int d,
                       int l2norm, float eps, int n_threads) {
    for (int t = 0; t < T; t++) {
#pragma omp parallel for schedule(static) num_threads(n_threads > 0 ? n_threads : 1) if (n_threads > 1)
        for (int h = 0; h < n_heads; h++) {
            size_t off = ((size_t)t * n_heads + h) * d;
            float* qq = (float*)malloc(sizeof(float) * (size_t)d);
            float* kk = (float*)malloc(sizeof(float) * (size_t)d);
            float* vv = (float*)malloc(sizeof(float) * (size_t)d);
            memcpy(qq, q + off, sizeof(float) * (size_t)d);
            memcpy(kk, k + off, sizeof(float) * (size_t)d);
            /* v_dst = finite_or_zero(v_src), math.rs:845 */
            for (int i = 0; i < d; i++) vv[i] = finite_or_zero(v[off + i]);
            if (l2norm) orc_deltanet_l2norm(qq, kk, d, eps);
            float g = finite_or_zero(expf(gate[(size_t)t * n_heads + h]));
            float b = finite_or_zero(beta[(size_t)t * n_heads + h]);
            orc_deltanet_head_step(state + (size_t)h * d * d, out + off, qq, kk, vv, g, b, d);
            free(qq);
            free(kk);
            free(vv);
        }
    }
}

/* sigmoid_mul_inplace, math.rs:396-403 (the x86 / portable branch): the Qwen3.5
 * packed-q output gate, d[i] = finite_or_zero(d[i] * (1 / (1 + exp(-g[i])))).
 * Pinned by: float64 sigmoid (closed form), g = +-inf and NaN special cases
 * (tests/test_oracle_attention.py). */
void orc_sigmoid_mul(float* d, const float* g, int n) {
    for (int i = 0; i < n; i++) {
        const float s = 1.0f / (1.0f + expf(-g[i]));
        d[i] = finite_or_zero(d[i] * s);
    }
}

/* ---------------------------------------------------------------- encoder attention */

/* dot_f32_simd on x86 with AVX2+FMA (quant.rs:741-763 dot_f32_avx2_ptr, via the
 * dispatch at 955-958): two 8-lane FMA accumulators over 16-element blocks, the
 * lanes of their sum added left to right, then a tail of separate multiply and
 * add. */
static float dot_f32_avx2(const float* a, const float* b, int n) {
    float acc0[8] = {0}, acc1[8] = {0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 8; l++) {
            acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
            acc1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], acc1[l]);
        }
    float sum = 0.0f;
    for (int l = 0; l < 8; l++) sum += acc0[l] + acc1[l];
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* encoder_self_attention_portable (multimodal/mod.rs:206-256): for each token of
 * each sequence and each head, an online softmax over the tokens of its own
 * sequence in order: score = dot * (1/sqrt(d)); on a new maximum the output is
 * rescaled by exp(old - new) when the running sum is positive; the weight
 * exp(score - max) is added to the sum and weight * v to the output (axpy); at
 * the end the output is multiplied by 1/sum.  Rows [token][heads * d].  The
 * reference parallelises over tokens (par_chunks_mut). */
void orc_encoder_self_attention(float* out, const float* q, const float* k, const float* v, int n_seq,
                                int tokens, int heads, int d, int n_threads) {
    const int dim = heads * d;
    const float inv_scale = 1.0f / sqrtf((float)d);
    const long total = (long)n_seq * tokens;
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (long t = 0; t < total; t++) {
        const long seq_start = (t / tokens) * tokens;
        for (int h = 0; h < heads; h++) {
            float* dst = out + t * dim + (long)h * d;
            const float* qv = q + t * dim + (long)h * d;
            for (int i = 0; i < d; i++) dst[i] = 0.0f;
            float maximum = -INFINITY, sum = 0.0f;
            for (int j = 0; j < tokens; j++) {
                const long src = (seq_start + j) * dim + (long)h * d;
                const float score = dot_f32_avx2(qv, k + src, d) * inv_scale;
                if (score > maximum) {
                    if (sum > 0.0f) {
                        const float rescale = expf(maximum - score);
                        for (int i = 0; i < d; i++) dst[i] *= rescale;
                        sum *= rescale;
                    }
                    maximum = score;
                }
                const float w = expf(score - maximum);
                sum += w;
                axpy_inplace(dst, w, v + src, d);
            }
            if (sum > 0.0f) {
                const float inv = 1.0f / sum;
                for (int i = 0; i < d; i++) dst[i] *= inv;
            }
        }
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
