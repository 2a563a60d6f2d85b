/*
 * gr_attn.h -- C ABI of the MI355X (gfx950) attention hot path of gguf-runner.
 *
 * Two layers, both plain C (pointers, sizes, POD structs; no torch types):
 *
 *  1. Device-pointer entry points (gr_decode_attention, gr_prefill_attention,
 *     gr_deltanet_*): every buffer already lives in HBM, work is enqueued on the
 *     caller's HIP stream, nothing is allocated (the caller passes a workspace
 *     sized by the matching *_workspace_size call) and nothing synchronises.
 *
 *  2. Run-state entry points (gr_malloc_run_state, gr_attention_token, ...):
 *     an opaque gr_run_state owns a HIP stream, the device KV cache and the
 *     DeltaNet state of one RunState (src/engine/types.rs:745-809) and takes the
 *     same host buffers the reference functions read and write (s.q, s.k, s.v,
 *     s.xb).  These are the drop-in replacements for the Rust call sites; each
 *     declaration cites the reference function it replaces.
 *
 * Error convention (src/engine/runtime/inference.rs:1533-1546, 2746-2749 use
 * Result<_, String>): every entry point returns GR_OK (0) or a negative status;
 * gr_last_error() returns the message of the last failure on the calling thread.
 * A run state is used by one thread at a time (like &mut RunState); distinct run
 * states are independent and may be used concurrently.
 */
#ifndef GR_ATTN_H
#define GR_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GR_ATTN_ABI_VERSION 5

/* Status codes. */
#define GR_OK 0
#define GR_ERR_ARG (-1)   /* invalid argument or unsupported shape */
#define GR_ERR_HIP (-2)   /* HIP runtime error (message carries hipGetErrorString) */
#define GR_ERR_RANGE (-3) /* position / range outside the context */
#define GR_ERR_OOM (-4)   /* device allocation failed */

/* Element types of activations and KV storage.  GR_DTYPE_Q8 is KV storage
 * only: KvCacheFormat::Q8 (inference.rs:1886-1917), int8 rows plus f32 scales,
 * one per kv_dim row or, in block mode (GGUF_Q8_BLOCK_SCALES), one per 32
 * elements of the row. */
typedef enum gr_dtype {
    GR_DTYPE_F32 = 0,
    GR_DTYPE_F16 = 1,
    GR_DTYPE_BF16 = 2,
    GR_DTYPE_Q8 = 3,
    GR_DTYPE_TURBO = 4 /* KvCacheFormat::Turbo (inference.rs:346-1334, the reference's
                        * default): per kv head 2-bit codes + residual sign bits + sigma,
                        * gamma; head_dim 64, 128 or 256 */
} gr_dtype;

/* RoPE pairing (apply_rope_qk, inference.rs:1817-1874). */
typedef enum gr_rope_mode {
    GR_ROPE_NONE = 0,
    GR_ROPE_ADJACENT = 1, /* pairs (2j, 2j+1): Llama, inference.rs:1853-1869 */
    GR_ROPE_NEOX = 2      /* pairs (i, i+rope_dim/2): Gemma3/Qwen2/Qwen3*, 1829-1852 */
} gr_rope_mode;

/* Message of the last failed call on this thread ("" if none). */
const char* gr_last_error(void);
int gr_abi_version(void);

/* ======================================================================
 * Decode: one new token per sequence attends over its cached keys.
 * Replaces attention_token (inference.rs:1970-2530) for a batch of
 * sequences; KV element (seq s, position t, kv head g, dim i) is at
 * s*seq_stride + t*row_stride + g*head_dim + i (reference layout
 * inference.rs:1880-1882 with row_stride = kv_dim).
 * ====================================================================== */
typedef struct gr_decode_args {
    int32_t n_seq;        /* independent sequences in the batch */
    int32_t n_heads;      /* query heads Hq */
    int32_t n_kv_heads;   /* KV heads Hkv (Hq % Hkv == 0, any ratio) */
    int32_t head_dim;     /* 64, 128 or 256 */
    int32_t kv_dtype;     /* gr_dtype of the cache */
    int32_t split_keys;   /* keys per split-K partition, 0 = automatic */
    int32_t max_kv_len;   /* >= kv_end[s] - kv_start[s] for every s (sizes the grid) */
    float score_scale;    /* 1/sqrt(head_dim); 1.0 for Gemma3 whose q is pre-scaled */
    const float* q;       /* [n_seq][n_heads][head_dim] f32, post-RoPE, 16-byte aligned */
    const void* k_cache;
    const void* v_cache;
    int64_t seq_stride;   /* elements between sequences */
    int64_t row_stride;   /* elements between positions */
    const int32_t* kv_start; /* [n_seq] device: first visible key (visible_keys, attention.rs:74-96) */
    const int32_t* kv_end;   /* [n_seq] device: one past the last visible key (pos + 1) */
    float* out;           /* [n_seq][n_heads][head_dim] f32 (s.xb rows) */
    void* workspace;      /* gr_decode_workspace_size() bytes, 256-byte aligned */
    /* GR_DTYPE_Q8 only (NULL / 0 otherwise): key_cache_scale / value_cache_scale.
     * The scale of (seq s, position t, kv head g, element i) is at
     * s*scale_seq_stride + t*scale_row_stride + (q8_block ? (g*head_dim + i)/32 : 0)
     * (inference.rs:1907-1916 row mode, 1888-1905 and 2021-2027 block mode). */
    const float* k_scale;
    const float* v_scale;
    int64_t scale_seq_stride;
    int64_t scale_row_stride;
    int32_t q8_block;     /* 1: one scale per 32 elements (GGUF_Q8_BLOCK_SCALES) */
    /* GR_DTYPE_TURBO only: k_cache / v_cache are key/value_cache_turbo_base (2-bit
     * codes, element e at byte e/4, bits 2(e%4)), k_sign / v_sign the
     * _turbo_sign arrays (bit e%8 of byte e/8), k_scale / v_scale sigma and
     * k_rnorm / v_rnorm gamma of (seq s, position t, kv head g) at
     * s*scale_seq_stride + t*scale_row_stride + g (turboquant_aux_index,
     * inference.rs:669-672).  turbo_signs points at the layer's rows of the
     * sign table (gr_turbo_sign_table): slot i of kv head g at
     * turbo_signs + i*turbo_slot_stride + g*head_dim/8. */
    const void* k_sign;
    const void* v_sign;
    const float* k_rnorm;
    const float* v_rnorm;
    const uint8_t* turbo_signs;
    int64_t turbo_slot_stride;
    /* Qwen3.5 packed-q output gate (qwen3next_packed_q_gate, inference.rs:3509-3519
     * decode, 3003-3016 batched prefill), fused into the kernel that writes out: when
     * non-NULL, out[r][h][i] = finite_or_zero(out[r][h][i] * sigmoid(g)) with
     * g = out_gate[r*out_gate_row_stride + h*out_gate_head_stride + i]
     * (sigmoid_mul_inplace, math.rs:396-403), r = the sequence.  The reference's packed
     * rows [q_h | gate_h] give out_gate = rows + head_dim, head stride 2*head_dim and
     * row stride 2*n_heads*head_dim.  NULL = no gate. */
    const float* out_gate;
    int64_t out_gate_row_stride;
    int32_t out_gate_head_stride;
} gr_decode_args;

size_t gr_decode_workspace_size(const gr_decode_args* a);
/* Enqueue split-K flash decoding on `stream` (a hipStream_t, NULL = default). */
int gr_decode_attention(const gr_decode_args* a, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc):
 * gr_decode_attention with the split-K partials in a library-owned device array
 * of GR_DECODE_NOALLOC_MAX_WORKSPACE bytes per GPU (held until the process
 * ends) instead of a caller workspace.  a->workspace is ignored; everything
 * else, the kernels and the results are those of gr_decode_attention.  Calls
 * whose gr_decode_workspace_size exceeds the maximum fail with GR_ERR_ARG
 * before any launch.  Allocates nothing.  Every call on one GPU uses the same
 * array: calls that overlap on one GPU (other streams or threads) race, so
 * serialise them.  The first call of each head shape and cache type on a device
 * also resolves the array's address and the kernels' occupancy (host-side
 * queries): make it before a graph capture; captured calls then record kernel
 * nodes only, and a replay reads q, the cache and kv_start / kv_end as they are
 * at replay time (kv_end at most the max_kv_len the capture was made with). */
#define GR_DECODE_NOALLOC_MAX_WORKSPACE (64u << 20)
int gr_decode_attention_noalloc(const gr_decode_args* a, void* stream);

/* ======================================================================
 * Prefill: a chunk of m new tokens of one sequence and one layer.
 * Replaces the serial per-token loop of transformer_prefill_batch
 * (inference.rs:2981-3017): for each token, qkv_bias_and_norm's QK-norm
 * (2535-2572), apply_rope_qk (1817-1874), kv_write_token (1877-1965, raw
 * storage) and attention_token (1970-2530).  Token i sits at position
 * base_pos + i and sees keys [start, base_pos + i] of the cache, where
 * start = 0 (window 0, global) or base_pos + i + 1 - window (sliding window,
 * attention.rs:74-96).  Q/K/V are pre-norm and pre-RoPE; the post-norm,
 * post-RoPE K and V rows are written into the cache at rows base_pos ..
 * base_pos + m - 1.  Cache rows [0, base_pos) must hold earlier tokens.
 * ====================================================================== */
typedef struct gr_prefill_args {
    int32_t n_tokens;     /* m */
    int32_t base_pos;
    int32_t n_heads;
    int32_t n_kv_heads;   /* n_heads % n_kv_heads == 0 */
    int32_t head_dim;     /* 64, 128 or 256 */
    int32_t dtype;        /* GR_DTYPE_F16 or GR_DTYPE_BF16: q/k/v inputs and cache.  The
                           * prepared queries are staged as f16 for both, so
                           * |q * score_scale * log2(e)| must stay below 65504; a bf16
                           * cache is read through exact f16 copies of its rows (in
                           * the workspace) unless a K / V value is beyond f16's range */
    int32_t window;       /* 0 = global causal, W > 0 = sliding window of W keys */
    int32_t rope_mode;    /* gr_rope_mode; GR_ROPE_ADJACENT needs rope_dim == head_dim */
    int32_t rope_dim;     /* rotated dims per head, even, <= head_dim */
    float rope_scale;     /* rope_scaling.global or .local of this layer (inference.rs:1502-1506) */
    const float* rope_freqs; /* device [rope_dim/2], see gr_rope_freqs */
    const float* q_norm;  /* device [head_dim] QK RMSNorm weights, 16-byte aligned, or NULL */
    const float* k_norm;  /* device [head_dim], 16-byte aligned, or NULL */
    float norm_eps;       /* rms_norm_eps (1e-5 when the model gives 0, inference.rs:2539-2543) */
    int32_t is_gemma3;    /* 1: q *= 1/sqrt(head_dim) after RoPE, scores unscaled (1871-1873, 1982) */
    const void* q;        /* [m][n_heads][head_dim] */
    const void* k;        /* [m][n_kv_heads][head_dim] */
    const void* v;
    void* k_cache;        /* [>= base_pos + m][n_kv_heads][head_dim] rows of this sequence and layer */
    void* v_cache;
    int64_t cache_row_stride; /* elements between cache rows (>= n_kv_heads*head_dim) */
    float* out;           /* [m][n_heads][head_dim] f32 (s.xb rows) */
    void* workspace;      /* gr_prefill_workspace_size() bytes, 256-byte aligned */
    int32_t bidirectional; /* 0: causal rows (visible_keys start..pos+1).  1: the m rows
                            * are one complete image block under
                            * ImageAttentionMode::Bidirectional: row pos sees
                            * [min(start(pos), base_pos), base_pos + m) with start(pos) =
                            * pos + 1 - window (saturating) or 0, i.e. every key of the
                            * block plus its causal / window history
                            * (LanguageAttentionPolicy::visible_keys, attention.rs:74-96). */
    /* Qwen3.5 packed-q output gate (qwen3next_packed_q_gate, inference.rs:3509-3519
     * decode, 3003-3016 batched prefill), fused into the kernel that writes out: when
     * non-NULL, out[r][h][i] = finite_or_zero(out[r][h][i] * sigmoid(g)) with
     * g = out_gate[r*out_gate_row_stride + h*out_gate_head_stride + i]
     * (sigmoid_mul_inplace, math.rs:396-403), r = the token.  The reference's packed
     * rows [q_h | gate_h] give out_gate = rows + head_dim, head stride 2*head_dim and
     * row stride 2*n_heads*head_dim.  NULL = no gate. */
    const float* out_gate;
    int64_t out_gate_row_stride;
    int32_t out_gate_head_stride;
    /* Qwen2 attention biases (qkv_bias_and_norm, inference.rs:2545-2559): device f32
     * q_bias [n_heads*head_dim], k_bias and v_bias [n_kv_heads*head_dim] of this layer,
     * added to every q / k / v row before the QK norm and RoPE.  All three or none
     * (NULL); 16-byte aligned. */
    const float* q_bias;
    const float* k_bias;
    const float* v_bias;
} gr_prefill_args;

size_t gr_prefill_workspace_size(const gr_prefill_args* a);
int gr_prefill_attention(const gr_prefill_args* a, void* stream);

/* turboquant_build_sign_table (inference.rs:370-395), host memory:
 * [4 slots: rot_pre, rot_post, res_pre, res_post][n_layers][n_kv_heads][ceil(head_size/8)],
 * bit i set = negate element i; bits from splitmix64 of the per-(slot, layer,
 * kv head) seed.  Copy it to the device for gr_decode_attention. */
int gr_turbo_sign_table(int32_t n_layers, int32_t n_kv_heads, int32_t head_size, uint8_t* out);

/* RoPE frequency table freq_i = 1 / theta^(2i / rope_dim), i < rope_dim/2, in
 * f32 with the host libm powf, exactly as malloc_run_state builds rope_freqs
 * (inference.rs:1590-1609).  Host memory; copy it to the device for the
 * device-pointer entry points. */
int gr_rope_freqs(float theta, int32_t rope_dim, float* freqs_out);

/* ======================================================================
 * Encoder self-attention: encoder_self_attention (src/engine/multimodal/
 * mod.rs:145-256), the attention of the vision / audio encoders.  q, k, v, out
 * are device f32 rows [n_seq * tokens][heads * head_dim]; each token attends to
 * every token of its own sequence (no mask, no cache), scores scaled by
 * 1/sqrt(head_dim).  head_dim <= 256.  Sizes of 0 are a no-op, like the
 * reference's required == 0 case; negative sizes fail with its "encoder
 * attention shape mismatch" message.  Enqueued on `stream`, allocates nothing.
 * ====================================================================== */
int gr_encoder_self_attention(float* out, const float* q, const float* k, const float* v,
                              int32_t n_seq, int32_t tokens, int32_t heads, int32_t head_dim,
                              void* stream);

/* ======================================================================
 * Gated DeltaNet linear attention (Qwen3-Next / Qwen3.5 SSM layers).
 * Per value head h and token t, with state S[h] (f32 [d][d], S[j][i]):
 *   S *= exp(gate); kv = S^T k; delta = beta (v - kv); S += k delta^T; o = S^T q
 * = qwen3next_state_head_step (src/engine/kernels/math.rs:492-546) applied over
 * heads (math.rs:890-934) and tokens (the serial scan inference.rs:2866-2885).
 * With l2norm = 1 the per-head normalisation of math.rs:833-846 is fused:
 * q <- q / sqrt(sum q^2 + eps) / sqrt(d), k <- k / sqrt(sum k^2 + eps).
 * q/k/v are the per-value-head rows (after the K->V head tiling, math.rs:826).
 * The reference's guards apply: finite_or_zero on the normalised q / k, on v
 * (math.rs:845), on exp(gate) and beta (869-874), on kv, delta and o (523-545).
 * ====================================================================== */
typedef enum gr_deltanet_algo {
    GR_DELTANET_AUTO = 0,      /* chunked for n_tokens >= 64, recurrent otherwise */
    GR_DELTANET_RECURRENT = 1, /* token by token, state slice in registers */
    GR_DELTANET_CHUNKED = 2    /* chunks of 64 tokens; from a chunk with a non-finite input or
                                  intermediate on, token by token with the guards above */
} gr_deltanet_algo;

typedef struct gr_deltanet_args {
    int32_t n_tokens;     /* T */
    int32_t n_heads;      /* value heads H */
    int32_t head_dim;     /* state size d: 64, 128 or 256 (the chunked algorithm at 128;
                           * other sizes run the token recurrence) */
    int32_t in_dtype;     /* gr_dtype of q/k/v */
    int32_t l2norm;       /* 1: fuse the q/k normalisation above */
    int32_t algo;         /* gr_deltanet_algo */
    float eps;            /* normalisation epsilon (rms_norm_eps) */
    const void* q;        /* [T][H][head_dim] */
    const void* k;
    const void* v;
    const float* gate;    /* [T][H] log decay: g = exp(gate) (math.rs:869-874) */
    const float* beta;    /* [T][H] sigmoid-ed beta (math.rs:862) */
    float* state;         /* [H][head_dim][head_dim] f32, updated in place */
    float* out;           /* [T][H][head_dim] f32 (ssm_proj before the gated norm) */
    void* workspace;      /* gr_deltanet_workspace_size() bytes (0 for recurrent), 256-aligned */
} gr_deltanet_args;

size_t gr_deltanet_workspace_size(const gr_deltanet_args* a);
int gr_deltanet_attention(const gr_deltanet_args* a, void* stream);

/* ======================================================================
 * Run state: device-resident KV cache, DeltaNet state and stream of one
 * RunState (src/engine/types.rs:745-809).  The entry points below take the
 * reference's own host buffers (s.q, s.k, s.v, s.xb as f32 rows) and return
 * when the results are back in host memory, so each one replaces the body of
 * the cited Rust function.  Device layout of the cache, per layer l and
 * sequence slot s: row t of kv_dim = n_kv_heads*head_dim elements at
 * ((l*n_seq + s)*seq_len + t)*kv_dim (the reference's (l*seq_len + t)*kv_dim,
 * inference.rs:1880-1882, with a slot index for batched decode).
 * ====================================================================== */
typedef struct gr_run_state gr_run_state;

typedef struct gr_attn_config {
    int32_t n_layers;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t seq_len;            /* cache rows per sequence (Config::seq_len) */
    int32_t n_seq;              /* sequence slots, one reference RunState each (>= 1) */
    int32_t kv_dtype;           /* gr_dtype of the device KV cache: raw F32/F16/BF16, Q8 or TURBO */
    int32_t rope_mode;          /* gr_rope_mode (NEOX for Gemma3/Qwen2/Qwen3*, ADJACENT for Llama) */
    int32_t rope_dim;           /* rotated dims, 0 -> head_dim (vendors/mod.rs:1015-1019) */
    float rope_theta;
    float rope_theta_swa;       /* <= 0 -> 10000 (inference.rs:1595-1599) */
    float rope_scale_global;    /* RopeScalingPolicy::global */
    float rope_scale_local;     /* RopeScalingPolicy::local */
    const int32_t* layer_windows; /* [n_layers] or NULL: window per layer, 0 = global
                                   * (LanguageAttentionPolicy::layer_windows, types.rs:614-621) */
    int32_t swa_pattern;        /* Config::swa_pattern, for is_swa_layer without layer_windows (1821-1825) */
    int32_t is_gemma3;          /* SWA RoPE table, q *= 1/sqrt(d), unscaled scores (1871-1873, 1982) */
    int32_t online_attn_fusion; /* accepted for parity; the device path is always online split-K */
    float rms_norm_eps;         /* <= 0 -> 1e-5 (inference.rs:2539-2543) */
    const float* q_norm;        /* host [n_layers][head_dim] QK-norm weights, or NULL */
    const float* k_norm;        /* host [n_layers][head_dim], or NULL */
    const uint8_t* qk_norm_present; /* host [n_layers] or NULL (= every layer when q_norm is set) */
    int32_t ssm_n_heads;        /* DeltaNet value heads, 0 = no SSM state */
    int32_t ssm_head_dim;       /* 64, 128 or 256 (ssm_state_size) */
    int32_t q8_block_scales;    /* Q8 cache: 1 = one scale per 32 elements (GGUF_Q8_BLOCK_SCALES,
                                 * inference.rs:1883), 0 = one scale per row */
    /* Qwen3.5 SSM layer weights for gr_qwen3next_ssm_layer (NULL when unused),
     * host memory copied at allocation (Qwen3NextLinearAttentionShape,
     * math.rs:549-620: n_v = ssm_n_heads = ssm_time_step_rank, n_k =
     * ssm_group_count, conv_dim = (n_v + 2 n_k) * ssm_head_dim). */
    int32_t ssm_n_k_heads;      /* ssm_group_count; ssm_n_heads % ssm_n_k_heads == 0 */
    int32_t ssm_conv_kernel;    /* ssm_conv_kernel, 1..9 */
    const float* ssm_conv1d;    /* [n_layers][conv_dim][ssm_conv_kernel] (blk.l.ssm_conv1d.weight) */
    const float* ssm_a;         /* [n_layers][ssm_n_heads] (ssm_a) */
    const float* ssm_dt_bias;   /* [n_layers][ssm_n_heads] (ssm_dt_bias) */
    const float* ssm_norm;      /* [n_layers][ssm_head_dim] (ssm_norm) */
} gr_attn_config;

/* malloc_run_state_with_kv_cache_format (inference.rs:1529-1748): validates
 * like 1533-1546 ("RoPE frequency scales must be finite and positive", one
 * positive window or global entry per layer), builds the RoPE tables
 * (1590-1609) and allocates the device cache, SSM state and stream. */
int gr_malloc_run_state(const gr_attn_config* cfg, gr_run_state** out);
void gr_free_run_state(gr_run_state* s);

/* qkv_bias_and_norm's per-head QK RMSNorm (inference.rs:2535-2572 ->
 * math.rs:164-184), in place on host q [n_heads*head_dim], k [n_kv_heads*head_dim]. */
int gr_qkv_norm(gr_run_state* s, int32_t layer, float* q, float* k);
/* apply_rope_qk (inference.rs:1817-1874), in place on host q and k. */
int gr_apply_rope_qk(gr_run_state* s, int32_t layer, int64_t pos, float* q, float* k);
/* kv_write_token (inference.rs:1877-1965): k, v -> cache row (layer, seq, pos),
 * raw storage or, for a Q8 cache, quantize_row_q8 per row / 32-element block
 * (inference.rs:166-268, 1886-1917). */
int gr_kv_write_token(gr_run_state* s, int32_t seq, int32_t layer, int64_t pos, const float* k,
                      const float* v);
/* attention_token (inference.rs:1970-2530): q (post-RoPE) -> xb over the
 * visible keys of (layer, pos) (attention.rs:74-96). */
int gr_attention_token(gr_run_state* s, int32_t seq, int32_t layer, int64_t pos, const float* q,
                       float* xb);
/* The four calls of layer_attention_token_staged (inference.rs:3499-3507)
 * fused into one device pass: QK-norm, RoPE, KV write and attention. */
int gr_attention_layer_token(gr_run_state* s, int32_t seq, int32_t layer, int64_t pos,
                             const float* q, const float* k, const float* v, float* xb);
/* The per-token attention loop of transformer_prefill_batch
 * (inference.rs:2981-3017) for m tokens at base_pos..base_pos+m-1:
 * q [m][n_heads*head_dim], k/v [m][kv_dim] pre-norm, pre-RoPE; xb [m][q_dim]. */
int gr_prefill_attention_chunk(gr_run_state* s, int32_t seq, int32_t layer, int64_t base_pos,
                               int32_t m, const float* q, const float* k, const float* v,
                               float* xb);
/* The attention of transformer_prefill_image_block (media_prefill.rs:15-124) for
 * one complete image block under ImageAttentionMode::Bidirectional: the m rows
 * at base_pos..base_pos+m-1 are normed, rotated and written to the cache first,
 * then row pos attends to [min(start(pos), base_pos), base_pos + m) (every key of
 * the block plus its causal / window history, attention.rs:87-94).  Same row
 * layout as gr_prefill_attention_chunk.  Fails with "image-block prefill must
 * evaluate one complete supported block within context" when the block does
 * not fit the context (media_prefill.rs:31-39). */
int gr_prefill_image_block(gr_run_state* s, int32_t seq, int32_t layer, int64_t base_pos, int32_t m,
                           const float* q, const float* k, const float* v, float* xb);
/* One decode step for n sequences at once (one token each, sequence slot
 * seqs[b] at position pos[b]): the per-sequence calls of
 * layer_attention_token_staged batched into one launch. */
int gr_decode_layer_batch(gr_run_state* s, int32_t layer, int32_t n, const int32_t* seqs,
                          const int64_t* pos, const float* q, const float* k, const float* v,
                          float* xb);
/* qwen3next_state_head_step over all value heads for one token
 * (math.rs:890-934): q, k already normalised, g the decay factor
 * (ssm_gate_exp), beta the sigmoid-ed gate; q/k/v/out [ssm_n_heads*ssm_head_dim]. */
int gr_qwen3next_state_step(gr_run_state* s, int32_t layer, const float* q, const float* k,
                            const float* v, const float* g, const float* beta, float* out);
/* The serial SSM prefill recurrence (inference.rs:2866-2885) for T tokens on the
 * chunk-64 device path: q/k raw (normalised in-kernel as math.rs:833-846),
 * gate the log decay, rows [T][ssm_n_heads*ssm_head_dim]. */
int gr_qwen3next_prefill(gr_run_state* s, int32_t layer, int32_t T, const float* q,
                         const float* k, const float* v, const float* gate, const float* beta,
                         float* out);
/* qwen3next_linear_attention_step_from_projections (math.rs:715-953) for T
 * consecutive tokens of layer `layer`, the serial loop of inference.rs:2866-2885
 * as one device pass: conv1d + SiLU over the layer's conv history, K -> V head
 * tiling, L2 norms, beta / decay gates, the gated delta rule on the layer's
 * state, gated RMSNorm with SiLU(z).  Host rows: qkv [T][conv_dim],
 * z [T][ssm_n_heads*ssm_head_dim], gate_a [T][2*ssm_n_heads] (fused ssm_ba,
 * gate_b NULL) or gate_a = alpha [T][ssm_n_heads] with gate_b = beta
 * [T][ssm_n_heads]; out [T][ssm_n_heads*ssm_head_dim] (ssm_proj). */
int gr_qwen3next_ssm_layer(gr_run_state* s, int32_t layer, int32_t T, const float* qkv, const float* z,
                           const float* gate_a, const float* gate_b, float* out);
/* The conv history of a layer ([ssm_conv_kernel - 1][conv_dim] f32, oldest row first). */
int gr_read_ssm_conv_state(gr_run_state* s, int32_t layer, float* out);
int gr_write_ssm_conv_state(gr_run_state* s, int32_t layer, const float* in);

/* Host copies of device state (for checks and snapshots): `n_rows` cache rows
 * of (layer, seq) starting at row0 as raw kv_dtype elements, and the SSM state
 * of a layer (f32 [ssm_n_heads][d][d]). */
int gr_read_kv_rows(gr_run_state* s, int32_t layer, int32_t seq, int64_t row0, int64_t n_rows,
                    void* k_out, void* v_out);
/* Q8 cache: the f32 scales of those rows (key_cache_scale / value_cache_scale),
 * 1 per row, or kv_dim/32 per row in block mode.  Turbo cache: sigma, n_kv_heads
 * per row. */
int gr_read_kv_scales(gr_run_state* s, int32_t layer, int32_t seq, int64_t row0, int64_t n_rows,
                      float* k_scale_out, float* v_scale_out);
/* Turbo cache only: code bytes (kv_dim/4 per row), sign bytes (kv_dim/8 per row)
 * and gamma (n_kv_heads per row) of those rows; any pointer may be NULL. */
int gr_read_turbo_rows(gr_run_state* s, int32_t layer, int32_t seq, int64_t row0, int64_t n_rows,
                       uint8_t* k_base, uint8_t* k_sign, float* k_rnorm, uint8_t* v_base,
                       uint8_t* v_sign, float* v_rnorm);
int gr_read_ssm_state(gr_run_state* s, int32_t layer, float* out);
int gr_write_ssm_state(gr_run_state* s, int32_t layer, const float* in);

/* Prefill cache (GPFC v1, src/app/prefill_cache.rs:1-19).  snapshot
 * (prefill_cache.rs:178-310): the blob of the first k rows of sequence slot
 * `seq` in every layer (Q8 or Turbo cache sections), the SSM conv history and
 * state of every layer, the k prompt tokens and the caller's model fingerprint
 * (model_fingerprint, prefill_cache.rs:65-68).  The q8_block byte is
 * cfg.q8_block_scales (the reference writes GGUF_Q8_BLOCK_SCALES for either
 * format).  out == NULL: only *size_out (the blob's byte size) is set; else
 * cap must hold the blob.  Errors: "prefill cache requires kv_dim % 8 == 0",
 * a raw (F32/F16/BF16) cache, k > seq_len. */
int gr_prefill_cache_snapshot(gr_run_state* s, int32_t seq, const int32_t* tokens, int32_t k,
                              uint64_t model_len, uint64_t model_head_fnv, uint8_t* out,
                              uint64_t cap, uint64_t* size_out);
/* PrefixCache::parse + inject (prefill_cache.rs:316-352, 380-507): copies the
 * blob's k rows into rows 0..k-1 of slot `seq` (re-strided to this state's
 * seq_len) and its SSM arrays into the state; *k_out = k.  Same messages as the
 * reference ("prefill cache truncated", "...: bad magic", "...: unsupported
 * version N", "...: bad kv format N", "...: model/config mismatch", "...: prefix
 * longer than context", "...: section size mismatch", "...: bad f32 section
 * length", "...: ssm state size mismatch"); every check runs before the first
 * copy, so a rejected blob leaves the state unchanged.  The prompt-token match
 * (match_len, prefill_cache.rs:366-377) stays with the caller. */
int gr_prefill_cache_inject(gr_run_state* s, int32_t seq, const uint8_t* blob, uint64_t len,
                            int32_t* k_out);

#ifdef __cplusplus
}
#endif

#endif /* GR_ATTN_H */
