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

#define GR_ATTN_ABI_VERSION 1

/* Status codes. */
#define GR_OK 0
#define GR_ERR_ARG (-1)   /* invalid argument or unsupported shape */
#define GR_ERR_HIP (-2)   /* HIP runtime error (message carries hipGetErrorString) */
#define GR_ERR_RANGE (-3) /* position / range outside the context */
#define GR_ERR_OOM (-4)   /* device allocation failed */

/* Element types of activations and KV storage. */
typedef enum gr_dtype { GR_DTYPE_F32 = 0, GR_DTYPE_F16 = 1, GR_DTYPE_BF16 = 2 } gr_dtype;

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
    int32_t n_kv_heads;   /* KV heads Hkv; Hq/Hkv in {1,2,4,8} */
    int32_t head_dim;     /* 64, 128 or 256 */
    int32_t kv_dtype;     /* gr_dtype of the cache */
    int32_t split_keys;   /* keys per split-K partition, 0 = automatic */
    int32_t max_kv_len;   /* >= kv_end[s] - kv_start[s] for every s (sizes the grid) */
    float score_scale;    /* 1/sqrt(head_dim); 1.0 for Gemma3 whose q is pre-scaled */
    const float* q;       /* [n_seq][n_heads][head_dim] f32, post-RoPE */
    const void* k_cache;
    const void* v_cache;
    int64_t seq_stride;   /* elements between sequences */
    int64_t row_stride;   /* elements between positions */
    const int32_t* kv_start; /* [n_seq] device: first visible key (visible_keys, attention.rs:74-96) */
    const int32_t* kv_end;   /* [n_seq] device: one past the last visible key (pos + 1) */
    float* out;           /* [n_seq][n_heads][head_dim] f32 (s.xb rows) */
    void* workspace;      /* gr_decode_workspace_size() bytes, 256-byte aligned */
} gr_decode_args;

size_t gr_decode_workspace_size(const gr_decode_args* a);
/* Enqueue split-K flash decoding on `stream` (a hipStream_t, NULL = default). */
int gr_decode_attention(const gr_decode_args* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GR_ATTN_H */
