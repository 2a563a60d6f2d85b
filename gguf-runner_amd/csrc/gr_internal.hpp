// Launch descriptors shared between the C-ABI layer (api.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gr {

// Split-K decode.  Partials: ws_o [n_seq][n_heads][n_splits][head_dim],
// ws_ml [n_seq][n_heads][n_splits][2] = (m, l) in log2 units.
// Qwen3.5 output gate of output row r (decode: batch entry, prefill: token), head
// h: out *= sigmoid(gate[r * row_stride + h * head_stride + i]) (gate null = none).
struct OutGate {
    const float* gate = nullptr;
    int64_t row_stride = 0;
    int head_stride = 0;
    __device__ __forceinline__ const float* at(int64_t r, int h) const {
        return gate ? gate + r * row_stride + (int64_t)h * head_stride : nullptr;
    }
};

// Sequences per launch on the stream schedule (per-workgroup LDS tables).
constexpr int kStreamMaxSeq = 1024;

struct DecodeLaunch {
    int n_seq, n_heads, n_kv_heads, head_dim, kv_dtype;
    int split_keys, n_splits;
    float score_scale;
    const float* q;
    const void* k_cache;
    const void* v_cache;
    int64_t seq_stride, row_stride;
    const int32_t* kv_start;
    const int32_t* kv_end;
    const int32_t* seq_slot;  // [n_seq] cache sequence slot of batch entry s, or nullptr (= s)
    float* out;
    float* ws_o;
    float* ws_ml;
    int use_mfma;  // 16-bit / Q8 caches: MFMA split kernel (decode_mfma.hip) instead of VALU
    // Stream schedule (the MFMA and Turbo split kernels, stream_sched.hpp): when
    // set, the grid is one row of workgroups that cut the flattened (sequence,
    // column, key) space into equal ranges of at least stream_min_keys keys;
    // partial slot j of (s, head) comes from the j-th range that meets the keys
    // of the head's pair, n_splits bounds the slots.  stream_sched[0 .. n_seq)
    // receives the pair offsets off_s of every sequence and stream_sched[n_seq]
    // the range size, for the combine kernel.
    int* stream_sched;
    int stream_min_keys;
    // Stream schedule: every non-empty (sequence, column) pair also counts
    // stream_seg_cost virtual keys ahead of its own (a segment start costs a
    // pipeline refill and a partial), so ranges that cross into a pair take
    // correspondingly fewer keys.  The split and combine kernels share it.
    int stream_seg_cost;
    // Q8 cache: scale of (seq slot, row t, kv head g, element i) at
    // slot*scale_seq_stride + t*scale_row_stride + (q8_block ? (g*head_dim + i)/32 : 0).
    const float* k_scale;
    const float* v_scale;
    int64_t scale_seq_stride, scale_row_stride;
    int q8_block;
    // Turbo cache: k_cache / v_cache hold the 2-bit codes (element e at byte e/4),
    // k_sign / v_sign the residual sign bits (byte e/8); k_scale / v_scale sigma and
    // k_rnorm / v_rnorm gamma of (slot, row t, kv head g) at
    // slot*scale_seq_stride + t*scale_row_stride + g; turbo_signs the layer's sign
    // table rows (slot i at turbo_signs + i*turbo_slot_stride, kv head g at + g*d/8);
    // ws_q the prepared query operands, turbo_query_ws_dwords(d) dwords per
    // (batch entry, head).
    const void* k_sign;
    const void* v_sign;
    const float* k_rnorm;
    const float* v_rnorm;
    const uint8_t* turbo_signs;
    int64_t turbo_slot_stride;
    float* ws_q;
    // Token-packed Turbo prefill (tok_pack > 0; one cache sequence, seq_slot
    // null): batch entries are n_seq consecutive query tokens; the split kernel
    // runs one workgroup row per group of tok_pack tokens, whose MFMA columns are
    // (token, query head of the GQA group) pairs.  kv_start / kv_end of every
    // token hold its group's key range (the split and merge ranges), col_start /
    // col_end the token's own visible keys.
    int tok_pack;
    const int32_t* col_start;
    const int32_t* col_end;
    OutGate gate;  // written by the combine kernels
    // Query heads of a GQA group split over n_sub workgroup columns (kv_mul above
    // what one workgroup takes: 16 MFMA columns, 8 VALU heads): column vg of the
    // grid is KV head vg / n_sub with query heads (vg / n_sub) * kv_mul + (vg % n_sub)
    // * sub_heads .. + min(sub_heads, kv_mul - (vg % n_sub) * sub_heads).  0 = 1.
    int n_sub = 0, sub_heads = 0;
};

hipError_t launch_decode(const DecodeLaunch& p, hipStream_t st);
bool decode_mfma_supported(const DecodeLaunch& p);
hipError_t launch_decode_mfma_split(const DecodeLaunch& p, hipStream_t st);

// Per-token Q/K/V preparation: optional QK RMSNorm (math.rs:164-184), RoPE
// (inference.rs:1817-1874), Gemma q scale, then
//   K, V rows -> cache (dtype `cache_dtype`) at rows pos0 + i,
//   Q rows -> q_out (f32, or 16-bit `q_out_dtype`) multiplied by q_out_scale.
struct QkvPrepLaunch {
    int n_tokens, n_heads, n_kv_heads, head_dim;
    int in_dtype;          // dtype of q/k/v inputs
    const int32_t* pos;    // [n_tokens] positions (device), or nullptr -> pos0 + i
    int64_t pos0;
    int rope_mode, rope_dim;
    float rope_scale;
    const float* rope_freqs;
    const float* q_norm;
    const float* k_norm;
    // Qwen2 biases added to the loaded q / k / v rows before the norm (nullable;
    // [n_heads*head_dim] / [n_kv_heads*head_dim])
    const float* q_bias;
    const float* k_bias;
    const float* v_bias;
    float eps;
    int gemma_q_scale;
    const void* q;
    const void* k;
    const void* v;
    int64_t q_row_stride, kv_row_stride;  // input row strides (elements)
    void* q_out;
    void* q_out_lo;        // 16-bit q_out only: residual x - round(x) in the same dtype, or nullptr
    int q_out_dtype;
    float q_out_scale;
    void* k_cache;
    void* v_cache;
    int cache_dtype;
    const int32_t* cache_row;   // [n_tokens] destination row per token (device), or nullptr -> pos
    int64_t cache_seq_stride;   // elements, used with cache_seq
    const int32_t* cache_seq;   // [n_tokens] sequence slot per token, or nullptr -> 0
    int64_t cache_row_stride;
    int cache_by_index;         // 1: token i's K/V go to row i of the cache (staging), slot 0
    float* rope_cs_out;         // [n_tokens][rope_dim / 2][2] (cos, sin) of each token, or nullptr
    // bf16 caches feeding the f16 MFMA prefill: each K / V row written to the cache
    // is also written as f16 (exact: a bf16 significand fits f16's) to row
    // (cache row - f16_row0) of k_f16 / v_f16 (row stride f16_row_stride
    // elements); a value f16 cannot hold (|x| >= 65536, inf, NaN) stores f16_epoch
    // to *f16_flag.  k_f16 = nullptr: no copy.
    void* k_f16;
    void* v_f16;
    int64_t f16_row0, f16_row_stride;
    uint32_t* f16_flag;
    uint32_t f16_epoch;
    // n_copy int32 values copied from copy_src to copy_dst by workgroup 0, for a
    // kernel launched after this one (the decode's sequence slots and key ranges
    // when the caller's copies sit in host memory); n_copy = 0: none.
    const int32_t* copy_src;
    int32_t* copy_dst;
    int n_copy;
};

hipError_t launch_qkv_prep(const QkvPrepLaunch& p, hipStream_t st);

// f16 copies of cache rows [row0, row0 + n_rows) of a bf16 K and V cache (row
// stride cache_row_stride elements, kv_dim elements per row) into rows 0.. of
// k_f16 / v_f16 (row stride kv_dim), with the range flag of QkvPrepLaunch.
struct Bf16CopyLaunch {
    int64_t n_rows, row0;
    int kv_dim;
    const uint16_t* k_cache;
    const uint16_t* v_cache;
    int64_t cache_row_stride;
    uint16_t* k_f16;
    uint16_t* v_f16;
    uint32_t* f16_flag;
    uint32_t f16_epoch;
};

hipError_t launch_bf16_rows_to_f16(const Bf16CopyLaunch& p, hipStream_t st);

// Q8 KV write (kv_write_token's Q8 branch, inference.rs:1886-1917): n_rows f32
// rows of kv_dim elements (k_rows / v_rows, row stride kv_dim) are quantised
// into int8 cache rows with one scale per row or per 32-element block.
// Destination row i: sequence slot (cache_seq ? cache_seq[i] : 0) and position
// (cache_row ? cache_row[i] : row0 + i).
struct Q8WriteLaunch {
    int n_rows, kv_dim, block;
    const float* k_rows;
    const float* v_rows;
    int8_t* k_cache;
    int8_t* v_cache;
    float* k_scale;
    float* v_scale;
    int64_t cache_seq_stride, cache_row_stride;  // elements
    int64_t scale_seq_stride, scale_row_stride;  // floats
    const int32_t* cache_row;
    const int32_t* cache_seq;
    int64_t row0;
};

hipError_t launch_q8_write(const Q8WriteLaunch& p, hipStream_t st);

// Turbo KV write (kv_write_token's Turbo branch, inference.rs:1918-1963): n_rows
// f32 rows of n_kv_heads*head_dim elements quantised per kv head into 2-bit
// codes + residual sign bits + (sigma, gamma).  Destination row i: slot
// (cache_seq ? cache_seq[i] : 0), position (cache_row ? cache_row[i] : row0 + i);
// element strides for the code / sign arrays, float strides for the aux arrays
// (aux index slot*aux_seq_stride + row*aux_row_stride + kv head).
struct TurboWriteLaunch {
    int n_rows, n_kv_heads, head_dim;
    const float* k_rows;
    const float* v_rows;
    uint8_t* k_base;
    uint8_t* v_base;
    uint8_t* k_sign;
    uint8_t* v_sign;
    float* k_scale;
    float* v_scale;
    float* k_rnorm;
    float* v_rnorm;
    const uint8_t* signs;   // the layer's sign table rows (see DecodeLaunch::turbo_signs)
    int64_t slot_stride;
    int64_t cache_seq_stride, cache_row_stride;
    int64_t aux_seq_stride, aux_row_stride;
    const int32_t* cache_row;
    const int32_t* cache_seq;
    int64_t row0;
};

hipError_t launch_turbo_write(const TurboWriteLaunch& p, hipStream_t st);

// Qwen3.5 SSM layer pre/post around the DeltaNet recurrence for a chunk of
// n_tokens tokens.  qkv [T][conv_dim] (conv_dim = (n_v + 2 n_k) head_dim),
// z [T][n_v head_dim], gate_a [T][2 n_v] fused (gate_b == nullptr) or [T][n_v]
// with gate_b [T][n_v]; conv_w [conv_dim][conv_kernel]; conv_hist
// [(conv_kernel - 1)][conv_dim] read by the pre pass and advanced past the chunk.
// Outputs of the pre pass: q/k/v [T][n_v][head_dim] (q, k before their L2 norms),
// beta and log-decay gate [T][n_v].  The post pass maps o [T][n_v][head_dim] to out.
struct SsmLaunch {
    int n_tokens, n_k_heads, n_v_heads, head_dim, conv_kernel;
    float eps;
    const float* qkv;
    const float* z;
    const float* gate_a;
    const float* gate_b;
    const float* conv_w;
    const float* dt_bias;
    const float* ssm_a;
    const float* ssm_norm;
    float* conv_hist;
    float* q_out;
    float* k_out;
    float* v_out;
    float* beta_out;
    float* gate_out;
    const float* o;
    float* out;
};

hipError_t launch_ssm_pre(const SsmLaunch& p, hipStream_t st);
hipError_t launch_ssm_post(const SsmLaunch& p, hipStream_t st);
bool decode_turbo_supported(const DecodeLaunch& p);
hipError_t launch_decode_turbo(const DecodeLaunch& p, hipStream_t st);
// ws_q dwords per (batch entry, head) of the Turbo decode (prepared query operands).
size_t turbo_query_ws_dwords(int head_dim);
// Rows per group of the token-packed Turbo prefill (DecodeLaunch::tok_pack).
int turbo_pack_rows(int head_dim, int kv_mul);
// Turbo decode: the split kernel carries the hi and lo query pieces as separate
// MFMA columns when a workgroup's query heads fit twice in 16 columns.
constexpr bool turbo_split_pieces(int kv_mul) { return 2 * (kv_mul < 16 ? kv_mul : 16) <= 16; }
// Turbo decode shapes that run on the stream schedule: every one but head_dim
// 256 with unsplit pieces (groups above 8 query heads), which keeps the fixed
// split grid (its stream build faulted on the GPU with no cause found).
constexpr bool turbo_stream_ok(int head_dim, bool split_pieces) { return head_dim != 256 || split_pieces; }

// Flash prefill over the KV cache (MFMA).  q is the prepared 16-bit Q
// [m][n_heads][d] already multiplied by score_scale*log2(e); for bf16, q_lo
// holds the bf16 residual q - q_hi so that q_hi + q_lo carries ~16 mantissa bits.
struct PrefillLaunch {
    int n_tokens, n_heads, n_kv_heads, head_dim, dtype;
    int64_t base_pos;
    int window;
    int bidirectional;  // the n_tokens rows form one image block (see gr_prefill_args)
    const void* q;      // prepared Q: 16-bit rows [n_tokens][n_heads][head_dim] x q scale
    const void* q_lo;   // bf16: the residuals of q
    // Fused Q preparation (head_dim 128, q_raw set; q / q_lo unused): raw Q rows
    // (q_in_dtype, row stride q_row_stride elements) are QK-normed with q_norm
    // (nullable, eps norm_eps), rotated with the token's (cos, sin) pairs
    // rope_cs[token][rope_dim / 2] (rope_mode; NeoX needs rope_dim % 32 == 0),
    // multiplied by q_pre_scale (Gemma3 1/sqrt(d), else 1) and then q_scale.
    const void* q_raw;
    int q_in_dtype;
    int64_t q_row_stride;
    const float* q_bias;  // Qwen2 q bias [n_heads][head_dim] added to the raw row, or null
    const float* q_norm;
    float norm_eps;
    int rope_mode, rope_dim;
    const float* rope_cs;
    float q_pre_scale, q_scale;
    const void* k_cache;
    const void* v_cache;
    int64_t cache_row_stride;
    float* out;
    OutGate gate;
    // bf16 caches (dtype BF16): when k_f16 is set, the rows [f16_row0, base_pos +
    // n_tokens) of the cache are also in k_f16 / v_f16 as exact f16 values (row
    // stride f16_row_stride), and unless *f16_flag == f16_epoch (a value f16
    // cannot hold was found) the kernel runs the single-pass f16 MFMA path on them;
    // otherwise the bf16 hi + lo path on the cache.  q (staged, head_dim 256)
    // then holds f16 values, which the bf16 path splits exactly into hi + lo.
    const void* k_f16;
    const void* v_f16;
    int64_t f16_row0, f16_row_stride;
    const uint32_t* f16_flag;
    uint32_t f16_epoch;
};

hipError_t launch_prefill(const PrefillLaunch& p, hipStream_t st);

// Prefill over a Q8 KV cache (prefill_q8.hip).  q: f32 rows
// [n_tokens][n_heads][head_dim] after RoPE / QK norm (score_scale applied in the
// kernel); k_codes / v_codes: int8 row 0 of the sequence (row stride row_stride
// bytes, KV head g at g * head_dim); scales of row t: k_scale[t * scale_row_stride]
// (block = 0) or k_scale[t * scale_row_stride + g * head_dim / 32 + b] (block = 1).
// Visibility as PrefillLaunch (window, bidirectional).
struct PrefillQ8Launch {
    int n_tokens, n_heads, n_kv_heads, head_dim;
    int64_t base_pos;
    int window, bidirectional, block;
    float score_scale;
    const float* q;
    const int8_t* k_codes;
    const int8_t* v_codes;
    int64_t row_stride;
    const float* k_scale;
    const float* v_scale;
    int64_t scale_row_stride;
    float* out;
    OutGate gate;
};

hipError_t launch_prefill_q8(const PrefillQ8Launch& p, hipStream_t st);

// Encoder self-attention (encoder.hip): rows [n_seq * tokens][heads * head_dim] f32.
struct EncoderLaunch {
    int n_seq, tokens, heads, head_dim;
    const float* q;
    const float* k;
    const float* v;
    float* out;
};

hipError_t launch_encoder_attention(const EncoderLaunch& p, hipStream_t st);

// Gated DeltaNet.
struct DeltaNetLaunch {
    int n_tokens, n_heads, head_dim, in_dtype, l2norm;
    float eps;
    const void* q;
    const void* k;
    const void* v;
    const float* gate;
    const float* beta;
    float* state;
    float* out;
    float* ws;   // chunked algorithm workspace
    int chunk;
    int gate_is_log;  // 1: g = exp(gate[t][h]); 0: gate already holds the decay factor g
    // step kernel after a chunked scan: [H][128 / 16] chunks each 16-column scan
    // block completed; column i starts at token 64 * first_bad[h][i / 16]
    const int* first_bad = nullptr;
};

hipError_t launch_deltanet_scan(const DeltaNetLaunch& p, hipStream_t st);
hipError_t launch_deltanet_chunked(const DeltaNetLaunch& p, hipStream_t st);
size_t deltanet_chunked_ws_bytes(int n_tokens, int n_heads, int head_dim, int chunk);

}  // namespace gr
