// C-ABI entry points of libgr_attn: argument validation, workspace carving and
// kernel dispatch for the device-pointer API.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "gr_api_util.hpp"
#include "gr_attn.h"
#include "gr_internal.hpp"

namespace gr {

static thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(GR_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

void clear_error() { g_last_error.clear(); }

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ---------------------------------------------------------------- Turbo sign table

// splitmix64, inference.rs:674-679.
static uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// turboquant_build_sign_table, inference.rs:370-395 (salts 352-355).
void turbo_sign_table_host(int n_layers, int n_kv_heads, int head_size, uint8_t* table) {
    static const uint64_t salts[4] = {0x9E3779B97F4A7C15ull, 0xC2B2AE3D27D4EB4Full, 0x165667B19E3779F9ull,
                                      0xD6E8FEB86659FD93ull};
    const size_t bytes = (size_t)(head_size + 7) / 8;
    const size_t stride = (size_t)n_layers * n_kv_heads * bytes;
    memset(table, 0, 4 * stride);
    for (int slot = 0; slot < 4; slot++)
        for (int l = 0; l < n_layers; l++)
            for (int g = 0; g < n_kv_heads; g++) {
                const uint64_t seed = splitmix64(((uint64_t)l << 32) ^ (uint64_t)g ^ salts[slot]);
                uint8_t* bits = table + slot * stride + ((size_t)l * n_kv_heads + g) * bytes;
                for (int i = 0; i < head_size; i++)
                    if (splitmix64(seed ^ (uint64_t)i) & 1) bits[i / 8] |= (uint8_t)(1u << (i & 7));
            }
}

// ---------------------------------------------------------------- decode
namespace {

struct DecodePlan {
    int split_keys;
    int n_splits;
    bool stream;  // stream schedule (see DecodeLaunch::stream_sched)
    int stream_min_keys, stream_seg_cost;
    size_t ws_o_bytes;
    size_t ws_ml_bytes;
    size_t ws_q_bytes;      // Turbo: rotated / projected queries
    size_t ws_sched_bytes;  // stream: pair offsets per sequence + range size
    bool valu = false;      // 16-bit cache on the VALU split kernel (small calls, GQA groups <= 2)
};

// Stream schedule of the MFMA split kernel (16-bit and Q8 caches).  Keys per
// workgroup range never drop below kStreamMinKeys, which bounds the partial
// slots per (sequence, head) by ceil(max_kv_len / kStreamMinKeys) + 1.
constexpr int kStreamMinKeys = 256;
// Virtual keys charged per (sequence, KV head) pair on the stream schedule: what a
// segment start costs a workgroup (the pipeline refill of its 8 waves, the partial
// written and combined) in keys' worth of streaming.  512 measured best over
// ragged batches (+2-10% against no charge, +59% on 64 sequences of 256-4096 keys)
// and costs 0.5% on 16 equal 32k sequences; 256 and 768 were each below it.
constexpr int kStreamSegCost = 512;
// The same for the Turbo split kernel (whose segment start also loads the
// prepared query operands of its columns): ranges of at least 1024 keys, 512
// virtual keys per pair.  Against the fixed 1024-key split grid: 16 x 32k keys
// 0.120 -> 0.107 ms, config-3 lengths 0.110 -> 0.095 ms, 64 sequences of 256-4096
// keys 0.081 -> 0.062 ms; charges of 0, 1024 and 2048 keys were within 1-15% of it.
constexpr int kTurboStreamMinKeys = 1024;
constexpr int kTurboStreamSegCost = 512;
// Automatic splits of 16-bit caches: calls up to this many keys per sequence that
// need at most this many fixed-grid workgroups run the fixed grid (plan_decode).
constexpr int kSmallCallMaxLen = 4096;
constexpr int64_t kSmallCallMaxWorkgroups = 512;
// The same for Q8 and Turbo caches: calls up to 8192 keys per sequence on at most
// 512 fixed-grid workgroups take splits of max(128, max_len / 32) keys.
constexpr int kQuantSmallCallMaxLen = 8192;

// Split size: aim for ~2048 (sequence, KV head, split) work units so the 256
// CUs stay fed even when sequences are ragged; never below 64 keys.
DecodePlan plan_decode(const gr_decode_args* a) {
    DecodePlan pl{};
    const int max_len = a->max_kv_len > 0 ? a->max_kv_len : 1;
    int split = a->split_keys;
    // Automatic splitting on the MFMA path (16-bit and Q8 caches) and the Turbo
    // path uses the stream schedule: one workgroup per resident slot, equal key
    // ranges, so ragged batches leave no tail.  Explicit split_keys keeps the
    // fixed split grid.
    const int kv_mul = a->n_kv_heads > 0 ? a->n_heads / a->n_kv_heads : 0;
    const bool turbo = a->kv_dtype == GR_DTYPE_TURBO;
    pl.stream_min_keys = turbo ? kTurboStreamMinKeys : kStreamMinKeys;
    pl.stream_seg_cost = turbo ? kTurboStreamSegCost : kStreamSegCost;
    pl.stream = split <= 0 &&
                (a->kv_dtype == GR_DTYPE_F16 || a->kv_dtype == GR_DTYPE_BF16 || a->kv_dtype == GR_DTYPE_Q8 ||
                 (turbo && turbo_stream_ok(a->head_dim, turbo_split_pieces(kv_mul)))) &&
                kv_mul >= 1 &&
                (a->head_dim == 64 || a->head_dim == 128 || a->head_dim == 256) &&
                a->n_seq <= kStreamMaxSeq &&
                (int64_t)a->n_seq * (max_len + pl.stream_seg_cost) * a->n_kv_heads * ((kv_mul + 15) / 16) <
                    (int64_t)1 << 30;
    // Small 16-bit calls (batch-1 decode of short contexts, a window layer): the
    // stream schedule's ranges of at least stream_min_keys keys leave few
    // workgroups, each with a long serial pipeline; the fixed grid with splits sized
    // for at most 16 partials per (sequence, column) runs more, shorter ones.
    // Measured (MI355X, us per call): Gemma-3-4B window layer (1024 keys, 4 KV
    // heads, bf16 d256) 20.5 stream -> 13.9 with 64-key splits; 4 x 2048 keys, 32 / 4
    // heads, f16 d128: 18.1 -> 15.0 with 128-key splits; the 8193-key global layer
    // stays faster on the stream schedule (25 vs 30 us).  With at most two query
    // heads per KV head those splits run faster on the VALU kernel, whose lanes
    // serve the group's heads without the MFMA kernel's 16-column tiles: window
    // layer 16.9 -> 13.4 us, 2 x 1024 keys, 16 / 8 heads, bf16 d128 15.5 -> 12.9-14.5;
    // larger groups are slower there (4 x 2048 keys, 32 / 4 heads: 15.2 -> 36.7).
    if (pl.stream && split <= 0 && (a->kv_dtype == GR_DTYPE_F16 || a->kv_dtype == GR_DTYPE_BF16) &&
        max_len <= kSmallCallMaxLen) {
        const int sk = std::max(64, (max_len + 16 * 64 - 1) / (16 * 64) * 64);
        const int64_t wgs = (int64_t)a->n_seq * a->n_kv_heads * ((kv_mul + 15) / 16) * ((max_len + sk - 1) / sk);
        if (wgs <= kSmallCallMaxWorkgroups) {
            pl.stream = false;
            split = sk;
            pl.valu = kv_mul <= 2;
        }
    }
    // Small Q8 and Turbo calls (batch-1 decode over the reference's own storage
    // formats): the stream schedule's ranges (1024 keys for Turbo, 256 for Q8)
    // leave few workgroups.  Measured (MI355X, us per call, stream -> fixed grid
    // with these splits): Turbo 1 x 1024 keys, 16 / 8 heads 27.4 -> 17.2;
    // 1 x 4096, 16 / 8 38.1 -> 19.4; 1 x 8192, 32 / 8 29.9 -> 22.2; 4 x 2048,
    // 32 / 4 30.4 -> 20.4 (the best of splits 64 ... 512 in each case, within
    // 0.2 us); Q8 rows 1 x 1024, 16 / 8 15.1 -> 11.7; 1 x 8192, 32 / 8 20.7 ->
    // 18.1; 4 x 2048, 32 / 4 18.3 -> 14.6.
    if (pl.stream && split <= 0 && (turbo || a->kv_dtype == GR_DTYPE_Q8) && max_len <= kQuantSmallCallMaxLen) {
        const int sk = std::max(128, (max_len + 32 * 64 - 1) / (32 * 64) * 64);
        const int64_t wgs = (int64_t)a->n_seq * a->n_kv_heads * ((kv_mul + 15) / 16) * ((max_len + sk - 1) / sk);
        if (wgs <= kSmallCallMaxWorkgroups) {
            pl.stream = false;
            split = sk;
        }
    }
    const size_t per_part = turbo ? 2 : 1;  // Turbo: base + residual
    pl.ws_q_bytes = turbo ? align_up((size_t)a->n_seq * a->n_heads * turbo_query_ws_dwords(a->head_dim) * 4, 256) : 0;
    if (pl.stream) {
        pl.split_keys = pl.stream_min_keys;
        pl.n_splits = (max_len + pl.stream_min_keys - 1) / pl.stream_min_keys + 1;
        const size_t parts = (size_t)a->n_seq * a->n_heads * pl.n_splits;
        pl.ws_o_bytes = align_up(parts * per_part * a->head_dim * sizeof(float), 256);
        pl.ws_ml_bytes = align_up(parts * 2 * sizeof(float), 256);
        pl.ws_sched_bytes = align_up((size_t)(a->n_seq + 1) * sizeof(int32_t), 256);
        return pl;
    }
    if (split <= 0) {
        // Fixed grid (VALU kernel, Turbo shapes off the stream schedule): about
        // 2048 (sequence, KV head, split) units.  For the VALU kernel, splits of
        // at least 256 keys once sequences reach 4096 keys: shorter splits of a
        // long sequence cost more in partials and merging than their extra
        // parallelism gains (MI355X, us per call, automatic split -> 256:
        // f32 1 x 32768 keys, 8 KV heads 87.9 -> 65.6; f32 4 x 8192, 8 KV heads
        // 76.6 -> 62.2; f16 d64 1 x 32768, 2 KV heads 91.3 -> 41.8), while short
        // calls keep the small splits their latency needs (config 1, 1024 keys:
        // 64; f32 4 x 2048 keys, 8 KV heads: 26.7 us at 64, 31.3 at 256).
        const long pairs = (long)a->n_seq * a->n_kv_heads;
        long want = (2048 + pairs - 1) / pairs;
        if (want < 1) want = 1;
        split = (int)((max_len + want - 1) / want);
        split = (split + 63) / 64 * 64;
        if (split < 64) split = 64;
        if (!turbo && max_len >= 4096 && split < 256) split = 256;
    }
    pl.split_keys = split;
    pl.n_splits = (max_len + split - 1) / split;
    const size_t parts = (size_t)a->n_seq * a->n_heads * pl.n_splits;
    pl.ws_o_bytes = align_up(parts * per_part * a->head_dim * sizeof(float), 256);
    pl.ws_ml_bytes = align_up(parts * 2 * sizeof(float), 256);
    return pl;
}

}  // namespace

int check_decode(const gr_decode_args* a) {
    if (!a) return fail(GR_ERR_ARG, "gr_decode_attention: null args");
    if (a->n_seq <= 0 || a->n_heads <= 0 || a->n_kv_heads <= 0)
        return fail(GR_ERR_ARG, "gr_decode_attention: n_seq/n_heads/n_kv_heads must be > 0");
    if (a->n_heads % a->n_kv_heads != 0)
        return fail(GR_ERR_ARG, "gr_decode_attention: n_heads %d not a multiple of n_kv_heads %d",
                    a->n_heads, a->n_kv_heads);
    if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
        return fail(GR_ERR_ARG, "gr_decode_attention: head_dim %d unsupported (64,128,256)",
                    a->head_dim);
    if (a->kv_dtype < GR_DTYPE_F32 || a->kv_dtype > GR_DTYPE_TURBO)
        return fail(GR_ERR_ARG, "gr_decode_attention: bad kv_dtype %d", a->kv_dtype);
    if (a->kv_dtype == GR_DTYPE_TURBO) {
        if (!a->k_sign || !a->v_sign || !a->k_scale || !a->v_scale || !a->k_rnorm || !a->v_rnorm ||
            !a->turbo_signs)
            return fail(GR_ERR_ARG, "gr_decode_attention: Turbo KV needs sign, scale, rnorm and sign-table arrays");
        const int64_t al = a->head_dim / 2;  // elements: code rows stay 4*(D/64)-byte, sign rows 2*(D/64)-byte aligned
        if (a->row_stride % al != 0 || a->seq_stride % al != 0 ||
            ((uintptr_t)a->k_cache | (uintptr_t)a->v_cache | (uintptr_t)a->k_sign | (uintptr_t)a->v_sign) % 16 != 0)
            return fail(GR_ERR_ARG,
                        "gr_decode_attention: Turbo arrays must be 16-byte aligned with element strides "
                        "that are multiples of head_dim / 2");
        if (a->scale_row_stride < a->n_kv_heads || a->scale_seq_stride < 0 || a->turbo_slot_stride <= 0)
            return fail(GR_ERR_ARG, "gr_decode_attention: bad Turbo aux or sign-table strides");
    }
    if (a->kv_dtype == GR_DTYPE_Q8) {
        if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
            return fail(GR_ERR_ARG, "gr_decode_attention: Q8 KV needs head_dim 64, 128 or 256");
        if (!a->k_scale || !a->v_scale)
            return fail(GR_ERR_ARG, "gr_decode_attention: Q8 KV needs k_scale and v_scale");
        if (a->q8_block && a->scale_row_stride < (int64_t)a->n_kv_heads * a->head_dim / 32)
            return fail(GR_ERR_ARG, "gr_decode_attention: Q8 block scales need scale_row_stride >= kv_dim/32");
        if (a->scale_row_stride < 0 || a->scale_seq_stride < 0)
            return fail(GR_ERR_ARG, "gr_decode_attention: negative scale stride");
    }
    if (a->max_kv_len <= 0) return fail(GR_ERR_ARG, "gr_decode_attention: max_kv_len must be > 0");
    if (a->out_gate && (a->out_gate_row_stride < 0 || a->out_gate_head_stride < 0))
        return fail(GR_ERR_ARG, "gr_decode_attention: negative out_gate stride");
    if (a->split_keys < 0) return fail(GR_ERR_ARG, "gr_decode_attention: split_keys < 0");
    if (!a->q || !a->k_cache || !a->v_cache || !a->kv_start || !a->kv_end || !a->out ||
        !a->workspace)
        return fail(GR_ERR_ARG, "gr_decode_attention: null buffer");
    if (a->row_stride < (int64_t)a->n_kv_heads * a->head_dim)
        return fail(GR_ERR_ARG, "gr_decode_attention: row_stride %lld < n_kv_heads*head_dim",
                    (long long)a->row_stride);
    const int eb = a->kv_dtype == GR_DTYPE_F32 ? 4 : (a->kv_dtype == GR_DTYPE_Q8 || a->kv_dtype == GR_DTYPE_TURBO ? 1 : 2);
    if (a->kv_dtype != GR_DTYPE_TURBO &&
        (((uintptr_t)a->k_cache | (uintptr_t)a->v_cache) % 16 != 0 || (a->row_stride * eb) % 16 != 0 ||
         (a->seq_stride * eb) % 16 != 0))
        return fail(GR_ERR_ARG, "gr_decode_attention: caches and strides must be 16-byte aligned");
    if ((uintptr_t)a->workspace % 256 != 0)
        return fail(GR_ERR_ARG, "gr_decode_attention: workspace must be 256-byte aligned");
    if ((uintptr_t)a->q % 16 != 0) return fail(GR_ERR_ARG, "gr_decode_attention: q must be 16-byte aligned");
    return GR_OK;
}

int decode_enqueue(const gr_decode_args* a, hipStream_t st) { return decode_enqueue_ex(a, nullptr, st); }

// seq_slot: optional device map from batch entry to cache sequence slot.
int decode_enqueue_ex(const gr_decode_args* a, const int32_t* seq_slot, hipStream_t st) {
    return decode_enqueue_ex(a, seq_slot, st, 0, nullptr, nullptr);
}

int decode_enqueue_ex(const gr_decode_args* a, const int32_t* seq_slot, hipStream_t st, int tok_pack,
                      const int32_t* col_start, const int32_t* col_end) {
    int rc = check_decode(a);
    if (rc) return rc;
    if (tok_pack > 0 && (a->kv_dtype != GR_DTYPE_TURBO || seq_slot || !col_start || !col_end || a->split_keys <= 0 ||
                         tok_pack * (a->n_heads / a->n_kv_heads) > 16))
        return fail(GR_ERR_ARG, "token-packed decode: Turbo cache, one sequence, explicit split and <= 16 columns");
    const DecodePlan pl = plan_decode(a);
    DecodeLaunch p{};
    p.n_seq = a->n_seq;
    p.n_heads = a->n_heads;
    p.n_kv_heads = a->n_kv_heads;
    p.head_dim = a->head_dim;
    p.kv_dtype = a->kv_dtype;
    p.split_keys = pl.split_keys;
    p.n_splits = pl.n_splits;
    p.score_scale = a->score_scale;
    p.q = a->q;
    p.k_cache = a->k_cache;
    p.v_cache = a->v_cache;
    p.seq_stride = a->seq_stride;
    p.row_stride = a->row_stride;
    p.kv_start = a->kv_start;
    p.kv_end = a->kv_end;
    p.seq_slot = seq_slot;
    p.out = a->out;
    p.gate.gate = a->out_gate;
    p.gate.row_stride = a->out_gate_row_stride;
    p.gate.head_stride = a->out_gate_head_stride;
    p.ws_o = (float*)a->workspace;
    p.ws_ml = (float*)((char*)a->workspace + pl.ws_o_bytes);
    p.use_mfma = pl.valu ? 0 : 1;
    if (pl.stream) {  // workspace: partials o | (m, l) | Turbo queries | schedule
        p.stream_sched = (int*)((char*)a->workspace + pl.ws_o_bytes + pl.ws_ml_bytes + pl.ws_q_bytes);
        p.stream_min_keys = pl.stream_min_keys;
        p.stream_seg_cost = pl.stream_seg_cost;
    }
    if (a->kv_dtype == GR_DTYPE_Q8) {
        p.k_scale = a->k_scale;
        p.v_scale = a->v_scale;
        p.scale_seq_stride = a->scale_seq_stride;
        p.scale_row_stride = a->scale_row_stride;
        p.q8_block = a->q8_block ? 1 : 0;
    }
    if (a->kv_dtype == GR_DTYPE_TURBO) {
        p.k_scale = a->k_scale;
        p.v_scale = a->v_scale;
        p.scale_seq_stride = a->scale_seq_stride;
        p.scale_row_stride = a->scale_row_stride;
        p.k_sign = a->k_sign;
        p.v_sign = a->v_sign;
        p.k_rnorm = a->k_rnorm;
        p.v_rnorm = a->v_rnorm;
        p.turbo_signs = a->turbo_signs;
        p.turbo_slot_stride = a->turbo_slot_stride;
        p.ws_q = (float*)((char*)a->workspace + pl.ws_o_bytes + pl.ws_ml_bytes);
        p.tok_pack = tok_pack;
        p.col_start = col_start;
        p.col_end = col_end;
    }
    hipError_t e = launch_decode(p, st);
    if (e != hipSuccess) return hip_fail(e, "gr_decode_attention launch");
    return GR_OK;
}

size_t decode_ws_bytes(const gr_decode_args* a) {
    if (check_decode_shape_only(a)) return 0;
    const DecodePlan pl = plan_decode(a);
    return pl.ws_o_bytes + pl.ws_ml_bytes + pl.ws_q_bytes + pl.ws_sched_bytes;
}

int check_decode_shape_only(const gr_decode_args* a) {
    if (!a || a->n_seq <= 0 || a->n_heads <= 0 || a->n_kv_heads <= 0 || a->head_dim <= 0)
        return GR_ERR_ARG;
    return GR_OK;
}

}  // namespace gr

extern "C" {

const char* gr_last_error(void) { return gr::g_last_error.c_str(); }

int gr_abi_version(void) { return GR_ATTN_ABI_VERSION; }

size_t gr_decode_workspace_size(const gr_decode_args* a) { return gr::decode_ws_bytes(a); }

int gr_decode_attention(const gr_decode_args* a, void* stream) {
    gr::clear_error();
    return gr::decode_enqueue(a, (hipStream_t)stream);
}

int gr_turbo_sign_table(int32_t n_layers, int32_t n_kv_heads, int32_t head_size, uint8_t* out) {
    gr::clear_error();
    if (n_layers <= 0 || n_kv_heads <= 0 || head_size <= 0 || !out)
        return gr::fail(GR_ERR_ARG, "gr_turbo_sign_table: bad arguments");
    gr::turbo_sign_table_host(n_layers, n_kv_heads, head_size, out);
    return GR_OK;
}

}  // extern "C"
