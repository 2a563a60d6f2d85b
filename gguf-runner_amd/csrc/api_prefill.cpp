// C-ABI entry points of the prefill path: validation, workspace carving, and
// the two launches (Q/K/V prep -> cache; MFMA flash attention).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>

#include "gr_api_util.hpp"
#include "gr_attn.h"
#include "gr_internal.hpp"

namespace gr {

namespace {

int check_prefill(const gr_prefill_args* a) {
    if (!a) return fail(GR_ERR_ARG, "gr_prefill_attention: null args");
    if (a->n_tokens < 0 || a->base_pos < 0)
        return fail(GR_ERR_ARG, "gr_prefill_attention: negative n_tokens/base_pos");
    if (a->n_heads <= 0 || a->n_kv_heads <= 0 || a->n_heads % a->n_kv_heads != 0)
        return fail(GR_ERR_ARG, "gr_prefill_attention: n_heads %d must be a positive multiple of n_kv_heads %d",
                    a->n_heads, a->n_kv_heads);
    if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
        return fail(GR_ERR_ARG, "gr_prefill_attention: head_dim %d unsupported (64, 128, 256)", a->head_dim);
    if (a->dtype != GR_DTYPE_F16 && a->dtype != GR_DTYPE_BF16)
        return fail(GR_ERR_ARG, "gr_prefill_attention: dtype must be f16 or bf16");
    if (a->window < 0) return fail(GR_ERR_ARG, "gr_prefill_attention: window < 0");
    if (a->rope_mode < GR_ROPE_NONE || a->rope_mode > GR_ROPE_NEOX)
        return fail(GR_ERR_ARG, "gr_prefill_attention: bad rope_mode %d", a->rope_mode);
    if (a->rope_mode != GR_ROPE_NONE) {
        if (a->rope_dim <= 0 || a->rope_dim > a->head_dim || (a->rope_dim & 1))
            return fail(GR_ERR_ARG, "gr_prefill_attention: rope_dim %d must be even and in (0, head_dim]",
                        a->rope_dim);
        if (a->rope_mode == GR_ROPE_ADJACENT && a->rope_dim != a->head_dim)
            return fail(GR_ERR_ARG, "gr_prefill_attention: adjacent-pair RoPE rotates whole heads (rope_dim == head_dim)");
        if (!a->rope_freqs) return fail(GR_ERR_ARG, "gr_prefill_attention: rope_freqs is NULL");
        if (!std::isfinite(a->rope_scale) || a->rope_scale <= 0.0f)
            return fail(GR_ERR_ARG, "RoPE frequency scales must be finite and positive");
    }
    if ((a->q_norm == nullptr) != (a->k_norm == nullptr))
        return fail(GR_ERR_ARG, "gr_prefill_attention: q_norm and k_norm must be both set or both NULL");
    if ((a->q_bias == nullptr) != (a->k_bias == nullptr) || (a->q_bias == nullptr) != (a->v_bias == nullptr))
        return fail(GR_ERR_ARG, "gr_prefill_attention: q_bias, k_bias and v_bias must be all set or all NULL");
    if (((uintptr_t)a->q_bias | (uintptr_t)a->k_bias | (uintptr_t)a->v_bias) % 16)
        return fail(GR_ERR_ARG, "gr_prefill_attention: q_bias, k_bias and v_bias must be 16-byte aligned");
    if (((uintptr_t)a->q_norm | (uintptr_t)a->k_norm) % 16)
        return fail(GR_ERR_ARG, "gr_prefill_attention: q_norm and k_norm must be 16-byte aligned");
    if (a->n_tokens > 0 && (!a->q || !a->k || !a->v || !a->k_cache || !a->v_cache || !a->out ||
                            !a->workspace))
        return fail(GR_ERR_ARG, "gr_prefill_attention: null buffer");
    if (a->out_gate && (a->out_gate_row_stride < 0 || a->out_gate_head_stride < 0))
        return fail(GR_ERR_ARG, "gr_prefill_attention: negative out_gate stride");
    if (a->cache_row_stride < (int64_t)a->n_kv_heads * a->head_dim || (a->cache_row_stride * 2) % 16)
        return fail(GR_ERR_ARG, "gr_prefill_attention: cache_row_stride must be >= n_kv_heads*head_dim and 16-byte aligned");
    if (((uintptr_t)a->k_cache | (uintptr_t)a->v_cache) % 16 || (uintptr_t)a->out % 16)
        return fail(GR_ERR_ARG, "gr_prefill_attention: cache and out must be 16-byte aligned");
    if ((uintptr_t)a->workspace % 256)
        return fail(GR_ERR_ARG, "gr_prefill_attention: workspace must be 256-byte aligned");
    return GR_OK;
}

size_t prefill_q_bytes(const gr_prefill_args* a) {
    return align_up((size_t)a->n_tokens * a->n_heads * a->head_dim * 2, 256);
}

// The attention kernel prepares Q itself (norm, RoPE, scale) for head_dim 128
// when every RoPE pair stays inside a lane's fragments; the prep pass then
// writes only K / V and each token's (cos, sin) table.
bool prefill_fused_q(const gr_prefill_args* a) {
    if (a->head_dim != 128) return false;
    if (a->rope_mode == GR_ROPE_NEOX) return a->rope_dim % 32 == 0;
    return true;
}

size_t prefill_cs_bytes(const gr_prefill_args* a) {
    return a->rope_mode == GR_ROPE_NONE ? 0 : align_up((size_t)a->n_tokens * a->rope_dim * 4, 256);
}

// Staging: the (cos, sin) table when Q is fused, else the prepared Q (16-bit;
// for bf16 caches the f16 values of the f16 path).  Both layouts fit the larger
// size.
size_t prefill_stage_bytes(const gr_prefill_args* a) {
    return prefill_q_bytes(a) > prefill_cs_bytes(a) ? prefill_q_bytes(a) : prefill_cs_bytes(a);
}

// bf16 caches run the f16 MFMA path on an exact f16 copy of the cache rows
// [f16_row0, base_pos + n_tokens): the first row any query of the launch sees,
// rounded down to 128 keys (the largest K / V tile, whose first rows the kernel
// loads and masks).
int64_t prefill_f16_row0(const gr_prefill_args* a) {
    const int64_t lo = a->window > 0 ? std::max<int64_t>(0, (int64_t)a->base_pos + 1 - a->window) : 0;
    return lo / 128 * 128;
}
size_t prefill_f16_copy_bytes(const gr_prefill_args* a) {
    const int64_t rows = (int64_t)a->base_pos + a->n_tokens - prefill_f16_row0(a);
    return align_up((size_t)rows * a->n_kv_heads * a->head_dim * 2, 256);
}

// [staging][K copy][V copy][flag, 256 B] for bf16, [staging] for f16.
size_t prefill_ws_total(const gr_prefill_args* a) {
    if (a->dtype != GR_DTYPE_BF16) return prefill_stage_bytes(a);
    return prefill_stage_bytes(a) + 2 * prefill_f16_copy_bytes(a) + 256;
}

// Per-launch tag of the bf16 range flag: a launch reads "out of f16 range" only
// from a flag word its own prep pass wrote (a stale word from an earlier launch
// holds another tag; a word that happens to match sends the launch down the
// exact bf16 path, which is always correct).
uint32_t next_f16_epoch() {
    static std::atomic<uint32_t> ctr{0x6a09e667u};
    uint32_t e;
    do e = ctr.fetch_add(0x9e3779b9u) + 0x9e3779b9u;
    while (e == 0u);
    return e;
}

}  // namespace

// in_dtype: element type of a->q / a->k / a->v (the public entry point uses
// a->dtype; the run-state path stages the reference's f32 rows directly).
int prefill_enqueue_ex(const gr_prefill_args* a, int in_dtype, hipStream_t st) {
    int rc = check_prefill(a);
    if (rc) return rc;
    if (a->n_tokens == 0) return GR_OK;
    const float score_scale = a->is_gemma3 ? 1.0f : 1.0f / std::sqrt((float)a->head_dim);

    QkvPrepLaunch pp{};
    pp.n_tokens = a->n_tokens;
    pp.n_heads = a->n_heads;
    pp.n_kv_heads = a->n_kv_heads;
    pp.head_dim = a->head_dim;
    pp.in_dtype = in_dtype;
    pp.pos = nullptr;
    pp.pos0 = a->base_pos;
    pp.rope_mode = a->rope_mode;
    pp.rope_dim = a->rope_dim;
    pp.rope_scale = a->rope_scale;
    pp.rope_freqs = a->rope_freqs;
    pp.q_norm = a->q_norm;
    pp.k_norm = a->k_norm;
    pp.q_bias = a->q_bias;
    pp.k_bias = a->k_bias;
    pp.v_bias = a->v_bias;
    pp.eps = a->norm_eps;
    pp.gemma_q_scale = a->is_gemma3;
    pp.q = a->q;
    pp.k = a->k;
    pp.v = a->v;
    pp.q_row_stride = (int64_t)a->n_heads * a->head_dim;
    pp.kv_row_stride = (int64_t)a->n_kv_heads * a->head_dim;
    const bool fused = prefill_fused_q(a);
    const bool bf16 = a->dtype == GR_DTYPE_BF16;
    pp.q_out = fused ? nullptr : a->workspace;
    pp.q_out_lo = nullptr;
    pp.rope_cs_out = fused && a->rope_mode != GR_ROPE_NONE ? (float*)a->workspace : nullptr;
    pp.q_out_dtype = GR_DTYPE_F16;  // bf16 caches too: the f16 path's operand (split exactly on the bf16 path)
    pp.q_out_scale = score_scale * 1.4426950408889634f;
    pp.k_cache = a->k_cache;
    pp.v_cache = a->v_cache;
    pp.cache_dtype = a->dtype;
    pp.cache_row = nullptr;
    pp.cache_seq = nullptr;
    pp.cache_seq_stride = 0;
    pp.cache_row_stride = a->cache_row_stride;
    const int kv_dim = a->n_kv_heads * a->head_dim;
    const int64_t row0 = prefill_f16_row0(a);
    uint16_t* k_f16 = nullptr;
    uint16_t* v_f16 = nullptr;
    uint32_t* flag = nullptr;
    uint32_t epoch = 0;
    hipError_t e = hipSuccess;
    if (bf16) {
        char* w = (char*)a->workspace + prefill_stage_bytes(a);
        k_f16 = (uint16_t*)w;
        v_f16 = (uint16_t*)(w + prefill_f16_copy_bytes(a));
        flag = (uint32_t*)(w + 2 * prefill_f16_copy_bytes(a));
        epoch = next_f16_epoch();
        pp.k_f16 = k_f16;
        pp.v_f16 = v_f16;
        pp.f16_row0 = row0;
        pp.f16_row_stride = kv_dim;
        pp.f16_flag = flag;
        pp.f16_epoch = epoch;
        // rows of earlier calls that this launch's queries see
        Bf16CopyLaunch hc{};
        hc.n_rows = a->base_pos - row0;
        hc.row0 = row0;
        hc.kv_dim = kv_dim;
        hc.k_cache = (const uint16_t*)a->k_cache;
        hc.v_cache = (const uint16_t*)a->v_cache;
        hc.cache_row_stride = a->cache_row_stride;
        hc.k_f16 = k_f16;
        hc.v_f16 = v_f16;
        hc.f16_flag = flag;
        hc.f16_epoch = epoch;
        e = launch_bf16_rows_to_f16(hc, st);
        if (e != hipSuccess) return hip_fail(e, "gr_prefill_attention bf16 copy launch");
    }
    e = launch_qkv_prep(pp, st);
    if (e != hipSuccess) return hip_fail(e, "gr_prefill_attention prep launch");

    PrefillLaunch pf{};
    pf.n_tokens = a->n_tokens;
    pf.n_heads = a->n_heads;
    pf.n_kv_heads = a->n_kv_heads;
    pf.head_dim = a->head_dim;
    pf.dtype = a->dtype;
    pf.base_pos = a->base_pos;
    pf.window = a->window;
    pf.bidirectional = a->bidirectional ? 1 : 0;
    pf.q = pp.q_out;
    pf.q_lo = pp.q_out_lo;
    if (fused) {
        pf.q_raw = a->q;
        pf.q_in_dtype = in_dtype;
        pf.q_row_stride = (int64_t)a->n_heads * a->head_dim;
        pf.q_bias = a->q_bias;
        pf.q_norm = a->q_norm;
        pf.norm_eps = a->norm_eps;
        pf.rope_mode = a->rope_mode;
        pf.rope_dim = a->rope_dim;
        pf.rope_cs = pp.rope_cs_out;
        pf.q_pre_scale = a->is_gemma3 ? 1.0f / std::sqrt((float)a->head_dim) : 1.0f;
        pf.q_scale = pp.q_out_scale;
    }
    pf.k_cache = a->k_cache;
    pf.v_cache = a->v_cache;
    pf.cache_row_stride = a->cache_row_stride;
    pf.out = a->out;
    pf.gate.gate = a->out_gate;
    pf.gate.row_stride = a->out_gate_row_stride;
    pf.gate.head_stride = a->out_gate_head_stride;
    if (bf16) {
        pf.k_f16 = k_f16;
        pf.v_f16 = v_f16;
        pf.f16_row0 = row0;
        pf.f16_row_stride = kv_dim;
        pf.f16_flag = flag;
        pf.f16_epoch = epoch;
    }
    e = launch_prefill(pf, st);
    if (e != hipSuccess) return hip_fail(e, "gr_prefill_attention launch");
    return GR_OK;
}

size_t prefill_ws_bytes(const gr_prefill_args* a) {
    if (!a || a->n_tokens < 0 || a->n_heads <= 0 || a->head_dim <= 0) return 0;
    return prefill_ws_total(a);
}

int rope_freqs_host(float theta, int rope_dim, float* out) {
    if (!out || rope_dim <= 0 || (rope_dim & 1))
        return fail(GR_ERR_ARG, "gr_rope_freqs: rope_dim %d must be positive and even", rope_dim);
    if (!std::isfinite(theta) || theta <= 0.0f)
        return fail(GR_ERR_ARG, "gr_rope_freqs: theta must be finite and positive");
    for (int i = 0; i < rope_dim / 2; i++)
        out[i] = 1.0f / powf(theta, (float)(i * 2) / (float)rope_dim);
    return GR_OK;
}

}  // namespace gr

extern "C" {

size_t gr_prefill_workspace_size(const gr_prefill_args* a) { return gr::prefill_ws_bytes(a); }

int gr_prefill_attention(const gr_prefill_args* a, void* stream) {
    gr::clear_error();
    return gr::prefill_enqueue_ex(a, a ? a->dtype : 0, (hipStream_t)stream);
}

int gr_rope_freqs(float theta, int32_t rope_dim, float* freqs_out) {
    gr::clear_error();
    return gr::rope_freqs_host(theta, rope_dim, freqs_out);
}

}  // extern "C"
