// Run-state entry points: the device-resident counterpart of the reference's
// RunState (src/engine/types.rs:745-809) and the functions that read and
// write it.  Each entry point takes the reference's host f32 rows, stages them
// on the state's stream, runs the kernels and returns once the results are
// back in host memory (the Rust call sites are synchronous).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <vector>

#include "gr_api_util.hpp"
#include "gr_attn.h"
#include "gr_internal.hpp"
#include "gr_runstate.hpp"

namespace gr {

int h2d(gr_run_state* s, void* dst, const void* src, size_t bytes) {
    hipError_t e = xfer_h2d(s->xfer, s->stream, dst, src, bytes);
    return e == hipSuccess ? GR_OK : hip_fail(e, "host to device copy");
}

int d2h_sync(gr_run_state* s, void* dst, const void* src, size_t bytes) {
    hipError_t e = xfer_d2h(s->xfer, s->stream, dst, src, bytes);
    return e == hipSuccess ? GR_OK : hip_fail(e, "device to host copy");
}

namespace {

// The small per-token calls (a few KB of rows) pay more for the runtime's
// pageable copies (a staging copy and a DMA per row array, each ~10 us) than
// for their kernels.  Their rows go through the state's device-mapped pinned
// buffer instead: the host copies the inputs in, the kernels read them and
// write the outputs there over PCIe, and after the stream synchronises the host
// copies the outputs out.  The buffer is reused call after call: every call
// returns only after its kernels have finished.
constexpr size_t kMappedBytes = size_t(4) << 20;

bool mapped_ready(gr_run_state* s) {
    if (s->mapped) return true;
    if (s->mapped_failed) return false;
    void* h = nullptr;
    void* d = nullptr;
    if (hipHostMalloc(&h, kMappedBytes, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
        (void)hipGetLastError();
        s->mapped_failed = true;
        return false;
    }
    if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipHostFree(h);
        s->mapped_failed = true;
        return false;
    }
    s->mapped = (char*)h;
    s->mapped_dev = (char*)d;
    return true;
}

// The rows of one small call in the mapped buffer: in() copies host rows in and
// returns their device address, out() reserves output rows; finish() waits for
// the stream and copies the reserved outputs to their host destinations.
struct MappedRows {
    gr_run_state* s;
    size_t off = 0;
    struct Out {
        void* dst;
        size_t off, bytes;
    };
    std::vector<Out> outs;
    explicit MappedRows(gr_run_state* st) : s(st) {}
    template <typename T>
    T* in(const T* src, size_t n) {
        host_copy(s->mapped + off, src, n * sizeof(T));
        T* d = (T*)(s->mapped_dev + off);
        off = align_up(off + n * sizeof(T), 256);
        return d;
    }
    template <typename T>
    T* out(T* dst, size_t n) {
        outs.push_back({dst, off, n * sizeof(T)});
        T* d = (T*)(s->mapped_dev + off);
        off = align_up(off + n * sizeof(T), 256);
        return d;
    }
    int finish() {
        const hipError_t e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) return hip_fail(e, "stream synchronize");
        for (const Out& o : outs) host_copy(o.dst, s->mapped + o.off, o.bytes);
        return GR_OK;
    }
};

// Whether a call with these row bytes (inputs + outputs, each array rounded up
// to 256 B) takes the mapped buffer.
bool use_mapped(gr_run_state* s, std::initializer_list<size_t> arrays) {
    size_t total = 0;
    for (size_t b : arrays) total += align_up(b, 256);
    return total <= kMappedBytes && mapped_ready(s);
}

// Staging arena: grows (never shrinks) and is carved per call.
struct Carve {
    char* base;
    size_t off = 0;
    explicit Carve(void* b) : base((char*)b) {}
    template <typename T>
    T* take(size_t n) {
        T* p = (T*)(base + off);
        off = align_up(off + n * sizeof(T), 256);
        return p;
    }
};

int ensure_stage(gr_run_state* s, size_t bytes) {
    if (bytes <= s->stage_bytes) return GR_OK;
    hipError_t e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return hip_fail(e, "staging resize sync");
    if (s->stage) (void)hipFree(s->stage);
    s->stage = nullptr;
    s->stage_bytes = 0;
    const size_t want = align_up(bytes + bytes / 4, 1 << 20);
    e = hipMalloc(&s->stage, want);
    if (e != hipSuccess) return fail(GR_ERR_OOM, "unable to allocate %zu bytes of device staging", want);
    s->stage_bytes = want;
    return GR_OK;
}

// is_swa_layer, inference.rs:1821-1825.
bool is_swa_layer(const gr_run_state* s, int l) {
    if (s->windows.empty()) {
        const int P = s->cfg.swa_pattern;
        return P > 0 && (l % P < P - 1);
    }
    return s->windows[l] > 0;
}

// visible_keys, attention.rs:74-96 (text tokens).
void visible(const gr_run_state* s, int l, int64_t pos, int32_t* start, int32_t* end) {
    const int64_t e = pos + 1;
    const int64_t w = s->windows.empty() ? 0 : s->windows[l];
    *start = (int32_t)(w > 0 && e > w ? e - w : 0);
    *end = (int32_t)e;
}

int check_layer(const gr_run_state* s, int l) {
    if (!s) return fail(GR_ERR_ARG, "null run state");
    if (l < 0 || l >= s->cfg.n_layers)
        return fail(GR_ERR_RANGE, "layer %d outside [0, %d)", l, s->cfg.n_layers);
    return GR_OK;
}

int check_pos(const gr_run_state* s, int seq, int64_t pos, int64_t count) {
    if (seq < 0 || seq >= s->cfg.n_seq)
        return fail(GR_ERR_RANGE, "sequence slot %d outside [0, %d)", seq, s->cfg.n_seq);
    if (pos < 0 || count < 0 || pos + count > s->cfg.seq_len)
        return fail(GR_ERR_RANGE, "batched prefill range exceeds context (%lld + %lld > %d)",
                    (long long)pos, (long long)count, s->cfg.seq_len);
    return GR_OK;
}

void* layer_k(gr_run_state* s, int l) { return (char*)s->k_cache + cache_bytes_at(s, (size_t)l * s->layer_stride); }
void* layer_v(gr_run_state* s, int l) { return (char*)s->v_cache + cache_bytes_at(s, (size_t)l * s->layer_stride); }

// Extra staging bytes a K/V write of n rows needs (Q8 / Turbo: f32 rows before quantising).
size_t q8_stage_bytes(const gr_run_state* s, size_t n) {
    return is_q8(s) || is_turbo(s) ? 8 * n * s->kv_dim + 512 : 0;
}

// Run the prep kernel and store its K/V rows into layer `l`'s cache.  Raw
// storage: the prep kernel writes the cache itself (p.k_cache / p.v_cache set by
// the caller, sequence slot `seq` already folded into them unless p.cache_seq is
// given).  Q8: the prep kernel writes f32 rows to staging and the Q8 write
// kernel quantises them into the cache rows (kv_write_token, inference.rs:1886-1917).
int prep_and_store(gr_run_state* s, int l, int seq, QkvPrepLaunch p, Carve& cv) {
    hipError_t e;
    if (!is_q8(s) && !is_turbo(s)) {
        e = launch_qkv_prep(p, s->stream);
        return e == hipSuccess ? GR_OK : hip_fail(e, "prep launch");
    }
    float* kst = cv.take<float>((size_t)p.n_tokens * s->kv_dim);
    float* vst = cv.take<float>((size_t)p.n_tokens * s->kv_dim);
    const size_t so = p.cache_seq ? 0 : (size_t)seq;
    if (is_turbo(s)) {
        TurboWriteLaunch w{};
        w.n_rows = p.n_tokens;
        w.n_kv_heads = s->cfg.n_kv_heads;
        w.head_dim = s->d;
        w.k_rows = kst;
        w.v_rows = vst;
        const size_t e0 = (size_t)l * s->layer_stride + so * s->seq_stride;
        w.k_base = (uint8_t*)s->k_cache + e0 / 4;
        w.v_base = (uint8_t*)s->v_cache + e0 / 4;
        w.k_sign = s->k_sign + e0 / 8;
        w.v_sign = s->v_sign + e0 / 8;
        const size_t a0 = (size_t)l * s->sc_layer_stride + so * s->sc_seq_stride;
        w.k_scale = s->k_scale + a0;
        w.v_scale = s->v_scale + a0;
        w.k_rnorm = s->k_rnorm + a0;
        w.v_rnorm = s->v_rnorm + a0;
        w.signs = s->turbo_table + (size_t)l * s->cfg.n_kv_heads * (s->d / 8);
        w.slot_stride = (int64_t)s->cfg.n_layers * s->cfg.n_kv_heads * (s->d / 8);
        w.cache_seq_stride = (int64_t)s->seq_stride;
        w.cache_row_stride = s->kv_dim;
        w.aux_seq_stride = (int64_t)s->sc_seq_stride;
        w.aux_row_stride = (int64_t)s->sc_per_row;
        w.cache_row = p.cache_row ? p.cache_row : p.pos;
        w.cache_seq = p.cache_seq;
        w.row0 = p.pos0;
        p.k_cache = kst;
        p.v_cache = vst;
        p.cache_dtype = GR_DTYPE_F32;
        p.cache_row_stride = s->kv_dim;
        p.cache_by_index = 1;
        e = launch_qkv_prep(p, s->stream);
        if (e != hipSuccess) return hip_fail(e, "prep launch");
        e = launch_turbo_write(w, s->stream);
        return e == hipSuccess ? GR_OK : hip_fail(e, "turbo kv write launch");
    }
    Q8WriteLaunch w{};
    w.n_rows = p.n_tokens;
    w.kv_dim = s->kv_dim;
    w.block = s->cfg.q8_block_scales ? 1 : 0;
    w.k_rows = kst;
    w.v_rows = vst;
    w.k_cache = (int8_t*)layer_k(s, l) + so * s->seq_stride;
    w.v_cache = (int8_t*)layer_v(s, l) + so * s->seq_stride;
    w.k_scale = s->k_scale + (size_t)l * s->sc_layer_stride + so * s->sc_seq_stride;
    w.v_scale = s->v_scale + (size_t)l * s->sc_layer_stride + so * s->sc_seq_stride;
    w.cache_seq_stride = (int64_t)s->seq_stride;
    w.cache_row_stride = s->kv_dim;
    w.scale_seq_stride = (int64_t)s->sc_seq_stride;
    w.scale_row_stride = (int64_t)s->sc_per_row;
    w.cache_row = p.cache_row ? p.cache_row : p.pos;
    w.cache_seq = p.cache_seq;
    w.row0 = p.pos0;
    p.k_cache = kst;
    p.v_cache = vst;
    p.cache_dtype = GR_DTYPE_F32;
    p.cache_row_stride = s->kv_dim;
    p.cache_by_index = 1;
    e = launch_qkv_prep(p, s->stream);
    if (e != hipSuccess) return hip_fail(e, "prep launch");
    e = launch_q8_write(w, s->stream);
    return e == hipSuccess ? GR_OK : hip_fail(e, "q8 kv write launch");
}

// Prep launch for one layer: QK-norm and/or RoPE as requested.
QkvPrepLaunch prep_for(gr_run_state* s, int l, int n_tokens, bool norm, bool rope) {
    QkvPrepLaunch p{};
    p.n_tokens = n_tokens;
    p.n_heads = s->cfg.n_heads;
    p.n_kv_heads = s->cfg.n_kv_heads;
    p.head_dim = s->d;
    p.in_dtype = GR_DTYPE_F32;
    const bool swa = is_swa_layer(s, l);
    p.rope_mode = rope ? s->cfg.rope_mode : GR_ROPE_NONE;
    p.rope_dim = s->rope_dim;
    p.rope_freqs = (s->cfg.is_gemma3 && swa) ? s->freqs_swa : s->freqs;
    p.rope_scale = swa ? s->cfg.rope_scale_local : s->cfg.rope_scale_global;
    if (norm && s->has_norm && s->norm_present[l]) {
        p.q_norm = s->qn + (size_t)l * s->d;
        p.k_norm = s->kn + (size_t)l * s->d;
    }
    p.eps = s->eps;
    p.gemma_q_scale = rope ? s->cfg.is_gemma3 : 0;
    p.q_row_stride = s->q_dim;
    p.kv_row_stride = s->kv_dim;
    p.q_out_dtype = GR_DTYPE_F32;
    p.q_out_scale = 1.0f;
    p.cache_dtype = s->cfg.kv_dtype;
    p.cache_row_stride = s->kv_dim;
    return p;
}

float score_scale(const gr_run_state* s) { return s->cfg.is_gemma3 ? 1.0f : 1.0f / std::sqrt((float)s->d); }

int validate_config(const gr_attn_config* c) {
    if (!c) return fail(GR_ERR_ARG, "null config");
    const float scales[2] = {c->rope_scale_global, c->rope_scale_local};
    for (float sc : scales)
        if (!std::isfinite(sc) || sc <= 0.0f) return fail(GR_ERR_ARG, "RoPE frequency scales must be finite and positive");
    if (c->layer_windows) {
        for (int l = 0; l < c->n_layers; l++)
            if (c->layer_windows[l] < 0)
                return fail(GR_ERR_ARG, "attention policy requires one positive window or global entry per layer");
    }
    if (c->n_layers <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->seq_len <= 0 || c->n_seq <= 0)
        return fail(GR_ERR_ARG, "n_layers, n_heads, n_kv_heads, seq_len and n_seq must be positive");
    if (c->n_heads % c->n_kv_heads)
        return fail(GR_ERR_ARG, "n_heads %d is not a multiple of n_kv_heads %d", c->n_heads, c->n_kv_heads);
    if (c->head_dim != 64 && c->head_dim != 128 && c->head_dim != 256)
        return fail(GR_ERR_ARG, "head_dim %d unsupported (64, 128, 256)", c->head_dim);
    if (c->kv_dtype < GR_DTYPE_F32 || c->kv_dtype > GR_DTYPE_TURBO) return fail(GR_ERR_ARG, "bad kv_dtype %d", c->kv_dtype);
    if (c->rope_mode < GR_ROPE_NONE || c->rope_mode > GR_ROPE_NEOX) return fail(GR_ERR_ARG, "bad rope_mode %d", c->rope_mode);
    const int rd = c->rope_dim > 0 ? c->rope_dim : c->head_dim;
    if (rd > c->head_dim || (rd & 1)) return fail(GR_ERR_ARG, "rope_dim %d must be even and <= head_dim", rd);
    if (c->rope_mode == GR_ROPE_ADJACENT && rd != c->head_dim)
        return fail(GR_ERR_ARG, "adjacent-pair RoPE rotates whole heads (rope_dim == head_dim)");
    if (c->rope_mode != GR_ROPE_NONE && (!std::isfinite(c->rope_theta) || c->rope_theta <= 0.0f))
        return fail(GR_ERR_ARG, "rope_theta must be finite and positive");
    if ((c->q_norm == nullptr) != (c->k_norm == nullptr))
        return fail(GR_ERR_ARG, "q_norm and k_norm must be both set or both NULL");
    if (c->ssm_n_heads < 0 ||
        (c->ssm_n_heads > 0 && c->ssm_head_dim != 64 && c->ssm_head_dim != 128 && c->ssm_head_dim != 256))
        return fail(GR_ERR_ARG, "DeltaNet state needs ssm_head_dim 64, 128 or 256");
    // One SSM state and conv history per layer, as one reference RunState holds:
    // the SSM entry points and the prefill-cache sections take no sequence slot.
    if (c->ssm_n_heads > 0 && c->n_seq != 1)
        return fail(GR_ERR_ARG, "an SSM state (ssm_n_heads > 0) needs n_seq == 1: the state has no sequence slots");
    if (c->ssm_conv1d) {
        if (c->ssm_n_heads <= 0 || c->ssm_n_k_heads <= 0 || c->ssm_conv_kernel < 1 || c->ssm_conv_kernel > 9)
            return fail(GR_ERR_ARG, "invalid qwen3next SSM config");
        if (c->ssm_n_heads % c->ssm_n_k_heads)
            return fail(GR_ERR_ARG, "unsupported qwen3next SSM shape: n_v_heads %d not divisible by n_k_heads %d",
                        c->ssm_n_heads, c->ssm_n_k_heads);
        if (!c->ssm_a || !c->ssm_dt_bias || !c->ssm_norm) return fail(GR_ERR_ARG, "missing qwen3next SSM tensors");
    }
    return GR_OK;
}

}  // namespace

int prefill_enqueue_ex(const gr_prefill_args* a, int in_dtype, hipStream_t st);
size_t prefill_ws_bytes(const gr_prefill_args* a);
int decode_enqueue_ex(const gr_decode_args* a, const int32_t* seq_slot, hipStream_t st);
int deltanet_enqueue(const gr_deltanet_args* a, hipStream_t st);
size_t deltanet_ws(const gr_deltanet_args* a);

}  // namespace gr

using namespace gr;

extern "C" {

int gr_malloc_run_state(const gr_attn_config* cfg, gr_run_state** out) {
    clear_error();
    if (!out) return fail(GR_ERR_ARG, "null output pointer");
    *out = nullptr;
    int rc = validate_config(cfg);
    if (rc) return rc;
    gr_run_state* s = new gr_run_state();
    s->cfg = *cfg;
    s->cfg.layer_windows = nullptr;
    s->cfg.q_norm = s->cfg.k_norm = nullptr;
    s->cfg.ssm_conv1d = s->cfg.ssm_a = s->cfg.ssm_dt_bias = s->cfg.ssm_norm = nullptr;  // copied to the device below
    s->cfg.qk_norm_present = nullptr;
    if (cfg->layer_windows) s->windows.assign(cfg->layer_windows, cfg->layer_windows + cfg->n_layers);
    s->d = cfg->head_dim;
    s->kv_dim = cfg->n_kv_heads * cfg->head_dim;
    s->q_dim = cfg->n_heads * cfg->head_dim;
    s->rope_dim = cfg->rope_dim > 0 ? cfg->rope_dim : cfg->head_dim;
    s->eps = cfg->rms_norm_eps > 0.0f ? cfg->rms_norm_eps : 1e-5f;
    s->has_norm = cfg->q_norm != nullptr;
    s->norm_present.assign(cfg->n_layers, s->has_norm ? 1 : 0);
    if (s->has_norm && cfg->qk_norm_present)
        for (int l = 0; l < cfg->n_layers; l++) s->norm_present[l] = cfg->qk_norm_present[l] ? 1 : 0;
    (void)hipGetDevice(&s->device);

    auto cleanup_fail = [&](int code) {
        gr_free_run_state(s);
        return code;
    };
    hipError_t e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (e != hipSuccess) return cleanup_fail(hip_fail(e, "stream create"));
    s->seq_stride = (size_t)cfg->seq_len * s->kv_dim;
    s->layer_stride = s->seq_stride * cfg->n_seq;
    const size_t cache_bytes = cache_bytes_at(s, s->layer_stride * cfg->n_layers);
    if (hipMalloc(&s->k_cache, cache_bytes) != hipSuccess || hipMalloc(&s->v_cache, cache_bytes) != hipSuccess)
        return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate KV cache (%zu bytes each); reduce --context-size", cache_bytes));
    (void)hipMemsetAsync(s->k_cache, 0, cache_bytes, s->stream);
    (void)hipMemsetAsync(s->v_cache, 0, cache_bytes, s->stream);
    if (cfg->kv_dtype == GR_DTYPE_TURBO) {
        const size_t total = s->layer_stride * cfg->n_layers;
        if (hipMalloc(&s->k_sign, total / 8) != hipSuccess || hipMalloc(&s->v_sign, total / 8) != hipSuccess)
            return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate Turbo sign caches (%zu bytes each)", total / 8));
        (void)hipMemsetAsync(s->k_sign, 0, total / 8, s->stream);
        (void)hipMemsetAsync(s->v_sign, 0, total / 8, s->stream);
        s->sc_per_row = (size_t)cfg->n_kv_heads;
        s->sc_seq_stride = (size_t)cfg->seq_len * s->sc_per_row;
        s->sc_layer_stride = s->sc_seq_stride * cfg->n_seq;
        const size_t sb = s->sc_layer_stride * cfg->n_layers * 4;
        if (hipMalloc(&s->k_scale, sb) != hipSuccess || hipMalloc(&s->v_scale, sb) != hipSuccess ||
            hipMalloc(&s->k_rnorm, sb) != hipSuccess || hipMalloc(&s->v_rnorm, sb) != hipSuccess)
            return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate Turbo scale / norm buffers (%zu bytes each)", sb));
        for (float* b : {s->k_scale, s->v_scale, s->k_rnorm, s->v_rnorm}) (void)hipMemsetAsync(b, 0, sb, s->stream);
        const size_t tb = 4 * (size_t)cfg->n_layers * cfg->n_kv_heads * (s->d / 8);
        std::vector<uint8_t> table(tb);
        turbo_sign_table_host(cfg->n_layers, cfg->n_kv_heads, s->d, table.data());
        if (hipMalloc(&s->turbo_table, tb) != hipSuccess)
            return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate the Turbo sign table"));
        e = hipMemcpy(s->turbo_table, table.data(), tb, hipMemcpyHostToDevice);
        if (e != hipSuccess) return cleanup_fail(hip_fail(e, "Turbo sign table upload"));
    }
    if (cfg->kv_dtype == GR_DTYPE_Q8) {
        s->sc_per_row = cfg->q8_block_scales ? (size_t)s->kv_dim / 32 : 1;
        s->sc_seq_stride = (size_t)cfg->seq_len * s->sc_per_row;
        s->sc_layer_stride = s->sc_seq_stride * cfg->n_seq;
        const size_t sb = s->sc_layer_stride * cfg->n_layers * 4;
        if (hipMalloc(&s->k_scale, sb) != hipSuccess || hipMalloc(&s->v_scale, sb) != hipSuccess)
            return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate KV scale buffers (%zu bytes each)", sb));
        (void)hipMemsetAsync(s->k_scale, 0, sb, s->stream);
        (void)hipMemsetAsync(s->v_scale, 0, sb, s->stream);
    }

    // RoPE tables (inference.rs:1590-1609), host powf.
    const int half = s->rope_dim / 2;
    std::vector<float> f(half > 0 ? half : 1), fs(half > 0 ? half : 1);
    if (cfg->rope_mode != GR_ROPE_NONE) {
        const float swa_theta = cfg->rope_theta_swa > 0.0f ? cfg->rope_theta_swa : 10000.0f;
        for (int i = 0; i < half; i++) {
            f[i] = 1.0f / powf(cfg->rope_theta, (float)(i * 2) / (float)s->rope_dim);
            fs[i] = 1.0f / powf(swa_theta, (float)(i * 2) / (float)s->rope_dim);
        }
    }
    if (hipMalloc(&s->freqs, f.size() * 4) != hipSuccess || hipMalloc(&s->freqs_swa, fs.size() * 4) != hipSuccess)
        return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate RoPE tables"));
    (void)hipMemcpyAsync(s->freqs, f.data(), f.size() * 4, hipMemcpyHostToDevice, s->stream);
    (void)hipMemcpyAsync(s->freqs_swa, fs.data(), fs.size() * 4, hipMemcpyHostToDevice, s->stream);
    if (s->has_norm) {
        const size_t nb = (size_t)cfg->n_layers * s->d * 4;
        if (hipMalloc(&s->qn, nb) != hipSuccess || hipMalloc(&s->kn, nb) != hipSuccess)
            return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate QK-norm weights"));
        (void)hipMemcpyAsync(s->qn, cfg->q_norm, nb, hipMemcpyHostToDevice, s->stream);
        (void)hipMemcpyAsync(s->kn, cfg->k_norm, nb, hipMemcpyHostToDevice, s->stream);
    }
    if (cfg->ssm_n_heads > 0) {
        s->ssm_layer = (size_t)cfg->ssm_n_heads * cfg->ssm_head_dim * cfg->ssm_head_dim;
        const size_t nb = s->ssm_layer * cfg->n_layers * 4;
        if (hipMalloc(&s->ssm, nb) != hipSuccess) return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate SSM state"));
        (void)hipMemsetAsync(s->ssm, 0, nb, s->stream);
    }
    if (cfg->ssm_conv1d) {
        const int d = cfg->ssm_head_dim, nv = cfg->ssm_n_heads, K = cfg->ssm_conv_kernel;
        s->ssm_conv_dim = (nv + 2 * cfg->ssm_n_k_heads) * d;
        const size_t L = (size_t)cfg->n_layers;
        const size_t wb = L * s->ssm_conv_dim * K * 4, vb = L * nv * 4, nb = L * d * 4;
        const size_t hb = std::max<size_t>(L * (K - 1) * s->ssm_conv_dim * 4, 4);
        if (hipMalloc(&s->ssm_conv_w, wb) != hipSuccess || hipMalloc(&s->ssm_a, vb) != hipSuccess ||
            hipMalloc(&s->ssm_dt, vb) != hipSuccess || hipMalloc(&s->ssm_nw, nb) != hipSuccess ||
            hipMalloc(&s->ssm_hist, hb) != hipSuccess)
            return cleanup_fail(fail(GR_ERR_OOM, "unable to allocate qwen3next SSM weights / conv state"));
        (void)hipMemcpyAsync(s->ssm_conv_w, cfg->ssm_conv1d, wb, hipMemcpyHostToDevice, s->stream);
        (void)hipMemcpyAsync(s->ssm_a, cfg->ssm_a, vb, hipMemcpyHostToDevice, s->stream);
        (void)hipMemcpyAsync(s->ssm_dt, cfg->ssm_dt_bias, vb, hipMemcpyHostToDevice, s->stream);
        (void)hipMemcpyAsync(s->ssm_nw, cfg->ssm_norm, nb, hipMemcpyHostToDevice, s->stream);
        (void)hipMemsetAsync(s->ssm_hist, 0, hb, s->stream);
    }
    e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return cleanup_fail(hip_fail(e, "run state initialisation"));
    *out = s;
    return GR_OK;
}

void gr_free_run_state(gr_run_state* s) {
    if (!s) return;
    DeviceScope ds(s->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    for (void* p : {s->k_cache, s->v_cache, (void*)s->k_scale, (void*)s->v_scale, (void*)s->k_sign,
                    (void*)s->v_sign, (void*)s->k_rnorm, (void*)s->v_rnorm, (void*)s->turbo_table, (void*)s->ssm_conv_w,
                    (void*)s->ssm_a, (void*)s->ssm_dt, (void*)s->ssm_nw, (void*)s->ssm_hist, (void*)s->freqs,
                    (void*)s->freqs_swa, (void*)s->qn, (void*)s->kn, (void*)s->ssm, s->stage})
        if (p) (void)hipFree(p);
    xfer_release(s->xfer);
    xfer_pipe_release(s->pipe);
    if (s->mapped) (void)hipHostFree(s->mapped);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
}

static int norm_or_rope(gr_run_state* s, int32_t layer, int64_t pos, float* q, float* k, bool norm, bool rope) {
    int rc = check_layer(s, layer);
    if (rc) return rc;
    if (!q || !k) return fail(GR_ERR_ARG, "null q/k");
    if (norm && !(s->has_norm && s->norm_present[layer])) return GR_OK;  // no QK-norm weights: no-op
    DeviceScope dsc(s->device);
    rc = ensure_stage(s, 4 * ((size_t)s->q_dim * 2 + (size_t)s->kv_dim * 2) + 4096);
    if (rc) return rc;
    Carve cv(s->stage);
    const size_t qb = 4 * (size_t)s->q_dim, kb = 4 * (size_t)s->kv_dim;
    const bool mp = use_mapped(s, {qb, kb, qb, kb});
    MappedRows mr(s);
    float* qin = mp ? mr.in(q, s->q_dim) : cv.take<float>(s->q_dim);
    float* kin = mp ? mr.in(k, s->kv_dim) : cv.take<float>(s->kv_dim);
    float* qout = mp ? mr.out(q, s->q_dim) : cv.take<float>(s->q_dim);
    float* kout = mp ? mr.out(k, s->kv_dim) : cv.take<float>(s->kv_dim);
    float* vdump = cv.take<float>(s->kv_dim);
    if (!mp && ((rc = h2d(s, qin, q, qb)) || (rc = h2d(s, kin, k, kb)))) return rc;
    QkvPrepLaunch p = prep_for(s, layer, 1, norm, rope);
    p.pos0 = pos;
    p.q = qin;
    p.k = kin;
    p.v = kin;
    p.q_out = qout;
    p.k_cache = kout;
    p.v_cache = vdump;
    p.cache_dtype = GR_DTYPE_F32;
    p.cache_row_stride = 0;  // single row: ignore the position as a row index
    hipError_t e = launch_qkv_prep(p, s->stream);
    if (e != hipSuccess) return hip_fail(e, "prep launch");
    if (mp) return mr.finish();
    if ((rc = d2h_sync(s, q, qout, qb))) return rc;
    return d2h_sync(s, k, kout, kb);
}

int gr_qkv_norm(gr_run_state* s, int32_t layer, float* q, float* k) {
    clear_error();
    return norm_or_rope(s, layer, 0, q, k, true, false);
}

int gr_apply_rope_qk(gr_run_state* s, int32_t layer, int64_t pos, float* q, float* k) {
    clear_error();
    if (pos < 0) return fail(GR_ERR_RANGE, "negative position");
    return norm_or_rope(s, layer, pos, q, k, false, true);
}

int gr_kv_write_token(gr_run_state* s, int32_t seq, int32_t layer, int64_t pos, const float* k, const float* v) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc || (rc = check_pos(s, seq, pos, 1))) return rc;
    if (!k || !v) return fail(GR_ERR_ARG, "null k/v");
    DeviceScope dsc(s->device);
    if ((rc = ensure_stage(s, 8 * (size_t)s->kv_dim + q8_stage_bytes(s, 1) + 1024))) return rc;
    Carve cv(s->stage);
    const size_t kb = 4 * (size_t)s->kv_dim;
    const bool mp = use_mapped(s, {kb, kb});
    MappedRows mr(s);
    float* kin = mp ? mr.in(k, s->kv_dim) : cv.take<float>(s->kv_dim);
    float* vin = mp ? mr.in(v, s->kv_dim) : cv.take<float>(s->kv_dim);
    if (!mp && ((rc = h2d(s, kin, k, kb)) || (rc = h2d(s, vin, v, kb)))) return rc;
    QkvPrepLaunch p = prep_for(s, layer, 1, false, false);
    p.pos0 = pos;
    p.q = kin;
    p.k = kin;
    p.v = vin;
    p.q_out = nullptr;
    p.k_cache = (char*)layer_k(s, layer) + cache_bytes_at(s, (size_t)seq * s->seq_stride);
    p.v_cache = (char*)layer_v(s, layer) + cache_bytes_at(s, (size_t)seq * s->seq_stride);
    if ((rc = prep_and_store(s, layer, seq, p, cv))) return rc;
    hipError_t e = hipStreamSynchronize(s->stream);
    return e == hipSuccess ? GR_OK : hip_fail(e, "stream synchronize");
}

// Decode n queries whose prepared f32 q rows are at qdev; entry b reads cache
// slot slots[b] (or `seq` for all when slots_dev is null) with visible range
// [starts[b], ends[b]).
// Token-packed Turbo prefill of n rows of one sequence (DecodeLaunch::tok_pack):
// groups of tp = turbo_pack_rows consecutive rows share the split kernel's MFMA
// columns and read every K / V tile (and expand its codes) once.
struct TurboPack {
    int tp = 0;
    int split_keys = 0;
    int max_len = 1;            // longest group range
    std::vector<int32_t> host;  // [4][n]: group start, group end, own start, own end
};

static TurboPack plan_turbo_pack(const gr_run_state* s, int n, const std::vector<int32_t>& starts,
                                 const std::vector<int32_t>& ends) {
    TurboPack t;
    t.tp = turbo_pack_rows(s->d, s->cfg.n_heads / s->cfg.n_kv_heads);
    t.host.resize(4 * (size_t)n);
    for (int b = 0; b < n; b += t.tp) {
        const int e = std::min(n, b + t.tp);
        int32_t lo = starts[b], hi = ends[b];
        for (int i = b; i < e; i++) {
            lo = std::min(lo, starts[i]);
            hi = std::max(hi, ends[i]);
        }
        for (int i = b; i < e; i++) {
            t.host[i] = lo;
            t.host[n + i] = hi;
        }
        t.max_len = std::max(t.max_len, (int)(hi - lo));
    }
    for (int i = 0; i < n; i++) {
        t.host[2 * (size_t)n + i] = starts[i];
        t.host[3 * (size_t)n + i] = ends[i];
    }
    // ~2048 (group, KV head, split) workgroups; splits in whole 128-key rounds
    const long units = (long)((n + t.tp - 1) / t.tp) * s->cfg.n_kv_heads;
    const long want = std::max(1L, (2048 + units - 1) / units);
    t.split_keys = std::max(128, (int)((t.max_len + want - 1) / want + 127) / 128 * 128);
    return t;
}

static gr_decode_args turbo_pack_probe(const gr_run_state* s, int n, const TurboPack& t) {
    gr_decode_args a{};
    a.n_seq = n;
    a.n_heads = s->cfg.n_heads;
    a.n_kv_heads = s->cfg.n_kv_heads;
    a.head_dim = s->d;
    a.kv_dtype = s->cfg.kv_dtype;
    a.split_keys = t.split_keys;
    a.max_kv_len = t.max_len;
    return a;
}

// se_dev: the (start, end) arrays (or the pack's four arrays) already on the
// device; null: uploaded here on the state's stream.
static int run_decode(gr_run_state* s, int layer, int n, const float* qdev, const int32_t* slots_dev, int seq,
                      const std::vector<int32_t>& starts, const std::vector<int32_t>& ends, float* xb_dev,
                      Carve& cv, const TurboPack* pack = nullptr, const int32_t* se_dev = nullptr) {
    std::vector<int32_t> host(2 * (size_t)n);
    int max_len = 1;
    for (int b = 0; b < n; b++) {
        host[b] = starts[b];
        host[n + b] = ends[b];
        max_len = std::max(max_len, ends[b] - starts[b]);
    }
    if (pack) {
        host = pack->host;
        max_len = pack->max_len;
    }
    const int32_t* se = se_dev;
    if (!se) {
        int32_t* up = cv.take<int32_t>(host.size());
        const int rc = h2d(s, up, host.data(), host.size() * 4);
        if (rc) return rc;
        se = up;
    }
    gr_decode_args a{};
    a.n_seq = n;
    a.n_heads = s->cfg.n_heads;
    a.n_kv_heads = s->cfg.n_kv_heads;
    a.head_dim = s->d;
    a.kv_dtype = s->cfg.kv_dtype;
    a.split_keys = pack ? pack->split_keys : 0;
    a.max_kv_len = max_len;
    a.score_scale = score_scale(s);
    a.q = qdev;
    const size_t seq_el = slots_dev ? 0 : (size_t)seq * s->seq_stride;
    a.k_cache = (char*)layer_k(s, layer) + cache_bytes_at(s, seq_el);
    a.v_cache = (char*)layer_v(s, layer) + cache_bytes_at(s, seq_el);
    a.seq_stride = slots_dev ? (int64_t)s->seq_stride : 0;
    a.row_stride = s->kv_dim;
    a.kv_start = se;
    a.kv_end = se + n;
    a.out = xb_dev;
    if (is_turbo(s)) {
        const size_t so = (size_t)layer * s->sc_layer_stride + (slots_dev ? 0 : (size_t)seq * s->sc_seq_stride);
        const size_t e0 = (size_t)layer * s->layer_stride + seq_el;
        a.k_sign = s->k_sign + e0 / 8;
        a.v_sign = s->v_sign + e0 / 8;
        a.k_scale = s->k_scale + so;
        a.v_scale = s->v_scale + so;
        a.k_rnorm = s->k_rnorm + so;
        a.v_rnorm = s->v_rnorm + so;
        a.scale_seq_stride = slots_dev ? (int64_t)s->sc_seq_stride : 0;
        a.scale_row_stride = (int64_t)s->sc_per_row;
        a.turbo_signs = s->turbo_table + (size_t)layer * s->cfg.n_kv_heads * (s->d / 8);
        a.turbo_slot_stride = (int64_t)s->cfg.n_layers * s->cfg.n_kv_heads * (s->d / 8);
    }
    if (is_q8(s)) {
        const size_t so = slots_dev ? 0 : (size_t)seq * s->sc_seq_stride;
        a.k_scale = s->k_scale + (size_t)layer * s->sc_layer_stride + so;
        a.v_scale = s->v_scale + (size_t)layer * s->sc_layer_stride + so;
        a.scale_seq_stride = slots_dev ? (int64_t)s->sc_seq_stride : 0;
        a.scale_row_stride = (int64_t)s->sc_per_row;
        a.q8_block = s->cfg.q8_block_scales ? 1 : 0;
    }
    const size_t ws = decode_ws_bytes(&a);
    a.workspace = cv.take<char>(ws + 256);
    if (pack) return decode_enqueue_ex(&a, slots_dev, s->stream, pack->tp, se + 2 * (size_t)n, se + 3 * (size_t)n);
    return decode_enqueue_ex(&a, slots_dev, s->stream);
}

int gr_attention_token(gr_run_state* s, int32_t seq, int32_t layer, int64_t pos, const float* q, float* xb) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc || (rc = check_pos(s, seq, pos, 1))) return rc;
    if (!q || !xb) return fail(GR_ERR_ARG, "null q/xb");
    DeviceScope dsc(s->device);
    int32_t st, en;
    visible(s, layer, pos, &st, &en);
    gr_decode_args probe{};
    probe.n_seq = 1;
    probe.n_heads = s->cfg.n_heads;
    probe.n_kv_heads = s->cfg.n_kv_heads;
    probe.head_dim = s->d;
    probe.kv_dtype = s->cfg.kv_dtype;
    probe.max_kv_len = en - st;
    if ((rc = ensure_stage(s, 8 * (size_t)s->q_dim + decode_ws_bytes(&probe) + 4096))) return rc;
    Carve cv(s->stage);
    const size_t qb = 4 * (size_t)s->q_dim;
    const bool mp = use_mapped(s, {qb, 8, qb});
    MappedRows mr(s);
    const int32_t se[2] = {st, en};
    float* qin = mp ? mr.in(q, s->q_dim) : cv.take<float>(s->q_dim);
    const int32_t* se_dev = mp ? mr.in(se, 2) : nullptr;
    float* xo = mp ? mr.out(xb, s->q_dim) : cv.take<float>(s->q_dim);
    if (!mp && (rc = h2d(s, qin, q, qb))) return rc;
    if ((rc = run_decode(s, layer, 1, qin, nullptr, seq, {st}, {en}, xo, cv, nullptr, se_dev))) return rc;
    return mp ? mr.finish() : d2h_sync(s, xb, xo, qb);
}

int gr_attention_layer_token(gr_run_state* s, int32_t seq, int32_t layer, int64_t pos, const float* q,
                             const float* k, const float* v, float* xb) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc || (rc = check_pos(s, seq, pos, 1))) return rc;
    if (!q || !k || !v || !xb) return fail(GR_ERR_ARG, "null buffer");
    DeviceScope dsc(s->device);
    int32_t st, en;
    visible(s, layer, pos, &st, &en);
    gr_decode_args probe{};
    probe.n_seq = 1;
    probe.n_heads = s->cfg.n_heads;
    probe.n_kv_heads = s->cfg.n_kv_heads;
    probe.head_dim = s->d;
    probe.kv_dtype = s->cfg.kv_dtype;
    probe.max_kv_len = en - st;
    if ((rc = ensure_stage(s, 4 * (3 * (size_t)s->q_dim + 2 * (size_t)s->kv_dim) + decode_ws_bytes(&probe) +
                                  q8_stage_bytes(s, 1) + 8192)))
        return rc;
    Carve cv(s->stage);
    const size_t qb = 4 * (size_t)s->q_dim, kb = 4 * (size_t)s->kv_dim;
    const bool mp = use_mapped(s, {qb, kb, kb, 8, qb});
    MappedRows mr(s);
    const int32_t se[2] = {st, en};
    float* qin = mp ? mr.in(q, s->q_dim) : cv.take<float>(s->q_dim);
    float* kin = mp ? mr.in(k, s->kv_dim) : cv.take<float>(s->kv_dim);
    float* vin = mp ? mr.in(v, s->kv_dim) : cv.take<float>(s->kv_dim);
    const int32_t* se_host = mp ? mr.in(se, 2) : nullptr;
    int32_t* se_dev = mp ? cv.take<int32_t>(2) : nullptr;  // the prep copies the range here
    float* qp = cv.take<float>(s->q_dim);
    float* xo = mp ? mr.out(xb, s->q_dim) : cv.take<float>(s->q_dim);
    if (!mp && ((rc = h2d(s, qin, q, qb)) || (rc = h2d(s, kin, k, kb)) || (rc = h2d(s, vin, v, kb)))) return rc;
    QkvPrepLaunch p = prep_for(s, layer, 1, true, true);
    if (mp) {
        p.copy_src = se_host;
        p.copy_dst = se_dev;
        p.n_copy = 2;
    }
    p.pos0 = pos;
    p.q = qin;
    p.k = kin;
    p.v = vin;
    p.q_out = qp;
    p.k_cache = (char*)layer_k(s, layer) + cache_bytes_at(s, (size_t)seq * s->seq_stride);
    p.v_cache = (char*)layer_v(s, layer) + cache_bytes_at(s, (size_t)seq * s->seq_stride);
    if ((rc = prep_and_store(s, layer, seq, p, cv))) return rc;
    if ((rc = run_decode(s, layer, 1, qp, nullptr, seq, {st}, {en}, xo, cv, nullptr, se_dev))) return rc;
    return mp ? mr.finish() : d2h_sync(s, xb, xo, qb);
}

// Large calls run their rows in pieces so that the uploads of piece p + 1, the
// kernels of piece p and the downloads of piece p - 1 overlap (xfer_pipeline):
// calls of at least kPipeMinBytes of host rows and 1024 rows.  The first and the
// last piece take 256 rows, the ones between ~512 or more (at most eight pieces),
// which shortens the upload before the first kernel and the kernels and download
// after the last upload.  (Over a Turbo cache a piece of >= 2048 (row group, KV
// head) workgroups gets one split per group, finished in the split kernel; the
// smaller ones a few splits and the combine kernel.  Measured, 2048 rows, 32 / 8
// heads: 2.06-2.34 ms as two 1024-row single-split pieces, 1.81-1.97 ms as 256,
// 512, 512, 512, 256.)  Causal rows only: an image block's rows see the whole
// block, so all of its K / V writes precede its attention.
constexpr size_t kPipeMinBytes = size_t(16) << 20;

static std::vector<int> row_pieces(int m, bool block, size_t bytes, int align = 1) {
    constexpr int kEdge = 256, kMid = 512;
    if (block || bytes < kPipeMinBytes || m < 2 * kMid) return {0, m};
    const int n_mid = std::max(1, std::min(XferPipe::kMaxPieces - 2, (m - 2 * kEdge + kMid / 2) / kMid));
    std::vector<int> cut = {0};
    for (int i = 0; i <= n_mid; i++)
        cut.push_back((kEdge + (int)((int64_t)(m - 2 * kEdge) * i / n_mid)) / align * align);
    cut.push_back(m);
    return cut;
}

// The pieces of a call: each piece's host rows `ups` go up, enqueue(pc) adds its
// kernels to the state's stream and its output rows `downs` come back.  Several
// pieces run pipelined (xfer_pipeline) when the pinned rings can be had, else
// one after another through the state's own copies.
static int run_pieces(gr_run_state* s, int n_pieces, const std::vector<XferRange>& ups,
                      const std::vector<XferRange>& downs, const std::function<int(int)>& enqueue) {
    int rc = GR_OK;
    if (n_pieces > 1 && xfer_pipe_prepare(s->xfer, s->pipe)) {
        const hipError_t e = xfer_pipeline(s->xfer, s->pipe, s->stream, n_pieces, ups, downs, enqueue, &rc);
        if (rc) return rc;
        return e == hipSuccess ? GR_OK : hip_fail(e, "pipelined host transfers");
    }
    size_t iu = 0, id = 0;
    for (int pc = 0; pc < n_pieces; pc++) {
        for (; iu < ups.size() && ups[iu].piece == pc; iu++)
            if ((rc = h2d(s, ups[iu].dev, ups[iu].host, ups[iu].bytes))) return rc;
        if ((rc = enqueue(pc))) return rc;
        for (; id < downs.size() && downs[id].piece == pc; id++)
            if ((rc = d2h_sync(s, downs[id].host, downs[id].dev, downs[id].bytes))) return rc;
    }
    return GR_OK;
}

// The rows base_pos..base_pos+m-1 of one layer: QK-norm, RoPE and KV write of
// every row, then attention of every row over its visible keys; block = the rows
// are one bidirectional image block (attention.rs:87-94), else causal.
static int prefill_rows(gr_run_state* s, int32_t seq, int32_t layer, int64_t base_pos, int32_t m,
                        const float* q, const float* k, const float* v, float* xb, bool block) {
    if (m == 0) return GR_OK;
    if (!q || !k || !v || !xb) return fail(GR_ERR_ARG, "null buffer");
    int rc = GR_OK;
    DeviceScope dsc(s->device);
    const size_t qb = 4 * (size_t)m * s->q_dim, kb = 4 * (size_t)m * s->kv_dim;
    const bool mfma = (s->cfg.kv_dtype == GR_DTYPE_F16 || s->cfg.kv_dtype == GR_DTYPE_BF16) &&
                      (s->d == 64 || s->d == 128 || s->d == 256);
    const int64_t w = s->windows.empty() ? 0 : s->windows[layer];
    std::vector<int32_t> starts(m), ends(m);
    for (int i = 0; i < m; i++) {
        visible(s, layer, base_pos + i, &starts[i], &ends[i]);
        if (block) {
            starts[i] = std::min(starts[i], (int32_t)base_pos);
            ends[i] = (int32_t)(base_pos + m);
        }
    }
    const std::vector<int> cut = row_pieces(m, block, 2 * qb + 2 * kb);
    const int n_pieces = (int)cut.size() - 1;
    const int kv_mul = s->cfg.n_heads / s->cfg.n_kv_heads;
    // the MFMA prefill's arguments for n rows from position pos0 (sizes first: its
    // workspace depends on them)
    auto pf_args = [&](int n, int64_t pos0) {
        gr_prefill_args a{};
        a.n_tokens = n;
        a.base_pos = (int32_t)pos0;
        a.n_heads = s->cfg.n_heads;
        a.n_kv_heads = s->cfg.n_kv_heads;
        a.head_dim = s->d;
        a.dtype = s->cfg.kv_dtype;
        a.window = (int32_t)w;
        a.rope_mode = s->cfg.rope_mode;
        a.rope_dim = s->rope_dim;
        return a;
    };
    // Per piece: its rows' key ranges, the decode path's range arrays (uploaded
    // with the piece's rows) and the scratch its kernels carve; the pieces run in
    // stream order, so they share one scratch region.
    std::vector<std::vector<int32_t>> pst(n_pieces), pen(n_pieces), se(n_pieces);
    std::vector<TurboPack> packs(n_pieces);
    size_t scratch = 0, se_bytes = 0;
    for (int pc = 0; pc < n_pieces; pc++) {
        const int r0 = cut[pc], n = cut[pc + 1] - r0;
        if (mfma) {
            const gr_prefill_args a = pf_args(n, base_pos + r0);
            scratch = std::max(scratch, prefill_ws_bytes(&a) + 256);
            continue;
        }
        pst[pc].assign(starts.begin() + r0, starts.begin() + r0 + n);
        pen[pc].assign(ends.begin() + r0, ends.begin() + r0 + n);
        size_t need = 4 * (size_t)n * s->q_dim + q8_stage_bytes(s, n) + 4 * 256;
        if (!is_q8(s)) {
            gr_decode_args probe{};
            probe.n_seq = n;
            probe.n_heads = s->cfg.n_heads;
            probe.n_kv_heads = s->cfg.n_kv_heads;
            probe.head_dim = s->d;
            probe.kv_dtype = s->cfg.kv_dtype;
            probe.max_kv_len = 1;
            for (int i = 0; i < n; i++) probe.max_kv_len = std::max(probe.max_kv_len, pen[pc][i] - pst[pc][i]);
            if (is_turbo(s) && turbo_pack_rows(s->d, kv_mul) * kv_mul <= 16) {
                packs[pc] = plan_turbo_pack(s, n, pst[pc], pen[pc]);
                probe = turbo_pack_probe(s, n, packs[pc]);
                se[pc] = packs[pc].host;
            } else {  // tp = 0: rows decoded one query row each (GQA groups above 16 heads)
                se[pc] = pst[pc];
                se[pc].insert(se[pc].end(), pen[pc].begin(), pen[pc].end());
            }
            need += decode_ws_bytes(&probe) + 256;
            se_bytes += align_up(4 * se[pc].size(), 256);
        }
        scratch = std::max(scratch, need);
    }
    if ((rc = ensure_stage(s, 2 * qb + 2 * kb + se_bytes + scratch + 1024 * (size_t)n_pieces + 16384))) return rc;
    // per piece, its q, k, v rows and range arrays back to back (one upload DMA)
    Carve cv(s->stage);
    std::vector<float*> qin(n_pieces), kin(n_pieces), vin(n_pieces);
    std::vector<int32_t*> se_dev(n_pieces, nullptr);
    for (int pc = 0; pc < n_pieces; pc++) {
        const size_t n = (size_t)(cut[pc + 1] - cut[pc]);
        qin[pc] = cv.take<float>(n * s->q_dim);
        kin[pc] = cv.take<float>(n * s->kv_dim);
        vin[pc] = cv.take<float>(n * s->kv_dim);
        if (!se[pc].empty()) se_dev[pc] = cv.take<int32_t>(se[pc].size());
    }
    float* xo = cv.take<float>((size_t)m * s->q_dim);
    // One piece whose rows fit the mapped buffer (the reference's 64-token chunks):
    // the kernels read q / k / v and write xb in host memory; the decode's range
    // arrays reach the device through the prep pass's copy.
    const bool mp = n_pieces == 1 && use_mapped(s, {qb, kb, kb, 4 * se[0].size(), qb});
    MappedRows mr(s);
    const int32_t* se_host = nullptr;
    if (mp) {
        qin[0] = mr.in(q, (size_t)m * s->q_dim);
        kin[0] = mr.in(k, (size_t)m * s->kv_dim);
        vin[0] = mr.in(v, (size_t)m * s->kv_dim);
        if (!se[0].empty()) se_host = mr.in(se[0].data(), se[0].size());
        xo = mr.out(xb, (size_t)m * s->q_dim);
    }
    const Carve scratch_base = cv;
    void* kc = (char*)layer_k(s, layer) + cache_bytes_at(s, (size_t)seq * s->seq_stride);
    void* vc = (char*)layer_v(s, layer) + cache_bytes_at(s, (size_t)seq * s->seq_stride);

    // the kernels of piece pc, on the state's stream, once its rows are on the device
    auto enqueue = [&](int pc) -> int {
        const int r0 = cut[pc], n = cut[pc + 1] - r0;
        const int64_t pos0 = base_pos + r0;
        Carve cw = scratch_base;
        float* qi = qin[pc];
        float* ki = kin[pc];
        float* vi = vin[pc];
        float* xi = xo + (size_t)r0 * s->q_dim;
        if (mfma) {
            gr_prefill_args a = pf_args(n, pos0);
            const size_t ws = prefill_ws_bytes(&a);
            const bool swa = is_swa_layer(s, layer);
            a.rope_scale = swa ? s->cfg.rope_scale_local : s->cfg.rope_scale_global;
            a.rope_freqs = (s->cfg.is_gemma3 && swa) ? s->freqs_swa : s->freqs;
            if (s->has_norm && s->norm_present[layer]) {
                a.q_norm = s->qn + (size_t)layer * s->d;
                a.k_norm = s->kn + (size_t)layer * s->d;
            }
            a.norm_eps = s->eps;
            a.is_gemma3 = s->cfg.is_gemma3;
            a.q = qi;
            a.k = ki;
            a.v = vi;
            a.k_cache = kc;
            a.v_cache = vc;
            a.cache_row_stride = s->kv_dim;
            a.out = xi;
            a.workspace = cw.take<char>(ws);
            a.bidirectional = block ? 1 : 0;
            return prefill_enqueue_ex(&a, GR_DTYPE_F32, s->stream);
        }
        float* qp = cw.take<float>((size_t)n * s->q_dim);
        QkvPrepLaunch p = prep_for(s, layer, n, true, true);
        p.pos0 = pos0;
        p.q = qi;
        p.k = ki;
        p.v = vi;
        p.q_out = qp;
        p.k_cache = kc;
        p.v_cache = vc;
        if (se_host && se_dev[pc]) {
            p.copy_src = se_host;
            p.copy_dst = se_dev[pc];
            p.n_copy = (int)se[pc].size();
        }
        int r = prep_and_store(s, layer, seq, p, cw);
        if (r) return r;
        if (is_q8(s)) {
            // one MFMA flash pass over the int8 rows (all n queries share each K / V tile)
            PrefillQ8Launch pq{};
            pq.n_tokens = n;
            pq.n_heads = s->cfg.n_heads;
            pq.n_kv_heads = s->cfg.n_kv_heads;
            pq.head_dim = s->d;
            pq.base_pos = pos0;
            pq.window = (int)w;
            pq.bidirectional = block ? 1 : 0;
            pq.block = s->cfg.q8_block_scales ? 1 : 0;
            pq.score_scale = score_scale(s);
            pq.q = qp;
            pq.k_codes = (const int8_t*)kc;
            pq.v_codes = (const int8_t*)vc;
            pq.row_stride = s->kv_dim;
            const size_t so = (size_t)layer * s->sc_layer_stride + (size_t)seq * s->sc_seq_stride;
            pq.k_scale = s->k_scale + so;
            pq.v_scale = s->v_scale + so;
            pq.scale_row_stride = (int64_t)s->sc_per_row;
            pq.out = xi;
            const hipError_t e = launch_prefill_q8(pq, s->stream);
            return e == hipSuccess ? GR_OK : hip_fail(e, "q8 prefill launch");
        }
        return run_decode(s, layer, n, qp, nullptr, seq, pst[pc], pen[pc], xi, cw,
                          packs[pc].tp > 0 ? &packs[pc] : nullptr, se_dev[pc]);
    };

    if (mp) {
        if ((rc = enqueue(0))) return rc;
        return mr.finish();
    }
    std::vector<XferRange> ups, downs;
    for (int pc = 0; pc < n_pieces; pc++) {
        const size_t r0 = (size_t)cut[pc], n = (size_t)(cut[pc + 1] - cut[pc]);
        ups.push_back({(char*)qin[pc], (char*)(q + r0 * s->q_dim), 4 * n * s->q_dim, pc});
        ups.push_back({(char*)kin[pc], (char*)(k + r0 * s->kv_dim), 4 * n * s->kv_dim, pc});
        ups.push_back({(char*)vin[pc], (char*)(v + r0 * s->kv_dim), 4 * n * s->kv_dim, pc});
        if (se_dev[pc]) ups.push_back({(char*)se_dev[pc], (char*)se[pc].data(), 4 * se[pc].size(), pc});
        downs.push_back({(char*)(xo + r0 * s->q_dim), (char*)(xb + r0 * s->q_dim), 4 * n * s->q_dim, pc});
    }
    return run_pieces(s, n_pieces, ups, downs, enqueue);
}

int gr_prefill_attention_chunk(gr_run_state* s, int32_t seq, int32_t layer, int64_t base_pos, int32_t m,
                               const float* q, const float* k, const float* v, float* xb) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc || (rc = check_pos(s, seq, base_pos, m))) return rc;
    return prefill_rows(s, seq, layer, base_pos, m, q, k, v, xb, false);
}

int gr_prefill_image_block(gr_run_state* s, int32_t seq, int32_t layer, int64_t base_pos, int32_t m,
                           const float* q, const float* k, const float* v, float* xb) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc) return rc;
    if (m <= 0 || base_pos < 0 || base_pos + m > s->cfg.seq_len)
        return fail(GR_ERR_RANGE, "image-block prefill must evaluate one complete supported block within context");
    if ((rc = check_pos(s, seq, base_pos, m))) return rc;
    return prefill_rows(s, seq, layer, base_pos, m, q, k, v, xb, true);
}

int gr_decode_layer_batch(gr_run_state* s, int32_t layer, int32_t n, const int32_t* seqs, const int64_t* pos,
                          const float* q, const float* k, const float* v, float* xb) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc) return rc;
    if (n <= 0) return n == 0 ? GR_OK : fail(GR_ERR_ARG, "n < 0");
    if (!seqs || !pos || !q || !k || !v || !xb) return fail(GR_ERR_ARG, "null buffer");
    std::vector<int32_t> starts(n), ends(n), pos32(n);
    int max_len = 1;
    for (int b = 0; b < n; b++) {
        if ((rc = check_pos(s, seqs[b], pos[b], 1))) return rc;
        visible(s, layer, pos[b], &starts[b], &ends[b]);
        pos32[b] = (int32_t)pos[b];
        max_len = std::max(max_len, ends[b] - starts[b]);
    }
    DeviceScope dsc(s->device);
    gr_decode_args probe{};
    probe.n_seq = n;
    probe.n_heads = s->cfg.n_heads;
    probe.n_kv_heads = s->cfg.n_kv_heads;
    probe.head_dim = s->d;
    probe.kv_dtype = s->cfg.kv_dtype;
    probe.max_kv_len = max_len;
    const size_t qb = 4 * (size_t)n * s->q_dim, kb = 4 * (size_t)n * s->kv_dim;
    if ((rc = ensure_stage(s, 3 * qb + 2 * kb + decode_ws_bytes(&probe) + 16 * (size_t)n + q8_stage_bytes(s, n) +
                                  16384)))
        return rc;
    Carve cv(s->stage);
    const bool mp = use_mapped(s, {qb, kb, kb, 4 * (size_t)n, 4 * (size_t)n, 8 * (size_t)n, qb});
    MappedRows mr(s);
    std::vector<int32_t> se(2 * (size_t)n);
    for (int b = 0; b < n; b++) {
        se[b] = starts[b];
        se[n + b] = ends[b];
    }
    float* qin = mp ? mr.in(q, (size_t)n * s->q_dim) : cv.take<float>((size_t)n * s->q_dim);
    float* kin = mp ? mr.in(k, (size_t)n * s->kv_dim) : cv.take<float>((size_t)n * s->kv_dim);
    float* vin = mp ? mr.in(v, (size_t)n * s->kv_dim) : cv.take<float>((size_t)n * s->kv_dim);
    // mapped: [slots | starts | ends] in one array, which the prep copies to the
    // device for the decode kernels (read by every workgroup)
    std::vector<int32_t> sse;
    if (mp) {
        sse.assign(seqs, seqs + n);
        sse.insert(sse.end(), se.begin(), se.end());
    }
    const int32_t* sse_host = mp ? mr.in(sse.data(), sse.size()) : nullptr;
    int32_t* sse_dev = mp ? cv.take<int32_t>(3 * (size_t)n) : nullptr;
    int32_t* slot_d = mp ? sse_dev : cv.take<int32_t>(n);
    int32_t* pos_d = mp ? mr.in(pos32.data(), n) : cv.take<int32_t>(n);
    const int32_t* se_dev = mp ? sse_dev + n : nullptr;
    float* qp = cv.take<float>((size_t)n * s->q_dim);
    float* xo = mp ? mr.out(xb, (size_t)n * s->q_dim) : cv.take<float>((size_t)n * s->q_dim);
    if (!mp && ((rc = h2d(s, qin, q, qb)) || (rc = h2d(s, kin, k, kb)) || (rc = h2d(s, vin, v, kb)) ||
                (rc = h2d(s, slot_d, seqs, 4 * (size_t)n)) || (rc = h2d(s, pos_d, pos32.data(), 4 * (size_t)n))))
        return rc;
    QkvPrepLaunch p = prep_for(s, layer, n, true, true);
    if (mp) {
        p.copy_src = sse_host;
        p.copy_dst = sse_dev;
        p.n_copy = 3 * n;
    }
    p.pos = pos_d;
    p.q = qin;
    p.k = kin;
    p.v = vin;
    p.q_out = qp;
    p.k_cache = layer_k(s, layer);
    p.v_cache = layer_v(s, layer);
    p.cache_seq = mp ? sse_host : slot_d;  // the prep's own reads: the device copy is not there yet
    p.cache_seq_stride = (int64_t)s->seq_stride;
    if ((rc = prep_and_store(s, layer, 0, p, cv))) return rc;
    if ((rc = run_decode(s, layer, n, qp, slot_d, 0, starts, ends, xo, cv, nullptr, se_dev))) return rc;
    return mp ? mr.finish() : d2h_sync(s, xb, xo, qb);
}

static int check_ssm(gr_run_state* s, int layer) {
    int rc = check_layer(s, layer);
    if (rc) return rc;
    if (!s->ssm) return fail(GR_ERR_ARG, "run state has no SSM state (ssm_n_heads == 0)");
    return GR_OK;
}

int gr_qwen3next_state_step(gr_run_state* s, int32_t layer, const float* q, const float* k, const float* v,
                            const float* g, const float* beta, float* out) {
    clear_error();
    int rc = check_ssm(s, layer);
    if (rc) return rc;
    if (!q || !k || !v || !g || !beta || !out) return fail(GR_ERR_ARG, "null buffer");
    DeviceScope dsc(s->device);
    const int H = s->cfg.ssm_n_heads, D = s->cfg.ssm_head_dim;
    const size_t rb = 4 * (size_t)H * D;
    if ((rc = ensure_stage(s, 4 * rb + 8 * (size_t)H + 4096))) return rc;
    Carve cv(s->stage);
    const bool mp = use_mapped(s, {rb, rb, rb, 4 * (size_t)H, 4 * (size_t)H, rb});
    MappedRows mr(s);
    const size_t hd = (size_t)H * D;
    float* qd = mp ? mr.in(q, hd) : cv.take<float>(hd);
    float* kd = mp ? mr.in(k, hd) : cv.take<float>(hd);
    float* vd = mp ? mr.in(v, hd) : cv.take<float>(hd);
    float* gd = mp ? mr.in(g, (size_t)H) : cv.take<float>(H);
    float* bd = mp ? mr.in(beta, (size_t)H) : cv.take<float>(H);
    float* od = mp ? mr.out(out, hd) : cv.take<float>(hd);
    if (!mp && ((rc = h2d(s, qd, q, rb)) || (rc = h2d(s, kd, k, rb)) || (rc = h2d(s, vd, v, rb)) ||
                (rc = h2d(s, gd, g, 4 * (size_t)H)) || (rc = h2d(s, bd, beta, 4 * (size_t)H))))
        return rc;
    DeltaNetLaunch p{};
    p.n_tokens = 1;
    p.n_heads = H;
    p.head_dim = D;
    p.in_dtype = GR_DTYPE_F32;
    p.l2norm = 0;
    p.eps = s->eps;
    p.q = qd;
    p.k = kd;
    p.v = vd;
    p.gate = gd;
    p.beta = bd;
    p.state = s->ssm + (size_t)layer * s->ssm_layer;
    p.out = od;
    p.gate_is_log = 0;
    hipError_t e = launch_deltanet_scan(p, s->stream);
    if (e != hipSuccess) return hip_fail(e, "deltanet step launch");
    return mp ? mr.finish() : d2h_sync(s, out, od, rb);
}

int gr_qwen3next_prefill(gr_run_state* s, int32_t layer, int32_t T, const float* q, const float* k,
                         const float* v, const float* gate, const float* beta, float* out) {
    clear_error();
    int rc = check_ssm(s, layer);
    if (rc) return rc;
    if (T < 0) return fail(GR_ERR_ARG, "T < 0");
    if (T == 0) return GR_OK;
    if (!q || !k || !v || !gate || !beta || !out) return fail(GR_ERR_ARG, "null buffer");
    DeviceScope dsc(s->device);
    const int H = s->cfg.ssm_n_heads, D = s->cfg.ssm_head_dim;
    const size_t rw = (size_t)H * D;  // floats per token row
    // Pieces at multiples of the chunked scan's 64 tokens (the state carries
    // over in device memory, in stream order): the chunks are those of one call.
    const std::vector<int> cut = row_pieces(T, false, 4 * (size_t)T * (4 * rw + 2 * H), 64);
    const int n_pieces = (int)cut.size() - 1;
    auto args = [&](int n) {
        gr_deltanet_args a{};
        a.n_tokens = n;
        a.n_heads = H;
        a.head_dim = D;
        a.in_dtype = GR_DTYPE_F32;
        a.l2norm = 1;
        a.algo = GR_DELTANET_AUTO;
        a.eps = s->eps;
        return a;
    };
    size_t ws = 0, in_bytes = 0;
    for (int pc = 0; pc < n_pieces; pc++) {
        const gr_deltanet_args a = args(cut[pc + 1] - cut[pc]);
        ws = std::max(ws, deltanet_ws(&a));
        in_bytes += align_up(4 * (size_t)(cut[pc + 1] - cut[pc]) * (3 * rw + 2 * H) + 4 * 256, 256);
    }
    if ((rc = ensure_stage(s, in_bytes + 4 * (size_t)T * rw + ws + 8192))) return rc;
    // per piece, its q, k, v, gate and beta rows back to back (one upload DMA)
    Carve cv(s->stage);
    std::vector<XferRange> ups, downs;
    std::vector<float*> qd(n_pieces), kd(n_pieces), vd(n_pieces), gd(n_pieces), bd(n_pieces);
    for (int pc = 0; pc < n_pieces; pc++) {
        const size_t t0 = (size_t)cut[pc], n = (size_t)(cut[pc + 1] - cut[pc]);
        qd[pc] = cv.take<float>(n * rw);
        kd[pc] = cv.take<float>(n * rw);
        vd[pc] = cv.take<float>(n * rw);
        gd[pc] = cv.take<float>(n * H);
        bd[pc] = cv.take<float>(n * H);
        ups.push_back({(char*)qd[pc], (char*)(q + t0 * rw), 4 * n * rw, pc});
        ups.push_back({(char*)kd[pc], (char*)(k + t0 * rw), 4 * n * rw, pc});
        ups.push_back({(char*)vd[pc], (char*)(v + t0 * rw), 4 * n * rw, pc});
        ups.push_back({(char*)gd[pc], (char*)(gate + t0 * H), 4 * n * H, pc});
        ups.push_back({(char*)bd[pc], (char*)(beta + t0 * H), 4 * n * H, pc});
    }
    float* od = cv.take<float>((size_t)T * rw);
    char* wsp = ws ? cv.take<char>(ws) : nullptr;  // shared by the pieces (stream order)
    // one piece that fits the mapped buffer: rows read and written in host memory
    const size_t tb = 4 * (size_t)T * rw, gb = 4 * (size_t)T * H;
    const bool mp = n_pieces == 1 && use_mapped(s, {tb, tb, tb, gb, gb, tb});
    MappedRows mr(s);
    if (mp) {
        qd[0] = mr.in(q, (size_t)T * rw);
        kd[0] = mr.in(k, (size_t)T * rw);
        vd[0] = mr.in(v, (size_t)T * rw);
        gd[0] = mr.in(gate, (size_t)T * H);
        bd[0] = mr.in(beta, (size_t)T * H);
        od = mr.out(out, (size_t)T * rw);
    }
    for (int pc = 0; pc < n_pieces; pc++) {
        const size_t t0 = (size_t)cut[pc], n = (size_t)(cut[pc + 1] - cut[pc]);
        downs.push_back({(char*)(od + t0 * rw), (char*)(out + t0 * rw), 4 * n * rw, pc});
    }
    auto enqueue = [&](int pc) {
        gr_deltanet_args a = args(cut[pc + 1] - cut[pc]);
        a.q = qd[pc];
        a.k = kd[pc];
        a.v = vd[pc];
        a.gate = gd[pc];
        a.beta = bd[pc];
        a.state = s->ssm + (size_t)layer * s->ssm_layer;
        a.out = od + (size_t)cut[pc] * rw;
        a.workspace = deltanet_ws(&a) ? wsp : nullptr;
        return deltanet_enqueue(&a, s->stream);
    };
    if (mp) {
        if ((rc = enqueue(0))) return rc;
        return mr.finish();
    }
    return run_pieces(s, n_pieces, ups, downs, enqueue);
}

int gr_qwen3next_ssm_layer(gr_run_state* s, int32_t layer, int32_t T, const float* qkv, const float* z,
                           const float* gate_a, const float* gate_b, float* out) {
    clear_error();
    int rc = check_ssm(s, layer);
    if (rc) return rc;
    if (!s->ssm_conv_w) return fail(GR_ERR_ARG, "missing qwen3next SSM tensors");
    if (T < 0) return fail(GR_ERR_ARG, "T < 0");
    if (T == 0) return GR_OK;
    if (!qkv || !z || !gate_a || !out) return fail(GR_ERR_ARG, "null buffer");
    DeviceScope dsc(s->device);
    const int nv = s->cfg.ssm_n_heads, d = s->cfg.ssm_head_dim, K = s->cfg.ssm_conv_kernel;
    const size_t cd = (size_t)s->ssm_conv_dim, di = (size_t)nv * d;
    const size_t ga_rows = gate_b ? (size_t)nv : 2 * (size_t)nv;
    const size_t gb_rows = gate_b ? (size_t)nv : 0;
    // Pieces at multiples of the chunked scan's 64 tokens; each piece's launches
    // read and update the conv history and the state like a call of their own.
    const std::vector<int> cut = row_pieces(T, false, 4 * (size_t)T * (cd + 2 * di + ga_rows + gb_rows), 64);
    const int n_pieces = (int)cut.size() - 1;
    auto args = [&](int n) {
        gr_deltanet_args a{};
        a.n_tokens = n;
        a.n_heads = nv;
        a.head_dim = d;
        a.in_dtype = GR_DTYPE_F32;
        a.l2norm = 1;
        a.algo = GR_DELTANET_AUTO;
        a.eps = s->eps;
        return a;
    };
    size_t ws = 0, in_bytes = 0;
    int max_n = 0;
    for (int pc = 0; pc < n_pieces; pc++) {
        const int n = cut[pc + 1] - cut[pc];
        const gr_deltanet_args a = args(n);
        ws = std::max(ws, deltanet_ws(&a));
        max_n = std::max(max_n, n);
        in_bytes += align_up(4 * (size_t)n * (cd + di + ga_rows + gb_rows) + 4 * 256, 256);
    }
    const size_t mid = 4 * ((size_t)max_n * (4 * di + 2 * nv)) + 8 * 256;  // one piece's q, k, v, o, beta, gate
    if ((rc = ensure_stage(s, in_bytes + mid + 4 * (size_t)T * di + ws + 16384))) return rc;
    Carve cv(s->stage);
    std::vector<XferRange> ups, downs;
    std::vector<float*> qkv_d(n_pieces), z_d(n_pieces), ga_d(n_pieces), gb_d(n_pieces, nullptr);
    for (int pc = 0; pc < n_pieces; pc++) {
        const size_t t0 = (size_t)cut[pc], n = (size_t)(cut[pc + 1] - cut[pc]);
        qkv_d[pc] = cv.take<float>(n * cd);
        z_d[pc] = cv.take<float>(n * di);
        ga_d[pc] = cv.take<float>(n * ga_rows);
        ups.push_back({(char*)qkv_d[pc], (char*)(qkv + t0 * cd), 4 * n * cd, pc});
        ups.push_back({(char*)z_d[pc], (char*)(z + t0 * di), 4 * n * di, pc});
        ups.push_back({(char*)ga_d[pc], (char*)(gate_a + t0 * ga_rows), 4 * n * ga_rows, pc});
        if (gate_b) {
            gb_d[pc] = cv.take<float>(n * gb_rows);
            ups.push_back({(char*)gb_d[pc], (char*)(gate_b + t0 * gb_rows), 4 * n * gb_rows, pc});
        }
    }
    // the intermediates of one piece, reused piece after piece (stream order)
    float* q_d = cv.take<float>((size_t)max_n * di);
    float* k_d = cv.take<float>((size_t)max_n * di);
    float* v_d = cv.take<float>((size_t)max_n * di);
    float* beta_d = cv.take<float>((size_t)max_n * nv);
    float* gate_d = cv.take<float>((size_t)max_n * nv);
    float* o_d = cv.take<float>((size_t)max_n * di);
    float* out_d = cv.take<float>((size_t)T * di);
    char* wsp = ws ? cv.take<char>(ws) : nullptr;
    // one piece that fits the mapped buffer (decode: T = 1): rows read and
    // written in host memory
    const bool mp = n_pieces == 1 && use_mapped(s, {4 * (size_t)T * cd, 4 * (size_t)T * di, 4 * (size_t)T * ga_rows,
                                                   4 * (size_t)T * gb_rows, 4 * (size_t)T * di});
    MappedRows mr(s);
    if (mp) {
        qkv_d[0] = mr.in(qkv, (size_t)T * cd);
        z_d[0] = mr.in(z, (size_t)T * di);
        ga_d[0] = mr.in(gate_a, (size_t)T * ga_rows);
        if (gate_b) gb_d[0] = mr.in(gate_b, (size_t)T * gb_rows);
        out_d = mr.out(out, (size_t)T * di);
    }
    for (int pc = 0; pc < n_pieces; pc++) {
        const size_t t0 = (size_t)cut[pc], n = (size_t)(cut[pc + 1] - cut[pc]);
        downs.push_back({(char*)(out_d + t0 * di), (char*)(out + t0 * di), 4 * n * di, pc});
    }
    auto enqueue = [&](int pc) {
        const int n = cut[pc + 1] - cut[pc];
        SsmLaunch p{};
        p.n_tokens = n;
        p.n_k_heads = s->cfg.ssm_n_k_heads;
        p.n_v_heads = nv;
        p.head_dim = d;
        p.conv_kernel = K;
        p.eps = s->eps;
        p.qkv = qkv_d[pc];
        p.z = z_d[pc];
        p.gate_a = ga_d[pc];
        p.gate_b = gb_d[pc];
        p.conv_w = s->ssm_conv_w + (size_t)layer * cd * K;
        p.dt_bias = s->ssm_dt + (size_t)layer * nv;
        p.ssm_a = s->ssm_a + (size_t)layer * nv;
        p.ssm_norm = s->ssm_nw + (size_t)layer * d;
        p.conv_hist = s->ssm_hist + (size_t)layer * (K - 1) * cd;
        p.q_out = q_d;
        p.k_out = k_d;
        p.v_out = v_d;
        p.beta_out = beta_d;
        p.gate_out = gate_d;
        p.o = o_d;
        p.out = out_d + (size_t)cut[pc] * di;
        hipError_t e = launch_ssm_pre(p, s->stream);
        if (e != hipSuccess) return hip_fail(e, "ssm pre launch");
        gr_deltanet_args a = args(n);
        a.q = q_d;
        a.k = k_d;
        a.v = v_d;
        a.gate = gate_d;
        a.beta = beta_d;
        a.state = s->ssm + (size_t)layer * s->ssm_layer;
        a.out = o_d;
        a.workspace = deltanet_ws(&a) ? wsp : nullptr;
        int r = deltanet_enqueue(&a, s->stream);
        if (r) return r;
        e = launch_ssm_post(p, s->stream);
        return e == hipSuccess ? GR_OK : hip_fail(e, "ssm post launch");
    };
    if (mp) {
        if ((rc = enqueue(0))) return rc;
        return mr.finish();
    }
    return run_pieces(s, n_pieces, ups, downs, enqueue);
}

int gr_read_ssm_conv_state(gr_run_state* s, int32_t layer, float* out) {
    clear_error();
    int rc = check_ssm(s, layer);
    if (rc) return rc;
    if (!s->ssm_conv_w) return fail(GR_ERR_ARG, "missing qwen3next SSM tensors");
    if (!out) return fail(GR_ERR_ARG, "null buffer");
    DeviceScope dsc(s->device);
    const size_t n = (size_t)(s->cfg.ssm_conv_kernel - 1) * s->ssm_conv_dim;
    return d2h_sync(s, out, s->ssm_hist + (size_t)layer * n, 4 * n);
}

int gr_write_ssm_conv_state(gr_run_state* s, int32_t layer, const float* in) {
    clear_error();
    int rc = check_ssm(s, layer);
    if (rc) return rc;
    if (!s->ssm_conv_w) return fail(GR_ERR_ARG, "missing qwen3next SSM tensors");
    if (!in) return fail(GR_ERR_ARG, "null buffer");
    DeviceScope dsc(s->device);
    const size_t n = (size_t)(s->cfg.ssm_conv_kernel - 1) * s->ssm_conv_dim;
    if ((rc = h2d(s, s->ssm_hist + (size_t)layer * n, in, 4 * n))) return rc;
    hipError_t e = hipStreamSynchronize(s->stream);
    return e == hipSuccess ? GR_OK : hip_fail(e, "stream synchronize");
}

int gr_read_kv_rows(gr_run_state* s, int32_t layer, int32_t seq, int64_t row0, int64_t n_rows, void* k_out,
                    void* v_out) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc || (rc = check_pos(s, seq, row0, n_rows))) return rc;
    DeviceScope dsc(s->device);
    const size_t off = cache_bytes_at(s, (size_t)seq * s->seq_stride + (size_t)row0 * s->kv_dim);
    const size_t nb = cache_bytes_at(s, (size_t)n_rows * s->kv_dim);
    if (k_out && (rc = d2h_sync(s, k_out, (char*)layer_k(s, layer) + off, nb))) return rc;
    if (v_out && (rc = d2h_sync(s, v_out, (char*)layer_v(s, layer) + off, nb))) return rc;
    return GR_OK;
}

int gr_read_turbo_rows(gr_run_state* s, int32_t layer, int32_t seq, int64_t row0, int64_t n_rows, uint8_t* k_base,
                       uint8_t* k_sign, float* k_rnorm, uint8_t* v_base, uint8_t* v_sign, float* v_rnorm) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc || (rc = check_pos(s, seq, row0, n_rows))) return rc;
    if (!is_turbo(s)) return fail(GR_ERR_ARG, "run state has no Turbo KV cache (kv_dtype %d)", s->cfg.kv_dtype);
    DeviceScope dsc(s->device);
    const size_t e0 = (size_t)layer * s->layer_stride + (size_t)seq * s->seq_stride + (size_t)row0 * s->kv_dim;
    const size_t ne = (size_t)n_rows * s->kv_dim;
    const size_t a0 = (size_t)layer * s->sc_layer_stride + (size_t)seq * s->sc_seq_stride + (size_t)row0 * s->sc_per_row;
    const size_t na = (size_t)n_rows * s->sc_per_row * 4;
    if (k_base && (rc = d2h_sync(s, k_base, (uint8_t*)s->k_cache + e0 / 4, ne / 4))) return rc;
    if (v_base && (rc = d2h_sync(s, v_base, (uint8_t*)s->v_cache + e0 / 4, ne / 4))) return rc;
    if (k_sign && (rc = d2h_sync(s, k_sign, s->k_sign + e0 / 8, ne / 8))) return rc;
    if (v_sign && (rc = d2h_sync(s, v_sign, s->v_sign + e0 / 8, ne / 8))) return rc;
    if (k_rnorm && (rc = d2h_sync(s, k_rnorm, s->k_rnorm + a0, na))) return rc;
    if (v_rnorm && (rc = d2h_sync(s, v_rnorm, s->v_rnorm + a0, na))) return rc;
    return GR_OK;
}

int gr_read_kv_scales(gr_run_state* s, int32_t layer, int32_t seq, int64_t row0, int64_t n_rows,
                      float* k_scale_out, float* v_scale_out) {
    clear_error();
    int rc = check_layer(s, layer);
    if (rc || (rc = check_pos(s, seq, row0, n_rows))) return rc;
    if (!is_q8(s) && !is_turbo(s))
        return fail(GR_ERR_ARG, "run state has no Q8 or Turbo KV cache (kv_dtype %d)", s->cfg.kv_dtype);
    DeviceScope dsc(s->device);
    const size_t off = (size_t)layer * s->sc_layer_stride + (size_t)seq * s->sc_seq_stride + (size_t)row0 * s->sc_per_row;
    const size_t nb = (size_t)n_rows * s->sc_per_row * 4;
    if (k_scale_out && (rc = d2h_sync(s, k_scale_out, s->k_scale + off, nb))) return rc;
    if (v_scale_out && (rc = d2h_sync(s, v_scale_out, s->v_scale + off, nb))) return rc;
    return GR_OK;
}

int gr_read_ssm_state(gr_run_state* s, int32_t layer, float* out) {
    clear_error();
    int rc = check_ssm(s, layer);
    if (rc) return rc;
    if (!out) return fail(GR_ERR_ARG, "null buffer");
    DeviceScope dsc(s->device);
    return d2h_sync(s, out, s->ssm + (size_t)layer * s->ssm_layer, 4 * s->ssm_layer);
}

int gr_write_ssm_state(gr_run_state* s, int32_t layer, const float* in) {
    clear_error();
    int rc = check_ssm(s, layer);
    if (rc) return rc;
    if (!in) return fail(GR_ERR_ARG, "null buffer");
    DeviceScope dsc(s->device);
    if ((rc = h2d(s, s->ssm + (size_t)layer * s->ssm_layer, in, 4 * s->ssm_layer))) return rc;
    hipError_t e = hipStreamSynchronize(s->stream);
    return e == hipSuccess ? GR_OK : hip_fail(e, "stream synchronize");
}

}  // extern "C"
