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

// ---------------------------------------------------------------- decode
namespace {

struct DecodePlan {
    int split_keys;
    int n_splits;
    size_t ws_o_bytes;
    size_t ws_ml_bytes;
};

// Split size: aim for ~2048 (sequence, KV head, split) work units so the 256
// CUs stay fed even when sequences are ragged; never below 64 keys.
DecodePlan plan_decode(const gr_decode_args* a) {
    DecodePlan pl{};
    const int max_len = a->max_kv_len > 0 ? a->max_kv_len : 1;
    int split = a->split_keys;
    if (split <= 0) {
        const long pairs = (long)a->n_seq * a->n_kv_heads;
        long want = (2048 + pairs - 1) / pairs;
        if (want < 1) want = 1;
        split = (int)((max_len + want - 1) / want);
        split = (split + 63) / 64 * 64;
        if (split < 64) split = 64;
    }
    pl.split_keys = split;
    pl.n_splits = (max_len + split - 1) / split;
    const size_t parts = (size_t)a->n_seq * a->n_heads * pl.n_splits;
    pl.ws_o_bytes = align_up(parts * a->head_dim * sizeof(float), 256);
    pl.ws_ml_bytes = align_up(parts * 2 * sizeof(float), 256);
    return pl;
}

int check_decode(const gr_decode_args* a) {
    if (!a) return fail(GR_ERR_ARG, "gr_decode_attention: null args");
    if (a->n_seq <= 0 || a->n_heads <= 0 || a->n_kv_heads <= 0)
        return fail(GR_ERR_ARG, "gr_decode_attention: n_seq/n_heads/n_kv_heads must be > 0");
    if (a->n_heads % a->n_kv_heads != 0)
        return fail(GR_ERR_ARG, "gr_decode_attention: n_heads %d not a multiple of n_kv_heads %d",
                    a->n_heads, a->n_kv_heads);
    const int kv_mul = a->n_heads / a->n_kv_heads;
    const bool pow2 = kv_mul == 1 || kv_mul == 2 || kv_mul == 4 || kv_mul == 8;
    if (a->kv_dtype == GR_DTYPE_F32 ? !pow2 : (kv_mul > 16 || (a->head_dim == 64 && !pow2)))
        return fail(GR_ERR_ARG,
                    "gr_decode_attention: kv_mul %d unsupported (f32 KV: 1,2,4,8; 16-bit / Q8 KV: <= 16)",
                    kv_mul);
    if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
        return fail(GR_ERR_ARG, "gr_decode_attention: head_dim %d unsupported (64,128,256)",
                    a->head_dim);
    if (a->kv_dtype < GR_DTYPE_F32 || a->kv_dtype > GR_DTYPE_Q8)
        return fail(GR_ERR_ARG, "gr_decode_attention: bad kv_dtype %d", a->kv_dtype);
    if (a->kv_dtype == GR_DTYPE_Q8) {
        if (a->head_dim != 128 && a->head_dim != 256)
            return fail(GR_ERR_ARG, "gr_decode_attention: Q8 KV needs head_dim 128 or 256");
        if (!a->k_scale || !a->v_scale)
            return fail(GR_ERR_ARG, "gr_decode_attention: Q8 KV needs k_scale and v_scale");
        if (a->q8_block &&
            (((uintptr_t)a->k_scale | (uintptr_t)a->v_scale) % 16 != 0 || a->scale_row_stride % 4 != 0 ||
             a->scale_seq_stride % 4 != 0 || a->scale_row_stride < (int64_t)a->n_kv_heads * a->head_dim / 32))
            return fail(GR_ERR_ARG,
                        "gr_decode_attention: Q8 block scales need 16-byte aligned scale arrays and "
                        "strides (multiples of 4 floats, row stride >= kv_dim/32)");
        if (a->scale_row_stride < 0 || a->scale_seq_stride < 0)
            return fail(GR_ERR_ARG, "gr_decode_attention: negative scale stride");
    }
    if (a->max_kv_len <= 0) return fail(GR_ERR_ARG, "gr_decode_attention: max_kv_len must be > 0");
    if (a->split_keys < 0) return fail(GR_ERR_ARG, "gr_decode_attention: split_keys < 0");
    if (!a->q || !a->k_cache || !a->v_cache || !a->kv_start || !a->kv_end || !a->out ||
        !a->workspace)
        return fail(GR_ERR_ARG, "gr_decode_attention: null buffer");
    if (a->row_stride < (int64_t)a->n_kv_heads * a->head_dim)
        return fail(GR_ERR_ARG, "gr_decode_attention: row_stride %lld < n_kv_heads*head_dim",
                    (long long)a->row_stride);
    const int eb = a->kv_dtype == GR_DTYPE_F32 ? 4 : (a->kv_dtype == GR_DTYPE_Q8 ? 1 : 2);
    if (((uintptr_t)a->k_cache | (uintptr_t)a->v_cache) % 16 != 0 ||
        (a->row_stride * eb) % 16 != 0 || (a->seq_stride * eb) % 16 != 0)
        return fail(GR_ERR_ARG, "gr_decode_attention: caches and strides must be 16-byte aligned");
    if ((uintptr_t)a->workspace % 256 != 0)
        return fail(GR_ERR_ARG, "gr_decode_attention: workspace must be 256-byte aligned");
    return GR_OK;
}

}  // namespace

int decode_enqueue(const gr_decode_args* a, hipStream_t st) { return decode_enqueue_ex(a, nullptr, st); }

// seq_slot: optional device map from batch entry to cache sequence slot.
int decode_enqueue_ex(const gr_decode_args* a, const int32_t* seq_slot, hipStream_t st) {
    int rc = check_decode(a);
    if (rc) return rc;
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
    p.ws_o = (float*)a->workspace;
    p.ws_ml = (float*)((char*)a->workspace + pl.ws_o_bytes);
    p.use_mfma = 1;
    if (a->kv_dtype == GR_DTYPE_Q8) {
        p.k_scale = a->k_scale;
        p.v_scale = a->v_scale;
        p.scale_seq_stride = a->scale_seq_stride;
        p.scale_row_stride = a->scale_row_stride;
        p.q8_block = a->q8_block ? 1 : 0;
    }
    hipError_t e = launch_decode(p, st);
    if (e != hipSuccess) return hip_fail(e, "gr_decode_attention launch");
    return GR_OK;
}

size_t decode_ws_bytes(const gr_decode_args* a) {
    if (check_decode_shape_only(a)) return 0;
    const DecodePlan pl = plan_decode(a);
    return pl.ws_o_bytes + pl.ws_ml_bytes;
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

}  // extern "C"
