// Prefill-cache (GPFC v1) export and import of a device run state: the
// reference's snapshot, PrefixCache::parse and PrefixCache::inject
// (src/app/prefill_cache.rs:178-310, 316-364, 380-507) with the KV rows and the
// SSM arrays moved straight between HBM and the caller's blob.
//
// Blob (little-endian): "GPFC" | version u16 = 1 | kv_format u8 (0 = Q8,
// 1 = Turbo) | q8_block u8 | n_layers u32 | kv_dim u32 | n_kv_heads u32 | k u32 |
// seq_len_at_render u32 | model_len u64 | model_head_fnv u64 | tokens i32 x k |
// sections, each a u64 byte length and the bytes.  Section order: Q8 key codes,
// value codes, key scales, value scales; Turbo key codes, value codes, key sign
// bits, value sign bits, key sigma, value sigma, key gamma, value gamma; then
// the SSM conv history and the SSM state of every layer (empty without SSM).
// A KV section holds the first k rows of every layer, layer after layer.
//
// The device rows of one (layer, sequence slot) are contiguous, so a KV section
// moves as one copy per layer.  Every check runs before the first byte is
// written to the device, so a rejected blob leaves the state as it was.
#include <hip/hip_runtime.h>

#include <string.h>

#include <vector>

#include "gr_api_util.hpp"
#include "gr_attn.h"
#include "gr_runstate.hpp"

namespace gr {

namespace {

constexpr uint16_t kGpfcVersion = 1;
constexpr size_t kGpfcHeader = 4 + 2 + 1 + 1 + 5 * 4 + 2 * 8;

// One section of the blob as it lies in HBM: `rows` rows of `row_bytes` per
// layer, layer l's first row at dev + l * pitch; or a flat array (pitch = 0).
struct Section {
    char* dev;
    size_t row_bytes;
    size_t pitch;
    size_t flat_bytes;
    bool f32;
};

// The sections of sequence slot `seq`, in blob order.
std::vector<Section> sections_of(gr_run_state* s, int seq) {
    std::vector<Section> out;
    const size_t e0 = (size_t)seq * s->seq_stride;
    const size_t a0 = (size_t)seq * s->sc_seq_stride;
    auto rows = [&](void* base, size_t row_bytes, size_t pitch, bool f32) {
        out.push_back(Section{(char*)base, row_bytes, pitch, 0, f32});
    };
    const size_t kv_row = cache_bytes_at(s, (size_t)s->kv_dim);
    const size_t kv_pitch = cache_bytes_at(s, s->layer_stride);
    rows((char*)s->k_cache + cache_bytes_at(s, e0), kv_row, kv_pitch, false);
    rows((char*)s->v_cache + cache_bytes_at(s, e0), kv_row, kv_pitch, false);
    const size_t sc_row = s->sc_per_row * 4, sc_pitch = s->sc_layer_stride * 4;
    if (is_turbo(s)) {
        rows(s->k_sign + e0 / 8, (size_t)s->kv_dim / 8, s->layer_stride / 8, false);
        rows(s->v_sign + e0 / 8, (size_t)s->kv_dim / 8, s->layer_stride / 8, false);
        rows(s->k_scale + a0, sc_row, sc_pitch, true);
        rows(s->v_scale + a0, sc_row, sc_pitch, true);
        rows(s->k_rnorm + a0, sc_row, sc_pitch, true);
        rows(s->v_rnorm + a0, sc_row, sc_pitch, true);
    } else {
        rows(s->k_scale + a0, sc_row, sc_pitch, true);
        rows(s->v_scale + a0, sc_row, sc_pitch, true);
    }
    const size_t L = (size_t)s->cfg.n_layers;
    const size_t conv = s->ssm_hist ? L * (size_t)(s->cfg.ssm_conv_kernel - 1) * s->ssm_conv_dim * 4 : 0;
    const size_t state = s->ssm ? L * s->ssm_layer * 4 : 0;
    out.push_back(Section{(char*)s->ssm_hist, 0, 0, conv, true});
    out.push_back(Section{(char*)s->ssm, 0, 0, state, true});
    return out;
}

size_t section_bytes(const Section& c, size_t n_layers, size_t k) {
    return c.pitch ? n_layers * k * c.row_bytes : c.flat_bytes;
}

void put(std::vector<uint8_t>* h, uint64_t v, int bytes) {
    for (int i = 0; i < bytes; i++) h->push_back((uint8_t)(v >> (8 * i)));
}

uint64_t get(const uint8_t* p, int bytes) {
    uint64_t v = 0;
    for (int i = 0; i < bytes; i++) v |= (uint64_t)p[i] << (8 * i);
    return v;
}

// Reader::take (prefill_cache.rs:90-98).
struct Reader {
    const uint8_t* b;
    uint64_t len;
    uint64_t at = 0;
    const uint8_t* take(uint64_t n) {
        if (n > len - at) return nullptr;
        const uint8_t* p = b + at;
        at += n;
        return p;
    }
};

int check_kv_format(const gr_run_state* s) {
    if (!is_q8(s) && !is_turbo(s))
        return fail(GR_ERR_ARG, "prefill cache requires a Q8 or Turbo KV cache (kv_dtype %d)", s->cfg.kv_dtype);
    return GR_OK;
}

}  // namespace

}  // namespace gr

using namespace gr;

extern "C" {

int gr_prefill_cache_snapshot(gr_run_state* s, int32_t seq, const int32_t* tokens, int32_t k, uint64_t model_len,
                              uint64_t model_head_fnv, uint8_t* out, uint64_t cap, uint64_t* size_out) {
    clear_error();
    if (!s) return fail(GR_ERR_ARG, "null run state");
    if (seq < 0 || seq >= s->cfg.n_seq)
        return fail(GR_ERR_RANGE, "sequence slot %d outside [0, %d)", seq, s->cfg.n_seq);
    if (k < 0 || (k > 0 && !tokens)) return fail(GR_ERR_ARG, "prefill cache: bad token list");
    if (k > s->cfg.seq_len) return fail(GR_ERR_RANGE, "prefill cache: prefix longer than context");
    if (s->kv_dim % 8 != 0) return fail(GR_ERR_ARG, "prefill cache requires kv_dim %% 8 == 0");
    int rc = check_kv_format(s);
    if (rc) return rc;

    const size_t L = (size_t)s->cfg.n_layers;
    const std::vector<Section> secs = sections_of(s, seq);
    size_t total = kGpfcHeader + 4 * (size_t)k;
    for (const Section& c : secs) total += 8 + section_bytes(c, L, (size_t)k);
    if (size_out) *size_out = total;
    if (!out) return GR_OK;
    if (cap < total)
        return fail(GR_ERR_ARG, "prefill cache buffer too small (%llu < %zu bytes)", (unsigned long long)cap, total);

    std::vector<uint8_t> h;
    h.reserve(kGpfcHeader);
    for (char c : {'G', 'P', 'F', 'C'}) h.push_back((uint8_t)c);
    put(&h, kGpfcVersion, 2);
    h.push_back(is_turbo(s) ? 1 : 0);
    h.push_back(s->cfg.q8_block_scales ? 1 : 0);
    put(&h, L, 4);
    put(&h, (uint64_t)s->kv_dim, 4);
    put(&h, (uint64_t)(s->cfg.n_kv_heads > 1 ? s->cfg.n_kv_heads : 1), 4);
    put(&h, (uint64_t)k, 4);
    put(&h, (uint64_t)s->cfg.seq_len, 4);
    put(&h, model_len, 8);
    put(&h, model_head_fnv, 8);
    memcpy(out, h.data(), h.size());
    size_t at = h.size();
    for (int32_t i = 0; i < k; i++, at += 4) {
        const uint32_t t = (uint32_t)tokens[i];
        for (int b = 0; b < 4; b++) out[at + b] = (uint8_t)(t >> (8 * b));
    }

    DeviceScope dsc(s->device);
    for (const Section& c : secs) {
        const size_t nb = section_bytes(c, L, (size_t)k);
        for (int b = 0; b < 8; b++) out[at + b] = (uint8_t)((uint64_t)nb >> (8 * b));
        at += 8;
        hipError_t e = hipSuccess;
        if (c.pitch) {
            const size_t lb = (size_t)k * c.row_bytes;
            for (size_t l = 0; l < L && lb && e == hipSuccess; l++)
                e = hipMemcpyAsync(out + at + l * lb, c.dev + l * c.pitch, lb, hipMemcpyDeviceToHost, s->stream);
        } else if (nb) {
            e = hipMemcpyAsync(out + at, c.dev, nb, hipMemcpyDeviceToHost, s->stream);
        }
        if (e != hipSuccess) return hip_fail(e, "prefill cache device to host copy");
        at += nb;
    }
    hipError_t e = hipStreamSynchronize(s->stream);
    return e == hipSuccess ? GR_OK : hip_fail(e, "stream synchronize");
}

int gr_prefill_cache_inject(gr_run_state* s, int32_t seq, const uint8_t* blob, uint64_t len, int32_t* k_out) {
    clear_error();
    if (!s) return fail(GR_ERR_ARG, "null run state");
    if (seq < 0 || seq >= s->cfg.n_seq)
        return fail(GR_ERR_RANGE, "sequence slot %d outside [0, %d)", seq, s->cfg.n_seq);
    if (!blob && len) return fail(GR_ERR_ARG, "null buffer");

    // PrefixCache::parse (prefill_cache.rs:316-352).
    Reader r{blob, len};
    const uint8_t* p = r.take(4);
    if (!p) return fail(GR_ERR_ARG, "prefill cache truncated");
    if (memcmp(p, "GPFC", 4) != 0) return fail(GR_ERR_ARG, "prefill cache: bad magic");
    if (!(p = r.take(2))) return fail(GR_ERR_ARG, "prefill cache truncated");
    const unsigned version = (unsigned)get(p, 2);
    if (version != kGpfcVersion) return fail(GR_ERR_ARG, "prefill cache: unsupported version %u", version);
    if (!(p = r.take(1))) return fail(GR_ERR_ARG, "prefill cache truncated");
    const unsigned fmt = p[0];
    if (fmt > 1) return fail(GR_ERR_ARG, "prefill cache: bad kv format %u", fmt);
    if (!(p = r.take(1 + 5 * 4 + 2 * 8))) return fail(GR_ERR_ARG, "prefill cache truncated");
    const bool q8_block = p[0] != 0;
    const uint64_t n_layers = get(p + 1, 4), kv_dim = get(p + 5, 4), n_kv = get(p + 9, 4);
    const uint64_t k = get(p + 13, 4);
    if (!r.take(4 * k)) return fail(GR_ERR_ARG, "prefill cache truncated");
    const int n_sections = (fmt == 0 ? 4 : 8) + 2;
    std::vector<const uint8_t*> sec(n_sections);
    std::vector<uint64_t> sec_len(n_sections);
    for (int i = 0; i < n_sections; i++) {
        if (!(p = r.take(8))) return fail(GR_ERR_ARG, "prefill cache truncated");
        sec_len[i] = get(p, 8);
        if (!(sec[i] = r.take(sec_len[i]))) return fail(GR_ERR_ARG, "prefill cache truncated");
    }

    // PrefixCache::inject (prefill_cache.rs:380-507), every check before any copy.
    const int state_fmt = is_q8(s) ? 0 : (is_turbo(s) ? 1 : -1);
    if (n_layers != (uint64_t)s->cfg.n_layers || kv_dim != (uint64_t)s->kv_dim ||
        n_kv != (uint64_t)(s->cfg.n_kv_heads > 1 ? s->cfg.n_kv_heads : 1) || (int)fmt != state_fmt ||
        q8_block != (s->cfg.q8_block_scales != 0))
        return fail(GR_ERR_ARG, "prefill cache: model/config mismatch");
    if (k > (uint64_t)s->cfg.seq_len) return fail(GR_ERR_RANGE, "prefill cache: prefix longer than context");

    const size_t L = (size_t)n_layers;
    const std::vector<Section> secs = sections_of(s, seq);
    const int n_kv_sec = n_sections - 2;
    // The reference scatters the byte sections (codes, sign bits), then converts
    // every f32 section of the format, then scatters those; the byte sections
    // come first in the blob, so three passes in blob order meet the checks in
    // the reference's order and the first failure names the same fault.
    for (int i = 0; i < n_kv_sec; i++)
        if (!secs[i].f32 && sec_len[i] != section_bytes(secs[i], L, k))
            return fail(GR_ERR_ARG, "prefill cache: section size mismatch");
    for (int i = 0; i < n_kv_sec; i++)
        if (secs[i].f32 && sec_len[i] % 4) return fail(GR_ERR_ARG, "prefill cache: bad f32 section length");
    for (int i = 0; i < n_kv_sec; i++)
        if (secs[i].f32 && sec_len[i] != section_bytes(secs[i], L, k))
            return fail(GR_ERR_ARG, "prefill cache: section size mismatch");
    for (int i = n_kv_sec; i < n_sections; i++)
        if (sec_len[i] % 4) return fail(GR_ERR_ARG, "prefill cache: bad f32 section length");
    for (int i = n_kv_sec; i < n_sections; i++)
        if (sec_len[i] != secs[i].flat_bytes) return fail(GR_ERR_ARG, "prefill cache: ssm state size mismatch");

    DeviceScope dsc(s->device);
    for (int i = 0; i < n_sections; i++) {
        const Section& c = secs[i];
        hipError_t e = hipSuccess;
        if (c.pitch) {
            const size_t lb = (size_t)k * c.row_bytes;
            for (size_t l = 0; l < L && lb && e == hipSuccess; l++)
                e = hipMemcpyAsync(c.dev + l * c.pitch, sec[i] + l * lb, lb, hipMemcpyHostToDevice, s->stream);
        } else if (sec_len[i]) {
            e = hipMemcpyAsync(c.dev, sec[i], sec_len[i], hipMemcpyHostToDevice, s->stream);
        }
        if (e != hipSuccess) return hip_fail(e, "prefill cache host to device copy");
    }
    hipError_t e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return hip_fail(e, "stream synchronize");
    if (k_out) *k_out = (int32_t)k;
    return GR_OK;
}

}  // extern "C"
