// The device-resident run state (the reference's RunState,
// src/engine/types.rs:745-809) shared by the run-state translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <vector>

#include "gr_attn.h"
#include "host_xfer.hpp"

struct gr_run_state {
    gr_attn_config cfg{};
    std::vector<int32_t> windows;      // [n_layers], 0 = global
    std::vector<uint8_t> norm_present;  // [n_layers]
    bool has_norm = false;
    int device = 0;
    int d = 0, kv_dim = 0, q_dim = 0, rope_dim = 0;
    float eps = 1e-5f;
    hipStream_t stream = nullptr;
    void* k_cache = nullptr;
    void* v_cache = nullptr;
    size_t seq_stride = 0;    // elements between sequence slots
    size_t layer_stride = 0;  // elements between layers
    // Q8 cache: key_cache_scale / value_cache_scale, sc_per_row scales per row
    // (1, or kv_dim/32 in block mode), same [layer][slot][row] order as the cache.
    float* k_scale = nullptr;
    float* v_scale = nullptr;
    size_t sc_per_row = 0, sc_seq_stride = 0, sc_layer_stride = 0;
    // Turbo cache: k_cache / v_cache hold the 2-bit codes (element e at byte e/4),
    // k_sign / v_sign the residual sign bits (byte e/8), k_scale / v_scale sigma
    // and k_rnorm / v_rnorm gamma with sc_per_row = n_kv_heads; the sign table
    // (turboquant_build_sign_table) lives on the device.
    uint8_t* k_sign = nullptr;
    uint8_t* v_sign = nullptr;
    float* k_rnorm = nullptr;
    float* v_rnorm = nullptr;
    uint8_t* turbo_table = nullptr;
    float* freqs = nullptr;
    float* freqs_swa = nullptr;
    float* qn = nullptr;
    float* kn = nullptr;
    float* ssm = nullptr;
    size_t ssm_layer = 0;  // floats per layer
    // Qwen3.5 SSM layer weights and conv history (ssm_conv_state)
    int ssm_conv_dim = 0;
    float* ssm_conv_w = nullptr;  // [n_layers][conv_dim][K]
    float* ssm_a = nullptr;       // [n_layers][n_v]
    float* ssm_dt = nullptr;      // [n_layers][n_v]
    float* ssm_nw = nullptr;      // [n_layers][head_dim]
    float* ssm_hist = nullptr;    // [n_layers][K-1][conv_dim]
    void* stage = nullptr;
    size_t stage_bytes = 0;
    gr::HostXfer xfer;  // pinned ring for the host rows of each call
    gr::XferPipe pipe;  // streams and download ring of the pipelined large calls
    // Pinned, device-mapped host buffer for the rows of the small per-token calls:
    // their kernels read the inputs and write the outputs there directly, with no
    // DMA copy on either side (allocated on first use, kMappedBytes).
    char* mapped = nullptr;      // host address
    char* mapped_dev = nullptr;  // the same memory's device address
    bool mapped_failed = false;  // allocation refused once: the copy path is used
};

namespace gr {

inline int elem_bytes(int dt) { return dt == GR_DTYPE_F32 ? 4 : (dt == GR_DTYPE_Q8 ? 1 : 2); }

inline bool is_turbo(const gr_run_state* s) { return s->cfg.kv_dtype == GR_DTYPE_TURBO; }
inline bool is_q8(const gr_run_state* s) { return s->cfg.kv_dtype == GR_DTYPE_Q8; }

// Byte offset of cache element `e` in the K/V storage (Turbo codes: 4 per byte).
inline size_t cache_bytes_at(const gr_run_state* s, size_t e) {
    return is_turbo(s) ? e / 4 : e * elem_bytes(s->cfg.kv_dtype);
}

// RAII: make the state's device current for the duration of a call.
struct DeviceScope {
    int prev = -1;
    explicit DeviceScope(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceScope() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Enqueue a host -> device copy on the state's stream.
int h2d(gr_run_state* s, void* dst, const void* src, size_t bytes);
// Device -> host copy on the state's stream, then wait for the stream.
int d2h_sync(gr_run_state* s, void* dst, const void* src, size_t bytes);

}  // namespace gr
