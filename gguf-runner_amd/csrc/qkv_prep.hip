// Per-token Q/K/V preparation on the device, one wavefront per head row:
//   qkv_bias_and_norm's QK RMSNorm  (reference inference.rs:2535-2572 -> math.rs:164-184)
//   apply_rope_qk                   (inference.rs:1817-1874; angle as rebuild_rope_cache 1485-1523)
//   Gemma3 q *= 1/sqrt(head_dim)    (inference.rs:1871-1873)
//   kv_write_token, raw storage     (inference.rs:1877-1965: the row goes to the cache)
// Q rows are written to a staging buffer (f32 for decode, or 16-bit already
// multiplied by the softmax scale * log2(e) for the MFMA prefill kernel).
#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

constexpr int kPrepThreads = 256;
constexpr int kPrepRowsPerBlock = kPrepThreads / 64;

__device__ __forceinline__ float load_elem(const void* base, size_t idx, int dt) {
    if (dt == GR_DTYPE_F32) return ((const float*)base)[idx];
    const uint16_t b = ((const uint16_t*)base)[idx];
    return dt == GR_DTYPE_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

__device__ __forceinline__ void store_elem(void* base, size_t idx, int dt, float v) {
    if (dt == GR_DTYPE_F32)
        ((float*)base)[idx] = v;
    else
        ((uint16_t*)base)[idx] = dt == GR_DTYPE_F16 ? f32_to_f16(v) : f32_to_bf16(v);
}

// Row r of the launch: token i = r / rows_per_token, then Q heads, K heads, V heads.
template <int D>
__global__ __launch_bounds__(kPrepThreads) void qkv_prep_kernel(const QkvPrepLaunch p) {
    constexpr int EPL = D / 64;  // elements per lane
    __shared__ float row_buf[kPrepRowsPerBlock][D];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rows_per_token = p.n_heads + 2 * p.n_kv_heads;
    const long total = (long)p.n_tokens * rows_per_token;
    const long r = (long)blockIdx.x * kPrepRowsPerBlock + wave;
    const bool active = r < total;
    const long rr = active ? r : 0;
    const int i = (int)(rr / rows_per_token);
    const int hr = (int)(rr % rows_per_token);
    const int kind = hr < p.n_heads ? 0 : (hr < p.n_heads + p.n_kv_heads ? 1 : 2);  // q, k, v
    const int head = kind == 0 ? hr : (kind == 1 ? hr - p.n_heads : hr - p.n_heads - p.n_kv_heads);
    const bool skip_q = (kind == 0 && p.q_out == nullptr);

    float x[EPL];
    const void* src = kind == 0 ? p.q : (kind == 1 ? p.k : p.v);
    const int64_t rs = kind == 0 ? p.q_row_stride : p.kv_row_stride;
    const size_t base = (size_t)i * rs + (size_t)head * D;
#pragma unroll
    for (int e = 0; e < EPL; e++) x[e] = active && !skip_q ? load_elem(src, base + lane + 64 * e, p.in_dtype) : 0.0f;

    const int64_t pos = p.pos ? (int64_t)p.pos[i] : p.pos0 + i;

    if (kind != 2) {
        // QK RMSNorm: ss = sum(x^2)/d + eps; x = w * ((1/sqrt(ss)) * x).
        const float* w = kind == 0 ? p.q_norm : p.k_norm;
        if (w) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; e++) ss += x[e] * x[e];
            ss = wave_sum<64>(ss);
            ss = ss / (float)D + p.eps;
            const float inv = 1.0f / sqrtf(ss);
#pragma unroll
            for (int e = 0; e < EPL; e++) x[e] = w[lane + 64 * e] * (inv * x[e]);
        }
    }
    // Stage the row so that RoPE can pair elements held by other lanes.
#pragma unroll
    for (int e = 0; e < EPL; e++) row_buf[wave][lane + 64 * e] = x[e];
    __syncthreads();
    if (kind != 2 && p.rope_mode != GR_ROPE_NONE) {
        const int half = p.rope_dim / 2;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            const int idx = lane + 64 * e;
            int fi, partner;
            bool first;
            if (p.rope_mode == GR_ROPE_NEOX) {
                if (idx >= p.rope_dim) continue;  // partial RoPE: tail untouched
                first = idx < half;
                fi = first ? idx : idx - half;
                partner = first ? idx + half : idx - half;
            } else {
                first = (idx & 1) == 0;
                fi = idx >> 1;
                partner = idx ^ 1;
            }
            const float val = ((float)pos * p.rope_freqs[fi]) * p.rope_scale;
            float sn, cs;
            sincosf(val, &sn, &cs);
            const float mine = row_buf[wave][idx];
            const float other = row_buf[wave][partner];
            // (v0, v1) -> (v0*c - v1*s, v0*s + v1*c)
            x[e] = first ? mine * cs - other * sn : other * sn + mine * cs;
        }
    }
    if (kind == 0 && p.gemma_q_scale) {
        const float sc = 1.0f / sqrtf((float)D);
#pragma unroll
        for (int e = 0; e < EPL; e++) x[e] *= sc;
    }
    if (!active || skip_q) return;
    if (kind == 0) {
        const size_t ob = ((size_t)i * p.n_heads + head) * D;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            const float xs = x[e] * p.q_out_scale;
            store_elem(p.q_out, ob + lane + 64 * e, p.q_out_dtype, xs);
            if (p.q_out_lo) {
                const float hi = load_elem(p.q_out, ob + lane + 64 * e, p.q_out_dtype);
                store_elem(p.q_out_lo, ob + lane + 64 * e, p.q_out_dtype, xs - hi);
            }
        }
    } else {
        const int64_t row = p.cache_row ? (int64_t)p.cache_row[i] : pos;
        const int64_t sq = p.cache_seq ? (int64_t)p.cache_seq[i] : 0;
        void* dst = kind == 1 ? p.k_cache : p.v_cache;
        const size_t ob = (size_t)sq * p.cache_seq_stride + (size_t)row * p.cache_row_stride +
                          (size_t)head * D;
#pragma unroll
        for (int e = 0; e < EPL; e++) store_elem(dst, ob + lane + 64 * e, p.cache_dtype, x[e]);
    }
}

hipError_t launch_qkv_prep(const QkvPrepLaunch& p, hipStream_t st) {
    const long rows = (long)p.n_tokens * (p.n_heads + 2 * p.n_kv_heads);
    const unsigned blocks = (unsigned)((rows + kPrepRowsPerBlock - 1) / kPrepRowsPerBlock);
    if (blocks == 0) return hipSuccess;
    switch (p.head_dim) {
        case 64: qkv_prep_kernel<64><<<blocks, kPrepThreads, 0, st>>>(p); break;
        case 128: qkv_prep_kernel<128><<<blocks, kPrepThreads, 0, st>>>(p); break;
        case 256: qkv_prep_kernel<256><<<blocks, kPrepThreads, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gr
