// Per-token Q/K/V preparation on the device (one workgroup per token):
//   qkv_bias_and_norm's QK RMSNorm  (reference inference.rs:2535-2572 -> math.rs:164-184)
//   apply_rope_qk                   (inference.rs:1817-1874; angle as rebuild_rope_cache 1485-1523)
//   Gemma3 q *= 1/sqrt(head_dim)    (inference.rs:1871-1873)
//   kv_write_token, raw storage     (inference.rs:1877-1965: the row goes to the cache)
// Q rows are written to a staging buffer (f32 for decode, or 16-bit already
// multiplied by the softmax scale * log2(e) for the MFMA prefill kernel), or
// skipped, with each token's RoPE (cos, sin) pairs written out instead for a
// consumer that prepares Q itself.
#include <algorithm>

#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

constexpr int kPrepThreads = 256;
constexpr int kPrepRowsPerBlock = kPrepThreads / 64;

// 8 consecutive elements (one 16-byte chunk of a 16-bit row, two of an f32 row).
__device__ __forceinline__ void load8(const void* base, size_t idx, int dt, float* v) {
    if (dt == GR_DTYPE_F32) {
        const float4 a = *(const float4*)((const float*)base + idx);
        const float4 b = *(const float4*)((const float*)base + idx + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
        return;
    }
    const uint4 u = *(const uint4*)((const uint16_t*)base + idx);
    if (dt == GR_DTYPE_F16) unpack16<F16>(u, v);
    else unpack16<BF16>(u, v);
}

__device__ __forceinline__ void store8(void* base, size_t idx, int dt, const float* v) {
    if (dt == GR_DTYPE_F32) {
        *(float4*)((float*)base + idx) = make_float4(v[0], v[1], v[2], v[3]);
        *(float4*)((float*)base + idx + 4) = make_float4(v[4], v[5], v[6], v[7]);
        return;
    }
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint16_t lo = dt == GR_DTYPE_F16 ? f32_to_f16(v[2 * k]) : f32_to_bf16(v[2 * k]);
        const uint16_t hi = dt == GR_DTYPE_F16 ? f32_to_f16(v[2 * k + 1]) : f32_to_bf16(v[2 * k + 1]);
        w[k] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *(uint4*)((uint16_t*)base + idx) = make_uint4(w[0], w[1], w[2], w[3]);
}

// T tokens per workgroup of four waves (T = 1: the four waves share a
// token's rows; T = 4, long prefill chunks: a wave per token, a quarter of the
// workgroups).  The token's RoPE cos/sin (rope_dim/2 values, the
// rebuild_rope_cache angle (pos*freq)*scale) are computed once into LDS; then
// each lane owns 8 consecutive elements of a head row, LPR = D/8 lanes cover a
// row and a wave processes 64/LPR rows at once: Q heads, K heads, V heads.
template <int D, int T>
__global__ __launch_bounds__(kPrepThreads) void qkv_prep_kernel(const QkvPrepLaunch p) {
    constexpr int LPR = D / 8;        // lanes per row
    constexpr int RPW = 64 / LPR;     // rows per wave step
    constexpr int WPT = kPrepRowsPerBlock / T;  // waves per token
    static_assert(T >= 1 && kPrepRowsPerBlock % T == 0, "tokens per workgroup");
    __shared__ float row_buf[kPrepRowsPerBlock][RPW][D];
    __shared__ __attribute__((aligned(16))) float cs_all[T][D / 2], sn_all[T][D / 2];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tsub = wave / WPT, wt = wave % WPT;  // token of the wave, wave within the token
    const int rsub = lane / LPR;      // row of this lane within the wave step
    const int c8 = (lane % LPR) * 8;  // first element owned by this lane
    const int i_raw = (int)blockIdx.x * T + tsub;
    const bool tok_ok = i_raw < p.n_tokens;
    const int i = tok_ok ? i_raw : p.n_tokens - 1;
    float* cs_t = cs_all[tsub];
    float* sn_t = sn_all[tsub];
    if (p.n_copy > 0 && blockIdx.x == 0 && blockIdx.y == 0)
        for (int t = threadIdx.x; t < p.n_copy; t += kPrepThreads) p.copy_dst[t] = p.copy_src[t];
    const int rows_per_token = p.n_heads + 2 * p.n_kv_heads;
    const int64_t pos = p.pos ? (int64_t)p.pos[i] : p.pos0 + i;
    const bool rope = p.rope_mode != GR_ROPE_NONE;
    const int half = p.rope_dim / 2;
    if (rope) {
        for (int f = wt * 64 + lane; f < half; f += WPT * 64) {
            const float val = ((float)pos * p.rope_freqs[f]) * p.rope_scale;
            float sn, cs;
            sincosf(val, &sn, &cs);
            cs_t[f] = cs;
            sn_t[f] = sn;
            if (p.rope_cs_out && tok_ok && blockIdx.y == 0)
                *(float2*)(p.rope_cs_out + ((size_t)i * half + f) * 2) = make_float2(cs, sn);
        }
    }
    __syncthreads();
    if (!tok_ok) return;  // no workgroup barrier below
    float* rb = row_buf[wave][rsub];
    const int64_t row = p.cache_by_index ? (int64_t)i : (p.cache_row ? (int64_t)p.cache_row[i] : pos);
    const int64_t sq = p.cache_by_index ? 0 : (p.cache_seq ? (int64_t)p.cache_seq[i] : 0);

    // Without a Q staging buffer the Q rows are left to the consumer (the MFMA
    // prefill kernel prepares them itself from rope_cs_out).
    // workgroup y of gridDim.y takes every gridDim.y-th group of WPT * RPW rows
    const int row0 = p.q_out ? 0 : p.n_heads;
    for (int hr0 = row0 + ((int)blockIdx.y * WPT + wt) * RPW; hr0 < rows_per_token;
         hr0 += (int)gridDim.y * WPT * RPW) {
        const int hr = hr0 + rsub;
        const bool valid = hr < rows_per_token;
        const int hrc = valid ? hr : rows_per_token - 1;
        const int kind = hrc < p.n_heads ? 0 : (hrc < p.n_heads + p.n_kv_heads ? 1 : 2);  // q, k, v
        const int head = kind == 0 ? hrc : (kind == 1 ? hrc - p.n_heads : hrc - p.n_heads - p.n_kv_heads);
        const bool skip = !valid || (kind == 0 && p.q_out == nullptr);
        const void* src = kind == 0 ? p.q : (kind == 1 ? p.k : p.v);
        const int64_t rs = kind == 0 ? p.q_row_stride : p.kv_row_stride;
        float x[8];
        if (!skip) load8(src, (size_t)i * rs + (size_t)head * D + c8, p.in_dtype, x);
        else
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = 0.0f;
        // Qwen2 attention biases, before the norm (qkv_bias_and_norm, inference.rs:2545-2559)
        const float* bias = kind == 0 ? p.q_bias : (kind == 1 ? p.k_bias : p.v_bias);
        if (bias && !skip) {
            float bv[8];
            load8(bias, (size_t)head * D + c8, GR_DTYPE_F32, bv);
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] += bv[e];
        }
        if (kind != 2) {
            // QK RMSNorm: ss = sum(x^2)/d + eps; x = w * ((1/sqrt(ss)) * x).
            const float* w = kind == 0 ? p.q_norm : p.k_norm;
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) ss += x[e] * x[e];
            ss = wave_sum<LPR>(ss);  // lanes of other rows never mix: groups are LPR-aligned
            if (w) {
                const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
                float wv[8];
                load8(w, c8, GR_DTYPE_F32, wv);
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = wv[e] * (inv * x[e]);
            }
            if (rope) {
                if (p.rope_mode == GR_ROPE_ADJACENT) {
                    // pairs (2j, 2j+1) sit inside the lane's 8 elements
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        const int fi = (c8 + e) >> 1;
                        const float cs = cs_t[fi], sn = sn_t[fi];
                        const float v0 = x[e], v1 = x[e + 1];
                        x[e] = v0 * cs - v1 * sn;
                        x[e + 1] = v0 * sn + v1 * cs;
                    }
                } else if (p.rope_dim == D) {
                    // NeoX pairs (i, i + D/2) of a fully rotated row: the partner
                    // elements of this lane's 8 are the 8 of lane ^ (LPR/2), in the
                    // same row's lane group
                    const bool first = c8 < half;
                    const int f0 = first ? c8 : c8 - half;
                    float csv[8], snv[8];
                    *(float4*)csv = *(const float4*)(cs_t + f0);
                    *(float4*)(csv + 4) = *(const float4*)(cs_t + f0 + 4);
                    *(float4*)snv = *(const float4*)(sn_t + f0);
                    *(float4*)(snv + 4) = *(const float4*)(sn_t + f0 + 4);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float other = __shfl_xor(x[e], LPR / 2, 64);
                        // (v0, v1) -> (v0*c - v1*s, v0*s + v1*c)
                        x[e] = first ? x[e] * csv[e] - other * snv[e] : other * snv[e] + x[e] * csv[e];
                    }
                } else {
                    // NeoX pairs (i, i + rope_dim/2) of a partial rotation live in
                    // other lanes: stage the row
#pragma unroll
                    for (int e = 0; e < 8; e++) rb[c8 + e] = x[e];
                    __builtin_amdgcn_wave_barrier();
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const int idx = c8 + e;
                        if (idx >= p.rope_dim) continue;  // partial RoPE: tail untouched
                        const bool first = idx < half;
                        const int fi = first ? idx : idx - half;
                        const float other = rb[first ? idx + half : idx - half];
                        const float cs = cs_t[fi], sn = sn_t[fi];
                        // (v0, v1) -> (v0*c - v1*s, v0*s + v1*c)
                        x[e] = first ? x[e] * cs - other * sn : other * sn + x[e] * cs;
                    }
                    __builtin_amdgcn_wave_barrier();  // reads done before the next rows' stores
                }
            }
            if (kind == 0 && p.gemma_q_scale) {
                const float sc = 1.0f / sqrtf((float)D);
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] *= sc;
            }
        }
        if (skip) continue;
        if (kind == 0) {
            const size_t ob = ((size_t)i * p.n_heads + head) * D + c8;
            float xs[8];
#pragma unroll
            for (int e = 0; e < 8; e++) xs[e] = x[e] * p.q_out_scale;
            if (p.q_out_lo) {
                // bf16 hi + lo pair of the MFMA operand (the hi rounding kept in
                // registers for the residual)
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    hw[w] = pack_bf16x2(xs[2 * w], xs[2 * w + 1]);
                    lw[w] = pack_bf16x2(xs[2 * w] - __uint_as_float(hw[w] << 16),
                                        xs[2 * w + 1] - __uint_as_float(hw[w] & 0xffff0000u));
                }
                *(uint4*)((uint16_t*)p.q_out + ob) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                *(uint4*)((uint16_t*)p.q_out_lo + ob) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            } else {
                store8(p.q_out, ob, p.q_out_dtype, xs);
            }
        } else {
            void* dst = kind == 1 ? p.k_cache : p.v_cache;
            const size_t ob = (size_t)sq * p.cache_seq_stride + (size_t)row * p.cache_row_stride +
                              (size_t)head * D + c8;
            if (p.k_f16) {
                // bf16 cache row plus its exact f16 copy for the f16 MFMA prefill
                uint32_t wb[4], wh[4];
                bool bad = false;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint16_t b0 = f32_to_bf16(x[2 * k]), b1 = f32_to_bf16(x[2 * k + 1]);
                    bad = bad || bf16_outside_f16(b0) || bf16_outside_f16(b1);
                    wb[k] = (uint32_t)b0 | ((uint32_t)b1 << 16);
                    wh[k] = (uint32_t)f32_to_f16(bf16_to_f32(b0)) | ((uint32_t)f32_to_f16(bf16_to_f32(b1)) << 16);
                }
                *(uint4*)((uint16_t*)dst + ob) = make_uint4(wb[0], wb[1], wb[2], wb[3]);
                uint16_t* cp = (uint16_t*)(kind == 1 ? p.k_f16 : p.v_f16);
                *(uint4*)(cp + (size_t)(row - p.f16_row0) * p.f16_row_stride + (size_t)head * D + c8) =
                    make_uint4(wh[0], wh[1], wh[2], wh[3]);
                if (bad) *p.f16_flag = p.f16_epoch;
            } else {
                store8(dst, ob, p.cache_dtype, x);
            }
        }
    }
}

// Existing bf16 cache rows (the history of a prefill chunk) to their f16 copy:
// 8 elements per thread, K then V.
__global__ __launch_bounds__(256) void bf16_rows_to_f16_kernel(const Bf16CopyLaunch p) {
    const int64_t per = (int64_t)p.n_rows * (p.kv_dim / 8);
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= 2 * per) return;
    const bool is_v = idx >= per;
    const int64_t j = is_v ? idx - per : idx;
    const int64_t r = j / (p.kv_dim / 8);
    const int c8 = (int)(j - r * (p.kv_dim / 8)) * 8;
    const uint16_t* src = (is_v ? p.v_cache : p.k_cache) + (p.row0 + r) * p.cache_row_stride + c8;
    uint16_t* dst = (is_v ? p.v_f16 : p.k_f16) + r * p.kv_dim + c8;
    const uint4 u = *(const uint4*)src;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    uint32_t h[4];
    bool bad = false;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint16_t b0 = (uint16_t)(w[k] & 0xffffu), b1 = (uint16_t)(w[k] >> 16);
        bad = bad || bf16_outside_f16(b0) || bf16_outside_f16(b1);
        h[k] = (uint32_t)f32_to_f16(bf16_to_f32(b0)) | ((uint32_t)f32_to_f16(bf16_to_f32(b1)) << 16);
    }
    *(uint4*)dst = make_uint4(h[0], h[1], h[2], h[3]);
    if (bad) *p.f16_flag = p.f16_epoch;
}

hipError_t launch_bf16_rows_to_f16(const Bf16CopyLaunch& p, hipStream_t st) {
    if (p.n_rows <= 0) return hipSuccess;
    const int64_t threads = 2 * p.n_rows * (p.kv_dim / 8);
    bf16_rows_to_f16_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, st>>>(p);
    return hipGetLastError();
}

// Long chunks (at least kPrepWaveTokens tokens): a wave per token, a quarter of
// the workgroups (MI355X: 8192 tokens, 32 / 8 heads, d128: 23.5 -> 18.7 us;
// Gemma-3-4B-shaped d256 layers -1.5%; 2048 tokens unchanged).
constexpr int kPrepWaveTokens = 1024;

template <int T>
static hipError_t launch_qkv_prep_t(const QkvPrepLaunch& p, hipStream_t st) {
    // A few tokens (decode, short chunks): the rows of a token spread over
    // workgroups of one row step per wave each, so every wave issues its loads
    // once (the inputs may sit in host memory, a PCIe round trip per step).
    int ygroups = 1;
    if (T == 1 && p.n_tokens <= 64) {
        const int rows = p.n_heads + 2 * p.n_kv_heads - (p.q_out ? 0 : p.n_heads);
        const int per_wg = kPrepRowsPerBlock * (64 / (p.head_dim / 8));  // waves x rows per wave step
        ygroups = std::max(1, (rows + per_wg - 1) / per_wg);
    }
    const dim3 blocks((unsigned)((p.n_tokens + T - 1) / T), (unsigned)ygroups);
    switch (p.head_dim) {
        case 64: qkv_prep_kernel<64, T><<<blocks, kPrepThreads, 0, st>>>(p); break;
        case 128: qkv_prep_kernel<128, T><<<blocks, kPrepThreads, 0, st>>>(p); break;
        case 256: qkv_prep_kernel<256, T><<<blocks, kPrepThreads, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_qkv_prep(const QkvPrepLaunch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    return p.n_tokens >= kPrepWaveTokens ? launch_qkv_prep_t<kPrepRowsPerBlock>(p, st) : launch_qkv_prep_t<1>(p, st);
}

}  // namespace gr
