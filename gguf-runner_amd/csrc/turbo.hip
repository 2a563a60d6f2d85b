// Turbo KV cache (KvCacheFormat::Turbo, reference inference.rs:346-1334) on the
// device: the quantising KV write and the merge + value finalisation of the
// split-K decode (the query preparation and the split kernel are in
// turbo_decode.hip).
//
// Per KV head of a row the reference stores (x86 scalar paths):
//   rotated  = S_post H S_pre x              (sign flips, FWHT / sqrt(n); 596-605)
//   sigma    = |rotated| / sqrt(n);  code = 2-bit Lloyd-Max code of rotated/sigma
//   residual = rotated - C[code] sigma;  gamma = |residual|
//   sign bit = (S'_post H S'_pre residual/gamma >= 0)
// and attention reads
//   score = sigma (q_rot . C[code]) + gamma sqrt(pi/2/n) (q_proj . sgn)
//   out   = R^-1 ( sum_t p_t sigma_t C[code_t] + R'^-1 sum_t p_t r_t sgn_t ) / l.
//
// The write keeps the reference's arithmetic order: the wave FWHT adds and
// subtracts in its stage order and the norms are sequential sums in element
// order, so the written codes, signs, sigma and gamma are bit-exact with the
// reference for the same f32 row (no FMA contraction in this file).
#pragma clang fp contract(off)

#include "gr_common.hpp"
#include "gr_internal.hpp"
#include "stream_sched.hpp"
#include "turbo_common.hpp"

namespace gr {

namespace {

__device__ __forceinline__ float tq_centroid(int code) {
    return code == 0 ? -tq::kC1 : code == 1 ? -tq::kC0 : code == 2 ? tq::kC0 : tq::kC1;
}

__device__ __forceinline__ int tq_code(float x) {
    return x < -tq::kTh ? 0 : (x < 0.0f ? 1 : (x < tq::kTh ? 2 : 3));
}

// l2_norm (math.rs:467-473): sequential sum in element order, every lane the same
template <int D>
__device__ __forceinline__ float wave_l2_sequential(const float (&x)[D / 64], float* buf, int lane) {
#pragma unroll
    for (int j = 0; j < D / 64; j++) buf[lane + 64 * j] = x[j];
    __syncthreads();  // one-wave workgroup
    float ss = 0.0f;
    for (int e = 0; e < D; e++) {
        const float v = buf[e];
        ss = ss + v * v;
    }
    __syncthreads();  // buf is reused by the caller
    return sqrtf(ss);
}

}  // namespace

// ---------------------------------------------------------------- KV write

// quantize_turboquant_head (inference.rs:855-925) for one (row, kv head, K|V):
// grid (n_rows, n_kv_heads, 2), one wave.
template <int D>
__global__ __launch_bounds__(64) void turbo_write_kernel(const TurboWriteLaunch p) {
    constexpr int J = D / 64;
    __shared__ float buf[D];
    __shared__ uint8_t codes[D];
    const int lane = threadIdx.x;
    const int i = blockIdx.x, g = blockIdx.y;
    const bool is_v = blockIdx.z != 0;
    const int kv_dim = p.n_kv_heads * D;
    const float* src = (is_v ? p.v_rows : p.k_rows) + (size_t)i * kv_dim + (size_t)g * D;
    const int64_t row = p.cache_row ? (int64_t)p.cache_row[i] : p.row0 + i;
    const int64_t sq = p.cache_seq ? (int64_t)p.cache_seq[i] : 0;
    const int64_t elem = sq * p.cache_seq_stride + row * p.cache_row_stride + (int64_t)g * D;
    uint8_t* base = (is_v ? p.v_base : p.k_base) + elem / 4;
    uint8_t* sign = (is_v ? p.v_sign : p.k_sign) + elem / 8;
    const int64_t aux = sq * p.aux_seq_stride + row * p.aux_row_stride + g;
    float* scale_out = (is_v ? p.v_scale : p.k_scale) + aux;
    float* rnorm_out = (is_v ? p.v_rnorm : p.k_rnorm) + aux;
    const uint8_t* sg = p.signs + (size_t)g * (D / 8);
    const int64_t ss = p.slot_stride;

    float x[J];
#pragma unroll
    for (int j = 0; j < J; j++) x[j] = src[lane + 64 * j];
    tq::wave_transform<D>(x, sg, sg + ss, lane);  // rot_pre, rot_post
    const float sigma = wave_l2_sequential<D>(x, buf, lane) / sqrtf((float)D);
    if (sigma == 0.0f) {
        if (lane == 0) {
            *scale_out = 0.0f;
            *rnorm_out = 0.0f;
        }
        if (lane < D / 4) base[lane] = 0;
        if (lane < D / 8) sign[lane] = 0xff;
        return;
    }
    const float inv_sigma = 1.0f / sigma;
    float r[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int c = tq_code(x[j] * inv_sigma);
        r[j] = x[j] - tq_centroid(c) * sigma;
        codes[lane + 64 * j] = (uint8_t)c;
    }
    const float gamma = wave_l2_sequential<D>(r, buf, lane);  // its barrier also publishes `codes`
    if (lane < D / 4)
        base[lane] = (uint8_t)(codes[4 * lane] | (codes[4 * lane + 1] << 2) | (codes[4 * lane + 2] << 4) |
                               (codes[4 * lane + 3] << 6));
    if (lane == 0) {
        *scale_out = sigma;
        *rnorm_out = gamma;
    }
    if (gamma == 0.0f) {
        if (lane < D / 8) sign[lane] = 0xff;
        return;
    }
#pragma unroll
    for (int j = 0; j < J; j++) r[j] = r[j] / gamma;
    tq::wave_transform<D>(r, sg + 2 * ss, sg + 3 * ss, lane);  // res_pre, res_post
#pragma unroll
    for (int j = 0; j < J; j++) {
        const uint64_t m = __ballot(r[j] >= 0.0f);  // bit l = element 64 j + l
        if (lane == 0) *(uint64_t*)(sign + 8 * j) = m;
    }
}

hipError_t launch_turbo_write(const TurboWriteLaunch& p, hipStream_t st) {
    if (p.n_rows <= 0) return hipSuccess;
    dim3 grid((unsigned)p.n_rows, (unsigned)p.n_kv_heads, 2);
    switch (p.head_dim) {
        case 64: turbo_write_kernel<64><<<grid, 64, 0, st>>>(p); break;
        case 128: turbo_write_kernel<128><<<grid, 64, 0, st>>>(p); break;
        case 256: turbo_write_kernel<256><<<grid, 64, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- merge + finalize

// One wave per (head, sequence): merge the split partials of the base and residual
// accumulators (log2-domain weights), divide by the softmax sum, then
// finalize_turboquant_value_head (inference.rs:1323-1334): residual <- R'^-1
// residual, base += residual, out = R^-1 base.
template <int D>
__global__ __launch_bounds__(256) void turbo_combine_kernel(const DecodeLaunch p) {
    constexpr int J = D / 64, U = 8;
    __shared__ float wsh_all[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* wsh = wsh_all[wave];
    const int h = 4 * blockIdx.x + wave, s = blockIdx.y;  // four heads per workgroup
    if (h >= p.n_heads) return;  // whole wave; only wave-level synchronisation below
    const int kv_mul = p.n_heads / p.n_kv_heads;
    const int g = h / kv_mul;
    const int t_len = p.kv_end[s] - p.kv_start[s];
    int n_used;
    if (p.stream_sched) {  // ranges that meet pair (s, column of h)
        const int n_sub = p.n_sub > 0 ? p.n_sub : 1;
        n_used = stream_partials(p, s, g * n_sub + (n_sub > 1 ? (h % kv_mul) / p.sub_heads : 0));
    } else {
        n_used = t_len > 0 ? (t_len + p.split_keys - 1) / p.split_keys : 0;
    }
    const size_t part0 = ((size_t)s * p.n_heads + h) * p.n_splits;
    float mx = -INFINITY;
    for (int sp = lane; sp < n_used; sp += 64) mx = fmaxf(mx, p.ws_ml[(part0 + sp) * 2]);
    mx = wave_max<64>(mx);
    float lt = 0.0f;
    float b[J], r[J];
#pragma unroll
    for (int j = 0; j < J; j++) b[j] = r[j] = 0.0f;
    for (int c0 = 0; c0 < n_used; c0 += 64) {
        const int nc = min(64, n_used - c0);
        // lane i: the weight of split c0 + i
        float w = 0.0f;
        if (lane < nc) {
            const size_t pt = part0 + c0 + lane;
            w = exp2f(p.ws_ml[pt * 2] - mx);
            lt += p.ws_ml[pt * 2 + 1] * w;
        }
        wsh[lane] = w;
        tq::wave_lds_sync();  // the wave's weights visible to all its lanes
        const float* o = p.ws_o + (part0 + c0) * 2 * D;
        int i = 0;
        for (; i + U <= nc; i += U) {  // U partials' loads in flight together
            float ob[U][J], orr[U][J];
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int j = 0; j < J; j++) {
                    ob[u][j] = o[(i + u) * 2 * D + lane + 64 * j];
                    orr[u][j] = o[(i + u) * 2 * D + D + lane + 64 * j];
                }
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int j = 0; j < J; j++) {
                    b[j] += ob[u][j] * wsh[i + u];
                    r[j] += orr[u][j] * wsh[i + u];
                }
        }
        for (; i < nc; i++)
#pragma unroll
            for (int j = 0; j < J; j++) {
                b[j] += o[i * 2 * D + lane + 64 * j] * wsh[i];
                r[j] += o[i * 2 * D + D + lane + 64 * j] * wsh[i];
            }
        tq::wave_lds_sync();  // wsh reads done before the next chunk's stores
    }
    lt = wave_sum<64>(lt);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        b[j] *= inv;
        r[j] *= inv;
    }
    const uint8_t* sg = p.turbo_signs + (size_t)g * (D / 8);
    const int64_t ss = p.turbo_slot_stride;
    tq::wave_transform<D>(r, sg + 3 * ss, sg + 2 * ss, lane);  // res_post, res_pre: inverse
#pragma unroll
    for (int j = 0; j < J; j++) b[j] += r[j];
    tq::wave_transform<D>(b, sg + ss, sg, lane);  // rot_post, rot_pre: inverse
    float* out = p.out + ((size_t)s * p.n_heads + h) * D;
    const float* gt = p.gate.at(s, h);  // Qwen3.5 output gate, or null
#pragma unroll
    for (int j = 0; j < J; j++) out[lane + 64 * j] = gt ? gate_mul(b[j], gt[lane + 64 * j]) : b[j];
}

hipError_t launch_turbo_combine(const DecodeLaunch& p, hipStream_t st) {
    const dim3 grid((p.n_heads + 3) / 4, p.n_seq);
    switch (p.head_dim) {
        case 64: turbo_combine_kernel<64><<<grid, 256, 0, st>>>(p); break;
        case 128: turbo_combine_kernel<128><<<grid, 256, 0, st>>>(p); break;
        case 256: turbo_combine_kernel<256><<<grid, 256, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gr
