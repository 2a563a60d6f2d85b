// The Qwen3.5 / Qwen3-Next SSM layer around the gated-DeltaNet recurrence
// (reference qwen3next_linear_attention_projected_state, math.rs:766-953) for a
// chunk of T tokens:
//   ssm_pre_kernel   causal depthwise conv1d over [history, qkv] + SiLU
//                    (800-817), periodic K -> V head tiling (826), the beta /
//                    log-decay gates from the fused or split projections (853-874)
//   (deltanet)       L2 norms fused in the recurrence kernels (833-846)
//   ssm_post_kernel  gated RMSNorm with SiLU(z) (478-488, 936-950)
//   ssm_hist_kernel  the conv history after the chunk (819-825)
// Every conv output depends only on the K raw inputs before it, so the pre pass
// is parallel over (token, channel); only the recurrence is sequential.
#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

namespace {

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float silu_ref(float x) { return x * sigmoid_ref(x); }
__device__ __forceinline__ float softplus_ref(float x) {
    return x > 20.0f ? x : (x < -20.0f ? expf(x) : logf(1.0f + expf(x)));
}

constexpr int kSsmThreads = 256;

// grid (T, ceil((conv_dim + n_v) / 256)): thread j < conv_dim is conv channel j,
// the next n_v threads are the gates of value head j - conv_dim.
__global__ __launch_bounds__(kSsmThreads) void ssm_pre_kernel(const SsmLaunch p) {
    const int t = blockIdx.x;
    const int j = blockIdx.y * kSsmThreads + threadIdx.x;
    const int d = p.head_dim, nk = p.n_k_heads, nv = p.n_v_heads, K = p.conv_kernel;
    const int conv_dim = (nv + 2 * nk) * d;
    if (j < conv_dim) {
        const float* w = p.conv_w + (size_t)j * K;
        float acc = p.qkv[(size_t)t * conv_dim + j] * w[K - 1];
        for (int r = 0; r < K - 1; r++) {
            const int u = t - (K - 1) + r;  // token of history row r
            const float x = u >= 0 ? p.qkv[(size_t)u * conv_dim + j] : p.conv_hist[(size_t)(K - 1 + u) * conv_dim + j];
            acc += x * w[r];
        }
        if (!is_finite_f(acc)) acc = 0.0f;
        const float y = silu_ref(acc);
        if (j < 2 * nk * d) {
            const bool is_k = j >= nk * d;
            const int kh = (is_k ? j - nk * d : j) / d, i = j % d;
            float* dst = is_k ? p.k_out : p.q_out;
            for (int h = kh; h < nv; h += nk) dst[((size_t)t * nv + h) * d + i] = y;  // periodic tiling
        } else {
            const int c = j - 2 * nk * d;
            p.v_out[(size_t)t * nv * d + c] = finite_or_zero(y);
        }
    } else if (j < conv_dim + nv) {
        const int h = j - conv_dim;
        float b, a;
        if (p.gate_b == nullptr) {  // fused [b | a] per key-head group
            const int hpg = nv / nk, grp = h / hpg, idx = h % hpg, base = grp * 2 * hpg;
            b = p.gate_a[(size_t)t * 2 * nv + base + idx];
            a = p.gate_a[(size_t)t * 2 * nv + base + hpg + idx];
        } else {
            b = p.gate_b[(size_t)t * nv + h];
            a = p.gate_a[(size_t)t * nv + h];
        }
        float gate = softplus_ref(a + p.dt_bias[h]) * p.ssm_a[h];
        if (!is_finite_f(gate)) gate = 0.0f;
        p.beta_out[(size_t)t * nv + h] = finite_or_zero(sigmoid_ref(b));
        p.gate_out[(size_t)t * nv + h] = gate;  // log decay: g = exp(gate)
    }
}

// New history after the chunk: row r (oldest first) = raw input T - (K-1) + r,
// or an older history row when the chunk is shorter than K - 1.
__global__ __launch_bounds__(kSsmThreads) void ssm_hist_kernel(const SsmLaunch p) {
    const int c = blockIdx.x * kSsmThreads + threadIdx.x;
    const int conv_dim = (p.n_v_heads + 2 * p.n_k_heads) * p.head_dim;
    const int H = p.conv_kernel - 1;
    if (c >= conv_dim || H <= 0) return;
    float nv[8];
    for (int r = 0; r < H; r++) {
        const int u = p.n_tokens - H + r;
        nv[r] = u >= 0 ? p.qkv[(size_t)u * conv_dim + c] : p.conv_hist[(size_t)(H + u) * conv_dim + c];
    }
    for (int r = 0; r < H; r++) p.conv_hist[(size_t)r * conv_dim + c] = nv[r];
}

// grid (T, n_v), one wave: gated RMSNorm of one head row.
template <int D>
__global__ __launch_bounds__(64) void ssm_post_kernel(const SsmLaunch p) {
    constexpr int J = D / 64;
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const size_t row = ((size_t)t * p.n_v_heads + h) * D;
    float o[J], ss = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        o[j] = p.o[row + lane + 64 * j];
        ss += o[j] * o[j];
    }
    ss = wave_sum<64>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int i = lane + 64 * j;
        p.out[row + i] = finite_or_zero(p.ssm_norm[i] * (o[j] * inv) * silu_ref(p.z[row + i]));
    }
}

}  // namespace

hipError_t launch_ssm_pre(const SsmLaunch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    const int conv_dim = (p.n_v_heads + 2 * p.n_k_heads) * p.head_dim;
    ssm_pre_kernel<<<dim3(p.n_tokens, (conv_dim + p.n_v_heads + kSsmThreads - 1) / kSsmThreads), kSsmThreads, 0,
                     st>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.conv_kernel <= 1) return e;
    ssm_hist_kernel<<<(conv_dim + kSsmThreads - 1) / kSsmThreads, kSsmThreads, 0, st>>>(p);
    return hipGetLastError();
}

hipError_t launch_ssm_post(const SsmLaunch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    dim3 grid(p.n_tokens, p.n_v_heads);
    switch (p.head_dim) {
        case 64: ssm_post_kernel<64><<<grid, 64, 0, st>>>(p); break;
        case 128: ssm_post_kernel<128><<<grid, 64, 0, st>>>(p); break;
        case 256: ssm_post_kernel<256><<<grid, 64, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gr
