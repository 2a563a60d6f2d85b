// Encoder self-attention (encoder_self_attention, reference
// src/engine/multimodal/mod.rs:145-256): f32 Q/K/V rows [token][heads * d] of
// n_seq sequences of `tokens` tokens each; every token attends to all tokens of
// its own sequence (no cache, no mask), scores scaled by 1/sqrt(d).
//
// fp32 throughout (the reference's f32 dot / axpy / exp): one lane per query,
// 256 queries of one (sequence, head) per workgroup.  Key / value rows go
// through LDS in tiles of 32 and every lane reads the same row (broadcast, no
// bank conflicts).  Per tile: 32 scores in registers, the tile maximum raises
// the running maximum (O and the sum rescaled), then P = 2^(s - m) and
// O += P V.  Head dims up to 128; a dim that is not one of the compiled sizes
// runs zero-padded in the next one (zeros add nothing to dots or outputs).
#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

constexpr int kEncThreads = 256;
constexpr int kEncKeys = 32;

template <int DP>
__global__ __launch_bounds__(kEncThreads, 1) void encoder_attention_kernel(const EncoderLaunch p) {
    __shared__ __attribute__((aligned(16))) float Ks[kEncKeys][DP];
    __shared__ __attribute__((aligned(16))) float Vs[kEncKeys][DP];
    const int d = p.head_dim;
    const int dim = p.heads * d;
    const int h = blockIdx.y;
    const int s = blockIdx.z;
    const int tid = threadIdx.x;
    const int qi = blockIdx.x * kEncThreads + tid;  // query token within the sequence
    const bool q_ok = qi < p.tokens;
    const size_t seq0 = (size_t)s * p.tokens;
    const float qscale = kLog2e / sqrtf((float)d);  // scores in log2 units

    float q[DP], o[DP];
    {
        const float* qr = p.q + (seq0 + (q_ok ? qi : 0)) * dim + (size_t)h * d;
#pragma unroll
        for (int i = 0; i < DP; i++) {
            q[i] = i < d ? qr[i] * qscale : 0.0f;
            o[i] = 0.0f;
        }
    }
    float mrow = -INFINITY, lrow = 0.0f;

    for (int t0 = 0; t0 < p.tokens; t0 += kEncKeys) {
        const int nk = min(kEncKeys, p.tokens - t0);
        __syncthreads();  // the previous tile is consumed
        for (int e = tid; e < kEncKeys * DP; e += kEncThreads) {
            const int r = e / DP, c = e % DP;
            const bool ok = r < nk && c < d;
            const size_t src = (seq0 + t0 + (ok ? r : 0)) * dim + (size_t)h * d + (ok ? c : 0);
            Ks[r][c] = ok ? p.k[src] : 0.0f;
            Vs[r][c] = ok ? p.v[src] : 0.0f;
        }
        __syncthreads();
        float sc[kEncKeys];
        float tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < kEncKeys; j++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < DP; i += 4) {
                const float4 kv = *(const float4*)&Ks[j][i];
                acc = fmaf(q[i], kv.x, acc);
                acc = fmaf(q[i + 1], kv.y, acc);
                acc = fmaf(q[i + 2], kv.z, acc);
                acc = fmaf(q[i + 3], kv.w, acc);
            }
            sc[j] = j < nk ? acc : -INFINITY;
            tmax = fmaxf(tmax, sc[j]);
        }
        if (tmax > mrow) {
            const float alpha = __builtin_amdgcn_exp2f(mrow - tmax);  // 0 on the first tile
            lrow *= alpha;
#pragma unroll
            for (int i = 0; i < DP; i++) o[i] *= alpha;
            mrow = tmax;
        }
#pragma unroll
        for (int j = 0; j < kEncKeys; j++) {
            const float pj = __builtin_amdgcn_exp2f(sc[j] - mrow);
            lrow += pj;
#pragma unroll
            for (int i = 0; i < DP; i += 4) {
                const float4 vv = *(const float4*)&Vs[j][i];
                o[i] = fmaf(pj, vv.x, o[i]);
                o[i + 1] = fmaf(pj, vv.y, o[i + 1]);
                o[i + 2] = fmaf(pj, vv.z, o[i + 2]);
                o[i + 3] = fmaf(pj, vv.w, o[i + 3]);
            }
        }
    }
    if (!q_ok) return;
    const float inv = lrow > 0.0f ? 1.0f / lrow : 0.0f;
    float* orow = p.out + (seq0 + qi) * dim + (size_t)h * d;
#pragma unroll
    for (int i = 0; i < DP; i++)
        if (i < d) orow[i] = o[i] * inv;
}

template <int DP>
static hipError_t launch_encoder_dp(const EncoderLaunch& p, hipStream_t st) {
    dim3 grid((p.tokens + kEncThreads - 1) / kEncThreads, p.heads, p.n_seq);
    encoder_attention_kernel<DP><<<grid, kEncThreads, 0, st>>>(p);
    return hipGetLastError();
}

hipError_t launch_encoder_attention(const EncoderLaunch& p, hipStream_t st) {
    const int d = p.head_dim;
    if (d <= 32) return launch_encoder_dp<32>(p, st);
    if (d <= 64) return launch_encoder_dp<64>(p, st);
    if (d <= 72) return launch_encoder_dp<72>(p, st);
    if (d <= 80) return launch_encoder_dp<80>(p, st);
    if (d <= 96) return launch_encoder_dp<96>(p, st);
    if (d <= 128) return launch_encoder_dp<128>(p, st);
    return hipErrorInvalidValue;
}

}  // namespace gr
