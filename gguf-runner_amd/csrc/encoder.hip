// Encoder self-attention (encoder_self_attention, reference
// src/engine/multimodal/mod.rs:145-256): f32 Q/K/V rows [token][heads * d] of
// n_seq sequences of `tokens` tokens each; every token attends to all tokens of
// its own sequence (no cache, no mask), scores scaled by 1/sqrt(d).
//
// fp32 throughout (the reference's f32 dot / axpy / exp).  VALU kernel (sequences
// under 64 tokens; the f32 MFMA kernel below takes longer ones): one lane per query,
// 256 queries of one (sequence, head) per workgroup.  Key / value rows go
// through LDS in tiles of 32 and every lane reads the same row (broadcast, no
// bank conflicts).  Per tile: 32 scores in registers, the tile maximum raises
// the running maximum (O and the sum rescaled), then P = 2^(s - m) and
// O += P V.  Head dims up to 128 here, up to 256 on the MFMA kernel; a dim that
// is not one of the compiled sizes runs zero-padded in the next one (zeros add
// nothing to dots or outputs).
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

// ---------------------------------------------------------------- f32 MFMA path
//
// Sequences of kEmMinTokens or more run on v_mfma_f32_32x32x2_f32: f32 operands,
// f32 products and sums (no 16-bit rounding anywhere).  Workgroup = 4 waves x 32
// queries of one (sequence, head); keys in tiles of 64 (two 32-key sub-tiles),
// K row-major and V transposed in LDS, zero beyond the head dim.  Per sub-tile
//   S^T = K . Q^T   k-step s: lane half lg carries dim lg * DP/2 + s, so a lane
//                   reads its K operands for 4 k-steps with one ds_read_b128;
//   O^T += V^T . P^T  k-step t pairs key 8 (t/4) + 4 lg + t%4 with lane half lg,
//                   which is exactly accumulator element t of S^T: the B operand
//                   is the lane's own P value, and the A operand (V^T row d,
//                   4 consecutive keys) one ds_read_b128 per 4 k-steps.
// Online softmax per query (lanes l and l ^ 32) with the lazy rescale.

typedef float em_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kEmThreads = 256;
constexpr int kEmBM = 128;         // queries per workgroup
constexpr int kEmBN = 64;          // keys per tile (32 for head dims above 128)
constexpr int kEmMinTokens = 64;   // shorter sequences take the VALU kernel
constexpr float kEmLazy = 8.0f;    // log2 units

__device__ __forceinline__ float em_xmax32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float em_xsum32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Head dims above 128 (DP 192, 256): one wave per SIMD and 32-key tiles (Q
// operands, O and the tile staging then fit the 512 registers of a lone wave).
template <int DP>
__global__ __launch_bounds__(kEmThreads, (DP <= 128 ? 2 : 1)) void encoder_mfma_kernel(const EncoderLaunch p) {
    constexpr int BN = DP <= 128 ? kEmBN : 32;
    constexpr int KS = DP / 2;           // k-steps over the head dim
    constexpr int DT = (DP + 31) / 32;   // O^T tiles of 32 dims
    constexpr int DP32 = DT * 32;
    constexpr int KST = DP + 4;          // K tile row stride (floats)
    constexpr int VST = BN + 4;          // V^T tile row stride (floats)
    static_assert(KS % 4 == 0, "head dims in multiples of 8");
    __shared__ __attribute__((aligned(16))) float Kt[BN * KST];
    __shared__ __attribute__((aligned(16))) float Vt[DP32 * VST];

    const int d = p.head_dim;
    const int dim = p.heads * d;
    const int h = blockIdx.y;
    const size_t seq0 = (size_t)blockIdx.z * p.tokens;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 31, lg = lane >> 5;
    const int qi = (int)blockIdx.x * kEmBM + wave * 32 + ln;
    const bool q_ok = qi < p.tokens;
    const float qscale = kLog2e / sqrtf((float)d);  // scores in log2 units

    float qv[KS];  // B operand of k-step s: dim lg * KS + s of this lane's query
    {
        const float* qr = p.q + (seq0 + (q_ok ? qi : p.tokens - 1)) * dim + (size_t)h * d;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const int i = lg * KS + s;
            qv[s] = i < d ? qr[i] * qscale : 0.0f;
        }
    }
    em_f32x16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[dt][e] = 0.0f;
    float mrow = -1e30f, lrow = 0.0f;

    // Tile staging: thread tid holds the 4-dim groups tid + 256 u (row c / (DP32/4),
    // dims 4 (c % (DP32/4)) .. +3) of K and V; the next tile's loads are in flight
    // while the current one is computed.  Rows past the sequence and dims past d
    // are zero.  float4 loads when the rows are 16-byte aligned (d % 4 == 0).
    constexpr int G4 = DP32 / 4;
    constexpr int NV4 = BN * G4 / kEmThreads;
    static_assert(BN * G4 % kEmThreads == 0, "tile staging");
    const bool vec = (d & 3) == 0;
    float4 kst[NV4], vst[NV4];
    auto load_tile = [&](int t0) {
        const int nk = min(BN, p.tokens - t0);
#pragma unroll
        for (int u = 0; u < NV4; u++) {
            const int c = tid + kEmThreads * u;
            const int r = c / G4, i = 4 * (c % G4);
            const bool rok = r < nk;
            const size_t src = (seq0 + t0 + (rok ? r : 0)) * dim + (size_t)h * d;
            if (vec) {
                const bool ok = rok && i < d;
                kst[u] = ok ? *(const float4*)(p.k + src + i) : make_float4(0.f, 0.f, 0.f, 0.f);
                vst[u] = ok ? *(const float4*)(p.v + src + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float kx[4], vx[4];
#pragma unroll
                for (int x = 0; x < 4; x++) {
                    const bool ok = rok && i + x < d;
                    kx[x] = ok ? p.k[src + i + x] : 0.0f;
                    vx[x] = ok ? p.v[src + i + x] : 0.0f;
                }
                kst[u] = make_float4(kx[0], kx[1], kx[2], kx[3]);
                vst[u] = make_float4(vx[0], vx[1], vx[2], vx[3]);
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int u = 0; u < NV4; u++) {
            const int c = tid + kEmThreads * u;
            const int r = c / G4, i = 4 * (c % G4);
            if (i < DP) *(float4*)(Kt + r * KST + i) = kst[u];
            Vt[(i + 0) * VST + r] = vst[u].x;
            Vt[(i + 1) * VST + r] = vst[u].y;
            Vt[(i + 2) * VST + r] = vst[u].z;
            Vt[(i + 3) * VST + r] = vst[u].w;
        }
    };

    load_tile(0);
    for (int t0 = 0; t0 < p.tokens; t0 += BN) {
        const int nk = min(BN, p.tokens - t0);
        __syncthreads();  // the previous tile is consumed
        store_tile();
        __syncthreads();
        if (t0 + BN < p.tokens) load_tile(t0 + BN);
#pragma unroll
        for (int sb = 0; sb < BN / 32; sb++) {
            const int ts = 32 * sb;  // first key of the sub-tile within the tile
            if (ts >= nk) break;
            em_f32x16 acc;
#pragma unroll
            for (int e = 0; e < 16; e++) acc[e] = 0.0f;
            const float* krow = Kt + (ts + ln) * KST + lg * KS;
#pragma unroll
            for (int j = 0; j < KS / 4; j++) {
                const float4 kx = *(const float4*)(krow + 4 * j);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kx.x, qv[4 * j + 0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kx.y, qv[4 * j + 1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kx.z, qv[4 * j + 2], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kx.w, qv[4 * j + 3], acc, 0, 0, 0);
            }
            // element e is key ts + 8 (e / 4) + 4 lg + e % 4 of the tile
            if (ts + 32 > nk) {
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (ts + 8 * (e >> 2) + 4 * lg + (e & 3) >= nk) acc[e] = -INFINITY;
            }
            float mx = acc[0];
#pragma unroll
            for (int e = 1; e < 16; e++) mx = fmaxf(mx, acc[e]);
            mx = em_xmax32(mx);
            if (__any(mx > mrow + kEmLazy)) {
                const float mnew = fmaxf(mrow, mx);
                const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
                mrow = mnew;
                lrow *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) o[dt] *= alpha;
            }
            float pv[16];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                pv[e] = __builtin_amdgcn_exp2f(acc[e] - mrow);
                lrow += pv[e];
            }
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const float* vrow = Vt + (32 * dt + ln) * VST + ts + 4 * lg;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float4 vx = *(const float4*)(vrow + 8 * j);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vx.x, pv[4 * j + 0], o[dt], 0, 0, 0);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vx.y, pv[4 * j + 1], o[dt], 0, 0, 0);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vx.z, pv[4 * j + 2], o[dt], 0, 0, 0);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vx.w, pv[4 * j + 3], o[dt], 0, 0, 0);
                }
            }
        }
    }
    const float lsum = em_xsum32(lrow);
    if (!q_ok) return;
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float* orow = p.out + (seq0 + qi) * dim + (size_t)h * d;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int i = 32 * dt + 8 * (e >> 2) + 4 * lg + (e & 3);
            if (i < d) orow[i] = o[dt][e] * inv;
        }
}

template <int DP>
static hipError_t launch_encoder_dp(const EncoderLaunch& p, hipStream_t st) {
    // head dims above 128 take the MFMA kernel at every length (the VALU kernel's
    // per-lane query and output rows would not fit its registers); it masks the keys
    // past a short sequence's end and skips its query rows
    if constexpr (DP <= 128) {
        if (p.tokens < kEmMinTokens) {
            dim3 grid((p.tokens + kEncThreads - 1) / kEncThreads, p.heads, p.n_seq);
            encoder_attention_kernel<DP><<<grid, kEncThreads, 0, st>>>(p);
            return hipGetLastError();
        }
    }
    dim3 grid((p.tokens + kEmBM - 1) / kEmBM, p.heads, p.n_seq);
    encoder_mfma_kernel<DP><<<grid, kEmThreads, 0, st>>>(p);
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
    if (d <= 192) return launch_encoder_dp<192>(p, st);
    if (d <= 256) return launch_encoder_dp<256>(p, st);
    return hipErrorInvalidValue;
}

}  // namespace gr
