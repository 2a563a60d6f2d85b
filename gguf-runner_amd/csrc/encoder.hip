// Encoder self-attention (encoder_self_attention, reference
// src/engine/multimodal/mod.rs:145-256): f32 Q/K/V rows [token][heads * d] of
// n_seq sequences of `tokens` tokens each; every token attends to all tokens of
// its own sequence (no cache, no mask), scores scaled by 1/sqrt(d).
//
// f32 results (the reference's f32 dot / axpy / exp).  VALU kernel (sequences
// under 64 tokens; the MFMA kernels below take longer ones): one lane per query,
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
// Sequences of kEmMinTokens or more with head dims above 128 run on
// v_mfma_f32_32x32x2_f32: f32 operands, f32 products and sums.  Workgroup = 4 waves x 32
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

// ---------------------------------------------------------------- bf16-piece MFMA path
//
// Head dims up to 128: the same tiling on v_mfma_f32_32x32x16_bf16 with every f32
// operand cut into three exact bf16 pieces (x = hi + mid + lo, each the
// round-to-nearest bf16 of what the pieces before it leave: |mid| <= 2^-8 |x|,
// |lo| <= 2^-16 |x|, and lo holds the rest exactly) and each product taken as the
// six piece products hi hi, hi mid, mid hi, hi lo, mid mid, lo hi (the three
// dropped ones add at most ~2^-23 of |x y|, the size of the f32 rounding of the
// sum): products of bf16 values are exact and the MFMA sums them in fp32.  Six bf16 MFMAs of 16 dims cost 3/8 of the f32 MFMA time for the same
// dims (bf16 runs 16 x the f32 matrix rate on this part).  K and V tiles sit in
// LDS as pieces, row-major [key][dim]; the V^T operand comes from transposing
// reads (ds_read_b64_tr_b16); Q is cut once per query row, P once per sub-tile.

typedef __bf16 em_b8 __attribute__((ext_vector_type(8)));
typedef short em_s4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ em_f32x16 em_mma(const uint4& a, const uint4& b, const em_f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(em_b8, a), __builtin_bit_cast(em_b8, b), c, 0,
                                                   0, 0);
}
// the six piece products of A (pieces a[0..2]) and B (b[0..2]), largest first
__device__ __forceinline__ em_f32x16 em_mma6(const uint4* a, const uint4* b, em_f32x16 c) {
    c = em_mma(a[0], b[0], c);
    c = em_mma(a[0], b[1], c);
    c = em_mma(a[1], b[0], c);
    c = em_mma(a[0], b[2], c);
    c = em_mma(a[1], b[1], c);
    c = em_mma(a[2], b[0], c);
    return c;
}
typedef __bf16 em_b2 __attribute__((ext_vector_type(2)));
typedef float em_f2 __attribute__((ext_vector_type(2)));
// two floats as a word of two round-to-nearest bf16 (v_cvt_pk_bf16_f32), and back
__device__ __forceinline__ uint32_t em_bf2(em_f2 v) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, em_b2));
}
__device__ __forceinline__ em_f2 em_unbf2(uint32_t w) {
    return em_f2{__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
}
// pieces of 2 n floats as n words each (two bf16 per word, element 2 i low)
template <int N>
__device__ __forceinline__ void em_split_words(const float* x, uint32_t* hi, uint32_t* mid, uint32_t* lo) {
#pragma unroll
    for (int i = 0; i < N; i++) {
        const em_f2 v = {x[2 * i], x[2 * i + 1]};
        hi[i] = em_bf2(v);
        const em_f2 r1 = v - em_unbf2(hi[i]);  // exact
        mid[i] = em_bf2(r1);
        lo[i] = em_bf2(r1 - em_unbf2(mid[i]));  // exact (at most 8 significant bits left)
    }
}

template <int DP>
__global__ __launch_bounds__(kEmThreads, 2) void encoder_bf3_kernel(const EncoderLaunch p) {
    static_assert(DP <= 128, "one-wave-per-SIMD head dims stay on the f32 kernel");
    constexpr int BN = kEmBN;
    constexpr int DP16 = (DP + 15) / 16 * 16;   // S^T k-steps of 16 dims
    constexpr int KS = DP16 / 16;
    constexpr int DT = (DP + 31) / 32;          // O^T tiles of 32 dims
    constexpr int DP32 = DT * 32;
    // Piece row strides (bf16): K rows are read 16 bytes at a time by 16 lanes at
    // 16 consecutive keys (a stride of 4 mod 8 dwords puts them on distinct
    // banks); V rows by transposing reads of 4 keys x 64 bytes (a stride of 16
    // or 48 mod 64 dwords puts the 4 keys on distinct banks).
    constexpr int KRS = 2 * ((DP32 / 2 + 3) / 8 * 8 + 4);
    constexpr int VRS = 2 * (DP32 / 2 <= 16 ? 16 : DP32 / 2 <= 48 ? 48 : DP32 / 2 <= 80 ? 80 : 112);
    constexpr int KPB = BN * KRS, VPB = BN * VRS;  // one piece of a tile (bf16 elements)
    __shared__ __attribute__((aligned(16))) uint16_t Kp[3 * KPB];
    __shared__ __attribute__((aligned(16))) uint16_t Vp[3 * VPB];

    const int d = p.head_dim;
    const int dim = p.heads * d;
    const int h = blockIdx.y;
    const size_t seq0 = (size_t)blockIdx.z * p.tokens;
    const int tid = threadIdx.x, lane = tid & 63;
    const int ln = lane & 31, lg = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qi = (int)blockIdx.x * kEmBM + wave * 32 + ln;
    const bool q_ok = qi < p.tokens;
    const float qscale = kLog2e / sqrtf((float)d);  // scores in log2 units

    // Q^T B operand of k-step s: dims 16 s + 8 lg .. + 7 of this lane's query, as pieces
    uint4 qp[KS][3];
    {
        const float* qr = p.q + (seq0 + (q_ok ? qi : p.tokens - 1)) * dim + (size_t)h * d;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = 16 * s + 8 * lg + j;
                x[j] = i < d ? qr[i] * qscale : 0.0f;
            }
            uint32_t hw[4], mw[4], lw[4];
            em_split_words<4>(x, hw, mw, lw);
            qp[s][0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            qp[s][1] = make_uint4(mw[0], mw[1], mw[2], mw[3]);
            qp[s][2] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        }
    }
    em_f32x16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[dt][e] = 0.0f;
    float mrow = -1e30f, lrow = 0.0f;

    // Tile staging as the f32 kernel: thread tid holds the 4-dim groups tid + 256 u
    // (row c / (DP32/4), dims 4 (c % (DP32/4)) .. +3) of K and V, zero past the
    // sequence and past d; stored as pieces.
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
            const float kx[4] = {kst[u].x, kst[u].y, kst[u].z, kst[u].w};
            const float vx[4] = {vst[u].x, vst[u].y, vst[u].z, vst[u].w};
            uint32_t kh[2], km[2], kl[2], vh[2], vm[2], vl[2];
            em_split_words<2>(kx, kh, km, kl);
            em_split_words<2>(vx, vh, vm, vl);
            const int ko = r * KRS + i;
            *(uint2*)(Kp + ko) = make_uint2(kh[0], kh[1]);
            *(uint2*)(Kp + KPB + ko) = make_uint2(km[0], km[1]);
            *(uint2*)(Kp + 2 * KPB + ko) = make_uint2(kl[0], kl[1]);
            const int vo = r * VRS + i;
            *(uint2*)(Vp + vo) = make_uint2(vh[0], vh[1]);
            *(uint2*)(Vp + VPB + vo) = make_uint2(vm[0], vm[1]);
            *(uint2*)(Vp + 2 * VPB + vo) = make_uint2(vl[0], vl[1]);
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
            // S^T = K Q^T: A = key ts + ln, dims 16 s + 8 lg .. + 7
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const int off = (ts + ln) * KRS + 16 * s + 8 * lg;
                const uint4 ka[3] = {*(const uint4*)(Kp + off), *(const uint4*)(Kp + KPB + off),
                                     *(const uint4*)(Kp + 2 * KPB + off)};
                acc = em_mma6(ka, qp[s], acc);
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
            // P^T B operand of k-step t: slot j of lane half lg <-> key
            // 16 t + 8 (j / 4) + 4 lg + j % 4, which is accumulator element 8 t + j
#pragma unroll
            for (int t = 0; t < 2; t++) {
                uint32_t hw[4], mw[4], lw[4];
                em_split_words<4>(pv + 8 * t, hw, mw, lw);
                const uint4 pp[3] = {make_uint4(hw[0], hw[1], hw[2], hw[3]), make_uint4(mw[0], mw[1], mw[2], mw[3]),
                                     make_uint4(lw[0], lw[1], lw[2], lw[3])};
                // V^T A operand (dims 32 dt + 0..31, the same key slots): two
                // transposing reads per piece; lane i of 16-lane group G supplies key
                // k0 + i / 4, dims d0 + 4 (i % 4) .. + 3 and receives dim d0 + i of
                // keys k0 .. k0 + 3 (d0 = 32 dt + 16 (G % 2), k0 = ts + 16 t + 4 lg (+ 8))
                const int gi = lane & 15;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    uint4 va[3];
#pragma unroll
                    for (int pc = 0; pc < 3; pc++) {
                        em_s4 part[2];
#pragma unroll
                        for (int b = 0; b < 2; b++) {
                            const int key = ts + 16 * t + 8 * b + 4 * lg + (gi >> 2);
                            const int dd = 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (gi & 3);
                            part[b] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                (__attribute__((address_space(3))) em_s4*)(Vp + pc * VPB + key * VRS + dd));
                        }
                        const uint2 lo2 = __builtin_bit_cast(uint2, part[0]);
                        const uint2 hi2 = __builtin_bit_cast(uint2, part[1]);
                        va[pc] = make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
                    }
                    o[dt] = em_mma6(va, pp, o[dt]);
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
    if constexpr (DP <= 128)
        encoder_bf3_kernel<DP><<<grid, kEmThreads, 0, st>>>(p);
    else
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
