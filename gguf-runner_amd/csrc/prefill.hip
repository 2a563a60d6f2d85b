// Causal / sliding-window flash prefill on gfx950 MFMA (f16 or bf16 inputs,
// fp32 accumulation).  Replaces the token-serial attention of the prefill loop
// (reference inference.rs:2981-3017, one attention_token per token) with one
// launch per chunk: every query row sees keys [start(pos), pos] of the device KV
// cache, start = 0 for global layers and pos + 1 - W for window W
// (LanguageAttentionPolicy::visible_keys, attention.rs:74-96).
//
// Block = 4 waves = 128 query rows of one query head; KV tiles of 64 keys are
// staged in LDS (K row-major, V transposed).  Each wave computes
//   S^T = K . Q^T   (v_mfma_f32_32x32x16: A = K rows from LDS, B = Q from VGPRs)
//   O^T += V^T . P^T (A = V^T from LDS, B = P straight from the S^T accumulators)
// so both accumulators hold one query per lane column and the online-softmax
// statistics of a row live in the two lanes (l, l^32) that own it.
// Q arrives prepared: RoPE'd / normed and multiplied by softmax_scale*log2(e).
#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename DT>
struct Mfma32;
template <>
struct Mfma32<F16> {
    static __device__ __forceinline__ f32x16 mma(const uint4& a, const uint4& b, const f32x16& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a),
                                                      __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        return (uint32_t)f32_to_f16(lo) | ((uint32_t)f32_to_f16(hi) << 16);
    }
    static constexpr bool kSplit = false;
};
// bf16 keeps only 8 mantissa bits: Q and P are carried as hi + lo bf16 pairs
// (two MFMAs per product; K and V are exact bf16 values of the cache), which
// brings the products to ~1e-5 of an fp32 evaluation.
template <>
struct Mfma32<BF16> {
    static constexpr bool kSplit = true;
    static __device__ __forceinline__ f32x16 mma(const uint4& a, const uint4& b, const f32x16& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
    }
};

constexpr int kPfThreads = 256;
constexpr int kPfBM = 128;  // query rows per block (32 per wave)
constexpr int kPfBN = 64;   // keys per LDS tile

template <typename DT, int D>
__global__ __launch_bounds__(kPfThreads) void prefill_kernel(const PrefillLaunch p) {
    constexpr int BM = kPfBM, BN = kPfBN;
    constexpr int KS = D + 8;   // K tile row stride (elements)
    constexpr int VS = BN + 8;  // V^T tile row stride (elements)
    constexpr int DC = D / 8;   // 16-byte chunks per row
    constexpr int KCH = BN * DC / kPfThreads;        // K chunks per thread
    constexpr int VT = (BN / 4) * DC / kPfThreads;   // V 4-key tasks per thread
    static_assert(KCH >= 1 && VT >= 1, "tile too small for the block");
    using M = Mfma32<DT>;

    __shared__ __attribute__((aligned(16))) uint16_t Ks[BN * KS];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 31, lg = lane >> 5;
    const int h = blockIdx.x;
    const int qb = gridDim.y - 1 - blockIdx.y;  // heaviest causal blocks first
    const int kv_mul = p.n_heads / p.n_kv_heads;
    const int g = h / kv_mul;
    const int m = p.n_tokens;
    const int64_t P0 = p.base_pos;
    const int W = p.window;

    const int q0 = qb * BM;
    const int wr0 = q0 + wave * 32;
    const int my_row = wr0 + ln;
    const bool row_ok = my_row < m;
    const int my_row_c = row_ok ? my_row : m - 1;
    const int64_t my_pos = P0 + my_row_c;
    const bool wave_active = wr0 < m;
    const int64_t wpos_min = P0 + (wave_active ? wr0 : m - 1);
    const int64_t wpos_max = P0 + min(wr0 + 31, m - 1);

    // Q fragments (B operand): lane (query ln, group lg) holds d = 16 s + 8 lg .. +7.
    constexpr bool kSplit = M::kSplit;
    uint4 qf[D / 16];
    uint4 qfl[kSplit ? D / 16 : 1];
    {
        const size_t qoff = ((size_t)my_row_c * p.n_heads + h) * D + 8 * lg;
        const uint16_t* qrow = (const uint16_t*)p.q + qoff;
#pragma unroll
        for (int s = 0; s < D / 16; s++) qf[s] = *(const uint4*)(qrow + 16 * s);
        if constexpr (kSplit) {
            const uint16_t* qrl = (const uint16_t*)p.q_lo + qoff;
#pragma unroll
            for (int s = 0; s < D / 16; s++) qfl[s] = *(const uint4*)(qrl + 16 * s);
        }
    }

    const int last_row = min(q0 + BM, m) - 1;
    const int64_t kend = P0 + last_row + 1;  // keys [0, kend) exist in the cache
    int64_t kbeg = 0;
    if (W > 0) {
        kbeg = P0 + q0 + 1 - W;
        if (kbeg < 0) kbeg = 0;
    }
    const int64_t t_first = kbeg / BN * BN;
    const int n_tiles = (int)((kend - t_first + BN - 1) / BN);

    const uint16_t* kc = (const uint16_t*)p.k_cache + (size_t)g * D;
    const uint16_t* vc = (const uint16_t*)p.v_cache + (size_t)g * D;
    const int64_t rs = p.cache_row_stride;

    uint4 kreg[KCH];
    uint4 vreg[VT][4];
    auto load_tile = [&](int64_t t0) {
#pragma unroll
        for (int u = 0; u < KCH; u++) {
            const int c = tid + kPfThreads * u;
            int64_t key = t0 + c / DC;
            if (key >= kend) key = kend - 1;
            kreg[u] = *(const uint4*)(kc + key * rs + (c % DC) * 8);
        }
#pragma unroll
        for (int u = 0; u < VT; u++) {
            const int c = tid + kPfThreads * u;
            const int kg = c / DC, dc = c % DC;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int64_t key = t0 + 4 * kg + r;
                if (key >= kend) key = kend - 1;
                vreg[u][r] = *(const uint4*)(vc + key * rs + dc * 8);
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int u = 0; u < KCH; u++) {
            const int c = tid + kPfThreads * u;
            *(uint4*)(Ks + (c / DC) * KS + (c % DC) * 8) = kreg[u];
        }
#pragma unroll
        for (int u = 0; u < VT; u++) {
            const int c = tid + kPfThreads * u;
            const int kg = c / DC, dc = c % DC;
            const uint32_t w[4][4] = {{vreg[u][0].x, vreg[u][0].y, vreg[u][0].z, vreg[u][0].w},
                                      {vreg[u][1].x, vreg[u][1].y, vreg[u][1].z, vreg[u][1].w},
                                      {vreg[u][2].x, vreg[u][2].y, vreg[u][2].z, vreg[u][2].w},
                                      {vreg[u][3].x, vreg[u][3].y, vreg[u][3].z, vreg[u][3].w}};
#pragma unroll
            for (int dd = 0; dd < 8; dd++) {
                const int wi = dd >> 1;
                uint32_t lo, hi;
                if ((dd & 1) == 0) {
                    lo = (w[0][wi] & 0xffffu) | (w[1][wi] << 16);
                    hi = (w[2][wi] & 0xffffu) | (w[3][wi] << 16);
                } else {
                    lo = (w[0][wi] >> 16) | (w[1][wi] & 0xffff0000u);
                    hi = (w[2][wi] >> 16) | (w[3][wi] & 0xffff0000u);
                }
                *(uint2*)(Vt + (dc * 8 + dd) * VS + 4 * kg) = make_uint2(lo, hi);
            }
        }
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
        for (int j = 0; j < 16; j++) o[dt][j] = 0.0f;
    float mrow = -1e30f;  // finite start: alpha = exp2(m_old - m_new) never sees inf - inf
    float lrow = 0.0f;    // this lane's share of the row sum

    if (n_tiles > 0) load_tile(t_first);
    for (int it = 0; it < n_tiles; it++) {
        const int64_t t0 = t_first + (int64_t)it * BN;
        __syncthreads();
        store_tile();
        __syncthreads();
        if (it + 1 < n_tiles) load_tile(t0 + BN);

        if (!wave_active || t0 > wpos_max) continue;
        if (W > 0 && t0 + BN - 1 < wpos_min + 1 - W) continue;
        const bool need_mask = (t0 + BN - 1 > wpos_min) || (W > 0 && t0 < wpos_max + 1 - W);

        f32x16 sacc[2];
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
#pragma unroll
            for (int j = 0; j < 16; j++) sacc[sb][j] = 0.0f;
            const uint16_t* krow = Ks + (32 * sb + ln) * KS + 8 * lg;
#pragma unroll
            for (int s = 0; s < D / 16; s++) {
                const uint4 a = *(const uint4*)(krow + 16 * s);
                sacc[sb] = M::mma(a, qf[s], sacc[sb]);
                if constexpr (kSplit) sacc[sb] = M::mma(a, qfl[s], sacc[sb]);
            }
        }
        // S^T register j of sub-tile sb holds key t0 + 32 sb + 8 (j/4) + 4 lg + j%4.
        float mx = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int j = 0; j < 16; j++) {
                float sv = sacc[sb][j];
                if (need_mask) {
                    const int64_t key = t0 + 32 * sb + 8 * (j >> 2) + 4 * lg + (j & 3);
                    const bool vis = key <= my_pos && (W <= 0 || key > my_pos - W);
                    sv = vis ? sv : -INFINITY;
                    sacc[sb][j] = sv;
                }
                mx = fmaxf(mx, sv);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(mrow, mx);
        const float alpha = exp2f(mrow - mnew);
        mrow = mnew;
        float psum = 0.0f;
        uint4 pf[2][2];
        uint4 pfl[kSplit ? 2 : 1][2];
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            float pv[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                pv[j] = exp2f(sacc[sb][j] - mnew);
                psum += pv[j];
            }
#pragma unroll
            for (int t = 0; t < 2; t++) {
                pf[sb][t].x = M::pack2(pv[8 * t + 0], pv[8 * t + 1]);
                pf[sb][t].y = M::pack2(pv[8 * t + 2], pv[8 * t + 3]);
                pf[sb][t].z = M::pack2(pv[8 * t + 4], pv[8 * t + 5]);
                pf[sb][t].w = M::pack2(pv[8 * t + 6], pv[8 * t + 7]);
            }
            if constexpr (kSplit) {
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t hw[4] = {pf[sb][t].x, pf[sb][t].y, pf[sb][t].z, pf[sb][t].w};
                    uint32_t lw[4];
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        const float r0 = pv[8 * t + 2 * w] - __uint_as_float(hw[w] << 16);
                        const float r1 = pv[8 * t + 2 * w + 1] - __uint_as_float(hw[w] & 0xffff0000u);
                        lw[w] = M::pack2(r0, r1);
                    }
                    pfl[sb][t] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
                }
            }
        }
        lrow = lrow * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
#pragma unroll
            for (int j = 0; j < 16; j++) o[dt][j] *= alpha;
            const uint16_t* vrow = Vt + (32 * dt + ln) * VS + 4 * lg;
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const int kb = 32 * sb + 16 * t;
                    const uint2 lo = *(const uint2*)(vrow + kb);
                    const uint2 hi = *(const uint2*)(vrow + kb + 8);
                    const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    o[dt] = M::mma(a, pf[sb][t], o[dt]);
                    if constexpr (kSplit) o[dt] = M::mma(a, pfl[sb][t], o[dt]);
                }
        }
    }

    const float lsum = lrow + __shfl_xor(lrow, 32, 64);
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    if (!row_ok) return;
    float* orow = p.out + ((size_t)my_row * p.n_heads + h) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
            const int d0 = 32 * dt + 8 * jb + 4 * lg;
            float4 v;
            v.x = o[dt][4 * jb + 0] * inv;
            v.y = o[dt][4 * jb + 1] * inv;
            v.z = o[dt][4 * jb + 2] * inv;
            v.w = o[dt][4 * jb + 3] * inv;
            *(float4*)(orow + d0) = v;
        }
}

template <typename DT>
static hipError_t launch_prefill_dt(const PrefillLaunch& p, hipStream_t st) {
    const int n_qb = (p.n_tokens + kPfBM - 1) / kPfBM;
    dim3 grid(p.n_heads, n_qb);
    switch (p.head_dim) {
        case 128: prefill_kernel<DT, 128><<<grid, kPfThreads, 0, st>>>(p); break;
        case 256: prefill_kernel<DT, 256><<<grid, kPfThreads, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillLaunch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    switch (p.dtype) {
        case GR_DTYPE_F16: return launch_prefill_dt<F16>(p, st);
        case GR_DTYPE_BF16: return launch_prefill_dt<BF16>(p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace gr
