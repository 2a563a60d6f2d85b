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
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
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
    // one v_cvt_pk_f16_f32 (round to nearest even)
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, half2_t));
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

// Raw buffer access: wave-uniform base in a scalar descriptor, 32-bit byte
// offsets per lane (gfx9-family descriptor word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pf_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)0xffffffff, 0x00020000);
}
__device__ __forceinline__ uint4 pf_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

constexpr int kPfThreads = 256;
constexpr int kPfBM = 128;  // query rows per query block (32 per wave)
constexpr int kPfBN = 64;   // keys per LDS tile

// Softmax reference maxima are only raised when a row's tile maximum exceeds
// them by more than this (log2 units): until then P = 2^(s - m_ref) <= 2^8 and
// the accumulators need no rescale.  The final O / l is exact either way.
constexpr float kLazyRescale = 8.0f;

template <typename DT, int D>
// Two workgroups per CU (8 waves): keeps each wave within 256 registers, so the
// MFMA accumulators stay in VGPRs next to the softmax.
__global__ __launch_bounds__(kPfThreads, 2) void prefill_kernel(const PrefillLaunch p) {
    constexpr int BM = kPfBM, BN = kPfBN;
    constexpr int KS = D + 8;   // K tile row stride (elements)
    constexpr int VS = BN + 8;  // V^T tile row stride (elements)
    constexpr int DC = D / 8;   // 16-byte chunks per row
    constexpr int KCH = BN * DC / kPfThreads;        // K chunks per thread
    constexpr int VT = (BN / 4) * DC / kPfThreads;   // V 4-key tasks per thread
    static_assert(KCH >= 1 && VT >= 1, "tile too small for the block");
    using M = Mfma32<DT>;
    constexpr bool kSplit = M::kSplit;

    // double-buffered K (row-major) and V^T tiles
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BN * KS];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[2][D * VS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 31, lg = lane >> 5;
    const int h = blockIdx.x;
    const int kv_mul = p.n_heads / p.n_kv_heads;
    const int g = h / kv_mul;
    const int m = p.n_tokens;
    const int P0 = (int)p.base_pos;
    const int W = p.window;
    const int n_qb = (m + BM - 1) / BM;
    const uint16_t* kc = (const uint16_t*)p.k_cache + (size_t)g * D;
    const uint16_t* vc = (const uint16_t*)p.v_cache + (size_t)g * D;
    const int64_t rs = p.cache_row_stride;

    // Each workgroup takes query blocks n_qb-1-j and j: causal work per workgroup
    // is then nearly constant.
    const int j = blockIdx.y;
    for (int pass = 0; pass < 2; pass++) {
        const int qblk = pass == 0 ? n_qb - 1 - j : j;
        if (pass == 1 && qblk >= n_qb - 1 - j) break;

        const int q0 = qblk * BM;
        const int wr0 = q0 + wave * 32;
        const int my_row = wr0 + ln;
        const bool row_ok = my_row < m;
        const int my_row_c = row_ok ? my_row : m - 1;
        const int my_pos = P0 + my_row_c;
        const bool wave_active = wr0 < m;
        const int wpos_min = P0 + (wave_active ? wr0 : m - 1);
        const int wpos_max = P0 + min(wr0 + 31, m - 1);

        // Q fragments (B operand): lane (query ln, group lg) holds d = 16 s + 8 lg .. +7.
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

        const int kend = P0 + min(q0 + BM, m);  // keys [0, kend) exist in the cache
        const int kbeg = W > 0 ? max(0, P0 + q0 + 1 - W) : 0;
        const int t_first = kbeg / BN * BN;
        const int n_tiles = (kend - t_first + BN - 1) / BN;

        uint4 kreg[KCH];
        uint4 vreg[VT][4];
        // Tiles that end inside the cache load through a descriptor at the tile's
        // first row plus per-thread byte offsets fixed for the whole loop; only
        // the last tile clamps its rows to kend - 1.
        auto load_tile = [&](int t0) {
            if (!kSplit && t0 + BN <= kend) {
                const __amdgpu_buffer_rsrc_t kr = pf_rsrc(kc + (int64_t)t0 * rs);
                const __amdgpu_buffer_rsrc_t vr = pf_rsrc(vc + (int64_t)t0 * rs);
                const int rsb = (int)rs * 2;
                // chunk c = tid + 256 u: row c / DC = tid / DC + u (256 / DC), column c % DC = tid % DC
                const int koff = (tid / DC) * rsb + (tid % DC) * 16;
                const int voff = 4 * (tid / DC) * rsb + (tid % DC) * 16;
#pragma unroll
                for (int u = 0; u < KCH; u++) kreg[u] = pf_load16(kr, koff, u * (kPfThreads / DC) * rsb);
#pragma unroll
                for (int u = 0; u < VT; u++)
#pragma unroll
                    for (int r = 0; r < 4; r++) vreg[u][r] = pf_load16(vr, voff, (4 * u * (kPfThreads / DC) + r) * rsb);
                return;
            }
            if (kSplit && t0 + BN <= kend) {  // bf16: plain strided addresses (fewer registers live)
                const uint16_t* kt = kc + (int64_t)t0 * rs;
                const uint16_t* vtp = vc + (int64_t)t0 * rs;
#pragma unroll
                for (int u = 0; u < KCH; u++) {
                    const int c = tid + kPfThreads * u;
                    kreg[u] = *(const uint4*)(kt + (c / DC) * rs + (c % DC) * 8);
                }
#pragma unroll
                for (int u = 0; u < VT; u++) {
                    const int c = tid + kPfThreads * u;
                    const int kg = c / DC, dc = c % DC;
                    const uint16_t* vr0 = vtp + (4 * kg) * rs + dc * 8;
#pragma unroll
                    for (int r = 0; r < 4; r++) vreg[u][r] = *(const uint4*)(vr0 + r * rs);
                }
                return;
            }
#pragma unroll
            for (int u = 0; u < KCH; u++) {
                const int c = tid + kPfThreads * u;
                const int key = min(t0 + c / DC, kend - 1);
                kreg[u] = *(const uint4*)(kc + (int64_t)key * rs + (c % DC) * 8);
            }
#pragma unroll
            for (int u = 0; u < VT; u++) {
                const int c = tid + kPfThreads * u;
                const int kg = c / DC, dc = c % DC;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = min(t0 + 4 * kg + r, kend - 1);
                    vreg[u][r] = *(const uint4*)(vc + (int64_t)key * rs + dc * 8);
                }
            }
        };
        auto store_tile = [&](int buf) {
#pragma unroll
            for (int u = 0; u < KCH; u++) {
                const int c = tid + kPfThreads * u;
                *(uint4*)(&Ks[buf][(c / DC) * KS + (c % DC) * 8]) = kreg[u];
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
                    *(uint2*)(&Vt[buf][(dc * 8 + dd) * VS + 4 * kg]) = make_uint2(lo, hi);
                }
            }
        };
        f32x16 o[D / 32];
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
            for (int e = 0; e < 16; e++) o[dt][e] = 0.0f;
        float mrow = -1e30f;  // reference maximum of this lane's row (finite start)
        float lrow = 0.0f;    // this lane's share of the row sum

        // S^T for the 32-key sub-tile sb of buffer buf
        auto qk = [&](int buf, int sb, f32x16& sacc) {
            const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                                 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            const uint16_t* krow = &Ks[buf][(32 * sb + ln) * KS + 8 * lg];
#pragma unroll
            for (int s = 0; s < D / 16; s++) {
                const uint4 a = *(const uint4*)(krow + 16 * s);
                sacc = M::mma(a, qf[s], s == 0 ? zero : sacc);
                if constexpr (kSplit) sacc = M::mma(a, qfl[s], sacc);
            }
        };

        // softmax of the 32-key sub-tile starting at key t0 (sub-tile sb of
        // buffer buf) and O += V^T P^T over those keys
        auto softmax_pv = [&](int t0, int buf, int sb, f32x16& sacc) {
            const bool need_mask = (t0 + 31 > wpos_min) || (W > 0 && t0 < wpos_max + 1 - W);
            // element e of the accumulator is key t0 + 8 (e/4) + 4 lg + e%4
            if (need_mask) {
                // visible iff lo <= key <= my_pos: one unsigned compare per element
                const int lo = W > 0 ? my_pos + 1 - W : 0;
                const unsigned range = (unsigned)(my_pos - lo);
                const int kb = t0 + 4 * lg - lo;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int off = 8 * (e >> 2) + (e & 3);
                    sacc[e] = (unsigned)(kb + off) <= range ? sacc[e] : -INFINITY;
                }
            }
            float mx = fmaxf(sacc[0], sacc[1]);
#pragma unroll
            for (int e = 2; e < 16; e++) mx = fmaxf(mx, sacc[e]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            if (__any(mx > mrow + kLazyRescale)) {
                const float mnew = fmaxf(mrow, mx);
                const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
                mrow = mnew;
                lrow *= alpha;
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++) o[dt] *= alpha;
            }
            float pv[16];
#pragma unroll
            for (int e = 0; e < 16; e++) pv[e] = __builtin_amdgcn_exp2f(sacc[e] - mrow);
            if constexpr (kSplit) {
                float psum = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) psum += pv[e];
                lrow += psum;
            }
            // B operand P^T, k-step t: k-slot r <-> key t0 + 16 t + 8 (r/4) + 4 lg + r%4
            uint4 pf[2];
            uint4 pfl[kSplit ? 2 : 1];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                pf[t].x = M::pack2(pv[8 * t + 0], pv[8 * t + 1]);
                pf[t].y = M::pack2(pv[8 * t + 2], pv[8 * t + 3]);
                pf[t].z = M::pack2(pv[8 * t + 4], pv[8 * t + 5]);
                pf[t].w = M::pack2(pv[8 * t + 6], pv[8 * t + 7]);
                if constexpr (kSplit) {
                    const uint32_t hw[4] = {pf[t].x, pf[t].y, pf[t].z, pf[t].w};
                    uint32_t lw[4];
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        const float r0 = pv[8 * t + 2 * w] - __uint_as_float(hw[w] << 16);
                        const float r1 = pv[8 * t + 2 * w + 1] - __uint_as_float(hw[w] & 0xffff0000u);
                        lw[w] = M::pack2(r0, r1);
                    }
                    pfl[t] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
                }
            }
            if constexpr (!kSplit) {
                // row sum of the f16 P that enters the product (v_dot2c_f32_f16 with 1.0)
                const half2_t one2 = {1.0f16, 1.0f16};
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    lrow = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, pf[t].x), one2, lrow, false);
                    lrow = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, pf[t].y), one2, lrow, false);
                    lrow = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, pf[t].z), one2, lrow, false);
                    lrow = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, pf[t].w), one2, lrow, false);
                }
            }
#pragma unroll
            for (int dt = 0; dt < D / 32; dt++) {
                const uint16_t* vrow = &Vt[buf][(32 * dt + ln) * VS + 32 * sb + 4 * lg];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint2 lo = *(const uint2*)(vrow + 16 * t);
                    const uint2 hi = *(const uint2*)(vrow + 16 * t + 8);
                    const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    o[dt] = M::mma(a, pf[t], o[dt]);
                    if constexpr (kSplit) o[dt] = M::mma(a, pfl[t], o[dt]);
                }
            }
        };

        __syncthreads();  // the previous pass is done with both LDS buffers
        load_tile(t_first);
        for (int it = 0; it < n_tiles; it++) {
            const int t0 = t_first + it * BN;
            const int cur = it & 1;
            store_tile(cur);  // buffer cur was last read two tiles ago
            __syncthreads();
            if (it + 1 < n_tiles) load_tile(t0 + BN);
#pragma unroll
            for (int sb = 0; sb < BN / 32; sb++) {
                const int ts = t0 + 32 * sb;
                if (!(wave_active && ts <= wpos_max && (W <= 0 || ts + 31 >= wpos_min + 1 - W))) continue;
                f32x16 sacc;
                qk(cur, sb, sacc);
                softmax_pv(ts, cur, sb, sacc);
            }
        }

        const float lsum = lrow + __shfl_xor(lrow, 32, 64);
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        if (row_ok) {
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
    }
}

template <typename DT>
static hipError_t launch_prefill_dt(const PrefillLaunch& p, hipStream_t st) {
    const int n_qb = (p.n_tokens + kPfBM - 1) / kPfBM;
    dim3 grid(p.n_heads, (n_qb + 1) / 2);  // query blocks paired heavy + light
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
