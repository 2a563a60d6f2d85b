// Split-K flash decoding on gfx950 MFMA for 16-bit (f16 / bf16) KV caches.
//
// Same work split and partial format as decode.hip (one workgroup per
// (sequence, KV head, split); partials merged by decode_combine_kernel), but
// the scores and the value accumulation run on v_mfma_f32_16x16x32 with the
// kv_mul (<= 16) query heads of a GQA group on the N axis:
//   S^T[key][q]  = K . Q^T        A = K rows straight from HBM (16 B per lane)
//   O^T[d][q]   += V^T . P^T      A = V^T from a per-wave LDS tile, B = P from
//                                 the S^T accumulators (same lane <-> query map)
// Each wave streams its own 32-key tiles (keys split between the 4 waves of
// the workgroup, next tile prefetched into registers while the current one is
// processed) and keeps its own online-softmax state; the waves merge in LDS.
// Q and P are carried as hi + lo 16-bit pairs (two MFMAs per product; K and V
// are exact 16-bit cache values), so the scores and weights keep ~fp32
// precision even for large unscaled logits.  Decode is HBM-bound with the
// matrix cores mostly idle, so the second MFMA costs no time.
#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename DT>
struct Mfma16;
template <>
struct Mfma16<F16> {
    static constexpr bool kSplit = true;
    static __device__ __forceinline__ f32x4 mma(const uint4& a, const uint4& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                      __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t cvt(float x) { return f32_to_f16(x); }
    static __device__ __forceinline__ float back(uint16_t x) { return f16_to_f32(x); }
};
template <>
struct Mfma16<BF16> {
    static constexpr bool kSplit = true;
    static __device__ __forceinline__ f32x4 mma(const uint4& a, const uint4& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t cvt(float x) { return f32_to_bf16(x); }
    static __device__ __forceinline__ float back(uint16_t x) { return bf16_to_f32(x); }
};

constexpr int kMdThreads = 256;
constexpr int kMdWaves = kMdThreads / 64;

// Raise a row's reference maximum only when a tile exceeds it by more than
// this (log2 units); P = 2^(s - m_ref) <= 2^8 meanwhile and O needs no rescale.
constexpr float kMdLazyRescale = 8.0f;

// NSUB groups of 32 keys per wave iteration.  1 is used: with 2, the d128
// kernel needs 300 registers (one wave per SIMD) and measured slower than two
// waves per SIMD streaming 32-key tiles.
template <typename DT, int D, int NSUB>
__global__ __launch_bounds__(kMdThreads) void decode_mfma_kernel(const DecodeLaunch p) {
    using M = Mfma16<DT>;
    constexpr bool kSplit = M::kSplit;
    constexpr int TILE = 32 * NSUB;              // keys per wave iteration
    constexpr int NS16 = TILE / 16;              // 16-key score sub-tiles
    constexpr int DC = D / 8;                    // 16-byte chunks per row
    constexpr int KS = D / 32;                   // MFMA k-steps over d
    constexpr int VTASK = (TILE / 4) * DC / 64;  // 4-key x 16-byte V tasks per lane
    constexpr int VS = TILE + 4;                 // V^T row stride (elements)
    static_assert(VTASK >= 1, "tile");

    // LDS: per-wave V^T tiles during the key loop, then (aliased) the wave merge.
    constexpr int kVtBytes = kMdWaves * D * VS * 2;
    constexpr int kMergeBytes = (kMdWaves * 16 * (D + 1) + 2 * kMdWaves * 16) * 4;
    __shared__ __attribute__((aligned(16))) char smem[kVtBytes > kMergeBytes ? kVtBytes : kMergeBytes];

    const int split = blockIdx.x;
    const int g = blockIdx.y;
    const int s = blockIdx.z;
    const int t_begin = p.kv_start[s] + split * p.split_keys;
    const int t_limit = p.kv_end[s];
    if (t_begin >= t_limit) return;
    const int t_stop = min(t_limit, t_begin + p.split_keys);
    const int kv_mul = p.n_heads / p.n_kv_heads;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g4 = lane >> 4;
    uint16_t* vt = (uint16_t*)smem + wave * D * VS;

    // Q fragments (B operand of S^T = K Q^T): lane (query l16, group g4) holds
    // d = 32 ks + 8 g4 .. +7, pre-scaled to log2 units; queries >= kv_mul are 0.
    uint4 qf[KS], qfl[kSplit ? KS : 1];
    {
        const bool qv = l16 < kv_mul;
        const float* qrow = p.q + ((size_t)s * p.n_heads + (size_t)g * kv_mul + (qv ? l16 : 0)) * D;
        const float qscale = p.score_scale * kLog2e;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const int d0 = 32 * k + 8 * g4 + 2 * w;
                const float x0 = qv ? qrow[d0] * qscale : 0.0f;
                const float x1 = qv ? qrow[d0 + 1] * qscale : 0.0f;
                const uint16_t h0 = M::cvt(x0), h1 = M::cvt(x1);
                hw[w] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                if constexpr (kSplit) {
                    lw[w] = (uint32_t)M::cvt(x0 - M::back(h0)) | ((uint32_t)M::cvt(x1 - M::back(h1)) << 16);
                }
            }
            qf[k] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            if constexpr (kSplit) qfl[k] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        }
    }

    const size_t slot = (size_t)(p.seq_slot ? p.seq_slot[s] : s);
    const uint16_t* kc = (const uint16_t*)p.k_cache + slot * p.seq_stride + (size_t)g * D;
    const uint16_t* vc = (const uint16_t*)p.v_cache + slot * p.seq_stride + (size_t)g * D;
    const int64_t rs = p.row_stride;

    uint4 kr[NS16][KS];
    uint4 vr[VTASK][4];
    auto load_tile = [&](int t0) {
        if (t0 + TILE <= t_stop) {  // whole tile inside the split: plain strided rows
            const uint16_t* kt = kc + (int64_t)t0 * rs + 8 * g4;
            const uint16_t* vtp = vc + (int64_t)t0 * rs;
#pragma unroll
            for (int sb = 0; sb < NS16; sb++) {
                const uint16_t* row = kt + (int64_t)(16 * sb + l16) * rs;
#pragma unroll
                for (int k = 0; k < KS; k++) kr[sb][k] = *(const uint4*)(row + 32 * k);
            }
#pragma unroll
            for (int u = 0; u < VTASK; u++) {
                const int task = lane + 64 * u;
                const int dc = task % DC, kg = task / DC;
                const uint16_t* v0 = vtp + (int64_t)(4 * kg) * rs + 8 * dc;
#pragma unroll
                for (int r = 0; r < 4; r++) vr[u][r] = *(const uint4*)(v0 + r * rs);
            }
            return;
        }
#pragma unroll
        for (int sb = 0; sb < NS16; sb++) {
            const int key = min(t0 + 16 * sb + l16, t_stop - 1);
            const uint16_t* row = kc + (int64_t)key * rs + 8 * g4;
#pragma unroll
            for (int k = 0; k < KS; k++) kr[sb][k] = *(const uint4*)(row + 32 * k);
        }
#pragma unroll
        for (int u = 0; u < VTASK; u++) {
            const int task = lane + 64 * u;
            const int dc = task % DC, kg = task / DC;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = min(t0 + 4 * kg + r, t_stop - 1);
                vr[u][r] = *(const uint4*)(vc + (int64_t)key * rs + 8 * dc);
            }
        }
    };

    f32x4 o[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrow = -1e30f, lrow = 0.0f;

    const int n_tiles = (t_stop - t_begin + TILE - 1) / TILE;
    int it = wave;
    if (it < n_tiles) load_tile(t_begin + it * TILE);
    for (; it < n_tiles; it += kMdWaves) {
        const int t0 = t_begin + it * TILE;
        // V tile -> LDS, transposed: Vt[d][key]
#pragma unroll
        for (int u = 0; u < VTASK; u++) {
            const int task = lane + 64 * u;
            const int dc = task % DC, kg = task / DC;
            const uint32_t w[4][4] = {{vr[u][0].x, vr[u][0].y, vr[u][0].z, vr[u][0].w},
                                      {vr[u][1].x, vr[u][1].y, vr[u][1].z, vr[u][1].w},
                                      {vr[u][2].x, vr[u][2].y, vr[u][2].z, vr[u][2].w},
                                      {vr[u][3].x, vr[u][3].y, vr[u][3].z, vr[u][3].w}};
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
                *(uint2*)(vt + (8 * dc + dd) * VS + 4 * kg) = make_uint2(lo, hi);
            }
        }
        // scores for the 16-key sub-tiles
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 sacc[NS16];
#pragma unroll
        for (int sb = 0; sb < NS16; sb++) {
#pragma unroll
            for (int k = 0; k < KS; k++) {
                sacc[sb] = M::mma(kr[sb][k], qf[k], k == 0 ? zero : sacc[sb]);
                if constexpr (kSplit) sacc[sb] = M::mma(kr[sb][k], qfl[k], sacc[sb]);
            }
        }
        // prefetch the wave's next tile while this one is finished
        if (it + kMdWaves < n_tiles) load_tile(t_begin + (it + kMdWaves) * TILE);

        // S^T register j of sub-tile sb holds key t0 + 16 sb + 4 g4 + j (query l16).
        float sv[4 * NS16];
        const bool tail = t0 + TILE > t_stop;
#pragma unroll
        for (int sb = 0; sb < NS16; sb++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int key = t0 + 16 * sb + 4 * g4 + j;
                sv[4 * sb + j] = (!tail || key < t_stop) ? sacc[sb][j] : -INFINITY;
            }
        float mx = sv[0];
#pragma unroll
        for (int e = 1; e < 4 * NS16; e++) mx = fmaxf(mx, sv[e]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        if (__any(mx > mrow + kMdLazyRescale)) {
            const float mnew = fmaxf(mrow, mx);
            const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
            mrow = mnew;
            lrow *= alpha;
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++) o[dt] *= alpha;
        }
        float pv[4 * NS16];
        float psum = 0.0f;
#pragma unroll
        for (int e = 0; e < 4 * NS16; e++) {
            pv[e] = __builtin_amdgcn_exp2f(sv[e] - mrow);
            psum += pv[e];
        }
        lrow += psum;
        // B operand P^T per 32-key k-step kk: k-slot r <-> key 32 kk + 16 (r/4) + 4 g4 + r%4
        uint4 pf[NSUB], pfl[kSplit ? NSUB : 1];
#pragma unroll
        for (int kk = 0; kk < NSUB; kk++) {
            uint32_t ph[4], pl[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float a0 = pv[8 * kk + 2 * w], a1 = pv[8 * kk + 2 * w + 1];
                const uint16_t h0 = M::cvt(a0), h1 = M::cvt(a1);
                ph[w] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                if constexpr (kSplit)
                    pl[w] = (uint32_t)M::cvt(a0 - M::back(h0)) | ((uint32_t)M::cvt(a1 - M::back(h1)) << 16);
            }
            pf[kk] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
            if constexpr (kSplit) pfl[kk] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
        }
        // LDS operations of one wave complete in issue order, so the V^T reads
        // below see this wave's stores; the barrier only pins the compiler's order.
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
            const uint16_t* vrow = vt + (16 * dt + l16) * VS + 4 * g4;
#pragma unroll
            for (int kk = 0; kk < NSUB; kk++) {
                const uint2 lo = *(const uint2*)(vrow + 32 * kk);
                const uint2 hi = *(const uint2*)(vrow + 32 * kk + 16);
                const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
                o[dt] = M::mma(a, pf[kk], o[dt]);
                if constexpr (kSplit) o[dt] = M::mma(a, pfl[kk], o[dt]);
            }
        }
        __builtin_amdgcn_wave_barrier();  // V^T reads done before the next tile overwrites it
    }

    // lane sums -> row sums (4 lanes share a query column)
    lrow += __shfl_xor(lrow, 16, 64);
    lrow += __shfl_xor(lrow, 32, 64);
    __syncthreads();  // every wave is done with its V^T tile: reuse the LDS for the merge
    float (*sh_o)[16][D + 1] = (float (*)[16][D + 1])smem;
    float (*sh_m)[16] = (float (*)[16])((float*)smem + kMdWaves * 16 * (D + 1));
    float (*sh_l)[16] = sh_m + kMdWaves;
    if (g4 == 0) {
        sh_m[wave][l16] = mrow;
        sh_l[wave][l16] = lrow;
    }
    // O^T register j of tile dt: d = 16 dt + 4 g4 + j, query l16
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++)
#pragma unroll
        for (int j = 0; j < 4; j++) sh_o[wave][l16][16 * dt + 4 * g4 + j] = o[dt][j];
    __syncthreads();
    const int n_splits = p.n_splits;
    for (int idx = tid; idx < kv_mul * D; idx += kMdThreads) {
        const int q = idx / D, i = idx % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kMdWaves; w++) mx = fmaxf(mx, sh_m[w][q]);
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int w = 0; w < kMdWaves; w++) {
            const float a = exp2f(sh_m[w][q] - mx);
            lt += sh_l[w][q] * a;
            ot += sh_o[w][q][i] * a;
        }
        const size_t part = ((size_t)s * p.n_heads + (size_t)g * kv_mul + q) * n_splits + split;
        p.ws_o[part * D + i] = ot;
        if (i == 0) {
            p.ws_ml[part * 2 + 0] = mx;
            p.ws_ml[part * 2 + 1] = lt;
        }
    }
}

template <typename DT>
static hipError_t launch_mfma_dt(const DecodeLaunch& p, hipStream_t st) {
    dim3 grid(p.n_splits, p.n_kv_heads, p.n_seq);
    switch (p.head_dim) {
        case 128: decode_mfma_kernel<DT, 128, 1><<<grid, kMdThreads, 0, st>>>(p); break;
        case 256: decode_mfma_kernel<DT, 256, 1><<<grid, kMdThreads, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool decode_mfma_supported(const DecodeLaunch& p) {
    const int kv_mul = p.n_heads / p.n_kv_heads;
    return (p.kv_dtype == GR_DTYPE_F16 || p.kv_dtype == GR_DTYPE_BF16) && kv_mul <= 16 &&
           (p.head_dim == 128 || p.head_dim == 256);
}

hipError_t launch_decode_mfma_split(const DecodeLaunch& p, hipStream_t st) {
    return p.kv_dtype == GR_DTYPE_F16 ? launch_mfma_dt<F16>(p, st) : launch_mfma_dt<BF16>(p, st);
}

}  // namespace gr
