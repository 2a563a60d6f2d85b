// Causal / sliding-window / image-block flash prefill over a Q8 KV cache
// (int8 codes with f32 scales per cache row or per 32-element block,
// kv_write_token, inference.rs:1886-1917) on gfx950 MFMA.  Replaces the
// token-serial attention of the prefill loop (inference.rs:2981-3017, one
// attention_token per token) for Q8 run states: one launch per chunk, every
// K / V tile read once per 128 (d64, d128) or 64 (d256) query rows.
//
// Workgroup = row groups of 32 query rows of one query head x 2 key halves,
// wave (row group, half) taking the 32-key sub-tiles 2 j + half of every tile;
// the two halves' (max, sum, O) merge through LDS at the end.  head_dim 64 and
// 128: 4 row groups, 128-key tiles, 8 waves (two per SIMD: the MFMAs of one overlap
// the VALU work of the other).  head_dim 256: 2 row groups, 64-key tiles, 4
// waves (one per SIMD, for the registers).  The tile goes global -> registers ->
// LDS (the next tile's loads are in flight while the current one is computed),
// the int8 codes converted to f16 on the way in (exact: |code| <= 127), K and V row-major with
// their 16-byte chunks XOR-swizzled per row like the f16 prefill kernel; the
// tile's k / v scales go to LDS as [block][key].  Each wave computes, on
// v_mfma_f32_32x32x16_f16,
//   S^T = K . Q^T     A = K codes (ds_read_b128), B = Q as an f16 hi + lo pair
//   O^T += V^T . P'^T A = V codes (ds_read_b64_tr_b16), B = P' as an f16 hi + lo pair
// The f32 scales stay outside the products, as in the Q8 decode kernel:
//   row scales    s = (codes . q) * k_scale[t];  P' = P * v_scale[t] * pw
//   block scales  one QK product per 32-element block (two k-steps), scaled
//                 and summed; one P' operand per V block (an O^T tile of 32 d
//                 rows is exactly one block)
// pw is a power of two that keeps the largest v_scale * pw of the tiles seen
// in [2^6, 2^7); when it has to drop, O is rescaled by the (exact) ratio, and
// it is divided out at the end.  Q is scaled per row by a power of two (max
// |q| in [2^14, 2^15)) before the split, undone on the scores.
#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
#define Q8P_LDS __attribute__((address_space(3)))

constexpr float kQ8Lazy = 8.0f;   // lazy softmax rescale threshold (log2 units)

// RG row groups of 32 query rows x KH key halves per workgroup (one wave each),
// BN keys per tile (each wave takes BN / 32 / KH sub-tiles between barriers).
// d64 / d128: 128 rows, 8 waves (two per SIMD).  d256: 64 rows, 4 waves (one per
// SIMD, which its registers need), so that 8-head models still launch one
// workgroup per CU for a 2048-token chunk.
template <int D>
struct Q8Tile {
    static constexpr int RG = D <= 128 ? 4 : 2;
    static constexpr int KH = 2;
    static constexpr int BN = D <= 128 ? 128 : 64;
    static constexpr int BM = 32 * RG;
    static constexpr int NT = 64 * RG * KH;
};

__device__ __forceinline__ f32x16 q8p_mma(const uint4& a, const uint4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                  0, 0, 0);
}

__device__ __forceinline__ uint32_t q8p_pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, half2_t));
}

// f16 hi + lo of (x0, x1): hi = f16(x), lo = f16(x - hi)
__device__ __forceinline__ uint32_t q8p_split2(float x0, float x1, uint32_t* lo) {
    const uint32_t h = q8p_pack2(x0, x1);
    const half2_t hh = __builtin_bit_cast(half2_t, h);
    *lo = q8p_pack2(x0 - (float)hh[0], x1 - (float)hh[1]);
    return h;
}

// 8 int8 codes (x = codes 0..3, y = codes 4..7) -> 8 exact f16.  With the sign
// bit flipped, u = c + 128 in [0, 255]; v_perm places u under the f16 exponent
// byte 0x64, i.e. the f16 1024 + u, and (1024 + u) - 1152 = c.
__device__ __forceinline__ uint4 q8p_cvt8(uint32_t x, uint32_t y) {
    const half2_t bias = {1152.0f16, 1152.0f16};
    auto two = [&](uint32_t w, uint32_t sel) {
        const uint32_t spread = __builtin_amdgcn_perm(0x64646464u, w, sel);
        return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, spread) - bias);
    };
    const uint32_t a = x ^ 0x80808080u, b = y ^ 0x80808080u;
    // selector bytes 0..3 pick bytes of the second operand, 4 a byte of 0x64646464
    return make_uint4(two(a, 0x04010400u), two(a, 0x04030402u), two(b, 0x04010400u), two(b, 0x04030402u));
}

__device__ __forceinline__ float q8p_xmax32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float q8p_xsum32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// floor(log2 x) for a positive normal float
__device__ __forceinline__ int q8p_ilog2(float x) { return (int)((__float_as_uint(x) >> 23) & 0xffu) - 127; }

// Position of 16-byte chunk c of tile row r: c ^ q8p_swz<D>(r & 15) (conflict-free
// K operand reads of 16 rows and V transpose reads of 4 rows x 4 chunks).  A
// head_dim-64 row is 8 chunks (half the banks): a 3-bit swizzle whose bit 2 is
// bit 1 of r keeps both read patterns conflict-free.
template <int D>
__device__ __forceinline__ int q8p_swz(int r) {
    if constexpr (D == 64) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    else return ((r << 2) ^ (r << 1) ^ (r >> 2)) & 15;
}

template <int D, bool BLOCK>
__global__ __launch_bounds__(Q8Tile<D>::NT, 1) void prefill_q8_kernel(const PrefillQ8Launch p) {
    constexpr int KH = Q8Tile<D>::KH, RG = Q8Tile<D>::RG;
    constexpr int NT = Q8Tile<D>::NT;     // threads
    constexpr int BM = Q8Tile<D>::BM, BN = Q8Tile<D>::BN;
    constexpr int NB = D / 32;            // 32-element blocks per head (k-step pairs, O^T tiles)
    constexpr int NBS = BLOCK ? NB : 1;   // scales per key and head
    constexpr int CPR = D / 16;           // 16-code chunks per cache row
    constexpr int KCH = BN * CPR / NT;    // chunks per thread per K (or V) tile
    constexpr int SCL = (2 * NBS * BN + NT - 1) / NT;  // scales per thread per tile
    static_assert(KCH >= 1 && BN * CPR % NT == 0, "tile");

    __shared__ __attribute__((aligned(16))) uint16_t KVt[2 * BN * D];
    uint16_t* const Kt = KVt;
    uint16_t* const Vt = KVt + BN * D;
    __shared__ __attribute__((aligned(16))) float Sc[2 * NBS * BN];  // [k|v][block][key]
    // key-half merge: O^T accumulators [row group][dt][e][lane], (m, l, pw) [row group][lane]
    // (O^T goes into the K / V tiles, free once the key loop is done)
    static_assert(RG * NB * 16 * 64 * 4 <= 2 * BN * D * 2, "merge buffer fits the tiles");
    float* const Mo = (float*)KVt;
    __shared__ float Ms[RG * (2 + NBS) * 64];
    // head_dim 256: the Q residual fragments live in LDS (per wave, [k-step][lane])
    // instead of 64 VGPRs, which the accumulators need
    constexpr bool kQloLds = D == 256;
    __shared__ __attribute__((aligned(16))) uint4 Qlo[kQloLds ? RG * (D / 16) * 64 : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave % RG, kh = wave / RG;  // row group, key half
    const int ln = lane & 31, lg = lane >> 5;
    const int m = p.n_tokens;
    const int P0 = (int)p.base_pos;
    const int W = p.window;
    const int n_qb = (m + BM - 1) / BM;
    const int h = blockIdx.x;
    const int qblk = n_qb - 1 - (int)blockIdx.y;  // the longest query blocks first
    const int kv_mul = p.n_heads / p.n_kv_heads;
    const int g = h / kv_mul;
    const int8_t* kc = p.k_codes + (size_t)g * D;
    const int8_t* vc = p.v_codes + (size_t)g * D;
    const int64_t rs = p.row_stride;
    const float* ksc = p.k_scale + (BLOCK ? (size_t)g * NB : 0);
    const float* vsc = p.v_scale + (BLOCK ? (size_t)g * NB : 0);
    const int64_t srs = p.scale_row_stride;

    const int q0 = qblk * BM;
    const int wr0 = q0 + rg * 32;
    const int my_row = wr0 + ln;
    const bool row_ok = my_row < m;
    const int my_row_c = row_ok ? my_row : m - 1;
    const int my_pos = P0 + my_row_c;
    const bool wave_active = wr0 < m;
    const int wpos_min = P0 + (wave_active ? wr0 : m - 1);
    const int wpos_max = P0 + min(wr0 + 31, m - 1);
    // Keys visible to the row at position pos: [row_lo(pos), row_hi(pos)]; causal
    // [pos + 1 - W (or 0), pos], image block [min(pos + 1 - W (or 0), P0), P0 + m - 1]
    // (LanguageAttentionPolicy::visible_keys, attention.rs:74-96).
    auto row_lo = [&](int pos) {
        const int wl = W > 0 ? pos + 1 - W : 0;
        return p.bidirectional ? min(wl, P0) : wl;
    };
    auto row_hi = [&](int pos) { return p.bidirectional ? P0 + m - 1 : pos; };
    const int lo_min = row_lo(wpos_min), lo_max = row_lo(wpos_max);
    const int hi_min = row_hi(wpos_min), hi_max = row_hi(wpos_max);

    // Q (B operand): lane (row ln, half lg) holds d = 16 s + 8 lg .. +7 of k-step s,
    // scaled by score_scale * log2(e) and a per-row power of two 2^eq.
    uint4 qf[D / 16], qfl[kQloLds ? 1 : D / 16];
    float qfac;
    {
        const float* qrow = p.q + ((size_t)my_row_c * p.n_heads + h) * D + 8 * lg;
        const float qs = p.score_scale * 1.44269504088896340736f;
        float qv[D / 16][8];
        float amax = 0.0f;
#pragma unroll
        for (int s = 0; s < D / 16; s++)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const float4 x = *(const float4*)(qrow + 16 * s + 4 * c);
                qv[s][4 * c + 0] = x.x * qs;
                qv[s][4 * c + 1] = x.y * qs;
                qv[s][4 * c + 2] = x.z * qs;
                qv[s][4 * c + 3] = x.w * qs;
#pragma unroll
                for (int e = 0; e < 4; e++) amax = fmaxf(amax, fabsf(qv[s][4 * c + e]));
            }
        amax = q8p_xmax32(amax);
        const int eq = amax > 0.0f ? min(100, max(-100, 14 - q8p_ilog2(amax))) : 0;
        const float up = ldexpf(1.0f, eq);
        qfac = ldexpf(1.0f, -eq);
#pragma unroll
        for (int s = 0; s < D / 16; s++) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int w = 0; w < 4; w++) hw[w] = q8p_split2(qv[s][2 * w] * up, qv[s][2 * w + 1] * up, &lw[w]);
            qf[s] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            const uint4 lo4 = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            if constexpr (kQloLds) Qlo[(rg * (D / 16) + s) * 64 + lane] = lo4;
            else qfl[s] = lo4;
        }
    }

    auto qlo = [&](int s) -> uint4 {
        if constexpr (kQloLds) return Qlo[(rg * (D / 16) + s) * 64 + lane];
        else return qfl[s];
    };

    // keys [kbeg, kend) are visible to some row of this block
    const int kend = p.bidirectional ? P0 + m : P0 + min(q0 + BM, m);
    const int kbeg = max(0, row_lo(P0 + q0));
    const int t_first = kbeg / BN * BN;
    const int n_tiles = (kend - t_first + BN - 1) / BN;

    // Tile staging registers; rows past kend - 1 are clamped to it (masked).
    uint4 kreg[KCH], vreg[KCH];
    float sreg[SCL];
    auto load_tile = [&](int t0) {
        const int last = kend - 1;
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int c = tid + NT * i;
            const int64_t off = (int64_t)min(t0 + c / CPR, last) * rs + (c % CPR) * 16;
            kreg[i] = *(const uint4*)(kc + off);
            vreg[i] = *(const uint4*)(vc + off);
        }
#pragma unroll
        for (int i = 0; i < SCL; i++) {
            const int c = tid + NT * i;
            if (c < 2 * NBS * BN) {
                const int kv = c / (NBS * BN), rem = c % (NBS * BN);
                const int b = rem / BN, key = rem % BN;
                sreg[i] = (kv ? vsc : ksc)[(int64_t)min(t0 + key, last) * srs + b];
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int c = tid + NT * i;
            const int r = c / CPR, cc = c % CPR, z = q8p_swz<D>(r & 15);
            uint16_t* kd = Kt + r * D;
            uint16_t* vd = Vt + r * D;
            *(uint4*)(kd + ((2 * cc) ^ z) * 8) = q8p_cvt8(kreg[i].x, kreg[i].y);
            *(uint4*)(kd + ((2 * cc + 1) ^ z) * 8) = q8p_cvt8(kreg[i].z, kreg[i].w);
            *(uint4*)(vd + ((2 * cc) ^ z) * 8) = q8p_cvt8(vreg[i].x, vreg[i].y);
            *(uint4*)(vd + ((2 * cc + 1) ^ z) * 8) = q8p_cvt8(vreg[i].z, vreg[i].w);
        }
#pragma unroll
        for (int i = 0; i < SCL; i++) {
            const int c = tid + NT * i;
            if (c < 2 * NBS * BN) Sc[c] = sreg[i];
        }
    };

    // V^T transpose reads (ds_read_b64_tr_b16): lane i of 16-lane group G supplies
    // row k0 + i/4, columns d0 + 4 (i%4) .. +3, k0 = 32 sb + 16 t + 8 b + 4 lg,
    // d0 = 32 dt + 16 (G & 1); it receives V[k0 + 0..3][d0 + i], i.e. A-operand
    // slots 4b .. 4b+3 of row d0 + i.
    const int gi = lane & 15;
    const int v_chunk = 2 * ((lane >> 4) & 1) + ((gi & 3) >> 1);
    int v_base[2], v_swz[2];
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const int r = 8 * b + 4 * lg + (gi >> 2);
        v_base[b] = r * D + (gi & 1) * 4;
        v_swz[b] = q8p_swz<D>(r & 15);
    }
    const int swz_k = q8p_swz<D>(ln & 15);

    f32x16 o[NB];
#pragma unroll
    for (int dt = 0; dt < NB; dt++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[dt][e] = 0.0f;
    float mrow = -1e30f;  // reference maximum of this lane's row (log2 units)
    float lrow = 0.0f;    // this lane's share of the row sum of P
    float pw[NBS];        // P' = P * v_scale * pw; 0 until a nonzero v scale is seen
#pragma unroll
    for (int b = 0; b < NBS; b++) pw[b] = 0.0f;

    auto subtile = [&](int sb, int ts) {
        const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const uint16_t* krow = Kt + (32 * sb + ln) * D;
        auto kop = [&](int s) { return *(const uint4*)(krow + (((2 * s + lg) ^ swz_k) << 3)); };
        // scales of this lane's keys 32 sb + 8 (e / 4) + 4 lg + e % 4 in block b
        auto lane_scales = [&](int kv, int b, float* out) {
            const float* src = Sc + (kv * NBS + b) * BN + 32 * sb + 4 * lg;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 x = *(const float4*)(src + 8 * q);
                out[4 * q + 0] = x.x, out[4 * q + 1] = x.y, out[4 * q + 2] = x.z, out[4 * q + 3] = x.w;
            }
        };
        f32x16 sacc;
        if constexpr (!BLOCK) {
            f32x16 acc = zero;
#pragma unroll
            for (int s = 0; s < D / 16; s++) {
                const uint4 a = kop(s);
                acc = q8p_mma(a, qf[s], acc);
                acc = q8p_mma(a, qlo(s), acc);
            }
            float ks[16];
            lane_scales(0, 0, ks);
#pragma unroll
            for (int e = 0; e < 16; e++) sacc[e] = acc[e] * (ks[e] * qfac);
        } else {
            sacc = zero;
#pragma unroll
            for (int u = 0; u < NB; u++) {
                const uint4 a0 = kop(2 * u), a1 = kop(2 * u + 1);
                f32x16 acc = q8p_mma(a0, qf[2 * u], zero);
                acc = q8p_mma(a0, qlo(2 * u), acc);
                acc = q8p_mma(a1, qf[2 * u + 1], acc);
                acc = q8p_mma(a1, qlo(2 * u + 1), acc);
                float ks[16];
                lane_scales(0, u, ks);
#pragma unroll
                for (int e = 0; e < 16; e++) sacc[e] = fmaf(acc[e], ks[e], sacc[e]);
            }
            sacc *= qfac;
        }

        // element e is key ts + 8 (e / 4) + 4 lg + e % 4
        if ((ts + 31 > hi_min) || (ts < lo_max)) {
            const int lo = row_lo(my_pos);
            const unsigned range = (unsigned)(row_hi(my_pos) - lo);
            const int kb0 = ts + 4 * lg - lo;
#pragma unroll
            for (int e = 0; e < 16; e++)
                sacc[e] = (unsigned)(kb0 + 8 * (e >> 2) + (e & 3)) <= range ? sacc[e] : -INFINITY;
        }
        float mx = sacc[0];
#pragma unroll
        for (int e = 1; e < 16; e++) mx = fmaxf(mx, sacc[e]);
        mx = q8p_xmax32(mx);
        if (__any(mx > mrow + kQ8Lazy)) {
            const float mnew = fmaxf(mrow, mx);
            const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
            mrow = mnew;
            lrow *= alpha;
#pragma unroll
            for (int dt = 0; dt < NB; dt++) o[dt] *= alpha;
        }
        float pv[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            pv[e] = __builtin_amdgcn_exp2f(sacc[e] - mrow);
            lrow += pv[e];
        }

        // P'^T operand (hi, lo) of block b, k-step t: slot r <-> key ts + 16 t + 8 (r/4) + 4 lg + r%4
        auto make_p = [&](int b, uint4* ph, uint4* pl) {
            float vs[16];
            lane_scales(1, b, vs);
            float vmax = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; e++) vmax = fmaxf(vmax, vs[e]);
            vmax = q8p_xmax32(vmax);  // the sub-tile's largest v scale (both halves of the row agree)
            if (vmax > 0.0f && (pw[b] == 0.0f || vmax * pw[b] >= 128.0f)) {
                const float pnew = ldexpf(1.0f, min(120, 6 - q8p_ilog2(vmax)));
                if (pw[b] != 0.0f) {
                    const float r = pnew / pw[b];
                    if constexpr (BLOCK) o[b] *= r;
                    else {
#pragma unroll
                        for (int dt = 0; dt < NB; dt++) o[dt] *= r;
                    }
                }
                pw[b] = pnew;
            }
#pragma unroll
            for (int t = 0; t < 2; t++) {
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const int e = 8 * t + 2 * w;
                    hw[w] = q8p_split2(pv[e] * vs[e] * pw[b], pv[e + 1] * vs[e + 1] * pw[b], &lw[w]);
                }
                ph[t] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                pl[t] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            }
        };
        // O^T += V^T P'^T for the 32 d rows of tile dt
        auto pv_block = [&](int dt, const uint4* ph, const uint4* pl) {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                i16x4 part[2];
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    const int off = (32 * sb + 16 * t) * D + v_base[b] + (((4 * dt + v_chunk) ^ v_swz[b]) << 3);
                    part[b] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((Q8P_LDS i16x4*)(Vt + off));
                }
                const uint2 lo = __builtin_bit_cast(uint2, part[0]);
                const uint2 hi = __builtin_bit_cast(uint2, part[1]);
                const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
                o[dt] = q8p_mma(a, ph[t], o[dt]);
                o[dt] = q8p_mma(a, pl[t], o[dt]);
            }
        };
        if constexpr (!BLOCK) {
            uint4 ph[2], pl[2];
            make_p(0, ph, pl);
#pragma unroll
            for (int dt = 0; dt < NB; dt++) pv_block(dt, ph, pl);
        } else {
#pragma unroll
            for (int dt = 0; dt < NB; dt++) {
                uint4 ph[2], pl[2];
                make_p(dt, ph, pl);
                pv_block(dt, ph, pl);
            }
        }
    };

    load_tile(t_first);
    for (int it = 0; it < n_tiles; it++) {
        const int t0 = t_first + it * BN;
        __syncthreads();  // every wave is done with the previous tile
        store_tile();
        __syncthreads();
        if (it + 1 < n_tiles) load_tile(t0 + BN);
#pragma unroll
        for (int sb = 0; sb < BN / 32; sb++) {
            if (KH == 2 && (sb & 1) != kh) continue;
            const int ts = t0 + 32 * sb;
            if (wave_active && ts <= hi_max && ts + 31 >= lo_min) subtile(sb, ts);
        }
    }

    // Merge the second key half into the first: both are partial softmax sums of
    // the same rows over disjoint keys.  A half with no keys has pw = 0, l = 0.
    float wa[NBS];  // final factor on O per block (1 / pw, or 1 after the merge)
    if constexpr (KH == 2) {
        __syncthreads();  // every wave is done with the tiles that Mo overlays
        if (kh == 1) {
#pragma unroll
            for (int dt = 0; dt < NB; dt++)
#pragma unroll
                for (int e = 0; e < 16; e++) Mo[((rg * NB + dt) * 16 + e) * 64 + lane] = o[dt][e];
            Ms[(rg * (2 + NBS) + 0) * 64 + lane] = mrow;
            Ms[(rg * (2 + NBS) + 1) * 64 + lane] = lrow;
#pragma unroll
            for (int b = 0; b < NBS; b++) Ms[(rg * (2 + NBS) + 2 + b) * 64 + lane] = pw[b];
        }
        __syncthreads();
        if (kh == 1) return;
        const float mb = Ms[(rg * (2 + NBS) + 0) * 64 + lane];
        const float lb = Ms[(rg * (2 + NBS) + 1) * 64 + lane];
        const float mm = fmaxf(mrow, mb);
        const float aa = __builtin_amdgcn_exp2f(mrow - mm), ab = __builtin_amdgcn_exp2f(mb - mm);
        lrow = lrow * aa + lb * ab;
#pragma unroll
        for (int b = 0; b < NBS; b++) {
            const float pb = Ms[(rg * (2 + NBS) + 2 + b) * 64 + lane];
            const float fa = pw[b] > 0.0f ? aa / pw[b] : 0.0f;
            const float fb = pb > 0.0f ? ab / pb : 0.0f;
#pragma unroll
            for (int dt = 0; dt < NB; dt++) {
                if (BLOCK && dt != b) continue;
#pragma unroll
                for (int e = 0; e < 16; e++)
                    o[dt][e] = o[dt][e] * fa + Mo[((rg * NB + dt) * 16 + e) * 64 + lane] * fb;
            }
            wa[b] = 1.0f;
        }
    } else {
#pragma unroll
        for (int b = 0; b < NBS; b++) wa[b] = pw[b] > 0.0f ? 1.0f / pw[b] : 0.0f;
    }

    const float lsum = q8p_xsum32(lrow);
    if (row_ok) {
        float* orow = p.out + ((size_t)my_row * p.n_heads + h) * D;
        const float* gt = p.gate.at(my_row, h);  // Qwen3.5 output gate, or null
        const float il = lsum > 0.0f ? 1.0f / lsum : 0.0f;
#pragma unroll
        for (int dt = 0; dt < NB; dt++) {
            const float inv = il * wa[BLOCK ? dt : 0];
#pragma unroll
            for (int jb = 0; jb < 4; jb++) {
                const int d0 = 32 * dt + 8 * jb + 4 * lg;
                float4 v;
                v.x = o[dt][4 * jb + 0] * inv;
                v.y = o[dt][4 * jb + 1] * inv;
                v.z = o[dt][4 * jb + 2] * inv;
                v.w = o[dt][4 * jb + 3] * inv;
                if (gt) {
                    v.x = gate_mul(v.x, gt[d0 + 0]);
                    v.y = gate_mul(v.y, gt[d0 + 1]);
                    v.z = gate_mul(v.z, gt[d0 + 2]);
                    v.w = gate_mul(v.w, gt[d0 + 3]);
                }
                *(float4*)(orow + d0) = v;
            }
        }
    }
}

template <int D, bool BLOCK>
hipError_t launch_q8_d(const PrefillQ8Launch& p, hipStream_t st) {
    const int n_qb = (p.n_tokens + Q8Tile<D>::BM - 1) / Q8Tile<D>::BM;
    prefill_q8_kernel<D, BLOCK><<<dim3(p.n_heads, n_qb), Q8Tile<D>::NT, 0, st>>>(p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_q8(const PrefillQ8Launch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    switch (p.head_dim) {
        case 64: return p.block ? launch_q8_d<64, true>(p, st) : launch_q8_d<64, false>(p, st);
        case 128: return p.block ? launch_q8_d<128, true>(p, st) : launch_q8_d<128, false>(p, st);
        case 256: return p.block ? launch_q8_d<256, true>(p, st) : launch_q8_d<256, false>(p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace gr
