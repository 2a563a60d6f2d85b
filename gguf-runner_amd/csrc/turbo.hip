// Turbo KV cache (KvCacheFormat::Turbo, reference inference.rs:346-1334) on the
// device: the quantising KV write, the query rotation, the split-K decode over
// the packed codes and the merge + value finalisation.
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
// Device layout per wave: a head of D (64, 128, 256) elements lives as
// x[j] = element lane + 64 j.  The FWHT runs its widths in the reference's
// order (1, 2, 4, ...: lanes via shuffles, then within the lane) and the norms
// are sequential sums in element order, so the written codes, signs, sigma and
// gamma are bit-exact with the reference for the same f32 row (no FMA
// contraction in this file).
//
// The decode keeps every product exact in f16: C[code] = c0 s + (c1 - c0) s_big
// with s, s_big, sgn in {-1, 0, +1}, so K and V enter the MFMAs as exact +-1/0
// operands and the f32 factors (c0, c1 - c0, sigma, gamma) ride on the other
// operand, carried as f16 hi + lo pairs (with power-of-two range scaling as in
// the Q8 decode).
#pragma clang fp contract(off)

#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kTqC0 = 0.45278f;    // TURBOQUANT_CENTROIDS, inference.rs:349
constexpr float kTqC1 = 1.510417f;
constexpr float kTqTh = 0.9815985f;  // TURBOQUANT_THRESHOLD_HI, inference.rs:351
constexpr float kFracPi2 = 1.5707964f;

__device__ __forceinline__ float tq_centroid(int code) {
    return code == 0 ? -kTqC1 : code == 1 ? -kTqC0 : code == 2 ? kTqC0 : kTqC1;
}

__device__ __forceinline__ int tq_code(float x) {
    return x < -kTqTh ? 0 : (x < 0.0f ? 1 : (x < kTqTh ? 2 : 3));
}

// sign flips of a wave-held head: bit i of `bits` set -> negate element i
template <int D>
__device__ __forceinline__ void wave_signs(float (&x)[D / 64], const uint8_t* bits, int lane) {
#pragma unroll
    for (int j = 0; j < D / 64; j++) {
        const int i = lane + 64 * j;
        if ((bits[i >> 3] >> (i & 7)) & 1) x[j] = -x[j];
    }
}

// turboquant_fwht_inplace_scalar (inference.rs:681-701) on a wave-held head
template <int D>
__device__ __forceinline__ void wave_fwht(float (&x)[D / 64], int lane) {
#pragma unroll
    for (int w = 1; w < 64; w <<= 1)
#pragma unroll
        for (int j = 0; j < D / 64; j++) {
            const float p = __shfl_xor(x[j], w, 64);
            x[j] = (lane & w) ? p - x[j] : x[j] + p;  // lower a+b, upper a-b
        }
#pragma unroll
    for (int w = 1; w < D / 64; w <<= 1)
#pragma unroll
        for (int j = 0; j < D / 64; j++)
            if (!(j & w)) {
                const float a = x[j], b = x[j | w];
                x[j] = a + b;
                x[j | w] = a - b;
            }
    const float sc = 1.0f / sqrtf((float)D);
#pragma unroll
    for (int j = 0; j < D / 64; j++) x[j] *= sc;
}

template <int D>
__device__ __forceinline__ void wave_transform(float (&x)[D / 64], const uint8_t* first, const uint8_t* second,
                                               int lane) {
    wave_signs<D>(x, first, lane);
    wave_fwht<D>(x, lane);
    wave_signs<D>(x, second, lane);
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
    wave_transform<D>(x, sg, sg + ss, lane);  // rot_pre, rot_post
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
    wave_transform<D>(r, sg + 2 * ss, sg + 3 * ss, lane);  // res_pre, res_post
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

// ---------------------------------------------------------------- query rotation

// turboquant_prepare_query (inference.rs:954-968): q_rot = R q, q_proj = R' q_rot,
// written as ws_q[s][h][2][D].  grid (n_heads, n_seq), one wave.
template <int D>
__global__ __launch_bounds__(64) void turbo_query_kernel(const DecodeLaunch p) {
    constexpr int J = D / 64;
    const int lane = threadIdx.x;
    const int h = blockIdx.x, s = blockIdx.y;
    const int g = h / (p.n_heads / p.n_kv_heads);
    const uint8_t* sg = p.turbo_signs + (size_t)g * (D / 8);
    const int64_t ss = p.turbo_slot_stride;
    const float* q = p.q + ((size_t)s * p.n_heads + h) * D;
    float* out = p.ws_q + ((size_t)s * p.n_heads + h) * 2 * D;
    float x[J];
#pragma unroll
    for (int j = 0; j < J; j++) x[j] = q[lane + 64 * j];
    wave_transform<D>(x, sg, sg + ss, lane);
#pragma unroll
    for (int j = 0; j < J; j++) out[lane + 64 * j] = x[j];
    wave_transform<D>(x, sg + 2 * ss, sg + 3 * ss, lane);
#pragma unroll
    for (int j = 0; j < J; j++) out[D + lane + 64 * j] = x[j];
}

// ---------------------------------------------------------------- split-K decode

namespace {

__device__ __forceinline__ f32x4 mma16(const uint4& a, const uint4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b),
                                                  c, 0, 0, 0);
}

typedef _Float16 tq_half2 __attribute__((ext_vector_type(2)));
typedef float tq_float2 __attribute__((ext_vector_type(2)));

// f16 hi/lo words of two floats (round to nearest even; one v_cvt_pk_f16_f32 each)
__device__ __forceinline__ void split2(float a0, float a1, uint32_t& hi, uint32_t& lo) {
    const tq_half2 h = __builtin_convertvector(tq_float2{a0, a1}, tq_half2);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(tq_float2{a0 - (float)h[0], a1 - (float)h[1]}, tq_half2));
}

// Lookup tables of the +-1 / 0 MFMA operands (f16 +1 = 0x3C00, -1 = 0xBC00):
//   lut_c[byte of 4 codes] = {a_s of elements 0-1, 2-3, a_sb of elements 0-1, 2-3}
//     a_s  = sign of the centroid (code bit 1), a_sb = a_s for the outer
//     centroids (codes 0, 3) and 0 for the inner ones: C = c0 a_s + (c1 - c0) a_sb;
//   lut_g[byte of 8 residual sign bits] = a_g of elements 0-7 (bit set = +1).
__device__ __forceinline__ void build_luts(uint4* lut_c, uint4* lut_g, int tid) {
    if (tid < 256) {
        uint32_t hs[4], hb[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int c = (tid >> (2 * e)) & 3;
            hs[e] = c >= 2 ? 0x3C00u : 0xBC00u;
            hb[e] = (c == 0 || c == 3) ? hs[e] : 0u;
        }
        lut_c[tid] = make_uint4(hs[0] | (hs[1] << 16), hs[2] | (hs[3] << 16), hb[0] | (hb[1] << 16),
                                hb[2] | (hb[3] << 16));
        uint32_t g[4];
#pragma unroll
        for (int w = 0; w < 4; w++)
            g[w] = (((tid >> (2 * w)) & 1) ? 0x3C00u : 0xBC00u) | ((((tid >> (2 * w + 1)) & 1) ? 0x3C00u : 0xBC00u) << 16);
        lut_g[tid] = make_uint4(g[0], g[1], g[2], g[3]);
    }
}

// 2-bit fields at bits 0-1 of each byte of v -> one byte (byte i at bits 2i)
__device__ __forceinline__ uint32_t gather2(uint32_t v) {
    v &= 0x03030303u;
    v |= v >> 6;
    v |= v >> 12;
    return v & 0xffu;
}
// bit 0 of each byte of v -> one nibble (byte i at bit i)
__device__ __forceinline__ uint32_t gather1(uint32_t v) {
    v &= 0x01010101u;
    v |= v >> 7;
    v |= v >> 14;
    return v & 0xfu;
}

// Raw buffer access: a wave-uniform base in a scalar descriptor plus a 32-bit
// byte offset per lane (gfx9-family descriptor word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)0xffffffff, 0x00020000);
}

__device__ __forceinline__ float pow2_for(float vmax, int top) {
    int ex;
    (void)frexpf(vmax, &ex);  // vmax = m 2^ex, m in [0.5, 1)
    return vmax > 0.0f ? ldexpf(1.0f, min(max(top - ex, -120), 120)) : 1.0f;
}

}  // namespace

constexpr int kTdThreads = 256;
constexpr int kTdWaves = kTdThreads / 64;

// One workgroup per (split, kv head, sequence); each wave streams 32-key tiles.
//   S^T[key][q] = sigma (c0 (A_s . B_rot) + (c1 - c0) (A_sb . B_rot)) + r (A_g . B_proj)
//     A = +-1/0 operands of the key row from the lookup tables (lane: key l16,
//     its D/4 contiguous dims), B = the rotated / projected query as f16 hi + lo;
//   O_base^T += A_s^T . (c0 P sigma) + A_sb^T . ((c1 - c0) P sigma),
//   O_res^T  += A_g^T . (P r)
//     A^T operands from the tile's code / sign bytes, staged byte-transposed in LDS.
// sigma and r = gamma sqrt(pi/2/D) of the tile's keys go through LDS as well
// (one coalesced load per lane).  Partials: ws_o [s][h][split][2][D] (base,
// residual), ws_ml as the other decodes.
// PACK: token-packed prefill (DecodeLaunch::tok_pack): column c of the MFMAs is
// token s * tok_pack + c / kv_mul, query head g * kv_mul + c % kv_mul, masked to
// that token's own visible keys.
template <int D, bool PACK>
__global__ __launch_bounds__(kTdThreads, 2) void decode_turbo_kernel(const DecodeLaunch p) {
    static_assert(D == 128, "decode_turbo_kernel: lane layouts are sized for head_dim 128");
    constexpr int TILE = 32;
    constexpr int KS = D / 32;   // MFMA k-steps over d
    constexpr int DQ = D / 4;    // dims per lane group in the score pass
    constexpr int NBC = D / 4;   // code bytes per head row
    constexpr int NSC = D / 8;   // sign bytes per head row
    constexpr int DT = D / 16;   // output tiles
    constexpr float kLazy = 8.0f;
    // LDS: lookup tables | per wave: codes [NBC][TILE] and signs [NSC][TILE] bytes
    // (byte-transposed), aux [4][TILE] floats (sigma_k, r_k, sigma_v, r_v)
    constexpr int kLutBytes = 2 * 256 * 16;
    constexpr int kWaveBytes = (NBC + NSC) * TILE + 4 * TILE * 4;
    constexpr int kLoopBytes = kLutBytes + kTdWaves * kWaveBytes;
    constexpr int kMergeBytes = (kTdWaves * 16 * (2 * D + 1) + 2 * kTdWaves * 16) * 4;
    __shared__ __attribute__((aligned(16))) char smem[kLoopBytes > kMergeBytes ? kLoopBytes : kMergeBytes];
    const int split = blockIdx.x, g = blockIdx.y, s = blockIdx.z;
    const int e_rng = PACK ? s * p.tok_pack : s;  // batch entry holding the key range
    const int t_begin = p.kv_start[e_rng] + split * p.split_keys;
    const int t_limit = p.kv_end[e_rng];
    if (t_begin >= t_limit) return;
    const int t_stop = min(t_limit, t_begin + p.split_keys);
    const int kv_mul = p.n_heads / p.n_kv_heads;
    // MFMA column c: batch entry col_tok(c), query head col_head(c)
    const int n_col = PACK ? p.tok_pack * kv_mul : kv_mul;
    auto col_tok = [&](int c) { return PACK ? s * p.tok_pack + c / kv_mul : s; };
    auto col_head = [&](int c) { return g * kv_mul + (PACK ? c % kv_mul : c); };
    auto col_ok = [&](int c) { return c < n_col && (!PACK || col_tok(c) < p.n_seq); };
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g4 = lane >> 4;
    uint4* lut_c = (uint4*)smem;
    uint4* lut_g = lut_c + 256;
    uint8_t* cT = (uint8_t*)smem + kLutBytes + wave * kWaveBytes;  // [NBC][TILE]
    uint8_t* sT = cT + NBC * TILE;                                 // [NSC][TILE]
    float* auxT = (float*)(sT + NSC * TILE);                       // [4][TILE]
    build_luts(lut_c, lut_g, tid);
    __syncthreads();

    // B operands of the score pass: lane (query l16, group g4), k-step k holds dims
    // DQ g4 + 8 k .. +7 (the same dims the A operand of the lane's key carries),
    // scaled by a power of two that puts the row maximum near 2^14.
    uint4 bq[KS], bql[KS], bp[KS], bpl[KS];
    float qback_c = 1.0f, qback_r = 1.0f;
    {
        const bool qv = col_ok(l16);
        const int qc = qv ? l16 : 0;
        const float* qr = p.ws_q + ((size_t)col_tok(qc) * p.n_heads + col_head(qc)) * 2 * D;
        const float qs = p.score_scale * kLog2e;
        float mr = 0.0f, mp = 0.0f;
#pragma unroll
        for (int e = 0; e < DQ; e++) {
            mr = fmaxf(mr, qv ? fabsf(qr[DQ * g4 + e]) : 0.0f);
            mp = fmaxf(mp, qv ? fabsf(qr[D + DQ * g4 + e]) : 0.0f);
        }
        mr = fmaxf(mr, __shfl_xor(mr, 16, 64));
        mr = fmaxf(mr, __shfl_xor(mr, 32, 64));
        mp = fmaxf(mp, __shfl_xor(mp, 16, 64));
        mp = fmaxf(mp, __shfl_xor(mp, 32, 64));
        const float pr = pow2_for(mr * qs, 14), pp = pow2_for(mp * qs, 14);
        qback_c = 1.0f / pr;
        qback_r = 1.0f / pp;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            uint32_t hr[4], lr[4], hp[4], lp[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const int d0 = DQ * g4 + 8 * k + 2 * w;
                split2(qv ? qr[d0] * qs * pr : 0.0f, qv ? qr[d0 + 1] * qs * pr : 0.0f, hr[w], lr[w]);
                split2(qv ? qr[D + d0] * qs * pp : 0.0f, qv ? qr[D + d0 + 1] * qs * pp : 0.0f, hp[w], lp[w]);
            }
            bq[k] = make_uint4(hr[0], hr[1], hr[2], hr[3]);
            bql[k] = make_uint4(lr[0], lr[1], lr[2], lr[3]);
            bp[k] = make_uint4(hp[0], hp[1], hp[2], hp[3]);
            bpl[k] = make_uint4(lp[0], lp[1], lp[2], lp[3]);
        }
    }

    // wave-uniform bases of (slot, kv head); per-key offsets in 32 bits
    const size_t slot = (size_t)(p.seq_slot ? p.seq_slot[s] : s);
    const int64_t e0 = (int64_t)slot * p.seq_stride + (int64_t)g * D;
    const __amdgpu_buffer_rsrc_t kbh = buf_rsrc((const uint8_t*)p.k_cache + e0 / 4);
    const __amdgpu_buffer_rsrc_t vbh = buf_rsrc((const uint8_t*)p.v_cache + e0 / 4);
    const __amdgpu_buffer_rsrc_t ksh = buf_rsrc((const uint8_t*)p.k_sign + e0 / 8);
    const __amdgpu_buffer_rsrc_t vsh = buf_rsrc((const uint8_t*)p.v_sign + e0 / 8);
    const int64_t a0 = (int64_t)slot * p.scale_seq_stride + g;
    const __amdgpu_buffer_rsrc_t ksig = buf_rsrc(p.k_scale + a0);
    const __amdgpu_buffer_rsrc_t kgam = buf_rsrc(p.k_rnorm + a0);
    const __amdgpu_buffer_rsrc_t vsig = buf_rsrc(p.v_scale + a0);
    const __amdgpu_buffer_rsrc_t vgam = buf_rsrc(p.v_rnorm + a0);
    const uint32_t rsc = (uint32_t)(p.row_stride / 4), rss = (uint32_t)(p.row_stride / 8);
    const uint32_t ars = (uint32_t)p.scale_row_stride;
    const float rfac = sqrtf(kFracPi2 / (float)D);

    // per-tile registers: K codes / signs of the lane's key in both 16-key sub-tiles,
    // V code / sign bytes for the staging (lane: key lane/2, half lane%2 of the row),
    // the lane's aux pair (key lane%32; K for lanes < 32, V above)
    // keys [c_lo, c_hi) of this split are visible to the lane's column
    int c_lo = t_begin, c_hi = t_stop;
    if constexpr (PACK) {
        const bool ok = col_ok(l16);
        c_lo = ok ? p.col_start[col_tok(l16)] : 0;
        c_hi = ok ? min(p.col_end[col_tok(l16)], t_stop) : 0;
    }

    uint2 kc[2];
    uint32_t ksb[2];
    uint4 vcw;
    uint2 vsw;
    float xs, xg;
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            const uint32_t key = (uint32_t)min(t0 + 16 * sb + l16, t_stop - 1);
            const auto v2 = __builtin_amdgcn_raw_buffer_load_b64(kbh, (int)(key * rsc + 8 * g4), 0, 0);
            kc[sb] = make_uint2(v2[0], v2[1]);
            ksb[sb] = __builtin_amdgcn_raw_buffer_load_b32(ksh, (int)(key * rss + 4 * g4), 0, 0);
        }
        {
            const uint32_t key = (uint32_t)min(t0 + (lane >> 1), t_stop - 1);
            const auto v4 = __builtin_amdgcn_raw_buffer_load_b128(vbh, (int)(key * rsc + 16 * (lane & 1)), 0, 0);
            vcw = make_uint4(v4[0], v4[1], v4[2], v4[3]);
            const auto v2 = __builtin_amdgcn_raw_buffer_load_b64(vsh, (int)(key * rss + 8 * (lane & 1)), 0, 0);
            vsw = make_uint2(v2[0], v2[1]);
        }
        {
            const int off = (int)((uint32_t)min(t0 + (lane & 31), t_stop - 1) * ars * 4);
            if (lane < 32) {
                xs = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ksig, off, 0, 0));
                xg = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(kgam, off, 0, 0));
            } else {
                xs = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(vsig, off, 0, 0));
                xg = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(vgam, off, 0, 0));
            }
        }
    };

    f32x4 ob[DT], orr[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) ob[dt] = orr[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrow = -1e30f, lrow = 0.0f;
    float pwb = 1.0f, pwr = 1.0f;  // power-of-two range factors of the two P operands
    bool pw_set = false;

    const int n_tiles = (t_stop - t_begin + TILE - 1) / TILE;
    int it = wave;
    if (it < n_tiles) load_tile(t_begin + it * TILE);
    for (; it < n_tiles; it += kTdWaves) {
        const int t0 = t_begin + it * TILE;
        // stage: V bytes transposed to [byte column][key]; aux as [4][key]
        {
            const int key = lane >> 1, col_c = (lane & 1) * (NBC / 2), col_s = (lane & 1) * (NSC / 2);
            const uint32_t wc[4] = {vcw.x, vcw.y, vcw.z, vcw.w};
            const uint32_t ws[2] = {vsw.x, vsw.y};
#pragma unroll
            for (int b = 0; b < 16; b++) cT[(col_c + b) * TILE + key] = (uint8_t)(wc[b >> 2] >> (8 * (b & 3)));
#pragma unroll
            for (int b = 0; b < 8; b++) sT[(col_s + b) * TILE + key] = (uint8_t)(ws[b >> 2] >> (8 * (b & 3)));
            const int a = 2 * (lane >> 5);
            auxT[a * TILE + (lane & 31)] = xs;
            auxT[(a + 1) * TILE + (lane & 31)] = xg * rfac;
        }
        // scores
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 s1[2], s2[2], sr[2];
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
#pragma unroll
            for (int k = 0; k < KS; k++) {
                const uint32_t c16 = (k < 2 ? kc[sb].x : kc[sb].y) >> (16 * (k & 1));
                const uint4 e0l = lut_c[c16 & 0xffu], e1l = lut_c[(c16 >> 8) & 0xffu];
                const uint4 ag = lut_g[(ksb[sb] >> (8 * k)) & 0xffu];
                const uint4 as = make_uint4(e0l.x, e0l.y, e1l.x, e1l.y);
                const uint4 asb = make_uint4(e0l.z, e0l.w, e1l.z, e1l.w);
                s1[sb] = mma16(as, bq[k], k == 0 ? zero : s1[sb]);
                s1[sb] = mma16(as, bql[k], s1[sb]);
                s2[sb] = mma16(asb, bq[k], k == 0 ? zero : s2[sb]);
                s2[sb] = mma16(asb, bql[k], s2[sb]);
                sr[sb] = mma16(ag, bp[k], k == 0 ? zero : sr[sb]);
                sr[sb] = mma16(ag, bpl[k], sr[sb]);
            }
        }
        __builtin_amdgcn_wave_barrier();  // aux stores precede the reads below (in-order LDS)
        float sv[8], vsg[8], vrr[8];
        const bool tail = t0 + TILE > t_stop;
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            const float4 ks4 = *(const float4*)(auxT + 0 * TILE + 16 * sb + 4 * g4);
            const float4 kr4 = *(const float4*)(auxT + 1 * TILE + 16 * sb + 4 * g4);
            const float4 vs4 = *(const float4*)(auxT + 2 * TILE + 16 * sb + 4 * g4);
            const float4 vr4 = *(const float4*)(auxT + 3 * TILE + 16 * sb + 4 * g4);
            const float ksv[4] = {ks4.x, ks4.y, ks4.z, ks4.w}, krv[4] = {kr4.x, kr4.y, kr4.z, kr4.w};
            const float vsv[4] = {vs4.x, vs4.y, vs4.z, vs4.w}, vrv[4] = {vr4.x, vr4.y, vr4.z, vr4.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = 4 * sb + j;
                const int key = t0 + 16 * sb + 4 * g4 + j;
                const float base = (kTqC0 * s1[sb][j] + (kTqC1 - kTqC0) * s2[sb][j]) * qback_c;
                const float v = ksv[j] * base + krv[j] * (sr[sb][j] * qback_r);
                if constexpr (PACK) sv[e] = (key >= c_lo && key < c_hi) ? v : -INFINITY;
                else sv[e] = (!tail || key < t_stop) ? v : -INFINITY;
                vsg[e] = vsv[j];
                vrr[e] = vrv[j];
            }
        }
        if (it + kTdWaves < n_tiles) load_tile(t_begin + (it + kTdWaves) * TILE);

        float mx = sv[0];
#pragma unroll
        for (int e = 1; e < 8; e++) mx = fmaxf(mx, sv[e]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        if (__any(mx > mrow + kLazy)) {
            const float mnew = fmaxf(mrow, mx);
            const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
            mrow = mnew;
            lrow *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                ob[dt] *= alpha;
                orr[dt] *= alpha;
            }
        }
        float pv[8], psum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            pv[e] = __builtin_amdgcn_exp2f(sv[e] - mrow);
            psum += pv[e];
        }
        lrow += psum;
        // range factors: the tile's largest sigma / r scaled into [2^5, 2^6)
        {
            float lb = 0.0f, lr = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                lb = fmaxf(lb, vsg[e]);
                lr = fmaxf(lr, vrr[e]);
            }
            if (!pw_set || __any(lb * pwb >= 64.0f || lr * pwr >= 64.0f)) {
                const float nb = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(pow2_for(wave_max<64>(lb), 6))));
                const float nr = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(pow2_for(wave_max<64>(lr), 6))));
                if (!pw_set) {
                    pwb = nb;
                    pwr = nr;
                } else {
                    if (nb < pwb) {
                        const float f = nb / pwb;
#pragma unroll
                        for (int dt = 0; dt < DT; dt++) ob[dt] *= f;
                        pwb = nb;
                    }
                    if (nr < pwr) {
                        const float f = nr / pwr;
#pragma unroll
                        for (int dt = 0; dt < DT; dt++) orr[dt] *= f;
                        pwr = nr;
                    }
                }
                pw_set = true;
            }
        }
        // P operands: k-slot r <-> key 16 (r/4) + 4 g4 + r%4, i.e. pv[r]
        uint4 pc0, pc0l, pc1, pc1l, pr, prl;
        {
            uint32_t h0[4], l0[4], h1[4], l1[4], hr[4], lr[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float b0 = pv[2 * w] * vsg[2 * w] * pwb, b1 = pv[2 * w + 1] * vsg[2 * w + 1] * pwb;
                split2(kTqC0 * b0, kTqC0 * b1, h0[w], l0[w]);
                split2((kTqC1 - kTqC0) * b0, (kTqC1 - kTqC0) * b1, h1[w], l1[w]);
                split2(pv[2 * w] * vrr[2 * w] * pwr, pv[2 * w + 1] * vrr[2 * w + 1] * pwr, hr[w], lr[w]);
            }
            pc0 = make_uint4(h0[0], h0[1], h0[2], h0[3]);
            pc0l = make_uint4(l0[0], l0[1], l0[2], l0[3]);
            pc1 = make_uint4(h1[0], h1[1], h1[2], h1[3]);
            pc1l = make_uint4(l1[0], l1[1], l1[2], l1[3]);
            pr = make_uint4(hr[0], hr[1], hr[2], hr[3]);
            prl = make_uint4(lr[0], lr[1], lr[2], lr[3]);
        }
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const int d = 16 * dt + l16;
            // codes / sign bits of dim d for keys 4 g4 + j and 16 + 4 g4 + j
            const uint32_t c_lo = *(const uint32_t*)(cT + (d >> 2) * TILE + 4 * g4);
            const uint32_t c_hi = *(const uint32_t*)(cT + (d >> 2) * TILE + 16 + 4 * g4);
            const uint32_t s_lo = *(const uint32_t*)(sT + (d >> 3) * TILE + 4 * g4);
            const uint32_t s_hi = *(const uint32_t*)(sT + (d >> 3) * TILE + 16 + 4 * g4);
            const int cs = 2 * (d & 3), bs = d & 7;
            const uint4 e0l = lut_c[gather2(c_lo >> cs)], e1l = lut_c[gather2(c_hi >> cs)];
            const uint4 ag = lut_g[gather1(s_lo >> bs) | (gather1(s_hi >> bs) << 4)];
            const uint4 as = make_uint4(e0l.x, e0l.y, e1l.x, e1l.y);
            const uint4 asb = make_uint4(e0l.z, e0l.w, e1l.z, e1l.w);
            ob[dt] = mma16(as, pc0, ob[dt]);
            ob[dt] = mma16(as, pc0l, ob[dt]);
            ob[dt] = mma16(asb, pc1, ob[dt]);
            ob[dt] = mma16(asb, pc1l, ob[dt]);
            orr[dt] = mma16(ag, pr, orr[dt]);
            orr[dt] = mma16(ag, prl, orr[dt]);
        }
        __builtin_amdgcn_wave_barrier();  // reads done before the next tile's stores
    }
    if (pw_set) {
        const float ib = 1.0f / pwb, ir = 1.0f / pwr;  // exact: powers of two
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            ob[dt] *= ib;
            orr[dt] *= ir;
        }
    }

    lrow += __shfl_xor(lrow, 16, 64);
    lrow += __shfl_xor(lrow, 32, 64);
    __syncthreads();
    float (*sh_o)[16][2 * D + 1] = (float (*)[16][2 * D + 1])smem;
    float (*sh_m)[16] = (float (*)[16])((float*)smem + kTdWaves * 16 * (2 * D + 1));
    float (*sh_l)[16] = sh_m + kTdWaves;
    if (g4 == 0) {
        sh_m[wave][l16] = mrow;
        sh_l[wave][l16] = lrow;
    }
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sh_o[wave][l16][16 * dt + 4 * g4 + j] = ob[dt][j];
            sh_o[wave][l16][D + 16 * dt + 4 * g4 + j] = orr[dt][j];
        }
    __syncthreads();
    const int n_splits = p.n_splits;
    for (int idx = tid; idx < n_col * 2 * D; idx += kTdThreads) {
        const int q = idx / (2 * D), i = idx % (2 * D);
        if (!col_ok(q)) continue;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kTdWaves; w++) mx = fmaxf(mx, sh_m[w][q]);
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int w = 0; w < kTdWaves; w++) {
            const float a = exp2f(sh_m[w][q] - mx);
            lt += sh_l[w][q] * a;
            ot += sh_o[w][q][i] * a;
        }
        const size_t part = ((size_t)col_tok(q) * p.n_heads + col_head(q)) * n_splits + split;
        p.ws_o[part * 2 * D + i] = ot;
        if (i == 0) {
            p.ws_ml[part * 2 + 0] = mx;
            p.ws_ml[part * 2 + 1] = lt;
        }
    }
}

// ---------------------------------------------------------------- merge + finalize

// One wave per (head, sequence): merge the split partials of the base and residual
// accumulators (log2-domain weights), divide by the softmax sum, then
// finalize_turboquant_value_head (inference.rs:1323-1334): residual <- R'^-1
// residual, base += residual, out = R^-1 base.
template <int D>
__global__ __launch_bounds__(64) void turbo_combine_kernel(const DecodeLaunch p) {
    constexpr int J = D / 64;
    const int lane = threadIdx.x;
    const int h = blockIdx.x, s = blockIdx.y;
    const int g = h / (p.n_heads / p.n_kv_heads);
    const int t_len = p.kv_end[s] - p.kv_start[s];
    const int n_used = t_len > 0 ? (t_len + p.split_keys - 1) / p.split_keys : 0;
    const size_t part0 = ((size_t)s * p.n_heads + h) * p.n_splits;
    float mx = -INFINITY;
    for (int sp = lane; sp < n_used; sp += 64) mx = fmaxf(mx, p.ws_ml[(part0 + sp) * 2]);
    mx = wave_max<64>(mx);
    float lt = 0.0f;
    for (int sp = lane; sp < n_used; sp += 64) lt += p.ws_ml[(part0 + sp) * 2 + 1] * exp2f(p.ws_ml[(part0 + sp) * 2] - mx);
    lt = wave_sum<64>(lt);
    float b[J], r[J];
#pragma unroll
    for (int j = 0; j < J; j++) b[j] = r[j] = 0.0f;
    for (int sp = 0; sp < n_used; sp++) {
        const float w = exp2f(p.ws_ml[(part0 + sp) * 2] - mx);
        const float* o = p.ws_o + (part0 + sp) * 2 * D;
#pragma unroll
        for (int j = 0; j < J; j++) {
            b[j] += o[lane + 64 * j] * w;
            r[j] += o[D + lane + 64 * j] * w;
        }
    }
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        b[j] *= inv;
        r[j] *= inv;
    }
    const uint8_t* sg = p.turbo_signs + (size_t)g * (D / 8);
    const int64_t ss = p.turbo_slot_stride;
    wave_transform<D>(r, sg + 3 * ss, sg + 2 * ss, lane);  // res_post, res_pre: inverse
#pragma unroll
    for (int j = 0; j < J; j++) b[j] += r[j];
    wave_transform<D>(b, sg + ss, sg, lane);  // rot_post, rot_pre: inverse
    float* out = p.out + ((size_t)s * p.n_heads + h) * D;
#pragma unroll
    for (int j = 0; j < J; j++) out[lane + 64 * j] = b[j];
}

bool decode_turbo_supported(const DecodeLaunch& p) {
    return p.head_dim == 128 && p.n_heads / p.n_kv_heads <= 16;
}

hipError_t launch_decode_turbo(const DecodeLaunch& p, hipStream_t st) {
    if (p.head_dim != 128) return hipErrorInvalidValue;
    turbo_query_kernel<128><<<dim3(p.n_heads, p.n_seq), 64, 0, st>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.tok_pack > 0)
        decode_turbo_kernel<128, true><<<dim3(p.n_splits, p.n_kv_heads, (p.n_seq + p.tok_pack - 1) / p.tok_pack),
                                         kTdThreads, 0, st>>>(p);
    else
        decode_turbo_kernel<128, false><<<dim3(p.n_splits, p.n_kv_heads, p.n_seq), kTdThreads, 0, st>>>(p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    turbo_combine_kernel<128><<<dim3(p.n_heads, p.n_seq), 64, 0, st>>>(p);
    return hipGetLastError();
}

}  // namespace gr
