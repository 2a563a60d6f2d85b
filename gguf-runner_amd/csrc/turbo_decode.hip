// Split-K decode over a Turbo KV cache (KvCacheFormat::Turbo, the reference's
// default; inference.rs:346-1334), head_dim 64, 128 or 256, on f16 MFMA.
//
// Per key t of a KV head the cache holds 2-bit codes c (bits b1 b0), residual
// sign bits g, sigma_t and gamma_t.  With alpha = (c0 + c1) / 2 and
// beta = (c1 - c0) / 2 every centroid is C(c) = alpha (2 b1 - 1) + beta (2 b0 - 1),
// so the reference's score and value sums (dot_/axpy_turboquant_head,
// inference.rs:1246-1310)
//   score_t = sigma_t q_rot . C(c_t) + r_t q_proj . (2 g_t - 1),   r_t = gamma_t sqrt(pi/2/D)
//   base    = sum_t p_t sigma_t C(c_t),   residual = sum_t p_t r_t (2 g_t - 1)
// become sums over single bits:
//   q_rot . C(c)   = 2 sum_i q_i (alpha b1_i + beta b0_i) - (alpha + beta) sum_i q_i
//   q_proj . (2g-1) = 2 sum_i q_i g_i - sum_i q_i
// (and the same for the value side with the running sums sum_t p_t sigma_t,
// sum_t p_t r_t).  The bit sums run on v_mfma_f32_16x16x32_f16 with A operands
// built by a shift and an AND per dword: a dword with single bits at positions p
// and 16 + p is the f16 pair (b 2^e(p), b' 2^e(p)) with 2^e(p) the value of bit p
// alone.  Only p = 10..14 are used (2^-14, 2^-13, 2^-11, 2^-7, 2): the matrix
// cores sum products of a subnormal single-bit A with 10 - p fewer significant
// bits (measured on MI355X), while normal A keeps the f32 sum exact to 2^-24.
// On the key side the factor 2^-e(p) rides on the query operand (f16 hi + lo,
// prepared once per query by turbo_query_kernel); on the value side it is one
// exact scale per output row.  Products are exact, sums are f32.
#include <algorithm>
#include <atomic>

#include "gr_common.hpp"
#include "gr_internal.hpp"
#include "stream_sched.hpp"
#include "turbo_common.hpp"

namespace gr {

hipError_t launch_turbo_combine(const DecodeLaunch& p, hipStream_t st);  // turbo.hip

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 th2 __attribute__((ext_vector_type(2)));
typedef float tf2 __attribute__((ext_vector_type(2)));

constexpr float kAlpha = 0.5f * (tq::kC0 + tq::kC1);  // weight of (2 b1 - 1)
constexpr float kBeta = 0.5f * (tq::kC1 - tq::kC0);   // weight of (2 b0 - 1)

// Shapes per head_dim.
template <int D>
struct Tq {
    static constexpr int NCW = D / 64;                   // code dwords per key and lane group (score pass)
    static constexpr int NSW = D >= 128 ? D / 128 : 0;   // sign dwords per key and lane group (D 64: a half)
    static constexpr int KSC = D / 16;                   // code k-steps (16 A dwords per code dword)
    static constexpr int KSS = D / 32;                   // sign k-steps
    static constexpr int KS = KSC + KSS;
    static constexpr int RT = D / 16;                    // value-pass row tiles = dims per lane field
    static constexpr int RB = D / 4 + D / 8;             // bytes per cached head row (codes | signs)
    static constexpr int QBW = 32 * KS + 16;             // ws_q dwords per (entry, head)
};

// Exponent of the f16 whose only set bit is p (10 <= p <= 14): 2^(2^(p-10) - 15).
__host__ __device__ constexpr int bit_exp(int p) { return (1 << (p - 10)) - 15; }

// Score pass: A dword a (0..15) of a 32-bit source word pairs the word's bits a
// (low half) and a + 16 (high half), moved by the shift ka_shift(a) (negative:
// right) to bit ka_pos(a) of each half; a = 0..4 -> 10..14, 5..9 -> 10..14, ...
__host__ __device__ constexpr int ka_shift(int a) { return 10 - 5 * (a / 5); }
__host__ __device__ constexpr int ka_pos(int a) { return a + ka_shift(a); }
// Value pass, code rows: dim j (0..7) of a 16-bit code field has its b1 bit at
// 2j + 1 and b0 at 2j; shifting the pair word by vc_shift(j) (b1) and
// vc_shift(j) + 1 (b0) puts both at vc_pos(j) in {10, 12, 14}.
__host__ __device__ constexpr int vc_shift(int j) { return 9 - 6 * (j / 3); }
__host__ __device__ constexpr int vc_pos(int j) { return 2 * j + 1 + vc_shift(j); }
// Value pass, sign rows: bit j of the field, shifted by vs_shift(j), at vs_pos(j).
__host__ __device__ constexpr int vs_shift(int j) { return 10 - 5 * (j / 5); }
__host__ __device__ constexpr int vs_pos(int j) { return j + vs_shift(j); }

template <int S>
__device__ __forceinline__ uint32_t shl(uint32_t x) {
    if constexpr (S >= 0) return x << S;
    else return x >> -S;
}

// The query slot behind dword m (half 0 / 1) of k-step s of lane group g4 in the
// score pass.  Code k-steps come in fours from one 32-bit code word w of the
// group (16 codes: bit 2i+1 = b1, bit 2i = b0 of element i); A dword a = 4 (s % 4)
// + m of the word carries its bits k = a (half 0) and a + 16 (half 1) at bit
// ka_pos(a).  Sign k-steps do the same over 32-bit sign words (D 64: a 16-bit
// half whose bits 8..15 are first moved to 16..23).
template <int D>
__host__ __device__ constexpr void score_slot(int g4, int s, int m, int half, bool& is_sign, int& dim, int& p,
                                              float& coef) {
    using S = Tq<D>;
    if (s < S::KSC) {
        const int a = 4 * (s & 3) + m, k = half ? a + 16 : a;
        p = ka_pos(a);
        dim = 16 * (g4 * S::NCW + (s >> 2)) + (k >> 1);
        coef = (k & 1) ? kAlpha : kBeta;
        is_sign = false;
        return;
    }
    const int s2 = s - S::KSC;
    is_sign = true;
    coef = 1.0f;
    if constexpr (D >= 128) {
        const int a = 4 * (s2 & 3) + m, k = half ? a + 16 : a;
        p = ka_pos(a);
        dim = 32 * (g4 * S::NSW + (s2 >> 2)) + k;
    } else {
        const int a = 4 * s2 + m;
        p = ka_pos(a);
        dim = 16 * g4 + (half ? 8 + a : a);
    }
}

// A dwords a = 4 q4 .. 4 q4 + 3 of a 32-bit source word (see score_slot)
template <int Q4>
__device__ __forceinline__ uint4 score_a(uint32_t w) {
    uint32_t r[4];
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const int a = 4 * Q4 + m;
        const uint32_t x = ka_shift(a) == 10 ? shl<10>(w) : ka_shift(a) == 5 ? shl<5>(w)
                         : ka_shift(a) == 0 ? w : shl<-5>(w);
        r[m] = x & (0x00010001u << ka_pos(a));
    }
    return make_uint4(r[0], r[1], r[2], r[3]);
}

// f16 hi / lo words of two floats (round to nearest even)
__device__ __forceinline__ void split2(float a0, float a1, uint32_t& hi, uint32_t& lo) {
    const th2 h = __builtin_convertvector(tf2{a0, a1}, th2);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(tf2{a0 - (float)h[0], a1 - (float)h[1]}, th2));
}

__device__ __forceinline__ f32x4 mma16(const uint4& a, const uint4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b),
                                                  c, 0, 0, 0);
}

// value of the lane's partner lane ^ 1 (DPP quad_perm [1, 0, 3, 2])
__device__ __forceinline__ float dpp_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}

// max / sum over the four lane rows l16 + 16 r (rows swapped in pairs, then halves)
__device__ __forceinline__ float rows_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// f16 words of two floats for a lane that carries piece `lo` of them: the f16
// rounding (lo = 0) or the f16 rounding of the residual x - f16(x) (lo = 1).
__device__ __forceinline__ uint32_t piece2(float a0, float a1, float lo) {
    const th2 h = __builtin_convertvector(tf2{a0, a1}, th2);
    return __builtin_bit_cast(uint32_t,
                              __builtin_convertvector(tf2{a0 - lo * (float)h[0], a1 - lo * (float)h[1]}, th2));
}

// Raw buffer access: a wave-uniform base in a scalar descriptor plus a 32-bit
// byte offset per lane (gfx9-family descriptor word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)0xffffffff, 0x00020000);
}

// n consecutive dwords (n = 1, 2, 4) at byte offset off
template <int N>
__device__ __forceinline__ void load_dwords(__amdgpu_buffer_rsrc_t r, int off, uint32_t* out) {
    if constexpr (N == 1) {
        out[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    } else if constexpr (N == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        out[0] = v[0];
        out[1] = v[1];
    } else {
        static_assert(N == 4, "load_dwords: 1, 2 or 4");
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        out[0] = v[0];
        out[1] = v[1];
        out[2] = v[2];
        out[3] = v[3];
    }
}

}  // namespace

// score_slot of every query-operand slot, tabulated at compile time for
// turbo_query_kernel: slot idx (lane + 64 i) and half h give the flat index
// (is_sign ? D : 0) + dim into the rotated / projected query and the factor
// coef * 2^-e(p).  The factor is coef scaled by a power of two (2^14 .. 2^-1), so
// factor * q rounds exactly as coef * q * 2^-e(p) does.
template <int D>
struct QSlots {
    static constexpr int NB = 16 * Tq<D>::KS;
    uint16_t idx[2][NB];
    float f[2][NB];
};

constexpr float pow2f(int e) {
    float r = 1.0f;
    for (; e > 0; e--) r *= 2.0f;
    for (; e < 0; e++) r *= 0.5f;
    return r;
}

template <int D>
constexpr QSlots<D> make_qslots() {
    QSlots<D> t{};
    for (int i = 0; i < QSlots<D>::NB; i++) {
        const int g4 = i / (4 * Tq<D>::KS), rem = i % (4 * Tq<D>::KS);
        for (int h = 0; h < 2; h++) {
            bool is_sign = false;
            int dim = 0, pp = 0;
            float coef = 0.0f;
            score_slot<D>(g4, rem >> 2, rem & 3, h, is_sign, dim, pp, coef);
            t.idx[h][i] = (uint16_t)((is_sign ? D : 0) + dim);
            t.f[h][i] = coef * pow2f(-bit_exp(pp));
        }
    }
    return t;
}

__constant__ QSlots<64> kQSlots64 = make_qslots<64>();
__constant__ QSlots<128> kQSlots128 = make_qslots<128>();
__constant__ QSlots<256> kQSlots256 = make_qslots<256>();

template <int D>
__device__ __forceinline__ const QSlots<D>& qslots() {
    if constexpr (D == 64) return kQSlots64;
    else if constexpr (D == 128) return kQSlots128;
    else return kQSlots256;
}

// ---------------------------------------------------------------- query preparation

// turboquant_prepare_query (inference.rs:954-968) for (head h, entry s), one wave:
// q_rot = R q, q_proj = R' q_rot, then the score pass's B operands in lane order,
// ws_q + (s * n_heads + h) * QBW:
//   [piece (hi, lo)][lane group g4][k-step][dword m]  f16 pairs of
//      coef * q * score_scale * log2(e) * 2^E / 2^e(p)  (score_slot gives the slot),
//      E = E_code for code k-steps, E_sign for sign k-steps (max |value| in [2^13, 2^14))
//   then 2^-E_code, 2^-E_sign, (alpha + beta) sum_i q_rot_i s, sum_i q_proj_i s.
template <int D>
__global__ __launch_bounds__(256) void turbo_query_kernel(const DecodeLaunch p) {
    using S = Tq<D>;
    constexpr int J = D / 64, KS = S::KS, NB = 16 * KS;
    __shared__ float qsh_all[4][2][D];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float (*qsh)[D] = qsh_all[wave];
    const int h = 4 * blockIdx.x + wave, s = blockIdx.y;  // four heads per workgroup
    if (h >= p.n_heads) return;  // whole wave; no workgroup barrier below
    const int g = h / (p.n_heads / p.n_kv_heads);
    const uint8_t* sg = p.turbo_signs + (size_t)g * (D / 8);
    const int64_t ss = p.turbo_slot_stride;
    const float* q = p.q + ((size_t)s * p.n_heads + h) * D;
    uint32_t* out = (uint32_t*)p.ws_q + ((size_t)s * p.n_heads + h) * S::QBW;
    const float qs = p.score_scale * kLog2e;
    float x[J];
#pragma unroll
    for (int j = 0; j < J; j++) x[j] = q[lane + 64 * j];
    tq::wave_transform<D>(x, sg, sg + ss, lane);  // rot_pre, rot_post
    float sr = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        qsh[0][lane + 64 * j] = x[j] * qs;
        sr += x[j] * qs;
    }
    tq::wave_transform<D>(x, sg + 2 * ss, sg + 3 * ss, lane);  // res_pre, res_post
    float sp = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        qsh[1][lane + 64 * j] = x[j] * qs;
        sp += x[j] * qs;
    }
    sr = wave_sum<64>(sr);
    sp = wave_sum<64>(sp);
    tq::wave_lds_sync();  // the wave's qsh stores precede its reads

    const float* qflat = &qsh[0][0];  // [rotated | projected]
    // one pass over the lane's slots (idx = lane + 64 i): values kept, maxima per plane
    constexpr int NI = (NB + 63) / 64;
    float v0[NI], v1[NI];
    bool sgn[NI];
    float mc = 0.0f, ms = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int idx = lane + 64 * i;
        v0[i] = v1[i] = 0.0f;
        sgn[i] = false;
        if (idx < NB) {
            const QSlots<D>& tab = qslots<D>();
            const int i0 = tab.idx[0][idx], i1 = tab.idx[1][idx];
            v0[i] = tab.f[0][idx] * qflat[i0];
            v1[i] = tab.f[1][idx] * qflat[i1];
            const bool is_sign = i0 >= D;  // the slot's k-step: both halves alike
            sgn[i] = is_sign;
            const float m = fmaxf(fabsf(v0[i]), fabsf(v1[i]));
            if (is_sign) ms = fmaxf(ms, m);
            else mc = fmaxf(mc, m);
        }
    }
    const float ec = tq::pow2_for(wave_max<64>(mc), 14), es = tq::pow2_for(wave_max<64>(ms), 14);
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int idx = lane + 64 * i;
        if (idx < NB) {
            const float sc = sgn[i] ? es : ec;
            uint32_t hi, lo;
            split2(v0[i] * sc, v1[i] * sc, hi, lo);
            out[idx] = hi;
            out[NB + idx] = lo;
        }
    }
    if (lane == 0) {
        float* c = (float*)(out + 2 * NB);
        c[0] = 1.0f / ec;
        c[1] = 1.0f / es;
        c[2] = (kAlpha + kBeta) * sr;
        c[3] = sp;
    }
}

// ---------------------------------------------------------------- split kernel

constexpr int kTsThreads = 256;
constexpr int kTsWaves = kTsThreads / 64;

// One workgroup per (split, kv head, sequence); each wave streams 32-key tiles
// (wave w: tiles w, w + 4, ...), keeps its own online-softmax state, and the
// waves merge in LDS.  Partials: ws_o [entry][head][split][2][D] (base and
// residual, rotated domain), ws_ml (m, l) in log2 units; turbo_combine_kernel
// merges the splits and applies the inverse rotations.
//
// Score pass, per 16-key sub-tile: A rows = keys (lane: key l16, group g4, which
// holds code dwords g4*NCW.. and sign dwords g4*NSW.. of its key), B = the
// prepared query slots; one accumulator for the code bits, one for the sign bits.
// Value pass: A rows = (lane field l16, row tile rt) = dim (D/16) l16 + rt, k =
// (key, bit plane) for the code rows and keys for the sign rows; the lane reads
// pair words [field bits of key a | field bits of key b] from the wave's staged
// V rows (as stored, no transpose); B = p sigma alpha / beta and p r.
//
// SPLIT: the hi and lo pieces of every B operand are separate MFMA columns
// (column 2i + piece = query column i, up to 8 of them), one MFMA per product;
// else the columns are the query columns (up to 16) and every product takes a hi
// and a lo MFMA.
// PACK: token-packed prefill (DecodeLaunch::tok_pack): query column i is token
// s * tok_pack + i / kv_mul, head g * kv_mul + i % kv_mul, masked to that
// token's own visible keys.
// STREAM: decode on the stream schedule (DecodeLaunch::stream_sched); else the
// fixed (split, column, entry) grid.
template <int D, bool PACK, bool SPLIT, bool STREAM>
__global__ __launch_bounds__(kTsThreads, (D <= 128 ? 2 : 1)) void turbo_split_kernel(const DecodeLaunch p) {
    static_assert(!(PACK && STREAM), "the token-packed prefill runs on the fixed grid");
    using S = Tq<D>;
    constexpr int TILE = 32;
    constexpr int NCW = S::NCW, NSW = S::NSW, KS = S::KS, KSC = S::KSC, RT = S::RT, RB = S::RB;
    constexpr int NF = D == 256 ? 2 : 1;  // 16-bit code fields per lane row in the value pass
    constexpr float kLazy = 8.0f;
    constexpr int kWaveBytes = TILE * RB + 4 * TILE * 4;  // V rows | aux [4][TILE]
    // !SPLIT: the lo pieces of the query operand, [g4][k-step][l16] uint4, in LDS
    // once for the four waves (they share the columns), read per MFMA
    constexpr int kBloBytes = SPLIT ? 0 : 4 * KS * 16 * 16;
    constexpr int kLoopBytes = kBloBytes + kTsWaves * kWaveBytes;
    constexpr int kMergeBytes = (kTsWaves * 16 * (2 * D + 1) + 2 * kTsWaves * 16) * 4;
    __shared__ __attribute__((aligned(16))) char smem[kLoopBytes > kMergeBytes ? kLoopBytes : kMergeBytes];

    // decode: column col = KV head g * n_sub + slice, query heads h0 .. h0 + n_col - 1
    // (DecodeLaunch::n_sub slices groups above 16 query heads)
    const int n_sub = (!PACK && p.n_sub > 0) ? p.n_sub : 1;
    const int kv_mul = p.n_heads / p.n_kv_heads;
    // Segment = keys [t_begin, t_stop) of entry s, column col; its partials go to
    // slot `split`.  Fixed grid: (split, column, entry) = blockIdx; decode on the
    // stream schedule (DecodeLaunch::stream_sched, stream_sched.hpp): the
    // segments of the workgroup's key range, one after another.
    constexpr bool stream = STREAM;
    __shared__ int st_len[STREAM ? kStreamMaxSeq : 1];
    __shared__ int st_off[STREAM ? kStreamMaxSeq : 1];
    __shared__ int st_first;
    __shared__ int st_wsum[kTsWaves];
    StreamCursor<kTsThreads> cur;
    int split, s, col, t_begin, t_stop;
    if (!stream) {
        split = blockIdx.x;
        // token-packed prefill: later row groups see more keys (causal), so they
        // are dispatched first and the short ones fill in behind them
        s = PACK ? (int)(gridDim.z - 1 - blockIdx.z) : (int)blockIdx.z;
        col = blockIdx.y;
        const int e_rng = PACK ? s * p.tok_pack : s;  // batch entry holding the key range
        t_begin = p.kv_start[e_rng] + split * p.split_keys;
        const int t_limit = p.kv_end[e_rng];
        if (t_begin >= t_limit) {
            if constexpr (PACK) {
                if (p.n_splits == 1) {  // no keys: the group's rows are zero (as the combine gives)
                    const int kv_mul = p.n_heads / p.n_kv_heads, n_col = p.tok_pack * kv_mul;
                    for (int i = threadIdx.x; i < n_col * D; i += kTsThreads) {
                        const int c = i / D, tok = s * p.tok_pack + c / kv_mul;
                        if (tok < p.n_seq) p.out[((size_t)tok * p.n_heads + blockIdx.y * kv_mul + c % kv_mul) * D + i % D] = 0.0f;
                    }
                }
            }
            return;
        }
        t_stop = min(t_limit, t_begin + p.split_keys);
    } else {
        if (!cur.init(p, p.n_kv_heads * n_sub, st_len, st_off, &st_first, st_wsum)) return;
        split = s = col = t_begin = t_stop = 0;  // set per segment below
    }
    for (;;) {
    if constexpr (stream) {
        if (!cur.segment(p, t_begin, t_stop, split)) break;  // the range ends inside the pair's virtual keys
        s = cur.s;
        col = cur.col;
        __syncthreads();  // the previous segment is done with the LDS
    }
    const int g = col / n_sub;
    const int h0 = g * kv_mul + (col % n_sub) * 16;
    const int n_col = PACK ? p.tok_pack * kv_mul : min(16, g * kv_mul + kv_mul - h0);
    auto col_tok = [&](int c) { return PACK ? s * p.tok_pack + c / kv_mul : s; };
    auto col_head = [&](int c) { return PACK ? g * kv_mul + c % kv_mul : h0 + c; };
    auto col_ok = [&](int c) { return c < n_col && (!PACK || col_tok(c) < p.n_seq); };
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g4 = lane >> 4;
    const int qc = SPLIT ? l16 >> 1 : l16;  // the lane's query column
    const bool qv = col_ok(qc);
    uint4* blo = (uint4*)smem;                                       // !SPLIT: [4][KS][16]
    uint8_t* vrow = (uint8_t*)smem + kBloBytes + wave * kWaveBytes;  // [TILE][RB]
    float* auxT = (float*)(vrow + TILE * RB);            // [4][TILE]: sigma_k, r_k, sigma_v, r_v

    // query operands and constants of the lane's column
    uint4 bq[KS];
    float cback, pback, qcorr, pcorr;
    {
        const int c0 = qv ? qc : 0;
        const uint32_t* qb = (const uint32_t*)p.ws_q + ((size_t)col_tok(c0) * p.n_heads + col_head(c0)) * S::QBW;
        const uint4* bh = (const uint4*)(qb + ((SPLIT ? (l16 & 1) * 4 : 0) + g4) * 4 * KS);
        const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < KS; k++) bq[k] = qv ? bh[k] : z;
        if constexpr (!SPLIT) {
            if (wave == 0) {
                const uint4* bl = (const uint4*)(qb + (4 + g4) * 4 * KS);
#pragma unroll
                for (int k = 0; k < KS; k++) blo[(g4 * KS + k) * 16 + l16] = qv ? bl[k] : z;
            }
            __syncthreads();
        }
        const float* cst = (const float*)(qb + 32 * KS);
        // SPLIT: the two piece columns each subtract half of the corrections
        const float half = SPLIT ? 0.5f : 1.0f;
        cback = qv ? 2.0f * cst[0] : 0.0f;
        pback = qv ? 2.0f * cst[1] : 0.0f;
        qcorr = qv ? half * cst[2] : 0.0f;
        pcorr = qv ? half * cst[3] : 0.0f;
    }

    // wave-uniform bases of (slot, kv head); per-key offsets in 32 bits
    const size_t slot = (size_t)(p.seq_slot ? p.seq_slot[s] : s);
    const int64_t e0 = (int64_t)slot * p.seq_stride + (int64_t)g * D;
    const __amdgpu_buffer_rsrc_t kbh = buf_rsrc((const uint8_t*)p.k_cache + e0 / 4);
    const __amdgpu_buffer_rsrc_t vbh = buf_rsrc((const uint8_t*)p.v_cache + e0 / 4);
    const __amdgpu_buffer_rsrc_t ksh = buf_rsrc((const uint8_t*)p.k_sign + e0 / 8);
    const __amdgpu_buffer_rsrc_t vsh = buf_rsrc((const uint8_t*)p.v_sign + e0 / 8);
    const int64_t a0 = (int64_t)slot * p.scale_seq_stride + g;
    const float* ksig_p = p.k_scale + a0;
    const float* kgam_p = p.k_rnorm + a0;
    const float* vsig_p = p.v_scale + a0;
    const float* vgam_p = p.v_rnorm + a0;
    const uint32_t rsc = (uint32_t)(p.row_stride / 4), rss = (uint32_t)(p.row_stride / 8);
    const uint32_t ars = (uint32_t)p.scale_row_stride;
    const float rfac = sqrtf(tq::kFracPi2 / (float)D);

    auto blo_at = [&](int k) { return blo[(g4 * KS + k) * 16 + l16]; };

    int c_lo = t_begin, c_hi = t_stop;  // keys visible to the lane's column
    int vis_lo = c_lo, vis_hi = c_hi;   // PACK: keys visible to every valid column (wave-uniform)
    if constexpr (PACK) {
        c_lo = qv ? p.col_start[col_tok(qc)] : 0;
        c_hi = qv ? min(p.col_end[col_tok(qc)], t_stop) : 0;
        int lo = qv ? c_lo : INT_MIN, hi = qv ? c_hi : INT_MAX;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            lo = max(lo, __shfl_xor(lo, o, 64));
            hi = min(hi, __shfl_xor(hi, o, 64));
        }
        vis_lo = __builtin_amdgcn_readfirstlane(lo);
        vis_hi = __builtin_amdgcn_readfirstlane(hi);
    }

    // per-tile registers: K code / sign dwords of the lane's key in both
    // sub-tiles; raw V bytes of the staging (lane: key lane/2, half lane%2 of
    // the row); the lane's aux pair (key lane%32; K below lane 32, V above)
    constexpr int NKS = NSW > 0 ? NSW : 1;
    constexpr int VCD = D / 32;  // code dwords per staging lane
    constexpr int VSD = D / 64;  // sign dwords per staging lane
    uint32_t kcw[2][NCW], ksw[2][NKS], vcw[VCD], vsw[VSD];
    float xs, xg;
    auto load_k = [&](int t0) {
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            const uint32_t key = (uint32_t)min(t0 + 16 * sb + l16, t_stop - 1);
            load_dwords<NCW>(kbh, (int)(key * rsc + 4 * NCW * g4), kcw[sb]);
            if constexpr (NSW > 0)
                load_dwords<NSW>(ksh, (int)(key * rss + 4 * NSW * g4), ksw[sb]);
            else
                ksw[sb][0] = __builtin_amdgcn_raw_buffer_load_b16(ksh, (int)(key * rss + 2 * g4), 0, 0);
        }
    };
    auto load_v = [&](int t0) {
        {
            const uint32_t key = (uint32_t)min(t0 + (lane >> 1), t_stop - 1);
            const int half = lane & 1;
            if constexpr (VCD == 8) {
                load_dwords<4>(vbh, (int)(key * rsc + 32 * half), vcw);
                load_dwords<4>(vbh, (int)(key * rsc + 32 * half + 16), vcw + 4);
            } else {
                load_dwords<VCD>(vbh, (int)(key * rsc + 4 * VCD * half), vcw);
            }
            load_dwords<VSD>(vsh, (int)(key * rss + 4 * VSD * half), vsw);
        }
        {
            // lanes 0..31: K sigma / gamma, 32..63: V; plain loads through a
            // per-lane pointer (a per-lane choice of buffer descriptor would
            // become a loop over the two descriptors around each load)
            const size_t off = (size_t)min(t0 + (lane & 31), t_stop - 1) * ars;
            xs = (lane < 32 ? ksig_p : vsig_p)[off];
            xg = (lane < 32 ? kgam_p : vgam_p)[off];
        }
    };

    f32x4 oc[RT], os[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) oc[r] = os[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrow = -1e30f, lrow = 0.0f, lsum_c = 0.0f, lsum_s = 0.0f;
    float pwc = 1.0f, pws = 1.0f;  // power-of-two range factors of the value-pass B operands
    bool pw_set = false;

    const int n_tiles = (t_stop - t_begin + TILE - 1) / TILE;
    int it = wave;
    if (it < n_tiles) {
        load_k(t_begin + it * TILE);
        load_v(t_begin + it * TILE);
    }
    for (; it < n_tiles; it += kTsWaves) {
        const int t0 = t_begin + it * TILE;
        // stage the V rows as stored and the aux values
        {
            const int key = lane >> 1, half = lane & 1;
            uint8_t* rowp = vrow + key * RB;
            if constexpr (VCD == 8) {
                *(uint4*)(rowp + 32 * half) = make_uint4(vcw[0], vcw[1], vcw[2], vcw[3]);
                *(uint4*)(rowp + 32 * half + 16) = make_uint4(vcw[4], vcw[5], vcw[6], vcw[7]);
                *(uint4*)(rowp + D / 4 + 16 * half) = make_uint4(vsw[0], vsw[1], vsw[2], vsw[3]);
            } else if constexpr (VCD == 4) {
                *(uint4*)(rowp + 16 * half) = make_uint4(vcw[0], vcw[1], vcw[2], vcw[3]);
                *(uint2*)(rowp + D / 4 + 8 * half) = make_uint2(vsw[0], vsw[1]);
            } else {
                *(uint2*)(rowp + 8 * half) = make_uint2(vcw[0], vcw[1]);
                *(uint32_t*)(rowp + D / 4 + 4 * half) = vsw[0];
            }
            const int a = 2 * (lane >> 5);
            auxT[a * TILE + (lane & 31)] = xs;
            auxT[(a + 1) * TILE + (lane & 31)] = xg * rfac;
        }
        // the V / aux registers are free: the next tile's loads get a whole iteration
        if (it + kTsWaves < n_tiles) load_v(t_begin + (it + kTsWaves) * TILE);
        // score pass: bit sums of the code and sign planes for both sub-tiles
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 sc[2], ssg[2];
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            sc[sb] = zero;
            ssg[sb] = zero;
            auto word4 = [&](uint32_t W, int ks0, f32x4& acc) {
                const uint4 A0 = score_a<0>(W), A1 = score_a<1>(W), A2 = score_a<2>(W), A3 = score_a<3>(W);
                acc = mma16(A0, bq[ks0], acc);
                if constexpr (!SPLIT) acc = mma16(A0, blo_at(ks0), acc);
                acc = mma16(A1, bq[ks0 + 1], acc);
                if constexpr (!SPLIT) acc = mma16(A1, blo_at(ks0 + 1), acc);
                acc = mma16(A2, bq[ks0 + 2], acc);
                if constexpr (!SPLIT) acc = mma16(A2, blo_at(ks0 + 2), acc);
                acc = mma16(A3, bq[ks0 + 3], acc);
                if constexpr (!SPLIT) acc = mma16(A3, blo_at(ks0 + 3), acc);
            };
#pragma unroll
            for (int w = 0; w < NCW; w++) word4(kcw[sb][w], 4 * w, sc[sb]);
            if constexpr (NSW > 0) {
#pragma unroll
                for (int w = 0; w < NSW; w++) word4(ksw[sb][w], KSC + 4 * w, ssg[sb]);
            } else {
                const uint32_t h = ksw[sb][0] & 0xffffu;
                const uint32_t H = (h & 0xffu) | ((h & 0xff00u) << 8);  // dims 0..7 | 8..15 at bits 0..7 | 16..23
                const uint4 A0 = score_a<0>(H), A1 = score_a<1>(H);
                ssg[sb] = mma16(A0, bq[KSC], ssg[sb]);
                if constexpr (!SPLIT) ssg[sb] = mma16(A0, blo_at(KSC), ssg[sb]);
                ssg[sb] = mma16(A1, bq[KSC + 1], ssg[sb]);
                if constexpr (!SPLIT) ssg[sb] = mma16(A1, blo_at(KSC + 1), ssg[sb]);
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
                float v = ksv[j] * (cback * sc[sb][j] - qcorr) + krv[j] * (pback * ssg[sb][j] - pcorr);
                if constexpr (SPLIT) v += dpp_xor1(v);  // the hi and lo columns' halves
                sv[e] = v;
                (void)key;
                vsg[e] = vsv[j];
                vrr[e] = vrv[j];
            }
        }
        if constexpr (PACK) {
            if (!(t0 >= vis_lo && t0 + TILE <= vis_hi)) {  // a column sees only part of the tile
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int key = t0 + 16 * (e >> 2) + 4 * g4 + (e & 3);
                    sv[e] = (key >= c_lo && key < c_hi) ? sv[e] : -INFINITY;
                }
            }
        }
        if constexpr (!PACK) {
            if (tail) {  // keys past the split end (the loads repeated the last one)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (t0 + 16 * (e >> 2) + 4 * g4 + (e & 3) >= t_stop) sv[e] = -INFINITY;
            }
        }
        if (it + kTsWaves < n_tiles) load_k(t_begin + (it + kTsWaves) * TILE);

        float mx = sv[0];
#pragma unroll
        for (int e = 1; e < 8; e++) mx = fmaxf(mx, sv[e]);
        mx = rows_max(mx);
        if (__any(mx > mrow + kLazy)) {
            const float mnew = fmaxf(mrow, mx);
            const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
            mrow = mnew;
            lrow *= alpha;
            lsum_c *= alpha;
            lsum_s *= alpha;
#pragma unroll
            for (int r = 0; r < RT; r++) {
                oc[r] *= alpha;
                os[r] *= alpha;
            }
        }
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            pv[e] = __builtin_amdgcn_exp2f(sv[e] - mrow);
            lrow += pv[e];
        }
        // range factors: the tile's largest sigma / r scaled into [2^5, 2^6)
        {
            float lb = 0.0f, lr = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                lb = fmaxf(lb, vsg[e]);
                lr = fmaxf(lr, vrr[e]);
            }
            if (!pw_set || __any(lb * pwc >= 64.0f || lr * pws >= 64.0f)) {
                // every lane of a row holds the same keys: the row maxima are the tile's
                const float nb = __int_as_float(
                    __builtin_amdgcn_readfirstlane(__float_as_int(tq::pow2_for(rows_max(lb), 6))));
                const float nr = __int_as_float(
                    __builtin_amdgcn_readfirstlane(__float_as_int(tq::pow2_for(rows_max(lr), 6))));
                if (!pw_set) {
                    pwc = nb;
                    pws = nr;
                } else {
                    if (nb < pwc) {
                        const float f = nb / pwc;
                        lsum_c *= f;
#pragma unroll
                        for (int r = 0; r < RT; r++) oc[r] *= f;
                        pwc = nb;
                    }
                    if (nr < pws) {
                        const float f = nr / pws;
                        lsum_s *= f;
#pragma unroll
                        for (int r = 0; r < RT; r++) os[r] *= f;
                        pws = nr;
                    }
                }
                pw_set = true;
            }
        }
        // value-pass B operands: pair i <-> keys (pv[2i], pv[2i+1])
        uint4 bc[2], bcl[2], bsg, bsgl;
        {
            float xc[8], xr[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                xc[e] = pv[e] * vsg[e] * pwc;
                xr[e] = pv[e] * vrr[e] * pws;
                lsum_c += xc[e];
                lsum_s += xr[e];
            }
            uint32_t h[12], l[12];
            if constexpr (SPLIT) {
                const float lo = (float)(l16 & 1);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    h[2 * i] = piece2(kAlpha * xc[2 * i], kAlpha * xc[2 * i + 1], lo);
                    h[2 * i + 1] = piece2(kBeta * xc[2 * i], kBeta * xc[2 * i + 1], lo);
                    h[8 + i] = piece2(xr[2 * i], xr[2 * i + 1], lo);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    split2(kAlpha * xc[2 * i], kAlpha * xc[2 * i + 1], h[2 * i], l[2 * i]);
                    split2(kBeta * xc[2 * i], kBeta * xc[2 * i + 1], h[2 * i + 1], l[2 * i + 1]);
                    split2(xr[2 * i], xr[2 * i + 1], h[8 + i], l[8 + i]);
                }
            }
            bc[0] = make_uint4(h[0], h[1], h[2], h[3]);
            bc[1] = make_uint4(h[4], h[5], h[6], h[7]);
            bsg = make_uint4(h[8], h[9], h[10], h[11]);
            if constexpr (!SPLIT) {
                bcl[0] = make_uint4(l[0], l[1], l[2], l[3]);
                bcl[1] = make_uint4(l[4], l[5], l[6], l[7]);
                bsgl = make_uint4(l[8], l[9], l[10], l[11]);
            }
        }
        // pair words of the lane's field (l16) for the key pairs of its group:
        // pair i = keys ka(i), ka(i) + 1 with ka(i) = 16 (i >> 1) + 4 g4 + 2 (i & 1)
        uint32_t pw[4][NF], spw[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint8_t* ra = vrow + (16 * (i >> 1) + 4 * g4 + 2 * (i & 1)) * RB;
            const uint8_t* rb = ra + RB;
            if constexpr (D == 64) {
                pw[i][0] = (uint32_t)ra[l16] | ((uint32_t)rb[l16] << 16);
                const int sh = 4 * (l16 & 1);
                spw[i] = (((uint32_t)ra[D / 4 + (l16 >> 1)] >> sh) & 0xfu) |
                         ((((uint32_t)rb[D / 4 + (l16 >> 1)] >> sh) & 0xfu) << 16);
            } else if constexpr (D == 128) {
                pw[i][0] = (uint32_t)*(const uint16_t*)(ra + 2 * l16) | ((uint32_t)*(const uint16_t*)(rb + 2 * l16) << 16);
                spw[i] = (uint32_t)ra[D / 4 + l16] | ((uint32_t)rb[D / 4 + l16] << 16);
            } else {
                const uint32_t wa = *(const uint32_t*)(ra + 4 * l16), wb = *(const uint32_t*)(rb + 4 * l16);
                pw[i][0] = __builtin_amdgcn_perm(wb, wa, 0x05040100u);
                pw[i][1] = __builtin_amdgcn_perm(wb, wa, 0x07060302u);
                spw[i] = (uint32_t)*(const uint16_t*)(ra + D / 4 + 2 * l16) |
                         ((uint32_t)*(const uint16_t*)(rb + D / 4 + 2 * l16) << 16);
            }
        }
        // value pass
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int f = rt >> 3, j2 = rt & 7;
            const uint32_t mk = 0x00010001u << vc_pos(j2);
            uint32_t au[4], av[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t w = pw[i][f];
                au[i] = (vc_shift(j2) == 9 ? shl<9>(w) : vc_shift(j2) == 3 ? shl<3>(w) : shl<-3>(w)) & mk;
                av[i] = (vc_shift(j2) == 9 ? shl<10>(w) : vc_shift(j2) == 3 ? shl<4>(w) : shl<-2>(w)) & mk;
            }
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const uint4 A = make_uint4(au[2 * m], av[2 * m], au[2 * m + 1], av[2 * m + 1]);
                oc[rt] = mma16(A, bc[m], oc[rt]);
                if constexpr (!SPLIT) oc[rt] = mma16(A, bcl[m], oc[rt]);
            }
            const uint32_t ms = 0x00010001u << vs_pos(rt);
            uint32_t as[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t w = spw[i];
                as[i] = (vs_shift(rt) == 10 ? shl<10>(w) : vs_shift(rt) == 5 ? shl<5>(w)
                         : vs_shift(rt) == 0 ? w : shl<-5>(w)) & ms;
            }
            const uint4 A = make_uint4(as[0], as[1], as[2], as[3]);
            os[rt] = mma16(A, bsg, os[rt]);
            if constexpr (!SPLIT) os[rt] = mma16(A, bsgl, os[rt]);
        }
        __builtin_amdgcn_wave_barrier();  // reads done before the next tile's stores
    }

    // per-wave totals of the lane's column: sums over the four key groups
    lrow = rows_sum(lrow);
    lsum_c = rows_sum(lsum_c);
    lsum_s = rows_sum(lsum_s);
    if constexpr (SPLIT) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                oc[r][j] += dpp_xor1(oc[r][j]);
                os[r][j] += dpp_xor1(os[r][j]);
            }
    }
    const float ipc = pw_set ? 1.0f / pwc : 0.0f, ips = pw_set ? 1.0f / pws : 0.0f;  // exact: powers of two
    const float cc = (kAlpha + kBeta) * lsum_c;
    __syncthreads();
    float (*sh_o)[16][2 * D + 1] = (float (*)[16][2 * D + 1])smem;
    float (*sh_m)[16] = (float (*)[16])((float*)smem + kTsWaves * 16 * (2 * D + 1));
    float (*sh_l)[16] = sh_m + kTsWaves;
    const bool writer = SPLIT ? (l16 & 1) == 0 : true;
    if (writer) {
        if (g4 == 0) {
            sh_m[wave][qc] = mrow;
            sh_l[wave][qc] = lrow;
        }
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const float sc_c = 2.0f * ldexpf(1.0f, -bit_exp(vc_pos(rt & 7)));
            const float sc_s = 2.0f * ldexpf(1.0f, -bit_exp(vs_pos(rt)));
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = (D / 16) * (4 * g4 + j) + rt;
                sh_o[wave][qc][d] = (oc[rt][j] * sc_c - cc) * ipc;
                sh_o[wave][qc][D + d] = (os[rt][j] * sc_s - lsum_s) * ips;
            }
        }
    }
    __syncthreads();
    const int n_splits = p.n_splits;
    if constexpr (PACK) {
        if (n_splits == 1) {
            // One split per row group (long chunks): the merged (O, l) of each
            // column is final, so the workgroup does turbo_combine_kernel's work
            // for it (1/l, the inverse residual rotation, the sum, the inverse
            // rotation, the output gate) and writes no partials; the host skips
            // the combine launch.
            constexpr int J = D / 64;
            const uint8_t* sg = p.turbo_signs + (size_t)g * (D / 8);
            const int64_t ss = p.turbo_slot_stride;
            for (int q = wave; q < n_col; q += kTsWaves) {
                if (!col_ok(q)) continue;  // wave-uniform
                float mx = -INFINITY;
#pragma unroll
                for (int w = 0; w < kTsWaves; w++) mx = fmaxf(mx, sh_m[w][q]);
                float lt = 0.0f, b[J], r[J];
#pragma unroll
                for (int j = 0; j < J; j++) b[j] = r[j] = 0.0f;
#pragma unroll
                for (int w = 0; w < kTsWaves; w++) {
                    const float a = exp2f(sh_m[w][q] - mx);
                    lt += sh_l[w][q] * a;
#pragma unroll
                    for (int j = 0; j < J; j++) {
                        b[j] += sh_o[w][q][lane + 64 * j] * a;
                        r[j] += sh_o[w][q][D + lane + 64 * j] * a;
                    }
                }
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
                for (int j = 0; j < J; j++) {
                    b[j] *= inv;
                    r[j] *= inv;
                }
                tq::wave_transform<D>(r, sg + 3 * ss, sg + 2 * ss, lane);  // res_post, res_pre: inverse
#pragma unroll
                for (int j = 0; j < J; j++) b[j] += r[j];
                tq::wave_transform<D>(b, sg + ss, sg, lane);  // rot_post, rot_pre: inverse
                const int tok = col_tok(q), hh = col_head(q);
                float* out = p.out + ((size_t)tok * p.n_heads + hh) * D;
                const float* gt = p.gate.at(tok, hh);  // Qwen3.5 output gate, or null
#pragma unroll
                for (int j = 0; j < J; j++) out[lane + 64 * j] = gt ? gate_mul(b[j], gt[lane + 64 * j]) : b[j];
            }
            break;
        }
    }
    for (int idx = tid; idx < n_col * 2 * D; idx += kTsThreads) {
        const int q = idx / (2 * D), i = idx % (2 * D);
        if (!col_ok(q)) continue;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kTsWaves; w++) mx = fmaxf(mx, sh_m[w][q]);
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int w = 0; w < kTsWaves; w++) {
            const float a = exp2f(sh_m[w][q] - mx);
            lt += sh_l[w][q] * a;
            ot += sh_o[w][q][i] * a;
        }
        if (split >= n_splits) break;  // a sequence longer than max_kv_len: slots end here
        const size_t part = ((size_t)col_tok(q) * p.n_heads + col_head(q)) * n_splits + split;
        p.ws_o[part * 2 * D + i] = ot;
        if (i == 0) {
            p.ws_ml[part * 2 + 0] = mx;
            p.ws_ml[part * 2 + 1] = lt;
        }
    }
    if constexpr (!stream) break;
    else if (!cur.advance()) break;
    }
}

int turbo_pack_rows(int head_dim, int kv_mul) {
    // Up to d128 the split kernel takes 16 query columns with a hi and a lo MFMA
    // per product; at d256 that form runs out of registers, so it carries 8
    // columns as hi / lo column pairs.
    return std::max(1, (head_dim == 256 ? 8 : 16) / std::max(1, kv_mul));
}

size_t turbo_query_ws_dwords(int head_dim) {
    switch (head_dim) {
        case 64: return Tq<64>::QBW;
        case 128: return Tq<128>::QBW;
        case 256: return Tq<256>::QBW;
        default: return 0;
    }
}

bool decode_turbo_supported(const DecodeLaunch& p) {
    return (p.head_dim == 64 || p.head_dim == 128 || p.head_dim == 256) &&
           (p.tok_pack == 0 || p.tok_pack * (p.n_heads / p.n_kv_heads) <= 16);
}

// Workgroups of the decode split kernel that fit on the current device at once
// (CUs x occupancy): the stream schedule's grid.  A device property, cached per
// (template instance, device); concurrent first calls compute the same value.
template <int D, bool SPLIT>
static int turbo_resident_wgs() {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cached[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    const int slot = dev >= 0 && dev < kMaxDev ? dev : -1;
    if (slot >= 0) {
        const int c = cached[slot].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int n_cu = 0, occ = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, turbo_split_kernel<D, false, SPLIT, true>, kTsThreads, 0) !=
            hipSuccess)
        return 256;
    const int v = std::max(1, n_cu * std::max(1, occ));
    if (slot >= 0) cached[slot].store(v, std::memory_order_relaxed);
    return v;
}

template <int D>
static hipError_t launch_turbo_d(const DecodeLaunch& p0, hipStream_t st) {
    DecodeLaunch p = p0;  // decode: groups above 16 query heads in columns of 16
    p.n_sub = p.tok_pack > 0 ? 1 : (p.n_heads / p.n_kv_heads + 15) / 16;
    p.sub_heads = 16;
    turbo_query_kernel<D><<<dim3((p.n_heads + 3) / 4, p.n_seq), 256, 0, st>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int kv_mul = p.n_heads / p.n_kv_heads;
    const int n_col = p.tok_pack > 0 ? p.tok_pack * kv_mul : std::min(kv_mul, 16);
    const bool split = 2 * n_col <= 16;  // hi / lo pieces as MFMA columns
    if (p.tok_pack > 0) {
        // token-packed prefill (turbo_pack_rows: 16 columns up to d128, 8 at d256)
        const dim3 grid(p.n_splits, p.n_kv_heads, (p.n_seq + p.tok_pack - 1) / p.tok_pack);
        if (split) turbo_split_kernel<D, true, true, false><<<grid, kTsThreads, 0, st>>>(p);
        else turbo_split_kernel<D, true, false, false><<<grid, kTsThreads, 0, st>>>(p);
    } else if (!p.stream_sched) {
        const dim3 grid(p.n_splits, p.n_kv_heads * p.n_sub, p.n_seq);
        if (split) turbo_split_kernel<D, false, true, false><<<grid, kTsThreads, 0, st>>>(p);
        else turbo_split_kernel<D, false, false, false><<<grid, kTsThreads, 0, st>>>(p);
    } else if (split) {
        turbo_split_kernel<D, false, true, true><<<dim3(turbo_resident_wgs<D, true>()), kTsThreads, 0, st>>>(p);
    } else if constexpr (turbo_stream_ok(D, false)) {
        turbo_split_kernel<D, false, false, true><<<dim3(turbo_resident_wgs<D, false>()), kTsThreads, 0, st>>>(p);
    } else {
        return hipErrorInvalidValue;  // the plan keeps this shape on the fixed grid
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (p.tok_pack > 0 && p.n_splits == 1) return hipSuccess;  // the split kernel finished the rows
    return launch_turbo_combine(p, st);
}

hipError_t launch_decode_turbo(const DecodeLaunch& p, hipStream_t st) {
    if (!decode_turbo_supported(p)) return hipErrorInvalidValue;
    switch (p.head_dim) {
        case 64: return launch_turbo_d<64>(p, st);
        case 128: return launch_turbo_d<128>(p, st);
        case 256: return launch_turbo_d<256>(p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace gr
