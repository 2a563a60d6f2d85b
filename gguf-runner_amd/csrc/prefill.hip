// Causal / sliding-window flash prefill on gfx950 MFMA (f16 or bf16 inputs,
// fp32 accumulation).  Replaces the token-serial attention of the prefill loop
// (reference inference.rs:2981-3017, one attention_token per token) with one
// launch per chunk: every query row sees keys [start(pos), pos] of the device KV
// cache, start = 0 for global layers and pos + 1 - W for window W
// (LanguageAttentionPolicy::visible_keys, attention.rs:74-96).
//
// Workgroup = NW waves x 32 query rows of one query head (NW = 8 for large
// launches, 4 for small ones), or, with KH = 2 key halves (d64 launches of at
// most one four-wave workgroup per CU), NW / 2 row groups of two waves that
// take alternate 32-key sub-tiles of every tile and merge their online-softmax
// states at the end.  K and V tiles of BN keys go from the cache
// straight into LDS (buffer_load ... lds, no register staging), both row-major
// with their 16-byte chunks XOR-swizzled per row so that every LDS read below
// is free of bank conflicts.  Each wave computes
//   S^T = K . Q^T    (v_mfma_f32_32x32x16: A = K rows (ds_read_b128), B = Q in VGPRs)
//   O^T += V^T . P^T (A = V^T via ds_read_b64_tr_b16 from the row-major V tile,
//                     B = P straight from the S^T accumulators)
// so both accumulators hold one query per lane column and the online-softmax
// statistics of a row live in the two lanes (l, l^32) that own it.
// For head_dim 128 the kernel prepares Q itself from the raw rows (QK RMSNorm,
// RoPE from a per-token (cos, sin) table, softmax_scale*log2(e)); otherwise Q
// arrives prepared that way by the prep pass.
#include <type_traits>

#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
#define GR_LDS __attribute__((address_space(3)))

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
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
};

// Raw buffer access: wave-uniform base in a scalar descriptor, 32-bit byte
// offsets per lane (gfx9-family descriptor word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pf_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)0xffffffff, 0x00020000);
}

// 16 bytes per lane from the buffer at byte offset voff into LDS at
// lds + 16 * lane (lds wave-uniform).  The builtin exists for the device pass
// only; the host pass of the kernel templates must not see it.
__device__ __forceinline__ void pf_dma16(__amdgpu_buffer_rsrc_t r, uint16_t* lds, int voff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (GR_LDS void*)lds, 16, voff, 0, 0, 0);
#endif
}

// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left at their maxima)
__device__ __forceinline__ void pf_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Position of 16-byte chunk c of tile row r: c ^ pf_swz<D>(r & 15).  With it the
// K reads (16 consecutive rows, one chunk each) and the V transpose reads (4
// consecutive rows x 4 chunks per 32 lanes) each touch distinct banks.  A
// head_dim-64 row is 8 chunks (128 B, half the banks): rows of one parity then
// need distinct chunk positions (K), and rows r and r + 2 opposite 4-chunk halves
// (V), which a 3-bit swizzle with bit 2 = bit 1 of r gives.
template <int D>
__device__ __forceinline__ int pf_swz(int r) {
    if constexpr (D == 64) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    else return ((r << 2) ^ (r << 1) ^ (r >> 2)) & 15;
}


// Workgroup = NW waves of 32 query rows each.  Large launches use 8 waves
// (256 query rows share every K / V tile, one workgroup per CU), small ones 4
// waves (twice the workgroups, so short prompts still fill the GPU), or, at d64,
// 8 waves as 4 row groups x 2 key halves (KH = 2: the four-wave kernel's
// workgroups with twice the waves).
template <int D, int NW, int KH = 1>
struct PfTile;
template <>
struct PfTile<128, 8> {
    static constexpr int BN = 128;      // keys per LDS tile
    static constexpr int kWaves = 2;    // waves per SIMD (one workgroup per CU, <= 256 VGPRs each)
};
template <>
struct PfTile<128, 4> {
    static constexpr int BN = 64;
    static constexpr int kWaves = 2;    // two workgroups per CU
};
template <>
struct PfTile<64, 8> {
    static constexpr int BN = 128;
    static constexpr int kWaves = 4;    // two workgroups per CU, <= 128 VGPRs each
};
template <>
struct PfTile<64, 4> {
    static constexpr int BN = 64;
    static constexpr int kWaves = 4;    // four workgroups per CU
};
template <>
struct PfTile<64, 8, 2> {
    static constexpr int BN = 128;      // 4 sub-tiles, two per key half
    static constexpr int kWaves = 4;    // two workgroups per CU
};
template <>
struct PfTile<256, 4> {
    static constexpr int BN = 32;
    static constexpr int kWaves = 1;    // one wave per SIMD (its registers)
};

// Softmax reference maxima are only raised when a row's tile maximum exceeds
// them by more than this (log2 units): until then P = 2^(s - m_ref) <= 2^8 and
// the accumulators need no rescale.  The final O / l is exact either way.
constexpr float kLazyRescale = 8.0f;

__device__ __forceinline__ float pf_xmax32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pf_xsum32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Fused Q preparation (head_dim 128).  Lane (query row, half lg) owns the
// elements d = 16 c + 8 lg .. +7 of its row, c = 0 .. D/16 - 1, i.e. exactly the
// B-operand fragments qf[c]; the QK RMSNorm sum pairs up with lane l ^ 32, and
// every RoPE pair stays inside the lane (adjacent pairs sit in one chunk; NeoX
// pairs (d, d + rope_dim / 2) are chunks c and c + rope_dim / 32).  The
// arithmetic follows qkv_prep_kernel expression for expression.
__device__ __forceinline__ void pf_load8(const void* base, size_t idx, int dt, float* v) {
    if (dt == GR_DTYPE_F32) {
        const float4 a = *(const float4*)((const float*)base + idx);
        const float4 b = *(const float4*)((const float*)base + idx + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
        return;
    }
    const uint4 u = *(const uint4*)((const uint16_t*)base + idx);
    if (dt == GR_DTYPE_F16) unpack16<F16>(u, v);
    else unpack16<BF16>(u, v);
}

template <int CS, int NC>
__device__ __forceinline__ void pf_rope_neox(float (&x)[NC][8], const float* cs, int lg) {
#pragma unroll
    for (int c = 0; c < CS; c++) {
        const float4* t = (const float4*)(cs + 2 * (16 * c + 8 * lg));
        float cv[8], sv[8];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float4 w = t[u];
            cv[2 * u] = w.x, sv[2 * u] = w.y, cv[2 * u + 1] = w.z, sv[2 * u + 1] = w.w;
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float v0 = x[c][e], v1 = x[c + CS][e];
            x[c][e] = v0 * cv[e] - v1 * sv[e];
            x[c + CS][e] = v0 * sv[e] + v1 * cv[e];
        }
    }
}

template <typename DT, int D>
__device__ __forceinline__ void pf_prepare_q(const PrefillLaunch& p, int row, int h, int lg, uint4* qf, uint4* qfl) {
    constexpr int NC = D / 16;
    float x[NC][8];
    const size_t base = (size_t)row * p.q_row_stride + (size_t)h * D + 8 * lg;
#pragma unroll
    for (int c = 0; c < NC; c++) pf_load8(p.q_raw, base + 16 * c, p.q_in_dtype, x[c]);
    if (p.q_bias) {  // Qwen2 q bias, before the norm (inference.rs:2545-2559)
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float bv[8];
            pf_load8(p.q_bias, (size_t)h * D + 16 * c + 8 * lg, GR_DTYPE_F32, bv);
#pragma unroll
            for (int e = 0; e < 8; e++) x[c][e] += bv[e];
        }
    }
    if (p.q_norm) {
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) ss += x[c][e] * x[c][e];
        ss = pf_xsum32(ss);
        const float inv = 1.0f / sqrtf(ss / (float)D + p.norm_eps);
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) x[c][e] = p.q_norm[16 * c + 8 * lg + e] * (inv * x[c][e]);
    }
    if (p.rope_mode == GR_ROPE_ADJACENT) {
        const float* cs = p.rope_cs + (size_t)row * (p.rope_dim / 2) * 2;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const float4* t = (const float4*)(cs + 2 * (8 * c + 4 * lg));  // pairs (16 c + 8 lg) / 2 ..
            const float4 w0 = t[0], w1 = t[1];
            const float cv[4] = {w0.x, w0.z, w1.x, w1.z}, sv[4] = {w0.y, w0.w, w1.y, w1.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float v0 = x[c][2 * u], v1 = x[c][2 * u + 1];
                x[c][2 * u] = v0 * cv[u] - v1 * sv[u];
                x[c][2 * u + 1] = v0 * sv[u] + v1 * cv[u];
            }
        }
    } else if (p.rope_mode == GR_ROPE_NEOX) {
        const float* cs = p.rope_cs + (size_t)row * (p.rope_dim / 2) * 2;
        switch (p.rope_dim / 32) {
            case 1: pf_rope_neox<1>(x, cs, lg); break;
            case 2: pf_rope_neox<2>(x, cs, lg); break;
            case 3: pf_rope_neox<3>(x, cs, lg); break;
            default: pf_rope_neox<NC / 2>(x, cs, lg); break;
        }
    }
    using M = Mfma32<DT>;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        float xs[8];
#pragma unroll
        for (int e = 0; e < 8; e++) xs[e] = (x[c][e] * p.q_pre_scale) * p.q_scale;
        uint32_t hw[4];
#pragma unroll
        for (int w = 0; w < 4; w++) hw[w] = M::pack2(xs[2 * w], xs[2 * w + 1]);
        qf[c] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        if constexpr (M::kSplit) {
            uint32_t lw[4];
#pragma unroll
            for (int w = 0; w < 4; w++)
                lw[w] = M::pack2(xs[2 * w] - __uint_as_float(hw[w] << 16), xs[2 * w + 1] - __uint_as_float(hw[w] & 0xffff0000u));
            qfl[c] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        }
    }
}

// The attention of one workgroup.  K / V rows t of the visible range are rows
// t - row0 of k_cache / v_cache (row stride rs elements); Ks0 .. Vs1 are the
// double-buffered tiles (BN * D each) and Qlo the bf16 d256 Q residuals, all in
// LDS and declared by the kernel (distinct arrays, so the compiler sees that the
// DMA into one buffer never aliases the reads of another).
template <typename DT, int D, int NW, int KH = 1>
__device__ __forceinline__ void prefill_body(const PrefillLaunch& p, const void* k_cache, const void* v_cache,
                                             const int64_t rs, const int64_t row0, uint16_t* Ks0, uint16_t* Ks1,
                                             uint16_t* Vs0, uint16_t* Vs1, uint4* Qlo) {
    constexpr int kPfThreads = NW * 64;
    constexpr int RW = NW / KH;                 // row groups of 32 query rows
    constexpr int BM = RW * 32, BN = PfTile<D, NW, KH>::BN;
    static_assert(KH == 1 || (KH == 2 && D <= 128 && BN / 32 % 2 == 0), "key halves: d <= 128, even sub-tiles");
    constexpr int CPR = D / 8;                   // 16-byte chunks per cache row
    constexpr int LD = BN * CPR / kPfThreads;    // DMA chunks per thread per K (or V) tile
    constexpr int RPU = kPfThreads / CPR;        // tile rows filled by one DMA round
    static_assert(LD >= 1 && BN % 32 == 0 && kPfThreads % CPR == 0, "tile shape");
    using M = Mfma32<DT>;
    constexpr bool kSplit = M::kSplit;
    // f16, d = 128: the S^T accumulators start from -m_off (a 16-register
    // broadcast), so the MFMAs deliver s - m_off and the exponent needs no
    // subtraction; the variants with more live registers subtract instead.
    constexpr bool kFold = D == 128 && !kSplit;

    // bf16 d256: the Q residual fragments live in LDS (per wave, [k-step][lane])
    // instead of 64 VGPRs, which the d256 accumulators need
    constexpr bool kQloLds = kSplit && D == 256;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int rw = KH > 1 ? wave % RW : wave, kh = KH > 1 ? wave / RW : 0;  // row group, key half
    const int ln = lane & 31, lg = lane >> 5;
    const int m = p.n_tokens;
    const int P0 = (int)p.base_pos;
    const int W = p.window;
    const int n_qb = (m + BM - 1) / BM;
    const int n_pairs = (n_qb + 1) / 2;

    // Work item = (query head, pair of query blocks), head-major.  Workgroup b
    // runs on XCD b % 8; giving each XCD a contiguous run of items keeps the
    // query heads of one GQA group (same K/V) in one XCD's L2.
    const int n_items = p.n_heads * n_pairs;
    const int per_xcd = (n_items + 7) / 8;
    const int item = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
    if (item >= n_items) return;
    const int h = item / n_pairs;
    const int j = item - h * n_pairs;
    const int kv_mul = p.n_heads / p.n_kv_heads;
    const int g = h / kv_mul;
    const uint16_t* kc = (const uint16_t*)k_cache + (size_t)g * D;
    const uint16_t* vc = (const uint16_t*)v_cache + (size_t)g * D;
    const int rsb = (int)rs * 2;

    // DMA: thread tid fills chunk position tid + NW * 64 * u of the tile: row
    // tid / CPR + u * RPU, position tid % CPR, which holds chunk
    // (tid % CPR) ^ swz(row) of that cache row.
    int dma_off[LD];  // byte offsets from the tile's first row (full tiles)
    int dma_row[LD];
    int dma_col[LD];  // byte offset of the source chunk within its row
#pragma unroll
    for (int u = 0; u < LD; u++) {
        const int r = tid / CPR + u * RPU;
        dma_row[u] = r;
        dma_col[u] = ((tid % CPR) ^ pf_swz<D>(r & 15)) * 16;
        dma_off[u] = r * rsb + dma_col[u];
    }
    // K fragment reads: row 32 sb + ln (row & 15 == ln & 15), chunk 2 s + lg.
    const int swz_k = pf_swz<D>(ln & 15);
    // V^T transpose reads (ds_read_b64_tr_b16): lane i of 16-lane group G
    // supplies row k0 + i/4, columns d0 + 4 (i%4) .. +3, with
    // k0 = 32 sb + 16 t + 8 b + 4 lg and d0 = 32 dt + 16 (G & 1); it receives
    // V[k0 + 0..3][d0 + i], i.e. A-operand slots 4b .. 4b+3 of row d0 + i.
    const int gi = lane & 15;
    const int v_chunk = 2 * ((lane >> 4) & 1) + ((gi & 3) >> 1);
    int v_base[2], v_swz[2];
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const int r = 8 * b + 4 * lg + (gi >> 2);
        v_base[b] = r * D + (gi & 1) * 4;
        v_swz[b] = pf_swz<D>(r & 15);
    }

    for (int pass = 0; pass < 2; pass++) {
        const int qblk = pass == 0 ? n_qb - 1 - j : j;
        if (pass == 1 && qblk >= n_qb - 1 - j) break;

        const int q0 = qblk * BM;
        const int wr0 = q0 + rw * 32;
        const int my_row = wr0 + ln;
        const bool row_ok = my_row < m;
        const int my_row_c = row_ok ? my_row : m - 1;
        const int my_pos = P0 + my_row_c;
        const bool wave_active = wr0 < m;
        const int wpos_min = P0 + (wave_active ? wr0 : m - 1);
        const int wpos_max = P0 + min(wr0 + 31, m - 1);
        // Keys visible to the row at position pos: [row_lo(pos), row_hi(pos)].
        // Causal: [pos + 1 - W (or 0), pos].  Bidirectional image block (the m
        // rows are one block, LanguageAttentionPolicy::visible_keys,
        // attention.rs:87-94): [min(pos + 1 - W (or 0), P0), P0 + m - 1].
        // Both ends are non-decreasing in pos.
        auto row_lo = [&](int pos) {
            const int wl = W > 0 ? pos + 1 - W : 0;
            return p.bidirectional ? min(wl, P0) : wl;
        };
        auto row_hi = [&](int pos) { return p.bidirectional ? P0 + m - 1 : pos; };
        const int lo_min = row_lo(wpos_min), lo_max = row_lo(wpos_max);
        const int hi_min = row_hi(wpos_min), hi_max = row_hi(wpos_max);

        // Q fragments (B operand): lane (query ln, group lg) holds d = 16 s + 8 lg .. +7.
        uint4 qf[D / 16];
        uint4 qfl[kSplit && !kQloLds ? D / 16 : 1];
        bool q_done = false;
        if constexpr (D == 128) {
            if (p.q_raw) {
                pf_prepare_q<DT, D>(p, my_row_c, h, lg, qf, qfl);
                q_done = true;
            }
        }
        if (!q_done) {
            const size_t qoff = ((size_t)my_row_c * p.n_heads + h) * D + 8 * lg;
            const uint16_t* qrow = (const uint16_t*)p.q + qoff;
#pragma unroll
            for (int s = 0; s < D / 16; s++) qf[s] = *(const uint4*)(qrow + 16 * s);
            if constexpr (kSplit) {
                if (p.k_f16) {
                    // staged f16 values (bf16 cache with an f16 copy): hi = bf16(x)
                    // and lo = x - hi are exact, an 11-bit significand in two 8-bit ones
#pragma unroll
                    for (int s = 0; s < D / 16; s++) {
                        float xv[8];
                        unpack16<F16>(qf[s], xv);
                        uint32_t hw[4], lw[4];
#pragma unroll
                        for (int w = 0; w < 4; w++) {
                            hw[w] = pack_bf16x2(xv[2 * w], xv[2 * w + 1]);
                            lw[w] = pack_bf16x2(xv[2 * w] - __uint_as_float(hw[w] << 16),
                                                xv[2 * w + 1] - __uint_as_float(hw[w] & 0xffff0000u));
                        }
                        qf[s] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                        const uint4 x = make_uint4(lw[0], lw[1], lw[2], lw[3]);
                        if constexpr (kQloLds) Qlo[(wave * (D / 16) + s) * 64 + lane] = x;
                        else qfl[s] = x;
                    }
                } else {
                    const uint16_t* qrl = (const uint16_t*)p.q_lo + qoff;
#pragma unroll
                    for (int s = 0; s < D / 16; s++) {
                        const uint4 x = *(const uint4*)(qrl + 16 * s);
                        if constexpr (kQloLds) Qlo[(wave * (D / 16) + s) * 64 + lane] = x;
                        else qfl[s] = x;
                    }
                }
            }
        }

        // keys [kbeg, kend) of the cache are visible to some row of this block
        const int kend = p.bidirectional ? P0 + m : P0 + min(q0 + BM, m);
        const int kbeg = max(0, row_lo(P0 + q0));
        const int t_first = kbeg / BN * BN;
        const int n_tiles = (kend - t_first + BN - 1) / BN;

        // Issue the DMA of the tile starting at key t0.  Rows past kend - 1 are
        // clamped to it (they are masked; the clamp keeps P.V free of stale data).
        auto dma_tile = [&](int t0, uint16_t* kdst, uint16_t* vdst) {
            const __amdgpu_buffer_rsrc_t kr = pf_rsrc(kc + (t0 - row0) * rs);
            const __amdgpu_buffer_rsrc_t vr = pf_rsrc(vc + (t0 - row0) * rs);
            if (t0 + BN <= kend) {
#pragma unroll
                for (int u = 0; u < LD; u++) {
                    const int dst = (wave * 64 + u * kPfThreads) * 8;
                    pf_dma16(kr, kdst + dst, dma_off[u]);
                    pf_dma16(vr, vdst + dst, dma_off[u]);
                }
            } else {
                const int last = kend - 1 - t0;
#pragma unroll
                for (int u = 0; u < LD; u++) {
                    const int off = min(dma_row[u], last) * rsb + dma_col[u];
                    const int dst = (wave * 64 + u * kPfThreads) * 8;
                    pf_dma16(kr, kdst + dst, off);
                    pf_dma16(vr, vdst + dst, off);
                }
            }
        };

        f32x16 o[D / 32];
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
            for (int e = 0; e < 16; e++) o[dt][e] = 0.0f;
        // Online-softmax state of this lane's row: mrow is the reference maximum
        // (finite start); with kFold, S^T arrives as s - m_off where m_off =
        // mrow once the row has seen a key and 0 before, and a rescale is due
        // when max(s - m_off) > thr = mrow + kLazyRescale - m_off.
        float mrow = -1e30f;
        float lrow = 0.0f;  // this lane's share of the row sum
        float m_off = 0.0f;
        float thr = -1e30f + kLazyRescale;
        f32x16 negm;
#pragma unroll
        for (int e = 0; e < 16; e++) negm[e] = 0.0f;

        // One 32-key sub-tile: rows 32 sb .. 32 sb + 31 of the tile in (kb, vb),
        // first key ts.
        auto subtile = [&](const uint16_t* kb, const uint16_t* vb, int sb, int ts) {
            const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                                 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            // Scheduling hint for the S^T region: LLVM's single-wave MFMA
            // interleave (iglp strategy 1) places the K fragment reads between
            // the MFMAs.  MI355X, A/B on one box, ms: d128 S = 2048 (one wave
            // per SIMD) 0.0655 -> 0.0640, S = 8192 unchanged; d256 window-1024
            // layer 0.147 -> 0.140, global 0.348 -> 0.333.  At d64 it made the
            // S = 8192 launch slower (0.167 -> 0.173), so d64 goes without it.
            if constexpr (D != 64) __builtin_amdgcn_iglp_opt(1);
            // S^T = K Q^T.  The waves raise their priority over their MFMA
            // groups (s_setprio 1) so the SIMD's arbiter favours the wave that has
            // matrix work ready while the other computes its softmax.
            __builtin_amdgcn_s_setprio(1);
            f32x16 sacc;
            const uint16_t* krow = kb + (32 * sb + ln) * D;
#pragma unroll
            for (int s = 0; s < D / 16; s++) {
                const int c = (2 * s + lg) ^ swz_k;
                const uint4 a = *(const uint4*)(krow + c * 8);
                sacc = M::mma(a, qf[s], s == 0 ? (kFold ? negm : zero) : sacc);
                if constexpr (kQloLds) sacc = M::mma(a, Qlo[(wave * (D / 16) + s) * 64 + lane], sacc);
                else if constexpr (kSplit) sacc = M::mma(a, qfl[s], sacc);
            }
            // V^T fragment (dt, t) of this sub-tile: two transpose reads
            auto load_va = [&](int dt, int t) {
                i16x4 part[2];
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    const int off = (32 * sb + 16 * t) * D + v_base[b] + (((4 * dt + v_chunk) ^ v_swz[b]) << 3);
                    part[b] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GR_LDS i16x4*)(vb + off));
                }
                const uint2 lo = __builtin_bit_cast(uint2, part[0]);
                const uint2 hi = __builtin_bit_cast(uint2, part[1]);
                return make_uint4(lo.x, lo.y, hi.x, hi.y);
            };
            // d <= 128: all V^T fragments are read before the softmax (they do not
            // depend on it); d = 256 reads them next to their MFMAs (registers).
            constexpr bool kPreV = D <= 128;
            uint4 va[kPreV ? D / 32 : 1][2];
            if constexpr (kPreV) {
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                    for (int t = 0; t < 2; t++) va[dt][t] = load_va(dt, t);
            }

            __builtin_amdgcn_s_setprio(0);
            // element e of the accumulator is key ts + 8 (e/4) + 4 lg + e%4
            const bool need_mask = (ts + 31 > hi_min) || (ts < lo_max);
            if (need_mask) {
                // visible iff lo <= key <= hi: one unsigned compare per element
                const int lo = row_lo(my_pos);
                const unsigned range = (unsigned)(row_hi(my_pos) - lo);
                const int kb0 = ts + 4 * lg - lo;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int off = 8 * (e >> 2) + (e & 3);
                    sacc[e] = (unsigned)(kb0 + off) <= range ? sacc[e] : -INFINITY;
                }
            }
            float mx = fmaxf(sacc[0], sacc[1]);
#pragma unroll
            for (int e = 2; e < 16; e++) mx = fmaxf(mx, sacc[e]);
            mx = pf_xmax32(mx);
            if constexpr (kFold) {
                if (__any(mx > thr)) {
                    const float mnew = fmaxf(mrow, mx + m_off);
                    const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
                    mrow = mnew;
                    lrow *= alpha;
#pragma unroll
                    for (int dt = 0; dt < D / 32; dt++) o[dt] *= alpha;
                    const float off_new = mnew > -1e29f ? mnew : 0.0f;
                    sacc += m_off - off_new;
                    m_off = off_new;
                    thr = mrow + kLazyRescale - m_off;
#pragma unroll
                    for (int e = 0; e < 16; e++) negm[e] = -m_off;
                }
            } else if (__any(mx > mrow + kLazyRescale)) {
                const float mnew = fmaxf(mrow, mx);
                const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
                mrow = mnew;
                lrow *= alpha;
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++) {
                    // d = 256: O lives in AGPRs (the MFMAs accumulate there).  The
                    // empty asm statements move it to VGPRs for the multiply and
                    // back here, inside this rarely taken branch; otherwise the
                    // compiler copies all of O out of the AGPRs on every tile.
                    if constexpr (D == 256) asm volatile("" : "+v"(o[dt]));
                    o[dt] *= alpha;
                    if constexpr (D == 256) asm volatile("" : "+a"(o[dt]));
                }
            }
            float pv[16];
#pragma unroll
            for (int e = 0; e < 16; e++) pv[e] = __builtin_amdgcn_exp2f(kFold ? sacc[e] : sacc[e] - mrow);
            if constexpr (kSplit) {
                float psum = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) psum += pv[e];
                lrow += psum;
            }
            // B operand P^T, k-step t: k-slot r <-> key ts + 16 t + 8 (r/4) + 4 lg + r%4
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
            __builtin_amdgcn_s_setprio(1);
            // O^T += V^T P^T; the V^T slot order matches P^T's: slots 0..3 are keys
            // 16 t + 4 lg + 0..3, slots 4..7 keys 16 t + 8 + 4 lg + 0..3.
#pragma unroll
            for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint4 a = kPreV ? va[kPreV ? dt : 0][t] : load_va(dt, t);
                    o[dt] = M::mma(a, pf[t], o[dt]);
                    if constexpr (kSplit) o[dt] = M::mma(a, pfl[t], o[dt]);
                }
            __builtin_amdgcn_s_setprio(0);
        };
        auto compute_tile = [&](const uint16_t* kb, const uint16_t* vb, int t0) {
#pragma unroll
            for (int sb = 0; sb < BN / 32; sb++) {
                const int ts = t0 + 32 * sb;
                if (KH > 1 && sb % KH != kh) continue;  // the other key half's sub-tile
                if (!(wave_active && ts <= hi_max && ts + 31 >= lo_min)) continue;
                subtile(kb, vb, sb, ts);
            }
        };

        __syncthreads();  // the previous pass is done with every LDS buffer
        dma_tile(t_first, Ks0, Vs0);
        for (int it = 0; it < n_tiles; it += 2) {
            const int t0 = t_first + it * BN;
            pf_wait_vmem();   // this thread's part of tile it is in LDS
            __syncthreads();  // ... everyone's, and tile it-1's buffers are free
            if (it + 1 < n_tiles) dma_tile(t0 + BN, Ks1, Vs1);
            compute_tile(Ks0, Vs0, t0);
            if (it + 1 >= n_tiles) break;
            pf_wait_vmem();
            __syncthreads();
            if (it + 2 < n_tiles) dma_tile(t0 + 2 * BN, Ks0, Vs0);
            compute_tile(Ks1, Vs1, t0 + BN);
        }

        if constexpr (KH > 1) {
            // Key half 1 hands (O, m, l) of its rows to key half 0 through the tile
            // buffers, free once every wave is past its last tile.  Both halves'
            // O and l are relative to their own reference maxima m (the row's
            // m_off of the folded S^T start is m once the row has seen a key,
            // and O = l = 0 before), so O = O0 2^(m0 - M) + O1 2^(m1 - M), M = max.
            constexpr int NO = D / 32 * 16;
            static_assert(2 * NO * 64 * 4 <= BN * D * 2 && RW * 2 * 64 * 4 <= BN * D * 2, "merge buffers");
            float* ob = (float*)(rw < 2 ? Ks0 : Ks1) + (size_t)(rw & 1) * NO * 64;
            float* mlb = (float*)Vs0 + (size_t)rw * 2 * 64;
            __syncthreads();
            if (kh == 1) {
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                    for (int e = 0; e < 16; e++) ob[(dt * 16 + e) * 64 + lane] = o[dt][e];
                mlb[lane] = mrow;
                mlb[64 + lane] = lrow;
            }
            __syncthreads();
            if (kh == 0) {
                const float m1 = mlb[lane], l1 = mlb[64 + lane];
                const float mm = fmaxf(mrow, m1);
                const float a0 = __builtin_amdgcn_exp2f(mrow - mm), a1 = __builtin_amdgcn_exp2f(m1 - mm);
                lrow = lrow * a0 + l1 * a1;
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                    for (int e = 0; e < 16; e++) o[dt][e] = o[dt][e] * a0 + ob[(dt * 16 + e) * 64 + lane] * a1;
            }
        }
        const float lsum = pf_xsum32(lrow);
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        if (row_ok && kh == 0) {
            float* orow = p.out + ((size_t)my_row * p.n_heads + h) * D;
            const float* gt = p.gate.at(my_row, h);  // Qwen3.5 output gate, or null
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

// The LDS of one workgroup: double-buffered K and V tiles (four distinct
// arrays) and, with QLO, the bf16 d256 Q residual fragments.
#define GR_PF_LDS(D, NW, KH, QLO)                                                      \
    __shared__ __attribute__((aligned(16))) uint16_t Ks0[PfTile<D, NW, KH>::BN * D];  \
    __shared__ __attribute__((aligned(16))) uint16_t Ks1[PfTile<D, NW, KH>::BN * D];  \
    __shared__ __attribute__((aligned(16))) uint16_t Vs0[PfTile<D, NW, KH>::BN * D];  \
    __shared__ __attribute__((aligned(16))) uint16_t Vs1[PfTile<D, NW, KH>::BN * D];  \
    __shared__ __attribute__((aligned(16))) uint4 Qlo[(QLO) ? NW * (D / 16) * 64 : 1]

template <typename DT, int D, int NW, int KH>
__global__ __launch_bounds__(NW * 64, (PfTile<D, NW, KH>::kWaves)) void prefill_kernel(const PrefillLaunch p) {
    GR_PF_LDS(D, NW, KH, Mfma32<DT>::kSplit && D == 256);
    prefill_body<DT, D, NW, KH>(p, p.k_cache, p.v_cache, p.cache_row_stride, 0, Ks0, Ks1, Vs0, Vs1, Qlo);
}

// bf16 cache with an exact f16 copy of its visible rows: the single-pass f16
// path on the copy, or, when the copy could not hold every value (the flag
// carries this launch's epoch), the bf16 hi + lo path on the cache itself.
template <int D, int NW, int KH>
__global__ __launch_bounds__(NW * 64, (PfTile<D, NW, KH>::kWaves)) void prefill_bf16x_kernel(const PrefillLaunch p) {
    GR_PF_LDS(D, NW, KH, D == 256);
    if (*p.f16_flag != p.f16_epoch)
        prefill_body<F16, D, NW, KH>(p, p.k_f16, p.v_f16, p.f16_row_stride, p.f16_row0, Ks0, Ks1, Vs0, Vs1, Qlo);
    else
        prefill_body<BF16, D, NW, KH>(p, p.k_cache, p.v_cache, p.cache_row_stride, 0, Ks0, Ks1, Vs0, Vs1, Qlo);
}
#undef GR_PF_LDS

template <typename DT, int D, int NW, int KH = 1>
static hipError_t launch_prefill_d(const PrefillLaunch& p, hipStream_t st) {
    constexpr int BM = NW / KH * 32;
    const int n_qb = (p.n_tokens + BM - 1) / BM;
    const int n_items = p.n_heads * ((n_qb + 1) / 2);  // query blocks paired heavy + light
    dim3 grid(8 * ((n_items + 7) / 8));
    if (std::is_same<DT, BF16>::value && p.k_f16)
        prefill_bf16x_kernel<D, NW, KH><<<grid, NW * 64, 0, st>>>(p);
    else
        prefill_kernel<DT, D, NW, KH><<<grid, NW * 64, 0, st>>>(p);
    return hipGetLastError();
}

// Workgroup shape (d <= 128): eight waves of 256 rows once those workgroups
// alone fill every CU (256 on MI355X); else four waves of 128 rows, or, at d64
// while those number at most one per CU, the same 128-row blocks on eight waves
// as two key halves.  Measured (MI355X): 14 / 2 heads, d64, S = 2048 (112
// workgroups) 44.0 -> 36.4 us per call; at d128 (32 / 8 heads, S = 2048, 256
// workgroups) the key halves were 1.5% slower than four waves.
enum { kPfWaves8 = 8, kPfWaves4 = 4, kPfKeyHalves = 2 };
static int prefill_pick(const PrefillLaunch& p) {
    constexpr int kCUs = 256;
    if (p.head_dim > 128) return kPfWaves4;
    const int n_qb8 = (p.n_tokens + 255) / 256, n_qb4 = (p.n_tokens + 127) / 128;
    if (p.n_heads * ((n_qb8 + 1) / 2) >= kCUs) return kPfWaves8;
    return p.head_dim == 64 && p.n_heads * ((n_qb4 + 1) / 2) <= kCUs ? kPfKeyHalves : kPfWaves4;
}

template <typename DT>
static hipError_t launch_prefill_dt(const PrefillLaunch& p, hipStream_t st) {
    switch (p.head_dim) {
        case 64:
            switch (prefill_pick(p)) {
                case kPfWaves8: return launch_prefill_d<DT, 64, 8>(p, st);
                case kPfKeyHalves: return launch_prefill_d<DT, 64, 8, 2>(p, st);
                default: return launch_prefill_d<DT, 64, 4>(p, st);
            }
        case 128:
            return prefill_pick(p) == kPfWaves8 ? launch_prefill_d<DT, 128, 8>(p, st) : launch_prefill_d<DT, 128, 4>(p, st);
        case 256: return launch_prefill_d<DT, 256, 4>(p, st);
        default: return hipErrorInvalidValue;
    }
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
