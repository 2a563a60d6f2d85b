// Split-K flash decoding on gfx950 MFMA for 16-bit (f16 / bf16) and Q8 KV caches.
//
// Same work split and partial format as decode.hip (one workgroup per
// (sequence, KV head, split); partials merged by decode_combine_kernel), but
// the scores and the value accumulation run on v_mfma_f32_16x16x32 with up to 16
// query heads of a GQA group on the N axis (larger groups: several workgroup
// columns per KV head, DecodeLaunch::n_sub):
//   S^T[key][q]  = K . Q^T        A = K rows (16-bit caches: from a per-wave
//                                 LDS tile; Q8: straight from HBM)
//   O^T[d][q]   += V^T . P^T      A = V^T from a per-wave LDS tile, B = P from
//                                 the S^T accumulators (same lane <-> query map)
// Each wave streams its own 32-key tiles (8 waves per workgroup for d128
// without block scales, else 4; wave w starts with tile w and then, with 8
// waves, claims the next unclaimed tile of its segment from an LDS counter,
// with 4 takes tile w + 4, w + 8, ...; the next tile is
// prefetched into registers while the current one is processed) and keeps its
// own online-softmax state; the waves merge in LDS.
// Q is carried as a hi + lo 16-bit pair (two MFMAs per product; K and V are
// exact 16-bit cache values), so the scores keep ~fp32 precision even for
// large unscaled logits; P is one operand for f16 caches and a hi + lo pair
// for bf16 and Q8.  Decode is HBM-bound with the matrix cores mostly idle.
//
// Q8 caches (KvCacheFormat::Q8, reference inference.rs:1337-1483): int8 codes
// are exact in f16, so K and V tiles are widened to f16 in registers and the
// same f16 MFMAs run; the f32 scales are applied outside the products:
//   row scales    score *= k_scale[t];  P[t] *= v_scale[t] before the PV product
//   block scales  one QK MFMA chain per 32-element block (an MFMA k-step is
//                 exactly one block), scaled and summed; one P operand per
//                 V block, scaled by that block's v scale.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "gr_common.hpp"
#include "gr_internal.hpp"
#include "stream_sched.hpp"

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
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    // f16 words of (a0, a1) (one v_cvt_pk_f16_f32, round to nearest even), and the
    // words of the residuals a - f16(a) given those words
    static __device__ __forceinline__ uint32_t pack2(float a0, float a1) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a0, a1}, h2));
    }
    static __device__ __forceinline__ uint32_t rest2(uint32_t hi, float a0, float a1) {
        const h2 h = __builtin_bit_cast(h2, hi);
        return pack2(a0 - (float)h[0], a1 - (float)h[1]);
    }
};
template <>
struct Mfma16<BF16> {
    static constexpr bool kSplit = true;
    static __device__ __forceinline__ f32x4 mma(const uint4& a, const uint4& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float a0, float a1) { return pack_bf16x2(a0, a1); }
    static __device__ __forceinline__ uint32_t rest2(uint32_t hi, float a0, float a1) {
        return pack2(a0 - __uint_as_float(hi << 16), a1 - __uint_as_float(hi & 0xffff0000u));
    }
};

// KV storage formats: Raw = one lane's 8-element chunk as loaded from HBM,
// to16() = the same 8 elements as 16-bit MFMA operands.
template <typename DT>
struct Kv16 {
    using M = Mfma16<DT>;
    using Raw = uint4;
    static constexpr bool kQ8 = false, kBlock = false;
    static __device__ __forceinline__ uint4 to16(const uint4& r) { return r; }
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// int8 -> f16, exact: with u = c + 128 (flip the sign bit), the f16 with
// exponent byte 0x64 and low byte u is 1024 + u, and (1024 + u) - 1152 = c.

template <bool BLOCK>
struct KvQ8 {
    using M = Mfma16<F16>;
    using Raw = uint2;
    static constexpr bool kQ8 = true, kBlock = BLOCK;
    // v_perm places the sign-flipped codes under the exponent byte 0x64 (selector
    // bytes 0..3 pick bytes of the code word, 4 a byte of 0x64646464)
    static __device__ __forceinline__ uint4 to16(const uint2& r) {
        const uint32_t a = r.x ^ 0x80808080u, b = r.y ^ 0x80808080u;
        auto two = [](uint32_t w, uint32_t sel) {
            const half2_t h = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, sel)) -
                              half2_t{1152.0f16, 1152.0f16};
            return __builtin_bit_cast(uint32_t, h);
        };
        return make_uint4(two(a, 0x04010400u), two(a, 0x04030402u), two(b, 0x04010400u), two(b, 0x04030402u));
    }
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Cache rows are read once per launch.  V tiles are read a row slice per
// 16 lanes (4 rows x 256 B per instruction for d128 f16), and those loads carry
// the nontemporal hint (streaming policy in the L2): a plain read of that
// pattern measured 6.0 TB/s with ordinary loads and 6.7 TB/s with the hint on
// MI355X.  K tiles are loaded in the MFMA operand layout, 64 B (f16, Q8 row
// scales) or 32 B (Q8 block scales) of each of 16 rows per instruction, i.e.
// part of a 128-byte line; with the hint the line leaves the L2 before the rest
// is read (5.8 -> 5.2 TB/s for that pattern), so K and all Q8 rows use plain loads.
__device__ __forceinline__ void ld_stream(uint4* r, const void* p) {
    const u32x4_t x = __builtin_nontemporal_load((const u32x4_t*)p);
    *r = make_uint4(x[0], x[1], x[2], x[3]);
}
__device__ __forceinline__ void ld_stream(uint2* r, const void* p) { *r = *(const uint2*)p; }
template <typename R>
__device__ __forceinline__ void ld_plain(R* r, const void* p) { *r = *(const R*)p; }

// Buffer descriptor for a wave-uniform base address (read from lane 0), for raw
// buffer loads with a scalar base and 32-bit per-lane offsets.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t md_rsrc(const void* p) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)(((uint64_t)hi << 32) | lo), 0, (int)0xffffffff,
                                             0x00020000);
}
// soff is wave-uniform at every call site (whole-tile or tail offsets of a
// wave-uniform tile); readfirstlane states it, so that a value the compiler
// cannot prove uniform is not turned into a loop over its distinct values
// around the load.
__device__ __forceinline__ uint2 md_ld8(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, __builtin_amdgcn_readfirstlane(soff), 0);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint4 md_ld16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, __builtin_amdgcn_readfirstlane(soff), 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float md_ldf(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, __builtin_amdgcn_readfirstlane(soff), 0));
}

// Waves per workgroup: 8 (one workgroup per CU, two waves per SIMD) where the
// registers (<= 256) and the per-wave LDS tiles allow it, else 4.
template <typename KV, int D>
struct MdWaves {
    static constexpr int value = D <= 128 && !KV::kBlock ? 8 : 4;
};

// Raise a row's reference maximum only when a tile exceeds it by more than
// this (log2 units); P = 2^(s - m_ref) <= 2^8 meanwhile and O needs no rescale.
constexpr float kMdLazyRescale = 8.0f;

// NSUB groups of 32 keys per wave iteration.  1 is used: with 2, the d128
// kernel needs 300 registers (one wave per SIMD) and measured slower than two
// waves per SIMD streaming 32-key tiles.  bf16 d128 needs the bound to stay
// within 256 registers (two waves per SIMD).
template <typename KV, int D, int NSUB>
__global__ __launch_bounds__((MdWaves<KV, D>::value * 64),
                             (D <= 128 && std::is_same<KV, Kv16<BF16>>::value ? 2 : 1)) void decode_mfma_kernel(const DecodeLaunch p) {
    constexpr int kMdWaves = MdWaves<KV, D>::value;
    constexpr int kMdThreads = kMdWaves * 64;
    using M = typename KV::M;
    using Raw = typename KV::Raw;
    constexpr bool kSplit = M::kSplit;
    constexpr bool kQ8 = KV::kQ8, kBlock = KV::kBlock;
    // P (<= 2^8 after the lazy rescale) as one f16 operand for f16 caches
    // (relative rounding 2^-12, against a bar of 2e-3 + 1e-2 |ref|); bf16 (2^-9)
    // and Q8 (fp32-level bar) keep the hi + lo pair.
    constexpr bool kSplitP = kSplit && (kQ8 || !std::is_same<M, Mfma16<F16>>::value);
    constexpr int NB = D / 32;                   // 32-element scale blocks per head (Q8 block mode)
    constexpr int TILE = 32 * NSUB;              // keys per wave iteration
    constexpr int NS16 = TILE / 16;              // 16-key score sub-tiles
    constexpr int DC = D / 8;                    // 16-byte chunks per row
    constexpr int KS = D / 32;                   // MFMA k-steps over d
    constexpr int VTASK = (TILE / 4) * DC / 64;  // 4-key x 16-byte V tasks per lane
    constexpr int VS = TILE + 4;                 // V^T row stride (elements)
    // V^T rows hold TILE / 4 quads of 4 keys; quad q of row d sits at quad
    // q ^ vswz(d), vswz(d) = ((d / 32) * (256 / D)) % 8: the transposing stores of
    // one instruction (rows 8 dc + dd, 16 dc values) then hit distinct banks, where
    // the row stride alone maps every fourth dc to the same banks
    auto vswz = [](int d) { return ((d >> 5) * (256 / D)) & 7; };
    static_assert(VTASK >= 1, "tile");

    // LDS: per-wave V^T tiles during the key loop, then (aliased) the wave merge.
    constexpr int kVtBytes = kMdWaves * D * VS * 2;
    // Q8 block mode: per-wave scale tile [K|V][block][32 keys] after the V^T tiles
    constexpr int kScBytes = kBlock ? kMdWaves * 2 * NB * TILE * 4 : 0;
    // 16-bit caches: per-wave K tile [TILE rows][DC chunks], 16-byte chunk c of
    // row r at chunk c ^ kswz(r), the rows fetched as full-line row slices like V.
    // d >= 128 (16+ chunks a row): kswz(r) = r & 15, conflict-free for the
    // row-slice writes and the 16-row MFMA operand reads.  d64 (8 chunks, two rows
    // per 256 bytes): kswz(r) = (r >> 1) & 7 keeps the operand reads of 16
    // consecutive rows on distinct bank groups (the row-slice writes, rows of one
    // parity per instruction, take two passes).
    // Q8 reads K straight from HBM in the operand layout: staging its rows through
    // the same tile (codes converted on the way in) measured slower at 32k keys,
    // 4.40 -> 3.73 TB/s with row scales and 3.39 -> 2.71 with block scales.
    constexpr bool kKLds = !kQ8;
    static_assert(!kKLds || DC >= 16 || DC == 8, "K tile swizzle: 8 or 16+ chunks a row");
    auto kswz = [](int r) { return DC >= 16 ? (r & 15) : ((r >> 1) & 7); };
    constexpr int kKBytes = kKLds ? kMdWaves * TILE * D * 2 : 0;
    constexpr int kLoopBytes = kVtBytes + kScBytes + kKBytes;
    constexpr int kMergeBytes = (kMdWaves * 16 * (D + 1) + 2 * kMdWaves * 16) * 4;
    __shared__ __attribute__((aligned(16))) char smem[kLoopBytes > kMergeBytes ? kLoopBytes : kMergeBytes];
    // d256 with block scales: the Q residual fragments live in LDS (per wave,
    // [k-step][lane]) instead of 32 VGPRs, which the per-block chains need
    constexpr bool kQloLds = kSplit && kBlock && D == 256;
    __shared__ __attribute__((aligned(16))) uint4 Qlo[kQloLds ? kMdWaves * KS * 64 : 1];

    const int kv_mul = p.n_heads / p.n_kv_heads;
    // grid / schedule columns: n_sub per KV head, 16 query heads each (DecodeLaunch::n_sub)
    const int n_sub = p.n_sub > 0 ? p.n_sub : 1;
    const int n_cols = p.n_kv_heads * n_sub;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l16 = lane & 15, g4 = lane >> 4;

    // Segment = keys [t_begin, t_stop) of sequence s, column g (KV head g / n_sub); its partial
    // goes to slot `split` of the (s, head) partial rows.
    int s, g, t_begin, t_stop, split;
    // stream schedule state (DecodeLaunch::stream_sched, stream_sched.hpp)
    __shared__ int st_len[kStreamMaxSeq];
    __shared__ int st_off[kStreamMaxSeq];
    __shared__ int st_first;
    __shared__ int st_wsum[kMdWaves];
    StreamCursor<kMdThreads> cur;
    // Tiles of the current segment: wave w starts with tile w, then claims the
    // next unclaimed one from this counter, so waves that get more issue slots
    // (the older wave of a SIMD) take more tiles and the waves finish together.
    __shared__ int tile_next;
    if (!p.stream_sched) {
        split = blockIdx.x;
        g = blockIdx.y;
        s = blockIdx.z;
        t_begin = p.kv_start[s] + split * p.split_keys;
        const int t_limit = p.kv_end[s];
        if (t_begin >= t_limit) return;
        t_stop = min(t_limit, t_begin + p.split_keys);
    } else {
        if (!cur.init(p, n_cols, st_len, st_off, &st_first, st_wsum)) return;
        t_begin = t_stop = split = 0;  // set per segment below
    }

    if (tid == 0) tile_next = kMdWaves;
    __syncthreads();
    for (;;) {
    if (p.stream_sched) {
        if (!cur.segment(p, t_begin, t_stop, split)) break;  // the range ends inside the pair's virtual keys
        s = cur.s;
        g = cur.col;
        __syncthreads();  // the previous segment is done with the LDS
    }
    // The segment bounds are wave-uniform; in SGPRs the whole-tile / tail choices
    // on them stay scalar branches instead of per-lane selects of load offsets.
    t_begin = __builtin_amdgcn_readfirstlane(t_begin);
    t_stop = __builtin_amdgcn_readfirstlane(t_stop);
    const int kvh = g / n_sub;                                     // KV head
    const int h0 = kvh * kv_mul + (g % n_sub) * 16;                // first query head
    const int nq = min(16, kvh * kv_mul + kv_mul - h0);            // query heads (MFMA columns)
    uint16_t* vt = (uint16_t*)smem + wave * D * VS;
    float* sct = (float*)(smem + kVtBytes) + wave * 2 * NB * TILE;  // block mode: [2][NB][TILE]
    uint4* kst = (uint4*)(smem + kVtBytes + kScBytes) + wave * TILE * DC;  // 16-bit: K tile

    // Element d of the head row behind slot e of k-step k in lane group g4: 32 k +
    // 8 g4 + e; Q8 with row scales pairs k-steps 2j, 2j + 1 on one 16-byte code
    // load per lane, d = 64 j + 16 g4 + 8 (k & 1) + e (the sum over d is the same;
    // block scales keep one 32-element block per k-step).
    constexpr bool kPairK = kQ8 && !kBlock && KS % 2 == 0;
    auto dperm = [](int k, int g) { return kPairK ? 64 * (k >> 1) + 16 * g + 8 * (k & 1) : 32 * k + 8 * g; };
    const size_t slot = (size_t)(p.seq_slot ? p.seq_slot[s] : s);
    // element pointers (one element = sizeof(Raw)/8 bytes)
    typedef typename std::conditional<kQ8, int8_t, uint16_t>::type Elem;
    const Elem* kc = (const Elem*)p.k_cache + slot * p.seq_stride + (size_t)kvh * D;
    const Elem* vc = (const Elem*)p.v_cache + slot * p.seq_stride + (size_t)kvh * D;
    const int64_t rs = p.row_stride;
    // Q8 scales: this lane's keys of S^T register j of sub-tile sb are
    // t0 + 16 sb + 4 g4 + j; block mode adds the kv head's block offset.
    const float* ksb = nullptr;
    const float* vsb = nullptr;
    int64_t srs = 0;
    if constexpr (kQ8) {
        const size_t so = slot * p.scale_seq_stride + (kBlock ? (size_t)kvh * NB : 0);
        ksb = p.k_scale + so;
        vsb = p.v_scale + so;
        srs = p.scale_row_stride;
    }
    // Row mode: each lane prefetches the k / v scales of its 4 NS16 keys.  Block
    // mode: the wave prefetches the tile's 32 x NB k and v block scales (NB/2 per
    // lane, coalesced along a row) and stages them in LDS for the score and P passes.
    constexpr int NRS = kQ8 && !kBlock ? 4 * NS16 : 1;
    constexpr int NBS = kBlock ? TILE * NB / 64 : 1;
    float ksc[NRS], vsc[NRS];
    float kbs[NBS], vbs[NBS];

    Raw kr[kKLds ? 1 : NS16][KS];   // Q8: K in the MFMA operand layout
    Raw krs[kKLds ? VTASK : 1][4];  // 16-bit: K rows in the V row-slice layout
    Raw vr[VTASK][4];
    // Q8 with row scales: raw buffer loads from the tile's first row (wave-uniform
    // base), so the lane offsets of a whole tile are the same for every tile and
    // the loop carries no 64-bit address arithmetic; the last tile of a range
    // clamps its keys to t_stop - 1.  Block scales keep plain loads.
    constexpr bool kBufLd = kQ8 && !kBlock;
    const int srsb = (int)srs * 4;  // scale row stride, bytes
    auto load_scales = [&](int t0) {
        const int last = t_stop - 1 - t0;  // last valid key, relative to t0
        const bool whole = t0 + TILE <= t_stop;
        (void)last;
        (void)whole;
        if constexpr (kBlock) {
            // block scales: plain loads (the four extra scalar descriptors of the
            // buffer path cost the block-scale kernel SGPR spills: 10% slower)
#pragma unroll
            for (int u = 0; u < NBS; u++) {
                const int e = lane + 64 * u;
                const int key = min(t0 + e / NB, t_stop - 1);
                kbs[u] = ksb[(int64_t)key * srs + e % NB];
                vbs[u] = vsb[(int64_t)key * srs + e % NB];
            }
        } else if constexpr (kQ8) {
            const __amdgpu_buffer_rsrc_t kr_ = md_rsrc(ksb + (int64_t)t0 * srs);
            const __amdgpu_buffer_rsrc_t vr_ = md_rsrc(vsb + (int64_t)t0 * srs);
#pragma unroll
            for (int e = 0; e < NRS; e++) {
                const int kk = 16 * (e >> 2) + (e & 3);  // key - 4 g4 - t0
                if (whole) {
                    ksc[e] = md_ldf(kr_, 4 * g4 * srsb, kk * srsb);
                    vsc[e] = md_ldf(vr_, 4 * g4 * srsb, kk * srsb);
                } else {
                    const int off = min(kk + 4 * g4, last) * srsb;
                    ksc[e] = md_ldf(kr_, off, 0);
                    vsc[e] = md_ldf(vr_, off, 0);
                }
            }
        }
    };
    // V and K of a tile are fetched separately: V as soon as the current V tile
    // is in LDS, K (and the Q8 scales) once the current scores are done, so each
    // is in flight for most of an iteration.
    auto load_v = [&](int t0) {
        if constexpr (kBufLd) {
            const __amdgpu_buffer_rsrc_t r_ = md_rsrc(vc + (int64_t)t0 * rs);
            const bool whole = t0 + TILE <= t_stop;
            const int last = t_stop - 1 - t0;
#pragma unroll
            for (int u = 0; u < VTASK; u++) {
                const int task = lane + 64 * u;
                const int dc = task % DC, kg = task / DC;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if (whole) vr[u][r] = md_ld8(r_, 4 * kg * (int)rs + 8 * dc, r * (int)rs);
                    else vr[u][r] = md_ld8(r_, min(4 * kg + r, last) * (int)rs + 8 * dc, 0);
                }
            }
            return;
        }
        if (t0 + TILE <= t_stop) {  // whole tile inside the split: plain strided rows
            const Elem* vtp = vc + (int64_t)t0 * rs;
#pragma unroll
            for (int u = 0; u < VTASK; u++) {
                const int task = lane + 64 * u;
                const int dc = task % DC, kg = task / DC;
                const Elem* v0 = vtp + (int64_t)(4 * kg) * rs + 8 * dc;
#pragma unroll
                for (int r = 0; r < 4; r++) ld_stream(&vr[u][r], v0 + r * rs);
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < VTASK; u++) {
            const int task = lane + 64 * u;
            const int dc = task % DC, kg = task / DC;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = min(t0 + 4 * kg + r, t_stop - 1);
                ld_stream(&vr[u][r], vc + (int64_t)key * rs + 8 * dc);
            }
        }
    };
    auto load_k = [&](int t0) {
        if constexpr (kKLds) {  // row slices, like V
            const bool whole = t0 + TILE <= t_stop;
#pragma unroll
            for (int u = 0; u < VTASK; u++) {
                const int task = lane + 64 * u;
                const int dc = task % DC, kg = task / DC;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = whole ? t0 + 4 * kg + r : min(t0 + 4 * kg + r, t_stop - 1);
                    ld_stream(&krs[u][r], kc + (int64_t)key * rs + 8 * dc);
                }
            }
        } else if constexpr (!kBufLd) {
            const Elem* kt = kc + (int64_t)t0 * rs + 8 * g4;
            const bool whole = t0 + TILE <= t_stop;
#pragma unroll
            for (int sb = 0; sb < NS16; sb++) {
                const int key = whole ? 16 * sb + l16 : min(16 * sb + l16, t_stop - 1 - t0);
                const Elem* row = kt + (int64_t)key * rs;
#pragma unroll
                for (int k = 0; k < KS; k++) ld_plain(&kr[sb][k], row + 32 * k);
            }
        } else {
        // this lane's operand chunks of K row 16 sb + l16 of the tile (row offset
        // voff + soff bytes from the tile's first row)
        const __amdgpu_buffer_rsrc_t r_ = md_rsrc(kc + (int64_t)t0 * rs);
        auto load_row = [&](int sb, int voff, int soff) {
            if constexpr (kPairK) {
#pragma unroll
                for (int j = 0; j < KS / 2; j++) {
                    const uint4 w = md_ld16(r_, voff + 64 * j + 16 * g4, soff);
                    kr[sb][2 * j] = make_uint2(w.x, w.y);
                    kr[sb][2 * j + 1] = make_uint2(w.z, w.w);
                }
            } else {
#pragma unroll
                for (int k = 0; k < KS; k++) kr[sb][k] = md_ld8(r_, voff + 32 * k + 8 * g4, soff);
            }
        };
        if (t0 + TILE <= t_stop) {
#pragma unroll
            for (int sb = 0; sb < NS16; sb++) load_row(sb, l16 * (int)rs, 16 * sb * (int)rs);
            return;
        }
#pragma unroll
        for (int sb = 0; sb < NS16; sb++) load_row(sb, min(16 * sb + l16, t_stop - 1 - t0) * (int)rs, 0);
        }
    };

    // The segment's first tile is requested before Q is prepared, so the Q
    // loads and their conversion run while it is in flight.
    const int n_tiles = (t_stop - t_begin + TILE - 1) / TILE;
    int it = wave;
    if (it < n_tiles) {
        load_scales(t_begin + it * TILE);
        load_k(t_begin + it * TILE);
        load_v(t_begin + it * TILE);
    }
    // Q fragments (B operand of S^T = K Q^T): lane (query l16, group g4) holds
    // d = dperm(ks, g4) .. +7, pre-scaled to log2 units; columns >= nq are 0.
    // f16: each query row is also multiplied by a power of two 2^e that puts its
    // largest element near 2^14, so that the lo halves of the hi/lo split stay
    // out of the f16 subnormal range; the scores are multiplied back by 2^-e.
    uint4 qf[KS], qfl[kSplit && !kQloLds ? KS : 1];
    float qback = 1.0f;
    {
        const bool qv = l16 < nq;
        const float* qrow = p.q + ((size_t)s * p.n_heads + h0 + (qv ? l16 : 0)) * D;
        float qscale = p.score_scale * kLog2e;
        // the lane's 8 consecutive elements per k-step as two 16-byte loads (q is
        // 16-byte aligned, checked by the API, and rows are D floats)
        float qx[KS][8];
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const float* src = qrow + dperm(k, g4);
            const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 a = qv ? *(const float4*)src : z;
            const float4 b = qv ? *(const float4*)(src + 4) : z;
            qx[k][0] = a.x, qx[k][1] = a.y, qx[k][2] = a.z, qx[k][3] = a.w;
            qx[k][4] = b.x, qx[k][5] = b.y, qx[k][6] = b.z, qx[k][7] = b.w;
        }
        if constexpr (std::is_same<M, Mfma16<F16>>::value) {
            float qmax = 0.0f;
#pragma unroll
            for (int k = 0; k < KS; k++)
#pragma unroll
                for (int e = 0; e < 8; e++) qmax = fmaxf(qmax, fabsf(qx[k][e] * qscale));
            qmax = fmaxf(qmax, __shfl_xor(qmax, 16, 64));
            qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
            if (qmax > 0.0f && qmax < 3.0e38f) {
                int ex;
                (void)frexpf(qmax, &ex);               // qmax = m 2^ex, m in [0.5, 1)
                const int e = min(max(14 - ex, -100), 100);
                qscale *= ldexpf(1.0f, e);
                qback = ldexpf(1.0f, -e);
            }
        }
#pragma unroll
        for (int k = 0; k < KS; k++) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float x0 = qx[k][2 * w] * qscale;
                const float x1 = qx[k][2 * w + 1] * qscale;
                hw[w] = M::pack2(x0, x1);
                if constexpr (kSplit) lw[w] = M::rest2(hw[w], x0, x1);
            }
            qf[k] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            if constexpr (kQloLds) Qlo[(wave * KS + k) * 64 + lane] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            else if constexpr (kSplit) qfl[k] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        }
    }

    f32x4 o[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrow = -1e30f, lrow = 0.0f;
    // Q8: P * v_scale is carried as P * v_scale * pw[pb] with a power of two pw
    // that keeps the tile's largest v_scale * pw in [2^6, 2^7): the f16 hi/lo
    // pair then stays clear of the subnormal range (whose 6e-8 floor, times int8
    // codes up to 127, would show in the output) and P * v_scale * pw <= 2^15.
    // O rows of block pb accumulate pw[pb] times the true value; pw only
    // decreases (O rescaled) and is divided out after the loop.
    constexpr int NPB = kBlock ? NB : 1;   // P operands (one per V scale block)
    float pw[kQ8 ? NPB : 1];
    bool pw_set = false;
    // O *= f inside the rarely taken rescale branches.  With block scales O lives
    // in AGPRs (the MFMAs accumulate there); the empty asm statements move a tile
    // to VGPRs for the multiply and back inside the branch, where otherwise the
    // compiler reads all of O out of the AGPRs before the branch on every tile.
    auto scale_o = [&](int dt, float f) {
        if constexpr (kBlock) asm volatile("" : "+v"(o[dt]));
        o[dt] *= f;
        if constexpr (kBlock) asm volatile("" : "+a"(o[dt]));
    };

    while (it < n_tiles) {
        const int t0 = t_begin + it * TILE;
        // V tile -> LDS, transposed: Vt[d][key]
#pragma unroll
        for (int u = 0; u < VTASK; u++) {
            const int task = lane + 64 * u;
            const int dc = task % DC, kg = task / DC;
            const int kq = kg ^ vswz(8 * dc);  // this lane's quad of keys, swizzled (rows 8 dc .. 8 dc + 7)
            const uint4 v16[4] = {KV::to16(vr[u][0]), KV::to16(vr[u][1]), KV::to16(vr[u][2]), KV::to16(vr[u][3])};
            const uint32_t w[4][4] = {{v16[0].x, v16[0].y, v16[0].z, v16[0].w},
                                      {v16[1].x, v16[1].y, v16[1].z, v16[1].w},
                                      {v16[2].x, v16[2].y, v16[2].z, v16[2].w},
                                      {v16[3].x, v16[3].y, v16[3].z, v16[3].w}};
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
                *(uint2*)(vt + (8 * dc + dd) * VS + 4 * kq) = make_uint2(lo, hi);
            }
        }
        float vbmax[kBlock ? NB : 1];  // block mode: the tile's largest v scale per block (wave-uniform)
        if constexpr (kBlock) {
            float vl = 0.0f;
#pragma unroll
            for (int u = 0; u < NBS; u++) {
                const int e = lane + 64 * u;  // block e % NB == lane % NB for every u
                sct[(e % NB) * TILE + e / NB] = kbs[u];
                sct[(NB + e % NB) * TILE + e / NB] = vbs[u];
                vl = fmaxf(vl, vbs[u]);
            }
#pragma unroll
            for (int m = NB; m < 64; m <<= 1) vl = fmaxf(vl, __shfl_xor(vl, m, 64));
#pragma unroll
            for (int b = 0; b < NB; b++) vbmax[b] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vl), b));
            __builtin_amdgcn_wave_barrier();
        }
        if constexpr (kKLds) {
#pragma unroll
            for (int u = 0; u < VTASK; u++) {
                const int task = lane + 64 * u;
                const int dc = task % DC, kg = task / DC;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = 4 * kg + r;
                    kst[row * DC + (dc ^ kswz(row))] = KV::to16(krs[u][r]);
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        // this tile's rows are in LDS: claim the wave's next tile, fetch its V (and 16-bit K).
        // Four-wave workgroups (one wave per SIMD) keep the fixed order it + 4: the
        // claim's LDS round trip measured slower there.
        int nxt = it + kMdWaves;
        if constexpr (kMdWaves == 8) {
            if (lane == 0) nxt = atomicAdd(&tile_next, 1);
            nxt = __builtin_amdgcn_readfirstlane(nxt);
        }
        if (nxt < n_tiles) {
            load_v(t_begin + nxt * TILE);
            if constexpr (kKLds) load_k(t_begin + nxt * TILE);
        }
        // scores for the 16-key sub-tiles
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 sacc[NS16];
#pragma unroll
        for (int sb = 0; sb < NS16; sb++) {
#pragma unroll
            for (int k = 0; k < KS; k++) {
                uint4 ka;
                if constexpr (kKLds) {
                    const int row = 16 * sb + l16;
                    ka = kst[row * DC + ((4 * k + g4) ^ kswz(row))];
                } else {
                    ka = KV::to16(kr[sb][k]);
                }
                if constexpr (kBlock) {
                    // k-step k is scale block k: its own product, then scaled
                    f32x4 part = M::mma(ka, qf[k], zero);
                    if constexpr (kQloLds) part = M::mma(ka, Qlo[(wave * KS + k) * 64 + lane], part);
                    else if constexpr (kSplit) part = M::mma(ka, qfl[k], part);
                    const float4 k4 = *(const float4*)(sct + k * TILE + 16 * sb + 4 * g4);
                    const float kb[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        sacc[sb][j] = k == 0 ? part[j] * kb[j] : fmaf(part[j], kb[j], sacc[sb][j]);
                } else {
                    sacc[sb] = M::mma(ka, qf[k], k == 0 ? zero : sacc[sb]);
                    if constexpr (kQloLds) sacc[sb] = M::mma(ka, Qlo[(wave * KS + k) * 64 + lane], sacc[sb]);
                    else if constexpr (kSplit) sacc[sb] = M::mma(ka, qfl[k], sacc[sb]);
                }
            }
            if constexpr (kQ8 && !kBlock) {
#pragma unroll
                for (int j = 0; j < 4; j++) sacc[sb][j] *= ksc[4 * sb + j] * qback;
            } else if constexpr (std::is_same<M, Mfma16<F16>>::value) {
#pragma unroll
                for (int j = 0; j < 4; j++) sacc[sb][j] *= qback;
            }
        }
        // row-mode V scales of this tile (the prefetch below overwrites vsc)
        float vcur[NRS];
#pragma unroll
        for (int e = 0; e < NRS; e++) vcur[e] = vsc[e];
        // Q8: the scales (and, without the K tile, the K rows) of the wave's next tile
        if constexpr (kQ8)
            if (nxt < n_tiles) {
                load_scales(t_begin + nxt * TILE);
                if constexpr (!kKLds) load_k(t_begin + nxt * TILE);
            }

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
            for (int dt = 0; dt < D / 16; dt++) scale_o(dt, alpha);
        }
        float pv[4 * NS16];
        float psum = 0.0f;
#pragma unroll
        for (int e = 0; e < 4 * NS16; e++) {
            pv[e] = __builtin_amdgcn_exp2f(sv[e] - mrow);
            psum += pv[e];
        }
        lrow += psum;
        // B operand P^T per 32-key k-step kk: k-slot r <-> key 32 kk + 16 (r/4) + 4 g4 + r%4,
        // i.e. pv[8 kk + r]; for Q8, P is multiplied by the v scale of its key (and,
        // in block mode, of the V block `vb` that the output tiles of this pass cover).
        // v scale of this lane's P slot r = 2 w + h of k-step kk, block vb
        auto vscale_of = [&](int vb, int kk, int r) -> float {
            if constexpr (kBlock) {
                // pv[8 kk + r] is key 32 kk + 16 (r/4) + 4 g4 + r%4
                return sct[(NB + vb) * TILE + 32 * kk + 16 * (r >> 2) + 4 * g4 + (r & 3)];
            } else {
                return vcur[kQ8 ? 8 * kk + r : 0];
            }
        };
        if constexpr (kQ8) {
#pragma unroll
            for (int pb = 0; pb < NPB; pb++) {
                float vloc = 0.0f;
                if constexpr (kBlock) {
                    vloc = vbmax[pb];
                } else {
#pragma unroll
                    for (int kk = 0; kk < NSUB; kk++)
#pragma unroll
                        for (int r = 0; r < 8; r++) vloc = fmaxf(vloc, vscale_of(pb, kk, r));
                }
                const bool grow = kBlock ? vloc * pw[pb] >= 128.0f : __any(vloc * pw[pb] >= 128.0f);
                if (!pw_set || grow) {
                    const float vmax = kBlock ? vloc : wave_max<64>(vloc);
                    int ex;
                    (void)frexpf(vmax, &ex);  // vmax = m 2^ex, m in [0.5, 1)
                    const float npw = __int_as_float(__builtin_amdgcn_readfirstlane(
                        __float_as_int(vmax > 0.0f ? ldexpf(1.0f, min(max(7 - ex, -120), 120)) : 1.0f)));
                    if (pw_set && npw < pw[pb]) {
                        const float f = npw / pw[pb];
#pragma unroll
                        for (int dd = 0; dd < (D / 16) / NPB; dd++) scale_o(pb * ((D / 16) / NPB) + dd, f);
                        pw[pb] = npw;
                    } else if (!pw_set) {
                        pw[pb] = npw;
                    }
                }
            }
            pw_set = true;
        }
        auto make_p = [&](int vb, uint4* pf, uint4* pfl) {
#pragma unroll
            for (int kk = 0; kk < NSUB; kk++) {
                uint32_t ph[4], pl[4];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    float a0 = pv[8 * kk + 2 * w], a1 = pv[8 * kk + 2 * w + 1];
                    if constexpr (kQ8) {
                        a0 *= vscale_of(vb, kk, 2 * w) * pw[vb];
                        a1 *= vscale_of(vb, kk, 2 * w + 1) * pw[vb];
                    }
                    ph[w] = M::pack2(a0, a1);
                    if constexpr (kSplitP) pl[w] = M::rest2(ph[w], a0, a1);
                }
                pf[kk] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
                if constexpr (kSplitP) pfl[kk] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
            }
        };
        // LDS operations of one wave complete in issue order, so the V^T reads
        // below see this wave's stores; the barrier only pins the compiler's order.
        __builtin_amdgcn_wave_barrier();
        constexpr int DTB = (D / 16) / NPB;    // 16-row output tiles per P operand
#pragma unroll
        for (int pb = 0; pb < NPB; pb++) {
            uint4 pf[NSUB], pfl[kSplitP ? NSUB : 1];
            make_p(pb, pf, pfl);
#pragma unroll
            for (int dd = 0; dd < DTB; dd++) {
                const int dt = pb * DTB + dd;
                const uint16_t* vrow = vt + (16 * dt + l16) * VS;
                const int sw = vswz(16 * dt);  // the same for the 16 rows of tile dt
#pragma unroll
                for (int kk = 0; kk < NSUB; kk++) {
                    const uint2 lo = *(const uint2*)(vrow + 4 * ((8 * kk + g4) ^ sw));
                    const uint2 hi = *(const uint2*)(vrow + 4 * ((8 * kk + 4 + g4) ^ sw));
                    const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    o[dt] = M::mma(a, pf[kk], o[dt]);
                    if constexpr (kSplitP) o[dt] = M::mma(a, pfl[kk], o[dt]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // V^T / K reads done before the next tile overwrites them
        it = nxt;
    }

    if constexpr (kQ8) {
        if (pw_set) {
#pragma unroll
            for (int pb = 0; pb < NPB; pb++) {
                const float inv = 1.0f / pw[pb];  // exact: pw is a power of two
#pragma unroll
                for (int dd = 0; dd < (D / 16) / NPB; dd++) o[pb * ((D / 16) / NPB) + dd] *= inv;
            }
        }
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
    for (int idx = tid; idx < nq * D; idx += kMdThreads) {
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
        if (split >= n_splits) break;  // a sequence longer than max_kv_len: slots end here
        const size_t part = ((size_t)s * p.n_heads + h0 + q) * n_splits + split;
        p.ws_o[part * D + i] = ot;
        if (i == 0) {
            p.ws_ml[part * 2 + 0] = mx;
            p.ws_ml[part * 2 + 1] = lt;
        }
    }
    if (!p.stream_sched || !cur.advance()) break;
    if (tid == 0) tile_next = kMdWaves;  // ordered before the next segment's claims by its barrier
    }
}

// Workgroups of kernel k that fit on the current device at once (CUs x
// occupancy).  A device property: computed once per (template instance, device)
// and cached read-only; concurrent first calls compute the same value.
template <typename KV, int D>
static int resident_wgs() {
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
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, decode_mfma_kernel<KV, D, 1>, MdWaves<KV, D>::value * 64, 0) !=
            hipSuccess)
        return 256;
    const int v = std::max(1, n_cu * std::max(1, occ));
    if (slot >= 0) cached[slot].store(v, std::memory_order_relaxed);
    return v;
}

template <typename KV, int D>
static hipError_t launch_mfma_kv_d(const DecodeLaunch& p, hipStream_t st) {
    const dim3 grid = p.stream_sched ? dim3(resident_wgs<KV, D>())
                                     : dim3(p.n_splits, p.n_kv_heads * (p.n_sub > 0 ? p.n_sub : 1), p.n_seq);
    decode_mfma_kernel<KV, D, 1><<<grid, MdWaves<KV, D>::value * 64, 0, st>>>(p);
    return hipGetLastError();
}

template <typename KV>
static hipError_t launch_mfma_kv(const DecodeLaunch& p, hipStream_t st) {
    switch (p.head_dim) {
        case 64: return launch_mfma_kv_d<KV, 64>(p, st);
        case 128: return launch_mfma_kv_d<KV, 128>(p, st);
        case 256: return launch_mfma_kv_d<KV, 256>(p, st);
        default: return hipErrorInvalidValue;
    }
}

bool decode_mfma_supported(const DecodeLaunch& p) {
    const int kv_mul = p.n_heads / p.n_kv_heads;
    return (p.kv_dtype == GR_DTYPE_F16 || p.kv_dtype == GR_DTYPE_BF16 || p.kv_dtype == GR_DTYPE_Q8) &&
           (kv_mul <= 16 || (p.n_sub > 0 && p.sub_heads == 16)) &&
           (p.head_dim == 64 || p.head_dim == 128 || p.head_dim == 256);
}

hipError_t launch_decode_mfma_split(const DecodeLaunch& p, hipStream_t st) {
    switch (p.kv_dtype) {
        case GR_DTYPE_F16: return launch_mfma_kv<Kv16<F16>>(p, st);
        case GR_DTYPE_BF16: return launch_mfma_kv<Kv16<BF16>>(p, st);
        case GR_DTYPE_Q8: return p.q8_block ? launch_mfma_kv<KvQ8<true>>(p, st) : launch_mfma_kv<KvQ8<false>>(p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace gr
