// Gated DeltaNet (gated delta rule) on gfx950, fp32 state [H][d][d], S[j][i]
// with j = key dim (row) and i = value dim (column), as in
// qwen3next_state_head_step (reference src/engine/kernels/math.rs:492-546):
//   S *= g;  kv_i = sum_j k_j S[j][i];  delta_i = beta (v_i - kv_i);
//   S[j][i] += k_j delta_i;  o_i = sum_j q_j S[j][i]
// q/k are optionally L2-normalised first (q also * 1/sqrt(d)), math.rs:833-846.
// Columns i are independent (the reference's guards are per element too), which
// is how every kernel here parallelises.
//
// 1. deltanet_step_kernel: the recurrence token by token with a 32-column
//    slice of the state in registers (decode, the recurrent algorithm, and the
//    chunked algorithm's continuation after a chunk with non-finite values).
// 2. Chunked prefill (chunk C = 64).  With S0 the state before the chunk,
//    gamma_t = prod_{s<=t} g_s (in-chunk) and the normalised rows q_t, k_t:
//      A[t][s] = beta_t (gamma_t / gamma_s) k_t.k_s  (s < t),   T = (I + A)^-1
//      X       = diag(beta) (V - diag(gamma) K S0)
//      Delta   = T X                      (row t = the token's delta)
//      O       = diag(gamma) Q S0 + P Delta,  P[t][s] = (gamma_t / gamma_s) q_t.k_s  (s <= t)
//      S_C     = gamma_last S0 + sum_s (gamma_last / gamma_s) k_s Delta_s^T
//    which is the token recurrence whenever every guard of the reference is a
//    no-op (all values finite).
//    deltanet_chunk_prep_kernel (chunk, head): T, P and per-row scales; the
//    Gram products on v_mfma_f32_16x16x4_f32, T by forward substitution.
//    deltanet_chunk_scan_kernel (head, 16 state columns): the sequential chunk
//    steps with the raw q / k rows as operands and their row scales applied to
//    the products' rows; T X and P Delta on v_mfma_f32_16x16x4_f32, and K S0,
//    Q S0 and the state update too for f32 / f16 rows, while bf16 rows (exact
//    bf16 operands) run those three on v_mfma_f32_16x16x32_bf16 against the f32
//    state / Delta cut into three exact bf16 pieces.
//    Non-finite values: the prep flags a chunk whose inputs, T or P are not all
//    finite, the scan one whose X, Delta, O or new state are not.  The scan stops
//    before such a chunk, keeping the state it started from, and the step kernel
//    runs from there token by token with the reference's guards.
#include <type_traits>

#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

__device__ __forceinline__ float dn_load(const void* p, size_t i, int dt) {
    if (dt == GR_DTYPE_F32) return ((const float*)p)[i];
    const uint16_t b = ((const uint16_t*)p)[i];
    return dt == GR_DTYPE_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

constexpr int kChunk = 64;
constexpr int kChunkThreads = 256;
constexpr int kScanCols = 16;                 // state columns per scan workgroup
constexpr int kScanBlocks = 128 / kScanCols;  // scan workgroups per head

// ------------------------------------------------------------------ recurrent step
constexpr int kStepThreads = 256;
constexpr int kStepCols = 32;
static_assert(kStepCols == 2 * kScanCols, "a step block covers two scan blocks");

template <int D>
__global__ __launch_bounds__(kStepThreads) void deltanet_step_kernel(const DeltaNetLaunch p) {
    constexpr int NJG = kStepThreads / kStepCols;  // 8 row groups
    constexpr int R = D / NJG;                     // rows per thread
    __shared__ float qs[D], ks[D];
    __shared__ float red[kStepThreads / 64][kStepCols];
    const int tid = threadIdx.x;
    const int ci = tid % kStepCols;
    const int jg = tid / kStepCols;
    const int wave = tid >> 6, lane = tid & 63;
    const int h = blockIdx.y;
    const int i = blockIdx.x * kStepCols + ci;
    const int H = p.n_heads;
    float* Sh = p.state + (size_t)h * D * D;

    // After a chunked scan (first_bad set): column i continues from the first
    // token of the first chunk its scan block did not complete.
    int start = 0, t_begin = 0;
    if (p.first_bad) {
        const int* fb = p.first_bad + h * kScanBlocks + blockIdx.x * (kStepCols / kScanCols);
        start = fb[ci / kScanCols] * kChunk;
        t_begin = min(fb[0], fb[1]) * kChunk;
        if (t_begin >= p.n_tokens) return;  // uniform: the scan completed every chunk
    }

    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = Sh[(size_t)(jg * R + r) * D + i];

    const float inv_scale_q = 1.0f / sqrtf((float)D);
    for (int t = t_begin; t < p.n_tokens; t++) {
        const bool act = t >= start;
        const size_t row = ((size_t)t * H + h) * D;
        if (wave < 2) {
            const void* src = wave == 0 ? p.q : p.k;
            float x[D / 64];
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < D / 64; e++) {
                x[e] = dn_load(src, row + lane + 64 * e, p.in_dtype);
                ss += x[e] * x[e];
            }
            float* dst = wave == 0 ? qs : ks;
            if (p.l2norm) {
                ss = wave_sum<64>(ss);
                const float inv = 1.0f / sqrtf(ss + p.eps);
#pragma unroll
                for (int e = 0; e < D / 64; e++)
                    dst[lane + 64 * e] = finite_or_zero(wave == 0 ? x[e] * inv * inv_scale_q : x[e] * inv);
            } else {
#pragma unroll
                for (int e = 0; e < D / 64; e++) dst[lane + 64 * e] = x[e];
            }
        }
        const float gv = p.gate[(size_t)t * H + h];
        const float g = act ? finite_or_zero(p.gate_is_log ? expf(gv) : gv) : 1.0f;
        const float beta = act ? finite_or_zero(p.beta[(size_t)t * H + h]) : 0.0f;
        const float vi = finite_or_zero(dn_load(p.v, row + i, p.in_dtype));
        __syncthreads();
        float part = 0.0f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            s[r] *= g;
            const float kj = ks[jg * R + r];
            if (kj != 0.0f) part = fmaf(kj, s[r], part);
        }
        part += shfl_xor(part, 32);
        if (lane < 32) red[wave][ci] = part;
        __syncthreads();
        float kv = 0.0f;
#pragma unroll
        for (int w = 0; w < kStepThreads / 64; w++) kv += red[w][ci];
        kv = finite_or_zero(kv);
        const float delta = finite_or_zero((vi - kv) * beta);
        float po = 0.0f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float kj = ks[jg * R + r];
            if (kj != 0.0f) s[r] = fmaf(kj, delta, s[r]);
            const float qj = qs[jg * R + r];
            if (qj != 0.0f) po = fmaf(qj, s[r], po);
        }
        po += shfl_xor(po, 32);
        __syncthreads();
        if (lane < 32) red[wave][ci] = po;
        __syncthreads();
        if (tid < kStepCols && act) {
            float o = 0.0f;
#pragma unroll
            for (int w = 0; w < kStepThreads / 64; w++) o += red[w][ci];
            p.out[row + i] = finite_or_zero(o);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) Sh[(size_t)(jg * R + r) * D + i] = s[r];
}

// ------------------------------------------------------------------ chunked prefill
typedef float dn_f32x4 __attribute__((ext_vector_type(4)));

// Per (chunk, head) block of the workspace, the unit the scan copies into LDS:
//   T, P: the ten 16x16 tiles on and below the diagonal of the 64x64 matrix,
//     tile (r, q) at index r (r + 1) / 2 + q; a tile is 16 rows of four 16-byte
//     pieces, piece g of row m at position 4 m + (g ^ (m / 4 % 4)), so the 16
//     lanes that read one piece column of 16 rows hit 16 distinct bank groups;
//   row scales [4][64] f32: beta_t;  beta_t gamma_t / |k_t|;
//     gamma_t / (|q_t| sqrt(d));  (gamma_last / gamma_t) / |k_t|   (|.| = 1
//     without l2norm, 0 for rows past the end of the sequence);
//   gamma_last (f32) and the chunk's non-finite flag (i32).
constexpr int kTpTiles = 10;
constexpr int kTpT = 0;
constexpr int kTpP = kTpT + kTpTiles * 1024;
constexpr int kTpScale = kTpP + kTpTiles * 1024;
constexpr int kTpGl = kTpScale + 4 * kChunk * 4;
constexpr int kTpBytes = 22 * 1024;  // 22 DMA rounds of 1 KB
static_assert(kTpGl + 8 <= kTpBytes, "block layout");

// Workspace: [H][kScanBlocks] i32 chunks completed by each scan block (256-byte
// aligned), then the (chunk, head) blocks.
__host__ __device__ constexpr size_t dn_ws_head(int H) { return ((size_t)H * kScanBlocks * 4 + 255) / 256 * 256; }

__device__ __forceinline__ int tp_tri(int r, int q) { return r * (r + 1) / 2 + q; }
// float offset of element (m, k) in a tile
__device__ __forceinline__ int tp_elem(int m, int k) { return (4 * m + ((k >> 2) ^ ((m >> 2) & 3))) * 4 + (k & 3); }

__device__ __forceinline__ dn_f32x4 mfma4(float a, float b, dn_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Sum over the four lanes of a quad (DPP quad_perm [1,0,3,2] then [2,3,0,1]).
__device__ __forceinline__ float quad_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    return v;
}

// MFMA 16x16x4 f32 operands: lane l holds A[l % 16][l / 16] and B[l / 16][l % 16];
// the result holds D[4 (l / 16) + i][l % 16] in element i.  Every product below
// gives lane group g = l / 16 the reduction indices 16 q + 4 g + i (i = 0..3)
// in A and B alike, so 4 consecutive indices come from one 16-byte read.
template <int DT>
__device__ __forceinline__ float2 dn_load2(const void* p, size_t i) {  // elements i, i + 1 (i even)
    if constexpr (DT == GR_DTYPE_F32) {
        return *(const float2*)((const float*)p + i);
    } else {
        const uint32_t b = *(const uint32_t*)((const uint16_t*)p + i);
        if constexpr (DT == GR_DTYPE_F16) return make_float2(f16_to_f32(b & 0xffffu), f16_to_f32(b >> 16));
        return make_float2(__uint_as_float(b << 16), __uint_as_float(b & 0xffff0000u));
    }
}

template <int DT>
__device__ __forceinline__ float dn_h2f(uint32_t b) {
    return DT == GR_DTYPE_F16 ? f16_to_f32((uint16_t)b) : __uint_as_float(b << 16);
}

typedef _Float16 dn_h8 __attribute__((ext_vector_type(8)));
typedef short dn_s4 __attribute__((ext_vector_type(4)));  // ds_read_b64_tr_b16 result
typedef __bf16 dn_b8 __attribute__((ext_vector_type(8)));

// 16x16x32 MFMA on 16-bit operands (8 consecutive reduction indices per lane,
// lane group g = l / 16 taking 8 g .. 8 g + 7): products of 16-bit values are
// exact and accumulate in fp32.
template <int DT>
__device__ __forceinline__ dn_f32x4 mfma32(const uint4& a, const uint4& b, dn_f32x4 c) {
    if constexpr (DT == GR_DTYPE_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dn_h8, a), __builtin_bit_cast(dn_h8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dn_b8, a), __builtin_bit_cast(dn_b8, b), c,
                                                       0, 0, 0);
}

// f32 x == hi + mid + lo exactly for three bf16 values made by truncation: hi
// keeps x's first 8 significant bits, mid the next 8 of the exact residual and
// lo the (at most 8) bits left.  (Normal values; the scan stops before a chunk
// whose state is not finite.)  Returned as the upper halves of three words.
__device__ __forceinline__ void dn_split3(float x, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
    hi = __float_as_uint(x) & 0xffff0000u;
    const float r1 = x - __uint_as_float(hi);
    mid = __float_as_uint(r1) & 0xffff0000u;
    lo = __float_as_uint(r1 - __uint_as_float(mid)) & 0xffff0000u;
}
// four floats as the three bf16 pieces of four consecutive B-operand slots
// (two words each); piece pc at out[pc]
__device__ __forceinline__ void dn_split3x4(const float* x, uint2* out) {
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) dn_split3(x[i], h[i], m[i], l[i]);
    out[0] = make_uint2((h[0] >> 16) | h[1], (h[2] >> 16) | h[3]);
    out[1] = make_uint2((m[0] >> 16) | m[1], (m[2] >> 16) | m[3]);
    out[2] = make_uint2((l[0] >> 16) | l[1], (l[2] >> 16) | l[3]);
}

template <int DT>
constexpr size_t dn_prep_lds() {
    // f32 inputs: normalised q, k rows [C][D + 4] f32; 16-bit inputs: raw q, k rows
    // [C][D + 8] (272-byte rows: 16 rows 4 banks apart); both hold A [C][C + 4] f32
    // once the products are done
    return DT == GR_DTYPE_F32 ? (size_t)2 * kChunk * (128 + 4) * 4 : (size_t)2 * kChunk * (128 + 8) * 2;
}

template <int DT>
__global__ __launch_bounds__(kChunkThreads, DT == GR_DTYPE_F32 ? 2 : 4) void deltanet_chunk_prep_kernel(
    const DeltaNetLaunch p) {
    constexpr int D = 128;
    constexpr int C = kChunk;
    constexpr bool RAW = DT != GR_DTYPE_F32;  // 16-bit rows, Gram products on 16-bit MFMA
    constexpr int RS = D + 4;   // f32 row stride (floats): rows 4 banks apart
    constexpr int RS16 = D + 8; // 16-bit row stride (elements)
    constexpr int AMS = C + 4;  // A row stride
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* qn = smem;                          // f32: [C][RS] normalised q rows
    float* kn = qn + C * RS;                   // f32: [C][RS] normalised k rows
    uint16_t* qr = (uint16_t*)smem;            // 16-bit: [C][RS16] raw q rows
    uint16_t* kr = qr + C * RS16;              // 16-bit: [C][RS16] raw k rows
    float* am = smem;                          // [C][AMS] A (strictly lower), over the rows once the products are done
    static_assert(C * AMS * 4 <= dn_prep_lds<DT>(), "A fits over the rows");
    // in-chunk cumulative log decay in double: with strong decays the prefix sums
    // reach ~-100 within a chunk, and a decay exp(lg[t] - lg[s]) taken from two
    // f32 prefix sums would carry ~100 ulp of absolute error in its exponent
    __shared__ double lg[C];
    __shared__ float bt[C], gm[C], kf[C], qi[C], ki[C];
    __shared__ int bad;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l16 = lane & 15, g = lane >> 4;
    const int c = blockIdx.x, h = blockIdx.y, H = p.n_heads;
    const int t0 = c * C;
    const int Cn = min(C, p.n_tokens - t0);
    char* blk = (char*)p.ws + dn_ws_head(H) + ((size_t)c * H + h) * kTpBytes;
    if (tid == 0) bad = 0;
    __syncthreads();

    const float inv_scale_q = 1.0f / sqrtf((float)D);
    if constexpr (RAW) {
        // 1. raw rows into LDS and their norms: wave w takes q and k rows
        //    16 w .. 16 w + 15, four rows per 16-byte load round (16 lanes a row)
        uint4 x[8];
#pragma unroll
        for (int r4 = 0; r4 < 8; r4++) {
            const int t = 16 * wave + 4 * (r4 & 3) + g;
            x[r4] = t < Cn ? *(const uint4*)((const uint16_t*)(r4 < 4 ? p.q : p.k) + ((size_t)(t0 + t) * H + h) * D +
                                             8 * l16)
                           : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r4 = 0; r4 < 8; r4++) {
            const int t = 16 * wave + 4 * (r4 & 3) + g;
            const bool isq = r4 < 4, valid = t < Cn;
            const uint32_t w[4] = {x[r4].x, x[r4].y, x[r4].z, x[r4].w};
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float lo = dn_h2f<DT>(w[e] & 0xffffu), hi = dn_h2f<DT>(w[e] >> 16);
                ss = fmaf(lo, lo, ss);
                ss = fmaf(hi, hi, ss);
            }
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) ss += shfl_xor(ss, m);
            *(uint4*)((isq ? qr : kr) + t * RS16 + 8 * l16) = x[r4];
            if (l16 == 0) {
                const float inv = 1.0f / sqrtf(ss + p.eps);
                (isq ? qi : ki)[t] = !valid ? 0.0f : !p.l2norm ? 1.0f : isq ? inv * inv_scale_q : inv;
                if (valid && !is_finite_f(ss)) bad = 1;
            }
        }
    } else {
        // 1. normalised rows (as math.rs:833-846) and the norms for the row scales:
        //    wave w takes q and k rows 16 w .. 16 w + 15, all 32 loads issued first
        float2 x[32];
#pragma unroll
        for (int k = 0; k < 32; k++) {
            const int t = 16 * wave + (k & 15);
            x[k] = t < Cn ? dn_load2<DT>(k < 16 ? p.q : p.k, ((size_t)(t0 + t) * H + h) * D + 2 * lane)
                          : make_float2(0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < 32; k++) {
            const int t = 16 * wave + (k & 15);
            const bool isq = k < 16, valid = t < Cn;
            const float ss = wave_sum<64>(x[k].x * x[k].x + x[k].y * x[k].y);
            float2* dst = (float2*)((isq ? qn : kn) + t * RS) + lane;
            float nrm = valid ? 1.0f : 0.0f;
            if (p.l2norm) {
                const float inv = 1.0f / sqrtf(ss + p.eps);
                *dst = isq ? make_float2(finite_or_zero(x[k].x * inv * inv_scale_q), finite_or_zero(x[k].y * inv * inv_scale_q))
                           : make_float2(finite_or_zero(x[k].x * inv), finite_or_zero(x[k].y * inv));
                nrm = valid ? (isq ? inv * inv_scale_q : inv) : 0.0f;
            } else {
                *dst = x[k];
            }
            if (lane == 0) {
                (isq ? qi : ki)[t] = nrm;
                if (valid && !is_finite_f(ss)) bad = 1;
            }
        }
    }
    // gates: padded tokens get log decay 0 and beta 0
    if (wave == 0) {
        const bool valid = lane < Cn;
        const float gv = valid ? p.gate[(size_t)(t0 + lane) * H + h] : 0.0f;
        const float bv = valid ? p.beta[(size_t)(t0 + lane) * H + h] : 0.0f;
        if (!is_finite_f(gv) || !is_finite_f(bv)) bad = 1;
        double gl = (double)gv;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(gl, off, 64);
            if (lane >= off) gl += o;
        }
        lg[lane] = gl;
        const double gl_last = __shfl(gl, 63, 64);
        gm[lane] = expf((float)gl);
        kf[lane] = expf((float)(gl_last - gl));
        bt[lane] = bv;
    }
    __syncthreads();

    // 2. K K^T (tiles 0..9) and Q K^T (10..19) on and below the diagonal, five per
    //    wave: of the normalised f32 rows, or exactly of the raw 16-bit rows (the
    //    norms are applied below)
    dn_f32x4 acc[5];
#pragma unroll
    for (int u = 0; u < 5; u++) {
        const int ti = wave + 4 * u;
        const int tt = ti < kTpTiles ? ti : ti - kTpTiles;
        const int r = tt < 1 ? 0 : tt < 3 ? 1 : tt < 6 ? 2 : 3;
        const int q = tt - r * (r + 1) / 2;
        dn_f32x4 a4 = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (RAW) {
            const uint16_t* ar = (ti < kTpTiles ? kr : qr) + (16 * r + l16) * RS16 + 8 * g;
            const uint16_t* br = kr + (16 * q + l16) * RS16 + 8 * g;
#pragma unroll
            for (int ks = 0; ks < D / 32; ks++)
                a4 = mfma32<DT>(*(const uint4*)(ar + 32 * ks), *(const uint4*)(br + 32 * ks), a4);
        } else {
            const float* ar = (ti < kTpTiles ? kn : qn) + (16 * r + l16) * RS + 4 * g;
            const float* br = kn + (16 * q + l16) * RS + 4 * g;
#pragma unroll
            for (int kk = 0; kk < D / 16; kk++) {
                const float4 a = *(const float4*)(ar + 16 * kk);
                const float4 b = *(const float4*)(br + 16 * kk);
                a4 = mfma4(a.x, b.x, a4);
                a4 = mfma4(a.y, b.y, a4);
                a4 = mfma4(a.z, b.z, a4);
                a4 = mfma4(a.w, b.w, a4);
            }
        }
        acc[u] = a4;
    }
    __syncthreads();  // every read of the rows is done: A goes over them
#pragma unroll
    for (int u = 0; u < 5; u++) {
        const int ti = wave + 4 * u;
        const int tt = ti < kTpTiles ? ti : ti - kTpTiles;
        const int r = tt < 1 ? 0 : tt < 3 ? 1 : tt < 6 ? 2 : 3;
        const int q = tt - r * (r + 1) / 2;
        const int s = 16 * q + l16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tl = 4 * g + i;
            const int t = 16 * r + tl;
            const float dec = s <= t ? expf((float)(lg[t] - lg[s])) : 0.0f;
            if (ti < kTpTiles) {
                const float gr = RAW ? ki[t] * ki[s] * acc[u][i] : acc[u][i];
                am[t * AMS + s] = s < t ? bt[t] * dec * gr : 0.0f;
            } else {
                const float pr = RAW ? qi[t] * ki[s] * acc[u][i] : acc[u][i];
                const float v = s <= t ? dec * pr : 0.0f;
                if (!is_finite_f(v)) bad = 1;
                *(float*)(blk + kTpP + tt * 1024 + 4 * tp_elem(tl, l16)) = v;
            }
        }
    }
    __syncthreads();

    // 3. T = (I + A)^-1, column col = 16 wave + lane / 4 by forward substitution
    //    x[t] = [t == col] - sum_{s<t} A[t][s] x[s]; the four lanes of a quad
    //    take the 4-blocks of s with (s / 4) % 4 == part and sum by DPP.
    {
        const int col = 16 * wave + (lane >> 2), part = lane & 3;
        float x[16];  // x[s] for s = 16 u + 4 part + e at x[4 u + e]
#pragma unroll
        for (int e = 0; e < 16; e++) x[e] = 0.0f;
#pragma unroll
        for (int t = 0; t < C; t++) {
            float su[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // four short chains instead of one long one
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (16 * u < t) {  // A[t][s >= t] is 0 and x[s >= t] is still 0
                    const float4 a = *(const float4*)(am + t * AMS + 16 * u + 4 * part);
                    su[u] = a.x * x[4 * u + 0];
                    su[u] = fmaf(a.y, x[4 * u + 1], su[u]);
                    su[u] = fmaf(a.z, x[4 * u + 2], su[u]);
                    su[u] = fmaf(a.w, x[4 * u + 3], su[u]);
                }
            }
            const float sum = quad_sum((su[0] + su[1]) + (su[2] + su[3]));
            const float val = (t == col ? 1.0f : 0.0f) - sum;
            // a select, not a branch: under a lane-dependent branch the compiler
            // copied the whole x array at every step
            const int xi = (t >> 4) * 4 + (t & 3);
            x[xi] = ((t >> 2) & 3) == part ? val : x[xi];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (u < wave) continue;  // T[s][col] = 0 above the diagonal tiles
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float v = x[4 * u + e];
                if (!is_finite_f(v)) bad = 1;
                *(float*)(blk + kTpT + tp_tri(u, wave) * 1024 + 4 * tp_elem(4 * part + e, lane >> 2)) = v;
            }
        }
    }
    // 4. row scales, gamma_last, flag
    if (tid < C) {
        const int t = tid;
        float* sc = (float*)(blk + kTpScale);
        const float v0 = bt[t], v1 = bt[t] * gm[t] * ki[t], v2 = gm[t] * qi[t], v3 = kf[t] * ki[t];
        sc[t] = v0;
        sc[C + t] = v1;
        sc[2 * C + t] = v2;
        sc[3 * C + t] = v3;
        if (!is_finite_f(v0) || !is_finite_f(v1) || !is_finite_f(v2) || !is_finite_f(v3)) bad = 1;
        if (t == C - 1) {
            const float gl = gm[C - 1];
            if (!is_finite_f(gl)) bad = 1;
            *(float*)(blk + kTpGl) = gl;
        }
    }
    __syncthreads();
    if (tid == 0) *(int*)(blk + kTpGl + 4) = bad;
}

// Raw buffer access: a buffer descriptor (base, stride 0, num_records = `bytes`:
// offsets at or past it read as zero) and 16 bytes per lane straight into LDS at
// lds + 16 * lane (buffer_load_dwordx4 ... lds; lds and the descriptor
// wave-uniform).  Issued as inline assembly so that the compiler does not see an
// LDS write: it would otherwise wait for the DMA before every later LDS read it
// cannot prove disjoint.  Completion is waited for explicitly (dn_wait_vmem)
// before the data is read; vmcnt waits the compiler places for its own loads
// count these rounds too and only wait longer, never shorter.
typedef int dn_i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ dn_i32x4 dn_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    dn_i32x4 r;
    r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
    r.z = __builtin_amdgcn_readfirstlane((int)bytes);
    r.w = 0x00020000;
    return r;
}
__device__ __forceinline__ void dn_dma16(dn_i32x4 r, void* lds, int voff) {
    const int m0 = __builtin_amdgcn_readfirstlane(
        (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
    // m0 (the LDS destination) is saved and restored inside the statement: the
    // compiler treats m0 as reserved and would not preserve a value of its own
    // across a clobber.  An SALU write of m0 followed by an LDS DMA needs one
    // wait state on gfx9-family parts, which the compiler cannot insert inside
    // the statement: hence the s_nop.
    int saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(m0), "v"(voff), "s"(r)
                 : "memory");
}
// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left at their maxima)
__device__ __forceinline__ void dn_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier for LDS data written with ds_write: waits for this wave's
// LDS operations (lgkmcnt) only, not for its outstanding global loads, stores and
// DMA rounds, which __syncthreads() (a fence of all memory, and the DMA rounds
// write LDS) would wait for too.  DMA rounds are waited for explicitly
// (dn_wait_vmem) before the barrier that publishes them.  The memory clobber
// keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void dn_lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// q / k chunk tiles in LDS: row t (D elements) as 16-byte pieces, piece p at
// position p ^ (t % 16).  Four consecutive elements 16 q + 4 g .. + 3 of row t:
template <int DT>
__device__ __forceinline__ void dn_arow(const char* tile, int t, int q, int g, float* a) {
    if constexpr (DT == GR_DTYPE_F32) {
        const int pos = (4 * q + g) ^ (t & 15);
        const float4 v = *(const float4*)(tile + t * 512 + pos * 16);
        a[0] = v.x;
        a[1] = v.y;
        a[2] = v.z;
        a[3] = v.w;
    } else {
        const int pos = (2 * q + (g >> 1)) ^ (t & 15);
        const uint2 v = *(const uint2*)(tile + t * 256 + pos * 16 + (g & 1) * 8);
        a[0] = dn_h2f<DT>(v.x & 0xffffu);
        a[1] = dn_h2f<DT>(v.x >> 16);
        a[2] = dn_h2f<DT>(v.y & 0xffffu);
        a[3] = dn_h2f<DT>(v.y >> 16);
    }
}
// element j of row s
template <int DT>
__device__ __forceinline__ float dn_elem(const char* tile, int s, int j) {
    if constexpr (DT == GR_DTYPE_F32) {
        return *(const float*)(tile + s * 512 + (((j >> 2) ^ (s & 15)) * 16) + (j & 3) * 4);
    } else {
        return dn_h2f<DT>(*(const uint16_t*)(tile + s * 256 + (((j >> 3) ^ (s & 15)) * 16) + (j & 7) * 2));
    }
}

// One workgroup per (head, 16 state columns), the chunks in order.  LDS holds the
// state slice, the chunk's raw K and Q tiles and its T / P / scale block, all
// copied by DMA (buffer_load ... lds) one chunk ahead into the other of two
// buffers (f32 inputs: one Q buffer, refilled after its last read in the chunk
// before, as two f32 Q tiles do not fit beside the rest).  Every buffer is its
// own array and the chunk loop is unrolled by two, so the compiler sees that a
// DMA never writes what the same chunk reads and adds no wait for it.
// Wave w computes rows 16 w .. 16 w + 15 of the chunk's X, Delta and O and state
// rows 32 w .. 32 w + 31.  Per chunk:
//   b: K S0 and Q S0 (raw rows; K = 128)
//   c: X = beta V - (beta gamma / |k|) (K S0)                    -> LDS
//   d: Delta = T X (the tiles on and below the diagonal)        -> LDS
//   e: O = (gamma / |q| sqrt(d)) (Q S0) + P Delta               -> out (stored a chunk later)
//      S' = gamma_last S0 + K^T ((gamma_last / gamma) / |k| Delta) -> LDS (own rows)
// Each product runs as two or four independent MFMA accumulator chains, and the
// next chunk's DMA rounds are issued between the MFMAs of steps b, d and e.
template <int DT>
__global__ __launch_bounds__(kChunkThreads, 1) void deltanet_chunk_scan_kernel(const DeltaNetLaunch p) {
    constexpr int C = kChunk, D = 128, NC = kScanCols;
    constexpr int ES = DT == GR_DTYPE_F32 ? 4 : 2;
    constexpr int KB = C * D * ES;        // one K / Q tile (bytes)
    constexpr bool Q2 = ES == 2;          // two Q buffers
    constexpr int PPR = D * ES / 16;      // 16-byte pieces per row
    constexpr int RPK = 1024 / (D * ES);  // rows per 1 KB DMA round
    constexpr int KR = KB / 1024 / 4;     // K (or Q) DMA rounds per wave
    constexpr int TR = (kTpBytes / 1024 + 3) / 4;  // T / P block rounds per wave (the last partly)
    __shared__ __attribute__((aligned(16))) char K0[KB];
    __shared__ __attribute__((aligned(16))) char K1[KB];
    __shared__ __attribute__((aligned(16))) char Q0[KB];
    __shared__ __attribute__((aligned(16))) char Q1[Q2 ? KB : 16];
    __shared__ __attribute__((aligned(16))) char TP0[kTpBytes];
    __shared__ __attribute__((aligned(16))) char TP1[kTpBytes];
    // S[16 q + 4 g + i][n] at (64 q + 16 g + n) * 4 + i: the four values of one
    // MFMA B operand (or result) of lane 16 g + n in one 16-byte read (write),
    // consecutive lanes on consecutive 16-byte words; X and Delta rows the same way
    __shared__ __attribute__((aligned(16))) float Sl[D * NC];
    __shared__ __attribute__((aligned(16))) float Xl[C * NC];
    __shared__ __attribute__((aligned(16))) float Dl[C * NC];
    // bf16 rows (raw k / q exact as bf16): the K S0, Q S0 and state-update products
    // run on v_mfma_f32_16x16x32_bf16 with the f32 operand as three exact bf16
    // pieces (hi + mid + lo, three MFMAs), a third of the matrix-core time of the
    // f32 MFMA.  The pieces in B-operand order: Sp[piece][k-step q][lane 16 g + n]
    // = state rows 32 q + 8 g .. + 7 of column n; Dp the same for the scaled Delta
    // rows (tokens).
    constexpr bool BF = DT == GR_DTYPE_BF16;
    __shared__ __attribute__((aligned(16))) uint4 Sp[BF ? 3 * (D / 32) * 64 : 1];
    __shared__ __attribute__((aligned(16))) uint4 Dp[BF ? 3 * (C / 32) * 64 : 1];
    __shared__ int flag;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l16 = lane & 15, g = lane >> 4;
    // blockIdx.x = head so that the column blocks of one head (linear ids
    // h + H * cb) share an XCD and its L2 copy of the chunk's rows and block
    const int h = blockIdx.x, cb = blockIdx.y;
    const int c0 = cb * NC;
    const int H = p.n_heads;
    const int rowstride = H * D * ES;  // bytes between token rows of q / k
    float* Sh = p.state + (size_t)h * D * D;
    const int n_chunks = (p.n_tokens + C - 1) / C;
    const char* tpg = (const char*)p.ws + dn_ws_head(H);

    for (int e = tid; e < D * NC; e += kChunkThreads) {
        const int i = e & 3, n = (e >> 2) & 15, gg = (e >> 6) & 3, q = e >> 8;
        Sl[e] = Sh[(size_t)(16 * q + 4 * gg + i) * D + c0 + n];
    }
    if (tid == 0) flag = 0;
    // this wave's state rows 32 w + 16 tt + 4 g + (0..3) (an MFMA result's rows) as
    // bf16 pieces: k-step w, lane 16 (2 tt + g / 2) + n, slots 4 (g % 2) ..
    auto store_state_pieces = [&](const float* v0, const float* v1) {
        if constexpr (BF) {
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                uint2 pcs[3];
                dn_split3x4(tt ? v1 : v0, pcs);
#pragma unroll
                for (int pc = 0; pc < 3; pc++)
                    *(uint2*)((char*)&Sp[(pc * (D / 32) + wave) * 64 + 16 * (2 * tt + (g >> 1)) + l16] + 8 * (g & 1)) =
                        pcs[pc];
            }
        }
    };
    if constexpr (BF) {
        __syncthreads();  // Sl complete
        float v0[4], v1[4];
        const float4 a = *(const float4*)(Sl + ((2 * wave) * 64 + lane) * 4);
        const float4 b = *(const float4*)(Sl + ((2 * wave + 1) * 64 + lane) * 4);
        v0[0] = a.x, v0[1] = a.y, v0[2] = a.z, v0[3] = a.w;
        v1[0] = b.x, v1[1] = b.y, v1[2] = b.z, v1[3] = b.w;
        store_state_pieces(v0, v1);
    }

    // DMA round k of this wave for a K / Q tile: round I = wave + 4 k (1 KB) fills
    // position l % PPR of row I * RPK + l / PPR (lane l) with the piece that
    // belongs there (piece p of row t at position p ^ (t % 16))
    auto rows_rsrc = [&](const void* src, int c) {
        const int r0 = c * C;
        const int cn = min(C, p.n_tokens - r0);
        return dn_rsrc((const char*)src + ((size_t)r0 * H + h) * D * ES,
                       (uint32_t)((cn - 1) * rowstride + D * ES));
    };
    auto dma_row_round = [&](dn_i32x4 rs, char* dst, int k) {
        const int I = wave + 4 * k;
        const int r = I * RPK + lane / PPR;
        dn_dma16(rs, dst + 1024 * I, r * rowstride + (((lane % PPR) ^ (r & 15)) * 16));
    };
    auto tp_rsrc = [&](int c) { return dn_rsrc(tpg + ((size_t)c * H + h) * kTpBytes, kTpBytes); };
    auto dma_tp_round = [&](dn_i32x4 rs, char* dst, int k) {
        const int I = wave + 4 * k;
        if (I < kTpBytes / 1024) dn_dma16(rs, dst + 1024 * I, 1024 * I + 16 * lane);
    };
    // V[t][c0 + n] for the rows of this lane's X elements
    //   as raw bits, converted where chunk c uses them (rows past the end are read
    //   from the last row and zeroed then): no branch and no arithmetic on the
    //   loaded registers here, so the compiler does not wait for the loads here
    auto load_v = [&](uint32_t* vr, int c) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = c * C + 16 * wave + 4 * g + i;
            const size_t e = ((size_t)min(t, p.n_tokens - 1) * H + h) * D + c0 + l16;
            vr[i] = DT == GR_DTYPE_F32 ? __float_as_uint(((const float*)p.v)[e]) : ((const uint16_t*)p.v)[e];
        }
    };
    auto v_value = [&](uint32_t raw, int t) {
        const float x = DT == GR_DTYPE_F32 ? __uint_as_float(raw) : dn_h2f<DT>(raw);
        return t < p.n_tokens ? x : 0.0f;
    };

    int done = n_chunks;     // chunks completed
    bool restore = false;    // state = s0own (the start of chunk done)
    dn_f32x4 s0own[2];
    // O rows of chunk `pend` wait in registers and are stored after the next
    // chunk's wait for its DMA rounds (which counts stores too), a chunk before
    // the wait that covers them
    float opend[4];
    int pend = -1;
    auto store_pending = [&]() {
        if (pend < 0) return;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = pend * C + 16 * wave + 4 * g + i;
            if (t < p.n_tokens) p.out[((size_t)t * H + h) * D + c0 + l16] = opend[i];
        }
        pend = -1;
    };
    uint32_t vcur[4], vnext[4];
    {
        const dn_i32x4 rk = rows_rsrc(p.k, 0), rq = rows_rsrc(p.q, 0), rt = tp_rsrc(0);
#pragma unroll
        for (int k = 0; k < KR; k++) {
            dma_row_round(rk, K0, k);
            dma_row_round(rq, Q0, k);
        }
#pragma unroll
        for (int k = 0; k < TR; k++) dma_tp_round(rt, TP0, k);
        load_v(vcur, 0);
    }

    // one chunk; PAR selects the buffers (compile time); false = stop the scan
    auto chunk = [&](const int c, auto par) -> bool {
        constexpr int P = decltype(par)::value;
        char* kt = P ? K1 : K0;
        char* qt = (Q2 && P) ? Q1 : Q0;
        const char* tp = P ? TP1 : TP0;
        char* kn = P ? K0 : K1;                // next chunk's buffers
        char* qn = Q2 ? (P ? Q0 : Q1) : Q0;
        char* tpn = P ? TP0 : TP1;
        dn_wait_vmem();   // this thread's DMA rounds for chunk c are in LDS
        dn_lds_barrier();  // ... everyone's; the state rows of chunk c - 1 are written
        store_pending();
        if (flag) {       // chunk c - 1 met a non-finite value: resume from its start
            done = c - 1;
            restore = true;
            return false;
        }
        if (*(const int*)(tp + kTpGl + 4)) {  // the prep flagged chunk c
            done = c;
            return false;
        }
        const int Cn = min(C, p.n_tokens - c * C);
        if (Cn < C) {  // rows past the end of the sequence: zero
            for (int e = Cn * D * ES / 16 + tid; e < KB / 16; e += kChunkThreads) {
                ((uint4*)kt)[e] = make_uint4(0, 0, 0, 0);
                ((uint4*)qt)[e] = make_uint4(0, 0, 0, 0);
            }
            dn_lds_barrier();
        }
        const bool more = c + 1 < n_chunks;
        if (more) load_v(vnext, c + 1);
        const float* scl = (const float*)(tp + kTpScale);
        bool nf = false;
        // b: K S0, Q S0 for rows 16 w + (0..15); four chains (K / Q x even / odd i);
        //    the next chunk's K (and 16-bit Q) rounds between the MFMAs
        dn_f32x4 ak0 = {0.0f, 0.0f, 0.0f, 0.0f}, ak1 = ak0, aq0 = ak0, aq1 = ak0;
        if constexpr (BF) {
            // bf16: A = the raw row piece (k-step q: dims 32 q + 8 g .. + 7), B = the
            // state's three pieces; ak1 / aq1 stay zero
            const dn_i32x4 rk = rows_rsrc(p.k, more ? c + 1 : c);
            const dn_i32x4 rq = rows_rsrc(p.q, more ? c + 1 : c);
            const int ta = 16 * wave + l16;
#pragma unroll
            for (int q = 0; q < D / 32; q++) {
                const int pos = (4 * q + g) ^ (ta & 15);
                const uint4 ka = *(const uint4*)(kt + ta * 256 + pos * 16);
                const uint4 qa = *(const uint4*)(qt + ta * 256 + pos * 16);
#pragma unroll
                for (int pc = 0; pc < 3; pc++) {
                    const uint4 sb = Sp[(pc * (D / 32) + q) * 64 + lane];
                    ak0 = mfma32<DT>(ka, sb, ak0);
                    aq0 = mfma32<DT>(qa, sb, aq0);
                }
                if (more && q < KR) {
                    dma_row_round(rk, kn, q);
                    if (Q2) dma_row_round(rq, qn, q);
                }
            }
            static_assert(!BF || KR <= D / 32, "the DMA rounds fit the k-steps");
        } else {
            const dn_i32x4 rk = rows_rsrc(p.k, more ? c + 1 : c);
            const dn_i32x4 rq = rows_rsrc(p.q, more ? c + 1 : c);
            const int ta = 16 * wave + l16;
#pragma unroll
            for (int q = 0; q < D / 16; q++) {
                const float4 sb = *(const float4*)(Sl + (q * 64 + lane) * 4);
                float ka[4], qa[4];
                dn_arow<DT>(kt, ta, q, g, ka);
                dn_arow<DT>(qt, ta, q, g, qa);
                ak0 = mfma4(ka[0], sb.x, ak0);
                aq0 = mfma4(qa[0], sb.x, aq0);
                ak1 = mfma4(ka[1], sb.y, ak1);
                aq1 = mfma4(qa[1], sb.y, aq1);
                ak0 = mfma4(ka[2], sb.z, ak0);
                aq0 = mfma4(qa[2], sb.z, aq0);
                ak1 = mfma4(ka[3], sb.w, ak1);
                aq1 = mfma4(qa[3], sb.w, aq1);
                if (more && q < KR) {
                    dma_row_round(rk, kn, q);
                    if (Q2) dma_row_round(rq, qn, q);
                }
            }
        }
        // c: X
        {
            float xv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * wave + 4 * g + i;
                xv[i] = scl[t] * v_value(vcur[i], c * C + t) - scl[C + t] * (ak0[i] + ak1[i]);
                nf |= !is_finite_f(xv[i]);
            }
            *(float4*)(Xl + (wave * 64 + lane) * 4) = make_float4(xv[0], xv[1], xv[2], xv[3]);
        }
        if (nf) flag = 1;
        dn_lds_barrier();  // X complete; Q of chunk c read
        // d: Delta = T X (two chains); the next chunk's T / P block rounds
        const int apos = 16 * (4 * l16 + (g ^ ((l16 >> 2) & 3)));  // this lane's piece in a T / P tile
        dn_f32x4 dl;
        {
            const dn_i32x4 rt = tp_rsrc(more ? c + 1 : c);
            dn_f32x4 d0 = {0.0f, 0.0f, 0.0f, 0.0f}, d1 = d0;
#pragma unroll
            for (int tq = 0; tq < 4; tq++) {
                if (tq <= wave) {
                    const float4 a = *(const float4*)(tp + kTpT + tp_tri(wave, tq) * 1024 + apos);
                    const float4 b = *(const float4*)(Xl + (tq * 64 + lane) * 4);
                    d0 = mfma4(a.x, b.x, d0);
                    d1 = mfma4(a.y, b.y, d1);
                    d0 = mfma4(a.z, b.z, d0);
                    d1 = mfma4(a.w, b.w, d1);
                }
                if (more) {
                    dma_tp_round(rt, tpn, tq);
                    if (tq < TR - 4) dma_tp_round(rt, tpn, tq + 4);
                }
            }
            dl = d0 + d1;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) nf |= !is_finite_f(dl[i]);
        *(float4*)(Dl + (wave * 64 + lane) * 4) = make_float4(dl[0], dl[1], dl[2], dl[3]);
        if constexpr (BF) {
            // the state update's B operand: Delta rows t = 16 w + 4 g + i scaled by
            // (gamma_last / gamma_t) / |k_t|, as pieces at k-step t / 32, lane
            // 16 ((t % 32) / 8) + n, slots t % 8
            const float4 sk = *(const float4*)(scl + 3 * C + 16 * wave + 4 * g);
            const float xs[4] = {dl[0] * sk.x, dl[1] * sk.y, dl[2] * sk.z, dl[3] * sk.w};
            uint2 pcs[3];
            dn_split3x4(xs, pcs);
#pragma unroll
            for (int pc = 0; pc < 3; pc++)
                *(uint2*)((char*)&Dp[(pc * (C / 32) + (wave >> 1)) * 64 + 16 * (2 * (wave & 1) + (g >> 1)) + l16] +
                          8 * (g & 1)) = pcs[pc];
        }
        if (nf) flag = 1;
        dn_lds_barrier();  // Delta complete
        if (!Q2 && more) {  // the single f32 Q buffer: its reads ended with step b
            const dn_i32x4 rq = rows_rsrc(p.q, c + 1);
#pragma unroll
            for (int k = 0; k < KR; k++) dma_row_round(rq, qn, k);
        }
        // e: O (two chains)
        {
            dn_f32x4 o0 = {0.0f, 0.0f, 0.0f, 0.0f}, o1 = o0;
#pragma unroll
            for (int tq = 0; tq < 4; tq++) {
                if (tq <= wave) {
                    const float4 a = *(const float4*)(tp + kTpP + tp_tri(wave, tq) * 1024 + apos);
                    const float4 b = *(const float4*)(Dl + (tq * 64 + lane) * 4);
                    o0 = mfma4(a.x, b.x, o0);
                    o1 = mfma4(a.y, b.y, o1);
                    o0 = mfma4(a.z, b.z, o0);
                    o1 = mfma4(a.w, b.w, o1);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * wave + 4 * g + i;
                opend[i] = scl[2 * C + t] * (aq0[i] + aq1[i]) + (o0[i] + o1[i]);
                nf |= !is_finite_f(opend[i]);
            }
            pend = c;
        }
        // e: S' for state rows 32 w .. 32 w + 31 (two tiles x even / odd i chains)
        {
            const float gl = *(const float*)(tp + kTpGl);
            float* srow0 = Sl + ((2 * wave) * 64 + lane) * 4;
            float* srow1 = Sl + ((2 * wave + 1) * 64 + lane) * 4;
            const float4 s0a = *(const float4*)srow0, s0b = *(const float4*)srow1;
            s0own[0] = dn_f32x4{s0a.x, s0a.y, s0a.z, s0a.w};
            s0own[1] = dn_f32x4{s0b.x, s0b.y, s0b.z, s0b.w};
            dn_f32x4 a0 = gl * s0own[0], a1 = gl * s0own[1];
            dn_f32x4 b0 = {0.0f, 0.0f, 0.0f, 0.0f}, b1 = b0;
            const int j0 = 32 * wave + l16, j1 = j0 + 16;
            if constexpr (BF) {
                // A = K^T (state rows 32 w + 16 tt + 0..15, tokens 32 ks + 8 g .. + 7):
                // two transposing reads of 4 tokens x 16 dims each (lane i of a
                // 16-lane group supplies token k0 + i / 4, dims d0 + 4 (i % 4) .. + 3,
                // and receives dims d0 + i of tokens k0 .. k0 + 3); B = the pieces of
                // the scaled Delta
#pragma unroll
                for (int ks = 0; ks < C / 32; ks++) {
                    uint4 at[2];
#pragma unroll
                    for (int tt = 0; tt < 2; tt++) {
                        dn_s4 part[2];
#pragma unroll
                        for (int hf = 0; hf < 2; hf++) {
                            const int t = 32 * ks + 8 * g + 4 * hf + (l16 >> 2);
                            const int e = 32 * wave + 16 * tt + 4 * (l16 & 3);
                            const int pos = (e >> 3) ^ (t & 15);
                            part[hf] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                (__attribute__((address_space(3))) dn_s4*)(kt + t * 256 + pos * 16 + (e & 7) * 2));
                        }
                        const uint2 lo2 = __builtin_bit_cast(uint2, part[0]);
                        const uint2 hi2 = __builtin_bit_cast(uint2, part[1]);
                        at[tt] = make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
                    }
#pragma unroll
                    for (int pc = 0; pc < 3; pc++) {
                        const uint4 db = Dp[(pc * (C / 32) + ks) * 64 + lane];
                        a0 = mfma32<DT>(at[0], db, a0);
                        a1 = mfma32<DT>(at[1], db, a1);
                    }
                }
            } else {
#pragma unroll
            for (int q = 0; q < C / 16; q++) {
                const float4 b = *(const float4*)(Dl + (q * 64 + lane) * 4);
                const float4 sk = *(const float4*)(scl + 3 * C + 16 * q + 4 * g);
                const int s = 16 * q + 4 * g;
                const float bs[4] = {b.x * sk.x, b.y * sk.y, b.z * sk.z, b.w * sk.w};
                a0 = mfma4(dn_elem<DT>(kt, s + 0, j0), bs[0], a0);
                a1 = mfma4(dn_elem<DT>(kt, s + 0, j1), bs[0], a1);
                b0 = mfma4(dn_elem<DT>(kt, s + 1, j0), bs[1], b0);
                b1 = mfma4(dn_elem<DT>(kt, s + 1, j1), bs[1], b1);
                a0 = mfma4(dn_elem<DT>(kt, s + 2, j0), bs[2], a0);
                a1 = mfma4(dn_elem<DT>(kt, s + 2, j1), bs[2], a1);
                b0 = mfma4(dn_elem<DT>(kt, s + 3, j0), bs[3], b0);
                b1 = mfma4(dn_elem<DT>(kt, s + 3, j1), bs[3], b1);
            }
            }
            a0 += b0;
            a1 += b1;
#pragma unroll
            for (int i = 0; i < 4; i++) nf |= !is_finite_f(a0[i]) || !is_finite_f(a1[i]);
            *(float4*)srow0 = make_float4(a0[0], a0[1], a0[2], a0[3]);
            *(float4*)srow1 = make_float4(a1[0], a1[1], a1[2], a1[3]);
            if constexpr (BF) {
                const float v0[4] = {a0[0], a0[1], a0[2], a0[3]}, v1[4] = {a1[0], a1[1], a1[2], a1[3]};
                store_state_pieces(v0, v1);
            }
        }
        if (nf) flag = 1;
#pragma unroll
        for (int i = 0; i < 4; i++) vcur[i] = vnext[i];
        return true;
    };

    int c = 0;
    bool all = true;
    for (; c < n_chunks; c += 2) {
        if (!chunk(c, std::integral_constant<int, 0>{})) { all = false; break; }
        if (c + 1 < n_chunks && !chunk(c + 1, std::integral_constant<int, 1>{})) { all = false; break; }
    }
    store_pending();
    if (all) {
        dn_lds_barrier();
        if (flag) {  // the last chunk met a non-finite value
            done = n_chunks - 1;
            restore = true;
        }
    }
#pragma unroll
    for (int r2 = 0; r2 < 2; r2++) {
        const int rt = 2 * wave + r2;
        const float4 sv = *(const float4*)(Sl + (rt * 64 + lane) * 4);
        const float v[4] = {restore ? s0own[r2][0] : sv.x, restore ? s0own[r2][1] : sv.y,
                            restore ? s0own[r2][2] : sv.z, restore ? s0own[r2][3] : sv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) Sh[(size_t)(16 * rt + 4 * g + i) * D + c0 + l16] = v[i];
    }
    if (tid == 0) ((int*)p.ws)[h * kScanBlocks + cb] = done;
}

size_t deltanet_chunked_ws_bytes(int n_tokens, int n_heads, int head_dim, int chunk) {
    if (head_dim != 128 || chunk != kChunk || n_tokens <= 0 || n_heads <= 0) return 0;
    const size_t n_chunks = (size_t)(n_tokens + kChunk - 1) / kChunk;
    return dn_ws_head(n_heads) + n_chunks * n_heads * kTpBytes;
}

// The token recurrence at any supported state size (64, 128, 256: 32 value
// columns per workgroup, D / 8 state rows per thread).
hipError_t launch_deltanet_scan(const DeltaNetLaunch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    DeltaNetLaunch q = p;
    q.first_bad = nullptr;
    const dim3 grid(p.head_dim / kStepCols, p.n_heads);
    switch (p.head_dim) {
        case 64: deltanet_step_kernel<64><<<grid, kStepThreads, 0, st>>>(q); break;
        case 128: deltanet_step_kernel<128><<<grid, kStepThreads, 0, st>>>(q); break;
        case 256: deltanet_step_kernel<256><<<grid, kStepThreads, 0, st>>>(q); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int DT>
static hipError_t launch_chunked_dt(const DeltaNetLaunch& p, hipStream_t st) {
    constexpr size_t lds_prep = dn_prep_lds<DT>();
    hipError_t e = hipFuncSetAttribute((const void*)deltanet_chunk_prep_kernel<DT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_prep);
    if (e != hipSuccess) return e;
    const int n_chunks = (p.n_tokens + kChunk - 1) / kChunk;
    deltanet_chunk_prep_kernel<DT><<<dim3(n_chunks, p.n_heads), kChunkThreads, lds_prep, st>>>(p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    deltanet_chunk_scan_kernel<DT><<<dim3(p.n_heads, kScanBlocks), kChunkThreads, 0, st>>>(p);
    return hipGetLastError();
}

hipError_t launch_deltanet_chunked(const DeltaNetLaunch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    if (p.head_dim != 128 || !p.ws) return hipErrorInvalidValue;
    constexpr int D = 128;
    hipError_t e;
    switch (p.in_dtype) {
        case GR_DTYPE_F32: e = launch_chunked_dt<GR_DTYPE_F32>(p, st); break;
        case GR_DTYPE_F16: e = launch_chunked_dt<GR_DTYPE_F16>(p, st); break;
        case GR_DTYPE_BF16: e = launch_chunked_dt<GR_DTYPE_BF16>(p, st); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    // columns whose scan stopped at a chunk with non-finite values continue token by token
    DeltaNetLaunch f = p;
    f.first_bad = (const int*)p.ws;
    deltanet_step_kernel<D><<<dim3(D / kStepCols, p.n_heads), kStepThreads, 0, st>>>(f);
    return hipGetLastError();
}

}  // namespace gr
