// Turbo KV cache (KvCacheFormat::Turbo, reference inference.rs:346-1334) on the
// device: the quantising KV write and the merge + value finalisation of the
// split-K decode (the query preparation and the split kernel are in
// turbo_decode.hip).
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
// The write keeps the reference's arithmetic order: the wave FWHT adds and
// subtracts in its stage order and the norms are sequential sums in element
// order, so the written codes, signs, sigma and gamma are bit-exact with the
// reference for the same f32 row (no FMA contraction in this file).
#pragma clang fp contract(off)

#include "gr_common.hpp"
#include "gr_internal.hpp"
#include "stream_sched.hpp"
#include "turbo_common.hpp"

namespace gr {

namespace {

__device__ __forceinline__ float tq_centroid(int code) {
    return code == 0 ? -tq::kC1 : code == 1 ? -tq::kC0 : code == 2 ? tq::kC0 : tq::kC1;
}

__device__ __forceinline__ int tq_code(float x) {
    return x < -tq::kTh ? 0 : (x < 0.0f ? 1 : (x < tq::kTh ? 2 : 3));
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
    tq::wave_transform<D>(x, sg, sg + ss, lane);  // rot_pre, rot_post
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
    tq::wave_transform<D>(r, sg + 2 * ss, sg + 3 * ss, lane);  // res_pre, res_post
#pragma unroll
    for (int j = 0; j < J; j++) {
        const uint64_t m = __ballot(r[j] >= 0.0f);  // bit l = element 64 j + l
        if (lane == 0) *(uint64_t*)(sign + 8 * j) = m;
    }
}

// The same write for long row sets (a prefill chunk): one wave quantises R
// consecutive units (unit = K|V, row, kv head; K units first).  Rotations, codes
// and sign bits are computed per unit across the wave as above; the two norms,
// sequential sums in element order, run in lanes 0..R-1, lane u summing unit u
// from an LDS copy ([R][D + 4]: the per-unit stores and the per-lane 16-byte
// reads are both free of bank conflicts).  One pass of the serial chain
// thus serves R units, with the same arithmetic and order as wave_l2_sequential.
template <int D, int R>
__global__ __launch_bounds__(64) void turbo_write_batch_kernel(const TurboWriteLaunch p) {
    constexpr int J = D / 64, LDR = D + 4;
    constexpr int SB = D / 2;                  // sign-table bytes per unit: 4 rows of D / 8
    constexpr int NSB = (SB + 63) / 64;
    __shared__ __attribute__((aligned(16))) float buf[R * LDR];
    __shared__ uint8_t codes[R * D];
    __shared__ uint8_t sgn[R * SB];            // unit u: rot_pre, rot_post, res_pre, res_post
    const int lane = threadIdx.x;
    const int per_kv = p.n_rows * p.n_kv_heads;
    const int u0 = (int)blockIdx.x * R;
    const int nu = min(R, 2 * per_kv - u0);
    const int kv_dim = p.n_kv_heads * D;
    const int64_t ss = p.slot_stride;

    struct Unit {
        bool is_v;
        int i, g;
    };
    auto unit = [&](int u) {
        const int x = u0 + u;
        Unit t;
        t.is_v = x >= per_kv;
        const int rem = t.is_v ? x - per_kv : x;
        t.i = rem / p.n_kv_heads;
        t.g = rem - t.i * p.n_kv_heads;
        return t;
    };
    auto elem_of = [&](const Unit& t) {
        const int64_t row = p.cache_row ? (int64_t)p.cache_row[t.i] : p.row0 + t.i;
        const int64_t sq = p.cache_seq ? (int64_t)p.cache_seq[t.i] : 0;
        return sq * p.cache_seq_stride + row * p.cache_row_stride + (int64_t)t.g * D;
    };
    auto aux_of = [&](const Unit& t) {
        const int64_t row = p.cache_row ? (int64_t)p.cache_row[t.i] : p.row0 + t.i;
        const int64_t sq = p.cache_seq ? (int64_t)p.cache_seq[t.i] : 0;
        return sq * p.aux_seq_stride + row * p.aux_row_stride + t.g;
    };
    // sequential sum of squares of lane's unit (lane < nu), as wave_l2_sequential
    auto lane_l2 = [&]() {
        float s2 = 0.0f;
        const float4* b4 = (const float4*)(buf + lane * LDR);
#pragma unroll 8
        for (int k = 0; k < D / 4; k++) {
            const float4 v = b4[k];
            s2 = s2 + v.x * v.x;
            s2 = s2 + v.y * v.y;
            s2 = s2 + v.z * v.z;
            s2 = s2 + v.w * v.w;
        }
        return sqrtf(s2);
    };
    auto bcast = [](float v, int u) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), u)); };

    // every unit's row and sign-table rows load in flight together (units past
    // nu re-read the last one); the sign rows go to LDS, then the rotations run
    // with the rows in registers, copied to buf
    float x[R][J];
    uint32_t sv[R][NSB];  // one byte per register: packing them would wait for each load
#pragma unroll
    for (int u = 0; u < R; u++) {
        const Unit t = unit(min(u, nu - 1));
        const float* src = (t.is_v ? p.v_rows : p.k_rows) + (size_t)t.i * kv_dim + (size_t)t.g * D;
#pragma unroll
        for (int j = 0; j < J; j++) x[u][j] = src[lane + 64 * j];
        const uint8_t* sg = p.signs + (size_t)t.g * (D / 8);
#pragma unroll
        for (int c = 0; c < NSB; c++) {
            const int k = min(lane + 64 * c, SB - 1);
            sv[u][c] = sg[(k / (D / 8)) * ss + k % (D / 8)];
        }
    }
#pragma unroll
    for (int u = 0; u < R; u++)
#pragma unroll
        for (int c = 0; c < NSB; c++)
            if (lane + 64 * c < SB) sgn[u * SB + lane + 64 * c] = (uint8_t)sv[u][c];
    tq::wave_lds_sync();
#pragma unroll
    for (int u = 0; u < R; u++) {
        if (u < nu) {
            const uint8_t* sg = sgn + u * SB;
            tq::wave_transform<D>(x[u], sg, sg + D / 8, lane);  // rot_pre, rot_post
#pragma unroll
            for (int j = 0; j < J; j++) buf[u * LDR + lane + 64 * j] = x[u][j];
        }
    }
    tq::wave_lds_sync();
    const float sig = lane < nu ? lane_l2() / sqrtf((float)D) : 0.0f;
    tq::wave_lds_sync();  // the sums' reads precede the residual stores below

    // codes and residuals (units with sigma 0 keep their rows: they are written as zero)
#pragma unroll
    for (int u = 0; u < R; u++) {
        const float sigma = bcast(sig, u);
        if (u < nu && sigma != 0.0f) {
            const float inv_sigma = 1.0f / sigma;
#pragma unroll
            for (int j = 0; j < J; j++) {
                const int c = tq_code(x[u][j] * inv_sigma);
                x[u][j] = x[u][j] - tq_centroid(c) * sigma;
                codes[u * D + lane + 64 * j] = (uint8_t)c;
                buf[u * LDR + lane + 64 * j] = x[u][j];
            }
        }
    }
    tq::wave_lds_sync();
    const float gam = (lane < nu && sig != 0.0f) ? lane_l2() : 0.0f;
    if (lane < nu) {
        const Unit t = unit(lane);
        const int64_t a = aux_of(t);
        (t.is_v ? p.v_scale : p.k_scale)[a] = sig;
        (t.is_v ? p.v_rnorm : p.k_rnorm)[a] = gam;
    }

    // packed codes and residual sign bits
#pragma unroll
    for (int u = 0; u < R; u++) {
        if (u < nu) {
            const Unit t = unit(u);
            const int64_t elem = elem_of(t);
            uint8_t* base = (t.is_v ? p.v_base : p.k_base) + elem / 4;
            uint8_t* sign = (t.is_v ? p.v_sign : p.k_sign) + elem / 8;
            const float sigma = bcast(sig, u), gamma = bcast(gam, u);
            if (lane < D / 4) {
                const uint8_t* cu = codes + u * D + 4 * lane;
                base[lane] = sigma == 0.0f ? (uint8_t)0 : (uint8_t)(cu[0] | (cu[1] << 2) | (cu[2] << 4) | (cu[3] << 6));
            }
            if (gamma == 0.0f) {  // also sigma 0
                if (lane < D / 8) sign[lane] = 0xff;
            } else {
                const uint8_t* sg = sgn + u * SB;
#pragma unroll
                for (int j = 0; j < J; j++) x[u][j] = x[u][j] / gamma;
                tq::wave_transform<D>(x[u], sg + 2 * (D / 8), sg + 3 * (D / 8), lane);  // res_pre, res_post
#pragma unroll
                for (int j = 0; j < J; j++) {
                    const uint64_t m = __ballot(x[u][j] >= 0.0f);  // bit l = element 64 j + l
                    if (lane == 0) *(uint64_t*)(sign + 8 * j) = m;
                }
            }
        }
    }
}

// Units (2 n_rows n_kv_heads) from which the batched write runs: below it the
// one-unit waves (142 VGPRs: about 3000 resident on the chip) all run at once and
// finish sooner.  Units per wave: a 2048-row, 8-head chunk (32768 units) takes
// 22.7 µs with 4, 25.6 with 8, 32.6 with 16, 27.1 with 2 and 47.1 in one-unit
// waves; four-wave workgroups were slower (24.5 with 4).
constexpr int kTurboWriteBatchMin = 4096;
constexpr int kTurboWriteBatch = 4;

hipError_t launch_turbo_write(const TurboWriteLaunch& p, hipStream_t st) {
    if (p.n_rows <= 0) return hipSuccess;
    const int64_t n_units = 2 * (int64_t)p.n_rows * p.n_kv_heads;
    if (n_units >= kTurboWriteBatchMin && n_units <= INT32_MAX) {
        const dim3 bgrid((unsigned)((n_units + kTurboWriteBatch - 1) / kTurboWriteBatch));
        switch (p.head_dim) {
            case 64: turbo_write_batch_kernel<64, kTurboWriteBatch><<<bgrid, 64, 0, st>>>(p); break;
            case 128: turbo_write_batch_kernel<128, kTurboWriteBatch><<<bgrid, 64, 0, st>>>(p); break;
            case 256: turbo_write_batch_kernel<256, kTurboWriteBatch><<<bgrid, 64, 0, st>>>(p); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    dim3 grid((unsigned)p.n_rows, (unsigned)p.n_kv_heads, 2);
    switch (p.head_dim) {
        case 64: turbo_write_kernel<64><<<grid, 64, 0, st>>>(p); break;
        case 128: turbo_write_kernel<128><<<grid, 64, 0, st>>>(p); break;
        case 256: turbo_write_kernel<256><<<grid, 64, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- merge + finalize

// One wave per (head, sequence): merge the split partials of the base and residual
// accumulators (log2-domain weights), divide by the softmax sum, then
// finalize_turboquant_value_head (inference.rs:1323-1334): residual <- R'^-1
// residual, base += residual, out = R^-1 base.
template <int D>
__global__ __launch_bounds__(256) void turbo_combine_kernel(const DecodeLaunch p) {
    constexpr int J = D / 64, U = 8;
    __shared__ float wsh_all[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* wsh = wsh_all[wave];
    const int h = 4 * blockIdx.x + wave, s = blockIdx.y;  // four heads per workgroup
    if (h >= p.n_heads) return;  // whole wave; only wave-level synchronisation below
    const int kv_mul = p.n_heads / p.n_kv_heads;
    const int g = h / kv_mul;
    const int t_len = p.kv_end[s] - p.kv_start[s];
    int n_used;
    if (p.stream_sched) {  // ranges that meet pair (s, column of h)
        const int n_sub = p.n_sub > 0 ? p.n_sub : 1;
        n_used = stream_partials(p, s, g * n_sub + (n_sub > 1 ? (h % kv_mul) / p.sub_heads : 0));
    } else {
        n_used = t_len > 0 ? (t_len + p.split_keys - 1) / p.split_keys : 0;
    }
    const size_t part0 = ((size_t)s * p.n_heads + h) * p.n_splits;
    float mx = -INFINITY;
    for (int sp = lane; sp < n_used; sp += 64) mx = fmaxf(mx, p.ws_ml[(part0 + sp) * 2]);
    mx = wave_max<64>(mx);
    float lt = 0.0f;
    float b[J], r[J];
#pragma unroll
    for (int j = 0; j < J; j++) b[j] = r[j] = 0.0f;
    for (int c0 = 0; c0 < n_used; c0 += 64) {
        const int nc = min(64, n_used - c0);
        // lane i: the weight of split c0 + i
        float w = 0.0f;
        if (lane < nc) {
            const size_t pt = part0 + c0 + lane;
            w = exp2f(p.ws_ml[pt * 2] - mx);
            lt += p.ws_ml[pt * 2 + 1] * w;
        }
        wsh[lane] = w;
        tq::wave_lds_sync();  // the wave's weights visible to all its lanes
        const float* o = p.ws_o + (part0 + c0) * 2 * D;
        int i = 0;
        for (; i + U <= nc; i += U) {  // U partials' loads in flight together
            float ob[U][J], orr[U][J];
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int j = 0; j < J; j++) {
                    ob[u][j] = o[(i + u) * 2 * D + lane + 64 * j];
                    orr[u][j] = o[(i + u) * 2 * D + D + lane + 64 * j];
                }
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int j = 0; j < J; j++) {
                    b[j] += ob[u][j] * wsh[i + u];
                    r[j] += orr[u][j] * wsh[i + u];
                }
        }
        for (; i < nc; i++)
#pragma unroll
            for (int j = 0; j < J; j++) {
                b[j] += o[i * 2 * D + lane + 64 * j] * wsh[i];
                r[j] += o[i * 2 * D + D + lane + 64 * j] * wsh[i];
            }
        tq::wave_lds_sync();  // wsh reads done before the next chunk's stores
    }
    lt = wave_sum<64>(lt);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        b[j] *= inv;
        r[j] *= inv;
    }
    const uint8_t* sg = p.turbo_signs + (size_t)g * (D / 8);
    const int64_t ss = p.turbo_slot_stride;
    tq::wave_transform<D>(r, sg + 3 * ss, sg + 2 * ss, lane);  // res_post, res_pre: inverse
#pragma unroll
    for (int j = 0; j < J; j++) b[j] += r[j];
    tq::wave_transform<D>(b, sg + ss, sg, lane);  // rot_post, rot_pre: inverse
    float* out = p.out + ((size_t)s * p.n_heads + h) * D;
    const float* gt = p.gate.at(s, h);  // Qwen3.5 output gate, or null
#pragma unroll
    for (int j = 0; j < J; j++) out[lane + 64 * j] = gt ? gate_mul(b[j], gt[lane + 64 * j]) : b[j];
}

hipError_t launch_turbo_combine(const DecodeLaunch& p, hipStream_t st) {
    const dim3 grid((p.n_heads + 3) / 4, p.n_seq);
    switch (p.head_dim) {
        case 64: turbo_combine_kernel<64><<<grid, 256, 0, st>>>(p); break;
        case 128: turbo_combine_kernel<128><<<grid, 256, 0, st>>>(p); break;
        case 256: turbo_combine_kernel<256><<<grid, 256, 0, st>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gr
