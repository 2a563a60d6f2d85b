// Split-K flash-decoding for one new token per sequence over a device KV cache.
//
// Replaces the per-head `for t in visible` loop of attention_token
// (reference src/engine/runtime/inference.rs:1970-2530) for every sequence of a
// batch at once.  Work unit = (sequence, KV head, split of `split_keys` keys):
// one workgroup reads each K/V row of its split exactly once and serves all
// kv_mul = Hq/Hkv query heads of that KV head (GQA, kv_head = h / kv_mul,
// inference.rs:2019).  Each workgroup leaves an online-softmax partial
// (running max m, sum l, unnormalised o[d]) in the workspace; a combine kernel
// merges the partials of a (sequence, head).
//
// Scores are kept in the log2 domain: s2 = (q.k) * score_scale * log2(e), so
// exp(s - m) == exp2(s2 - m2) with one v_exp_f32.
#include <type_traits>

#include "gr_common.hpp"
#include "gr_internal.hpp"
#include "stream_sched.hpp"

namespace gr {

constexpr int kDecodeThreads = 256;
constexpr int kDecodeWaves = kDecodeThreads / 64;
// Rows per row group per iteration (memory-level parallelism): 4, or 8 for f32
// splits that one 8-row iteration covers whole in grids of at most one
// workgroup per CU (a short split then costs one round trip to HBM instead of
// two: config 1, 1024 keys in 64-key splits, 128 workgroups, 11.9 -> 11.1 us
// per call).  Larger grids measured slower with 8 (f32, 4 x 2048 keys, 8 KV
// heads, 1024 workgroups: 26.7 -> 41 us), as did longer splits (4-5%).
constexpr int kDecodeUnroll = 4;
constexpr int64_t kDecodeUnroll8MaxWorkgroups = 256;

// One lane owns 16 bytes (EPL elements) of a key row; LPR lanes cover a row of
// D elements; a wave instruction covers RPW = 64 / LPR consecutive rows.
template <typename KV, int D>
struct DecodeGeom {
    static constexpr int EPL = 16 / KV::bytes;
    static constexpr int LPR = D / EPL;
    static constexpr int RPW = 64 / LPR;
    static_assert(LPR >= 1 && LPR <= 64 && 64 % LPR == 0, "row must map onto a wave");
};

// KVMUL: query heads per workgroup (the GQA group, or a slice of it: n_sub > 1).
template <typename KV, int D, int KVMUL, int U = kDecodeUnroll>
__global__ __launch_bounds__(kDecodeThreads) void decode_split_kernel(const DecodeLaunch p) {
    using G = DecodeGeom<KV, D>;
    constexpr int EPL = G::EPL, LPR = G::LPR, RPW = G::RPW;
    constexpr int STEP = kDecodeWaves * U * RPW;  // rows per block iteration

    const int split = blockIdx.x;
    const int n_sub = p.n_sub > 0 ? p.n_sub : 1;
    const int g = blockIdx.y / n_sub;  // KV head
    const int kv_mul = p.n_heads / p.n_kv_heads;
    const int h0 = g * kv_mul + (blockIdx.y % n_sub) * KVMUL;  // first query head
    const int nq = min(KVMUL, g * kv_mul + kv_mul - h0);       // query heads here
    const int s = blockIdx.z;
    const int t_begin = p.kv_start[s] + split * p.split_keys;
    const int t_limit = p.kv_end[s];
    if (t_begin >= t_limit) return;
    const int t_stop = min(t_limit, t_begin + p.split_keys);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rg = lane / LPR;   // row group within the wave
    const int sl = lane % LPR;   // slice of the row owned by this lane
    const int e0 = sl * EPL;

    // q slices for the kv_mul heads of this KV head, pre-scaled into log2 units.
    const float qscale = p.score_scale * kLog2e;
    float qv[KVMUL][EPL];
#pragma unroll
    for (int j = 0; j < KVMUL; j++) {
        const float* qh = p.q + ((size_t)s * p.n_heads + h0 + (j < nq ? j : 0)) * D + e0;
#pragma unroll
        for (int e = 0; e < EPL; e++) qv[j][e] = j < nq ? qh[e] * qscale : 0.0f;
    }

    float m[KVMUL], l[KVMUL], o[KVMUL][EPL];
#pragma unroll
    for (int j = 0; j < KVMUL; j++) {
        m[j] = -INFINITY;
        l[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; e++) o[j][e] = 0.0f;
    }

    const char* kbase = (const char*)p.k_cache +
                        ((size_t)(p.seq_slot ? p.seq_slot[s] : s) * p.seq_stride + (size_t)g * D + e0) * KV::bytes;
    const char* vbase = (const char*)p.v_cache +
                        ((size_t)(p.seq_slot ? p.seq_slot[s] : s) * p.seq_stride + (size_t)g * D + e0) * KV::bytes;
    const size_t row_bytes = (size_t)p.row_stride * KV::bytes;

    for (int tb = t_begin; tb < t_stop; tb += STEP) {
        uint4 kraw[U], vraw[U];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = tb + (wave * U + u) * RPW + rg;
            valid[u] = t < t_stop;
            const int tt = valid[u] ? t : t_begin;  // clamp: never read past the split
            kraw[u] = *(const uint4*)(kbase + (size_t)tt * row_bytes);
            vraw[u] = *(const uint4*)(vbase + (size_t)tt * row_bytes);
        }
        float sc[U][KVMUL];
#pragma unroll
        for (int u = 0; u < U; u++) {
            float kf[EPL];
            unpack16<KV>(kraw[u], kf);
#pragma unroll
            for (int j = 0; j < KVMUL; j++) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; e++) acc = fmaf(qv[j][e], kf[e], acc);
                sc[u][j] = acc;
            }
        }
        // Reduce partial dots across the LPR lanes of a row (butterfly: every
        // lane of the row group ends with the full score).
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int j = 0; j < KVMUL; j++) {
                float v = wave_sum<LPR>(sc[u][j]);
                sc[u][j] = valid[u] ? v : -INFINITY;
            }
#pragma unroll
        for (int j = 0; j < KVMUL; j++) {
            float mx = m[j];
#pragma unroll
            for (int u = 0; u < U; u++) mx = fmaxf(mx, sc[u][j]);
            // mx is finite whenever any row of this group was valid.
            const float alpha = (mx == -INFINITY) ? 1.0f : exp2f(m[j] - mx);
            float lsum = l[j] * alpha;
#pragma unroll
            for (int e = 0; e < EPL; e++) o[j][e] *= alpha;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float pu = (sc[u][j] == -INFINITY) ? 0.0f : exp2f(sc[u][j] - mx);
                lsum += pu;
                sc[u][j] = pu;
            }
            l[j] = lsum;
            m[j] = mx;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            float vf[EPL];
            unpack16<KV>(vraw[u], vf);
#pragma unroll
            for (int j = 0; j < KVMUL; j++)
#pragma unroll
                for (int e = 0; e < EPL; e++) o[j][e] = fmaf(sc[u][j], vf[e], o[j][e]);
        }
    }

    // Merge the RPW row groups of the wave (lanes with equal `sl`).
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
        for (int j = 0; j < KVMUL; j++) {
            const float m_o = shfl_xor(m[j], off);
            const float l_o = shfl_xor(l[j], off);
            const float mx = fmaxf(m[j], m_o);
            const float a = (m[j] == -INFINITY) ? 0.0f : exp2f(m[j] - mx);
            const float b = (m_o == -INFINITY) ? 0.0f : exp2f(m_o - mx);
            l[j] = l[j] * a + l_o * b;
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                const float oo = shfl_xor(o[j][e], off);
                o[j][e] = o[j][e] * a + oo * b;
            }
            m[j] = mx;
        }
    }

    // Merge the waves through LDS; wave 0 writes the partial.
    __shared__ float sh_m[kDecodeWaves][KVMUL];
    __shared__ float sh_l[kDecodeWaves][KVMUL];
    __shared__ float sh_o[kDecodeWaves][KVMUL][D];
    if (rg == 0) {
#pragma unroll
        for (int j = 0; j < KVMUL; j++) {
#pragma unroll
            for (int e = 0; e < EPL; e++) sh_o[wave][j][e0 + e] = o[j][e];
            if (sl == 0) {
                sh_m[wave][j] = m[j];
                sh_l[wave][j] = l[j];
            }
        }
    }
    __syncthreads();
    // Thread layout for the final merge: KVMUL*D outputs spread over the block.
    const int n_splits = p.n_splits;
    for (int idx = threadIdx.x; idx < nq * D; idx += kDecodeThreads) {
        const int j = idx / D;
        const int i = idx % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; w++) mx = fmaxf(mx, sh_m[w][j]);
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; w++) {
            const float a = (sh_m[w][j] == -INFINITY) ? 0.0f : exp2f(sh_m[w][j] - mx);
            lt += sh_l[w][j] * a;
            ot += sh_o[w][j][i] * a;
        }
        const int h = h0 + j;
        const size_t part = ((size_t)s * p.n_heads + h) * n_splits + split;
        p.ws_o[part * D + i] = ot;
        if (i == 0) {
            p.ws_ml[part * 2 + 0] = mx;
            p.ws_ml[part * 2 + 1] = lt;
        }
    }
}

// Merge the split partials of one (sequence, head), one wavefront each:
//   out = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M),  M = max_s m_s.
// Lanes first cover splits (weights), then dimensions (weighted sums, splits
// unrolled by 4 so the partial loads are in flight together).
constexpr int kCombineWaves = 4;

template <int D>
__global__ __launch_bounds__(64 * kCombineWaves) void decode_combine_kernel(const DecodeLaunch p) {
    __shared__ float wts[kCombineWaves][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = blockIdx.x * kCombineWaves + wave;
    const int s = blockIdx.y;
    if (h >= p.n_heads) return;
    const int len = p.kv_end[s] - p.kv_start[s];
    int nv;
    if (p.stream_sched) {  // ranges that meet pair (s, column of h)
        const int kv_mul = p.n_heads / p.n_kv_heads;
        const int n_sub = p.n_sub > 0 ? p.n_sub : 1;
        const int col = (h / kv_mul) * n_sub + (n_sub > 1 ? (h % kv_mul) / p.sub_heads : 0);
        nv = stream_partials(p, s, col);
    } else {  // the splits the grid has (keys past them are dropped, as on the stream schedule)
        nv = len > 0 ? min(p.n_splits, (len + p.split_keys - 1) / p.split_keys) : 0;
    }
    const size_t base = ((size_t)s * p.n_heads + h) * p.n_splits;
    float* out = p.out + ((size_t)s * p.n_heads + h) * D;
    const float* gt = p.gate.at(s, h);  // Qwen3.5 output gate, or null
    constexpr int EPL = D / 64;
    // Few partials (the usual case): every lane loads all (m, l) pairs and its
    // own o values at once and reduces them itself, one round trip to memory.
    constexpr int kFewSplits = 16;
    if (nv <= kFewSplits) {
        float mk[kFewSplits], lk[kFewSplits], ok[kFewSplits][EPL];
#pragma unroll
        for (int k = 0; k < kFewSplits; k++) {
            mk[k] = -INFINITY, lk[k] = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; e++) ok[k][e] = 0.0f;
            if (k < nv) {
                const float2 ml = *(const float2*)(p.ws_ml + (base + k) * 2);
                mk[k] = ml.x, lk[k] = ml.y;
#pragma unroll
                for (int e = 0; e < EPL; e++) ok[k][e] = p.ws_o[(base + k) * D + lane + 64 * e];
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < kFewSplits; k++) mx = fmaxf(mx, mk[k]);
        float lt = 0.0f, acc[EPL];
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < kFewSplits; k++) {
            const float w = mk[k] == -INFINITY ? 0.0f : exp2f(mk[k] - mx);
            lt += lk[k] * w;
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[e] += ok[k][e] * w;
        }
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            const float o = acc[e] * inv;
            out[lane + 64 * e] = gt ? gate_mul(o, gt[lane + 64 * e]) : o;
        }
        return;
    }
    // pass 1: global max and denominator, lanes over splits
    float mx = -INFINITY;
    for (int k = lane; k < nv; k += 64) mx = fmaxf(mx, p.ws_ml[(base + k) * 2]);
    mx = wave_max<64>(mx);
    float lt = 0.0f;
    for (int k = lane; k < nv; k += 64) {
        const float mk = p.ws_ml[(base + k) * 2];
        lt += p.ws_ml[(base + k) * 2 + 1] * (mk == -INFINITY ? 0.0f : exp2f(mk - mx));
    }
    lt = wave_sum<64>(lt);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    // pass 2: weighted sum of o, lanes over dimensions; weights staged per 64 splits
    float acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[e] = 0.0f;
    for (int k0 = 0; k0 < nv; k0 += 64) {
        const int k = k0 + lane;
        float wk = 0.0f;
        if (k < nv) {
            const float mk = p.ws_ml[(base + k) * 2];
            wk = mk == -INFINITY ? 0.0f : exp2f(mk - mx);
        }
        wts[wave][lane] = wk;
        __builtin_amdgcn_wave_barrier();
        const int kn = min(64, nv - k0);
        int kk = 0;
        for (; kk + 4 <= kn; kk += 4) {
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                const float* op = p.ws_o + (base + k0 + kk) * D + lane + 64 * e;
                const float a0 = op[0], a1 = op[D], a2 = op[2 * D], a3 = op[3 * D];
                acc[e] += wts[wave][kk] * a0 + wts[wave][kk + 1] * a1 + wts[wave][kk + 2] * a2 +
                          wts[wave][kk + 3] * a3;
            }
        }
        for (; kk < kn; kk++)
#pragma unroll
            for (int e = 0; e < EPL; e++)
                acc[e] += wts[wave][kk] * p.ws_o[(base + k0 + kk) * D + lane + 64 * e];
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int e = 0; e < EPL; e++) {
        const float o = acc[e] * inv;
        out[lane + 64 * e] = gt ? gate_mul(o, gt[lane + 64 * e]) : o;
    }
}

// Query heads per workgroup: the whole GQA group rounded up to 1, 2, 4 or 8
// (unused slots masked), groups above 8 in slices of 8 (n_sub columns per KV head).
static int valu_heads_per_block(int kv_mul) { return kv_mul <= 1 ? 1 : kv_mul <= 2 ? 2 : kv_mul <= 4 ? 4 : 8; }

template <typename KV, int D>
static hipError_t launch_kvmul(const DecodeLaunch& p0, int kv_mul, hipStream_t st) {
    DecodeLaunch p = p0;
    const int hb = valu_heads_per_block(kv_mul);
    p.n_sub = (kv_mul + hb - 1) / hb;
    p.sub_heads = hb;
    dim3 grid(p.n_splits, p.n_kv_heads * p.n_sub, p.n_seq);
    constexpr int kStep4 = kDecodeWaves * 4 * DecodeGeom<KV, D>::RPW;
    bool launched = false;
    if constexpr (std::is_same<KV, F32>::value) {
        if (p.split_keys > kStep4 && p.split_keys <= 2 * kStep4 &&
            (int64_t)grid.x * grid.y * grid.z <= kDecodeUnroll8MaxWorkgroups) {
            switch (hb) {
                case 1: decode_split_kernel<KV, D, 1, 8><<<grid, kDecodeThreads, 0, st>>>(p); break;
                case 2: decode_split_kernel<KV, D, 2, 8><<<grid, kDecodeThreads, 0, st>>>(p); break;
                case 4: decode_split_kernel<KV, D, 4, 8><<<grid, kDecodeThreads, 0, st>>>(p); break;
                case 8: decode_split_kernel<KV, D, 8, 8><<<grid, kDecodeThreads, 0, st>>>(p); break;
                default: return hipErrorInvalidValue;
            }
            launched = true;
        }
    }
    if (!launched) {
        switch (hb) {
            case 1: decode_split_kernel<KV, D, 1><<<grid, kDecodeThreads, 0, st>>>(p); break;
            case 2: decode_split_kernel<KV, D, 2><<<grid, kDecodeThreads, 0, st>>>(p); break;
            case 4: decode_split_kernel<KV, D, 4><<<grid, kDecodeThreads, 0, st>>>(p); break;
            case 8: decode_split_kernel<KV, D, 8><<<grid, kDecodeThreads, 0, st>>>(p); break;
            default: return hipErrorInvalidValue;
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    decode_combine_kernel<D><<<dim3((p.n_heads + kCombineWaves - 1) / kCombineWaves, p.n_seq),
                               64 * kCombineWaves, 0, st>>>(p);
    return hipGetLastError();
}

template <typename KV>
static hipError_t launch_dim(const DecodeLaunch& p, int kv_mul, hipStream_t st) {
    switch (p.head_dim) {
        case 64: return launch_kvmul<KV, 64>(p, kv_mul, st);
        case 128: return launch_kvmul<KV, 128>(p, kv_mul, st);
        case 256: return launch_kvmul<KV, 256>(p, kv_mul, st);
        default: return hipErrorInvalidValue;
    }
}

template <int D>
static hipError_t launch_combine(const DecodeLaunch& p, hipStream_t st) {
    decode_combine_kernel<D><<<dim3((p.n_heads + kCombineWaves - 1) / kCombineWaves, p.n_seq),
                               64 * kCombineWaves, 0, st>>>(p);
    return hipGetLastError();
}

hipError_t launch_decode(const DecodeLaunch& p, hipStream_t st) {
    const int kv_mul = p.n_heads / p.n_kv_heads;
    if (p.kv_dtype == GR_DTYPE_TURBO) return decode_turbo_supported(p) ? launch_decode_turbo(p, st) : hipErrorInvalidValue;
    DecodeLaunch pm = p;  // MFMA path: groups above 16 query heads in columns of 16
    pm.n_sub = (kv_mul + 15) / 16;
    pm.sub_heads = 16;
    if (p.use_mfma && decode_mfma_supported(pm)) {
        hipError_t e = launch_decode_mfma_split(pm, st);
        if (e != hipSuccess) return e;
        switch (p.head_dim) {
            case 64: return launch_combine<64>(pm, st);
            case 128: return launch_combine<128>(pm, st);
            case 256: return launch_combine<256>(pm, st);
            default: return hipErrorInvalidValue;
        }
    }
    switch (p.kv_dtype) {
        case GR_DTYPE_F32: return launch_dim<F32>(p, kv_mul, st);
        case GR_DTYPE_F16: return launch_dim<F16>(p, kv_mul, st);
        case GR_DTYPE_BF16: return launch_dim<BF16>(p, kv_mul, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace gr
