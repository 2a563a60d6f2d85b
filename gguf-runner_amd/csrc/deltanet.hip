// Gated DeltaNet (gated delta rule) on gfx950, fp32 state [H][d][d], S[j][i]
// with j = key dim (row) and i = value dim (column), as in
// qwen3next_state_head_step (reference src/engine/kernels/math.rs:492-546):
//   S *= g;  kv_i = sum_j k_j S[j][i];  delta_i = beta (v_i - kv_i);
//   S[j][i] += k_j delta_i;  o_i = sum_j q_j S[j][i]
// q/k are optionally L2-normalised first (q also * 1/sqrt(d)), math.rs:833-846.
// Columns i are independent, which is how both kernels parallelise.
//
// 1. deltanet_step_kernel: the recurrence token by token with a 32-column
//    slice of the state in registers (decode, and the serial scan).
// 2. Chunked prefill (chunk C = 64), WY form of the same recurrence:
//      gamma_t = prod_{s<=t} g_s (in-chunk),  A[t][s] = beta_t (gamma_t/gamma_s) k_t.k_s (s<t)
//      Delta = (I + A)^-1 [beta V - beta gamma K S0] = U - W S0
//      O     = diag(gamma) Q S0 + (Gamma-mask . Q K^T) Delta
//      S_C   = gamma_last S0 + Kd^T Delta,  Kd_s = (gamma_last/gamma_s) k_s
//    deltanet_chunk_prep_kernel builds U, W, P, Qg, Kd^T per (chunk, head) in
//    parallel; deltanet_chunk_scan_kernel carries S across chunks with the
//    state columns split over blocks of 4 (512 workgroups for 16 heads, two per
//    CU: the chunk steps are sequential and latency-bound, so more, smaller
//    blocks run faster even though each re-reads the chunk's W / Qg / P / Kd^T).
#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

__device__ __forceinline__ float dn_load(const void* p, size_t i, int dt) {
    if (dt == GR_DTYPE_F32) return ((const float*)p)[i];
    const uint16_t b = ((const uint16_t*)p)[i];
    return dt == GR_DTYPE_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

// ------------------------------------------------------------------ recurrent step
constexpr int kStepThreads = 256;
constexpr int kStepCols = 32;

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

    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = Sh[(size_t)(jg * R + r) * D + i];

    const float inv_scale_q = 1.0f / sqrtf((float)D);
    for (int t = 0; t < p.n_tokens; t++) {
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
        const float g = finite_or_zero(p.gate_is_log ? expf(gv) : gv);
        const float beta = finite_or_zero(p.beta[(size_t)t * H + h]);
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
        if (tid < kStepCols) {
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
constexpr int kChunk = 64;
constexpr int kChunkThreads = 256;

// Per (chunk, head) workspace block, floats: U, W, Qg [C][D]; KdT [D][C]; P [C][C]; gamma_last.
template <int D>
struct ChunkWs {
    static constexpr size_t U = 0;
    static constexpr size_t W = U + (size_t)kChunk * D;
    static constexpr size_t QG = W + (size_t)kChunk * D;
    static constexpr size_t KDT = QG + (size_t)kChunk * D;
    static constexpr size_t P = KDT + (size_t)D * kChunk;
    static constexpr size_t GL = P + (size_t)kChunk * kChunk;
    static constexpr size_t SIZE = (GL + 1 + 63) / 64 * 64;
};

template <int D>
__global__ __launch_bounds__(kChunkThreads) void deltanet_chunk_prep_kernel(const DeltaNetLaunch p) {
    constexpr int C = kChunk;
    constexpr int DS = D + 4;  // padded LDS row stride
    extern __shared__ float smem[];
    float* qs = smem;                   // [C][DS] normalised q
    float* ks = qs + C * DS;            // [C][DS] normalised k
    constexpr int AS = C + 4;           // A row stride (16-byte aligned rows)
    float* As = ks + C * DS;            // [C][AS] strictly lower-triangular A
    // [C] in-chunk cumulative log decay, in double: with strong decays the prefix
    // sums reach ~-100 within a chunk, and a decay exp(lg[t] - lg[s]) taken from two
    // f32 prefix sums would carry ~100 ulp of absolute error in its exponent
    double* lg = (double*)(As + C * AS);
    float* bt = (float*)(lg + C);       // [C] beta
    float* gm = bt + C;                 // [C] gamma_t = exp(lg[t])
    float* kf = gm + C;                 // [C] gamma_last / gamma_s = exp(lg[C-1] - lg[s])
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int c = blockIdx.x, h = blockIdx.y;
    const int H = p.n_heads;
    const int t0 = c * C;
    const int Cn = min(C, p.n_tokens - t0);  // tokens in this chunk
    float* ws = p.ws + ((size_t)c * H + h) * ChunkWs<D>::SIZE;

    // 1. normalised q, k rows (zero rows past the end of the sequence)
    const float inv_scale_q = 1.0f / sqrtf((float)D);
    for (int r = wave; r < 2 * C; r += kChunkThreads / 64) {
        const int t = r % C;
        const bool isq = r < C;
        float x[D / 64];
        float ss = 0.0f;
        const bool valid = t < Cn;
        const size_t row = ((size_t)(t0 + t) * H + h) * D;
#pragma unroll
        for (int e = 0; e < D / 64; e++) {
            x[e] = valid ? dn_load(isq ? p.q : p.k, row + lane + 64 * e, p.in_dtype) : 0.0f;
            ss += x[e] * x[e];
        }
        float* dst = (isq ? qs : ks) + t * DS;
        if (p.l2norm) {
            ss = wave_sum<64>(ss);
            const float inv = 1.0f / sqrtf(ss + p.eps);
#pragma unroll
            for (int e = 0; e < D / 64; e++)
                dst[lane + 64 * e] = valid ? finite_or_zero(isq ? x[e] * inv * inv_scale_q : x[e] * inv) : 0.0f;
        } else {
#pragma unroll
            for (int e = 0; e < D / 64; e++) dst[lane + 64 * e] = x[e];
        }
    }
    // in-chunk cumulative log decay (inclusive) and beta; padded tokens: gate 0, beta 0
    if (wave == 0) {
        const bool valid = lane < Cn;
        double gl = valid ? (double)p.gate[(size_t)(t0 + lane) * H + h] : 0.0;
        // inclusive prefix sum over the 64 lanes
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(gl, off, 64);
            if (lane >= off) gl += o;
        }
        lg[lane] = gl;
        gm[lane] = expf((float)gl);
        const double gl_last = __shfl(gl, 63, 64);
        kf[lane] = expf((float)(gl_last - gl));
        bt[lane] = valid ? finite_or_zero(p.beta[(size_t)(t0 + lane) * H + h]) : 0.0f;
    }
    __syncthreads();

    // 2. A (LDS) and P (workspace): thread -> row t, 16 columns s
    {
        const int t = tid >> 2;
        const int sb = (tid & 3) * 16;
        float akk[16], aqk[16];
#pragma unroll
        for (int u = 0; u < 16; u++) akk[u] = aqk[u] = 0.0f;
        for (int j = 0; j < D; j += 4) {
            const float4 kt = *(const float4*)(ks + t * DS + j);
            const float4 qt = *(const float4*)(qs + t * DS + j);
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const float4 kk = *(const float4*)(ks + (sb + u) * DS + j);
                akk[u] = fmaf(kt.x, kk.x, fmaf(kt.y, kk.y, fmaf(kt.z, kk.z, fmaf(kt.w, kk.w, akk[u]))));
                aqk[u] = fmaf(qt.x, kk.x, fmaf(qt.y, kk.y, fmaf(qt.z, kk.z, fmaf(qt.w, kk.w, aqk[u]))));
            }
        }
        const double lt = lg[t];
        const float bet = bt[t];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int s = sb + u;
            const float decay = s <= t ? expf((float)(lt - lg[s])) : 0.0f;
            As[t * AS + s] = s < t ? bet * decay * akk[u] : 0.0f;
            ws[ChunkWs<D>::P + t * C + s] = s <= t ? decay * aqk[u] : 0.0f;
        }
    }
    __syncthreads();

    // 3. Qg = gamma_t q_t and Kd^T[j][s] = (gamma_last / gamma_s) k_s[j]
    const double lglast = lg[C - 1];
    for (int e = tid; e < C * D; e += kChunkThreads) {
        const int t = e / D, j = e % D;
        ws[ChunkWs<D>::QG + e] = gm[t] * qs[t * DS + j];
    }
    for (int e = tid; e < D * C; e += kChunkThreads) {
        const int j = e / C, s2 = e % C;
        ws[ChunkWs<D>::KDT + e] = kf[s2] * ks[s2 * DS + j];
    }

    // 4. [U | W] = (I + A)^-1 [beta V | beta gamma K] by forward substitution,
    //    one right-hand-side column per thread, the whole column in registers:
    //    x[t] -= A[t][s] x[s] for s = 0 .. t-1 in order.
    for (int col = tid; col < 2 * D; col += kChunkThreads) {
        const bool isv = col < D;
        const int cc = isv ? col : col - D;
        float* dst = ws + (isv ? ChunkWs<D>::U : ChunkWs<D>::W);
        float x[C];
#pragma unroll
        for (int t = 0; t < C; t++)
            x[t] = isv ? (t < Cn ? bt[t] * finite_or_zero(dn_load(p.v, ((size_t)(t0 + t) * H + h) * D + cc, p.in_dtype))
                                 : 0.0f)
                       : bt[t] * gm[t] * ks[t * DS + cc];
#pragma unroll
        for (int t = 1; t < C; t++) {
            const float* arow = As + t * AS;
#pragma unroll
            for (int s4 = 0; s4 < t; s4 += 4) {
                const float4 a4 = *(const float4*)(arow + s4);
                const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (s4 + k < t) x[t] = fmaf(-av[k], x[s4 + k], x[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < C; t++) dst[t * D + cc] = x[t];
    }
    if (tid == 0) ws[ChunkWs<D>::GL] = expf((float)lglast);
}

constexpr int kScanCols = 4;

// Raw buffer access (wave-uniform base in a scalar descriptor, 32-bit byte
// offsets per lane) and 16 bytes per lane straight into LDS at lds + 16 * lane
// (lds wave-uniform).  The builtin exists for the device pass only.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dn_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)0xffffffff, 0x00020000);
}
__device__ __forceinline__ void dn_dma16(__amdgpu_buffer_rsrc_t r, float* lds, int voff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
#endif
}
// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left at their maxima)
__device__ __forceinline__ void dn_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The chunk steps are sequential, so every step's memory latency is exposed
// unless it is requested early: W and Qg (read only by phase A) go by DMA into
// LDS, the next chunk's as soon as phase A is done, and the P and Kd^T rows a
// thread needs in phases B and C are loaded into registers when the step starts.
// W / Qg tiles are [C][D] f32 rows of 32 16-byte chunks, chunk q of row r at
// position q ^ (r & 15), so the 16 rows a wave reads at once hit distinct banks.
template <int D>
__global__ __launch_bounds__(kChunkThreads) void deltanet_chunk_scan_kernel(const DeltaNetLaunch p) {
    constexpr int C = kChunk;
    constexpr int NC = kScanCols;
    constexpr int RQ = D / 4;                 // 16-byte chunks per W / Qg row
    static_assert(RQ == 32 && C * D * 4 == 4 * 8 * 1024, "tile DMA covers [C][D] in 4 waves x 8 KB");
    __shared__ __attribute__((aligned(16))) float Ss[D][NC];
    __shared__ __attribute__((aligned(16))) float Dl[C][NC];
    __shared__ __attribute__((aligned(16))) float Wl[C * D];
    __shared__ __attribute__((aligned(16))) float Ql[C * D];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    // blockIdx.x = head so that the column blocks of one head (linear ids
    // h + H*cb) land on the same XCD and share its L2 copy of the workspace.
    const int h = blockIdx.x;
    const int c0 = blockIdx.y * NC;
    const int H = p.n_heads;
    float* Sh = p.state + (size_t)h * D * D;
    for (int e = tid; e < D * NC; e += kChunkThreads) Ss[e / NC][e % NC] = Sh[(size_t)(e / NC) * D + c0 + e % NC];

    const int n_chunks = (p.n_tokens + C - 1) / C;
    // DMA: instruction k of wave w fills LDS bytes [1 KB (8 w + k), +1 KB): lane l
    // writes row 2 (8 w + k) + l / 32, position l % 32, which holds chunk
    // (l % 32) ^ (row & 15) of that row.
    int dma_off[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int r = 2 * (8 * wave + k) + (lane >> 5);
        dma_off[k] = (r * RQ + ((lane & 31) ^ (r & 15))) * 16;
    }
    auto dma_wq = [&](int c) {
        const float* ws = p.ws + ((size_t)c * H + h) * ChunkWs<D>::SIZE;
        const __amdgpu_buffer_rsrc_t rw = dn_rsrc(ws + ChunkWs<D>::W);
        const __amdgpu_buffer_rsrc_t rq = dn_rsrc(ws + ChunkWs<D>::QG);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            dn_dma16(rw, Wl + (8 * wave + k) * 256, dma_off[k]);
            dn_dma16(rq, Ql + (8 * wave + k) * 256, dma_off[k]);
        }
    };
    if (n_chunks > 0) dma_wq(0);

    const int ta = tid >> 2;          // phases A/B: row t
    const int ia = tid & 3;           //             column
    const int jc = tid >> 1;          // phase C: state row j (D = 128 rows over 256 threads / 2)
    const int ic = (tid & 1) * (NC / 2);
    const int swa = ta & 15;
    for (int c = 0; c < n_chunks; c++) {
        const float* ws = p.ws + ((size_t)c * H + h) * ChunkWs<D>::SIZE;
        dn_wait_vmem();   // this thread's part of chunk c's W / Qg is in LDS
        __syncthreads();  // ... everyone's (and the initial Ss)
        // the P and Kd^T rows for phases B and C, U and gamma_last
        float4 kd[C / 4], pr[C / 4];
        {
            const float* kr = ws + ChunkWs<D>::KDT + jc * C;
            const float* prr = ws + ChunkWs<D>::P + ta * C;
#pragma unroll
            for (int u = 0; u < C / 4; u++) {
                kd[u] = *(const float4*)(kr + 4 * u);
                pr[u] = *(const float4*)(prr + 4 * u);
            }
        }
        const float gl = ws[ChunkWs<D>::GL];
        const float u0 = ws[ChunkWs<D>::U + ta * D + c0 + ia];
        // A: Delta[t][i] = U[t][i] - sum_j W[t][j] S[j][i], and the first part of
        //    O[t][i], sum_j Qg[t][j] S[j][i], in the same pass over S
        float acc = 0.0f, acc_o = 0.0f;
#pragma unroll 8
        for (int q = 0; q < RQ; q++) {
            const int pos = (ta * RQ + (q ^ swa)) * 4;
            const float4 w4 = *(const float4*)(Wl + pos);
            const float4 q4 = *(const float4*)(Ql + pos);
            const int j = 4 * q;
            const float s0 = Ss[j][ia], s1 = Ss[j + 1][ia], s2 = Ss[j + 2][ia], s3 = Ss[j + 3][ia];
            acc = fmaf(-w4.x, s0, acc);
            acc = fmaf(-w4.y, s1, acc);
            acc = fmaf(-w4.z, s2, acc);
            acc = fmaf(-w4.w, s3, acc);
            acc_o = fmaf(q4.x, s0, acc_o);
            acc_o = fmaf(q4.y, s1, acc_o);
            acc_o = fmaf(q4.z, s2, acc_o);
            acc_o = fmaf(q4.w, s3, acc_o);
        }
        Dl[ta][ia] = u0 + acc;
        __syncthreads();  // Delta is complete; W / Qg of chunk c are no longer read
        if (c + 1 < n_chunks) dma_wq(c + 1);
        // B: O[t][i] += sum_{s<=t} P[t][s] Delta[s][i]
        {
#pragma unroll
            for (int u = 0; u < C / 4; u++) {
                const float pv[4] = {pr[u].x, pr[u].y, pr[u].z, pr[u].w};
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (4 * u + k <= ta) acc_o = fmaf(pv[k], Dl[4 * u + k][ia], acc_o);
            }
            const int t = c * C + ta;
            if (t < p.n_tokens) p.out[((size_t)t * H + h) * D + c0 + ia] = finite_or_zero(acc_o);
        }
        // C: S'[j][i] = gamma_last S[j][i] + sum_s KdT[j][s] Delta[s][i]
        float nv[NC / 2];
        {
#pragma unroll
            for (int u = 0; u < NC / 2; u++) nv[u] = gl * Ss[jc][ic + u];
#pragma unroll
            for (int q = 0; q < C / 4; q++) {
                const float kv[4] = {kd[q].x, kd[q].y, kd[q].z, kd[q].w};
#pragma unroll
                for (int w = 0; w < 4; w++)
#pragma unroll
                    for (int u = 0; u < NC / 2; u++) nv[u] = fmaf(kv[w], Dl[4 * q + w][ic + u], nv[u]);
            }
        }
        __syncthreads();  // every read of Ss / Dl for this chunk is done
#pragma unroll
        for (int u = 0; u < NC / 2; u++) Ss[jc][ic + u] = nv[u];
    }
    __syncthreads();
    for (int e = tid; e < D * NC; e += kChunkThreads) Sh[(size_t)(e / NC) * D + c0 + e % NC] = Ss[e / NC][e % NC];
}

size_t deltanet_chunked_ws_bytes(int n_tokens, int n_heads, int head_dim, int chunk) {
    if (head_dim != 128 || chunk != kChunk) return 0;
    const size_t n_chunks = (size_t)(n_tokens + kChunk - 1) / kChunk;
    return n_chunks * n_heads * ChunkWs<128>::SIZE * sizeof(float);
}

hipError_t launch_deltanet_scan(const DeltaNetLaunch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    if (p.head_dim != 128) return hipErrorInvalidValue;
    dim3 grid(128 / kStepCols, p.n_heads);
    deltanet_step_kernel<128><<<grid, kStepThreads, 0, st>>>(p);
    return hipGetLastError();
}

hipError_t launch_deltanet_chunked(const DeltaNetLaunch& p, hipStream_t st) {
    if (p.n_tokens <= 0) return hipSuccess;
    if (p.head_dim != 128) return hipErrorInvalidValue;
    constexpr int D = 128;
    constexpr size_t lds = (size_t)(2 * kChunk * (D + 4) + kChunk * (kChunk + 4) + 5 * kChunk) * sizeof(float);
    hipError_t ea = hipFuncSetAttribute((const void*)deltanet_chunk_prep_kernel<D>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (ea != hipSuccess) return ea;
    const int n_chunks = (p.n_tokens + kChunk - 1) / kChunk;
    deltanet_chunk_prep_kernel<D><<<dim3(n_chunks, p.n_heads), kChunkThreads, lds, st>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    deltanet_chunk_scan_kernel<D><<<dim3(p.n_heads, D / kScanCols), kChunkThreads, 0, st>>>(p);
    return hipGetLastError();
}

}  // namespace gr
