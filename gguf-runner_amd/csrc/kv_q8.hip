// Q8 KV-cache write: kv_write_token's KvCacheFormat::Q8 branch
// (reference inference.rs:1886-1917) over a batch of rows.
//
// quantize_row_q8 (inference.rs:249-268, x86 branch) on each row (row mode)
// or each 32-element block (GGUF_Q8_BLOCK_SCALES):
//   amax = max |x|;  amax == 0 -> scale 1, codes 0
//   scale = amax / 127;  code = clamp(round_half_away(x * (127 / amax)), -127, 127)
// Both divisions are IEEE round-to-nearest, so codes and scales are bit-exact
// with the reference for the same f32 input.
//
// One workgroup per (row, K|V); each lane owns 8 consecutive elements (one
// 8-byte store), so a 32-element block is 4 adjacent lanes.
#include "gr_common.hpp"
#include "gr_internal.hpp"

namespace gr {

constexpr int kQ8Threads = 256;

__device__ __forceinline__ int8_t q8_code(float x, float inv) {
    float r = roundf(x * inv);  // half away from zero, as Rust f32::round
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)(int)r;  // NaN converts to 0, as Rust's saturating `as i8`
}

__global__ __launch_bounds__(kQ8Threads) void q8_write_kernel(const Q8WriteLaunch p) {
    __shared__ float red[kQ8Threads / 64];
    const int i = blockIdx.x;
    const bool is_v = blockIdx.y != 0;
    const float* src = (is_v ? p.v_rows : p.k_rows) + (size_t)i * p.kv_dim;
    const int64_t row = p.cache_row ? (int64_t)p.cache_row[i] : p.row0 + i;
    const int64_t sq = p.cache_seq ? (int64_t)p.cache_seq[i] : 0;
    int8_t* dst = (is_v ? p.v_cache : p.k_cache) + sq * p.cache_seq_stride + row * p.cache_row_stride;
    float* sc = (is_v ? p.v_scale : p.k_scale) + sq * p.scale_seq_stride + row * p.scale_row_stride;
    const int n8 = p.kv_dim / 8;
    const int tid = threadIdx.x;

    float amax_row = 0.0f;
    if (!p.block) {
        for (int c = tid; c < n8; c += kQ8Threads) {
            const float4 a = *(const float4*)(src + 8 * c);
            const float4 b = *(const float4*)(src + 8 * c + 4);
            amax_row = fmaxf(amax_row, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
            amax_row = fmaxf(amax_row, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
        }
        amax_row = wave_max<64>(amax_row);
        if ((tid & 63) == 0) red[tid >> 6] = amax_row;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < kQ8Threads / 64; w++) amax_row = fmaxf(amax_row, red[w]);
        if (tid == 0) sc[0] = amax_row == 0.0f ? 1.0f : __fdiv_rn(amax_row, 127.0f);
    }
    for (int c = tid; c < n8; c += kQ8Threads) {
        const float4 a = *(const float4*)(src + 8 * c);
        const float4 b = *(const float4*)(src + 8 * c + 4);
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float amax = amax_row;
        if (p.block) {
            amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(x[e]));
            // the 4 lanes of a 32-element block are lanes 4k..4k+3 of this pass
            amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
            if ((c & 3) == 0) sc[c >> 2] = amax == 0.0f ? 1.0f : __fdiv_rn(amax, 127.0f);
        }
        uint32_t w0 = 0, w1 = 0;
        if (amax != 0.0f) {
            const float inv = __fdiv_rn(127.0f, amax);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                w0 |= (uint32_t)(uint8_t)q8_code(x[e], inv) << (8 * e);
                w1 |= (uint32_t)(uint8_t)q8_code(x[e + 4], inv) << (8 * e);
            }
        }
        *(uint2*)(dst + 8 * c) = make_uint2(w0, w1);
    }
}

hipError_t launch_q8_write(const Q8WriteLaunch& p, hipStream_t st) {
    if (p.n_rows <= 0) return hipSuccess;
    if (p.kv_dim <= 0 || p.kv_dim % 32 != 0) return hipErrorInvalidValue;
    q8_write_kernel<<<dim3((unsigned)p.n_rows, 2), kQ8Threads, 0, st>>>(p);
    return hipGetLastError();
}

}  // namespace gr
