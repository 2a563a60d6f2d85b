// Shared device helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gr_attn.h"

namespace gr {

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- element types
// KV / activation storage is handled as raw bit patterns; these tags select the
// conversion.  f16 uses the hardware cvt, bf16 is the upper half of an f32.
struct F32 {
    using storage = float;
    static constexpr int bytes = 4;
};
struct F16 {
    using storage = uint16_t;
    static constexpr int bytes = 2;
};
struct BF16 {
    using storage = uint16_t;
    static constexpr int bytes = 2;
};

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}
// Round-to-nearest-even, like gguf.rs fp32_to_fp16 / fp32_to_bf16.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

// A bf16 value whose f16 conversion is not exact or not finite: |x| >= 2^16
// (f16's largest finite value is 65504; bf16 has nothing between 65280 and
// 65536), inf or NaN.  Below f16's normal range the conversion rounds to a
// multiple of 2^-24, an absolute change under 2^-25.
__device__ __forceinline__ bool bf16_outside_f16(uint16_t b) { return (b & 0x7fffu) >= 0x4780u; }

// Two floats as a bf16 pair (low half = lo) with one v_cvt_pk_bf16_f32 (round to
// nearest even, as f32_to_bf16 for finite values); for MFMA operands.
typedef __bf16 gr_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float gr_f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(gr_f32x2_t{lo, hi}, gr_bf16x2_t));
}

template <typename T>
__device__ __forceinline__ float to_f32(typename T::storage v);
template <>
__device__ __forceinline__ float to_f32<F32>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<F16>(uint16_t v) { return f16_to_f32(v); }
template <>
__device__ __forceinline__ float to_f32<BF16>(uint16_t v) { return bf16_to_f32(v); }

template <typename T>
__device__ __forceinline__ typename T::storage from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<F32>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t from_f32<F16>(float v) { return f32_to_f16(v); }
template <>
__device__ __forceinline__ uint16_t from_f32<BF16>(float v) { return f32_to_bf16(v); }

// Unpack a 16-byte vector of T into floats (16/bytes of them).
template <typename T>
__device__ __forceinline__ void unpack16(const uint4& u, float* out);
template <>
__device__ __forceinline__ void unpack16<F32>(const uint4& u, float* out) {
    out[0] = __uint_as_float(u.x);
    out[1] = __uint_as_float(u.y);
    out[2] = __uint_as_float(u.z);
    out[3] = __uint_as_float(u.w);
}
template <>
__device__ __forceinline__ void unpack16<F16>(const uint4& u, float* out) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        out[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffffu));
        out[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
    }
}
template <>
__device__ __forceinline__ void unpack16<BF16>(const uint4& u, float* out) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

// ---------------------------------------------------------------- wave helpers
__device__ __forceinline__ float shfl_xor(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

template <int WIDTH>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = WIDTH / 2; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}

template <int WIDTH>
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = WIDTH / 2; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ bool is_finite_f(float x) {
    return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u;
}
__device__ __forceinline__ float finite_or_zero(float x) { return is_finite_f(x) ? x : 0.0f; }

// sigmoid_mul_inplace for one element (math.rs:396-403, the x86 branch):
// x * (1 / (1 + exp(-g))), non-finite results to 0.
__device__ __forceinline__ float gate_mul(float x, float g) {
    const float s = 1.0f / (1.0f + expf(-g));
    return finite_or_zero(x * s);
}

}  // namespace gr
