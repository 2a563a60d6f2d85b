// Device helpers shared by the Turbo KV kernels (turbo.hip, turbo_decode.hip):
// the format's constants and the wave-held sign flips / FWHT of one head.
//
// A head of D (64, 128, 256) elements lives in a wave as x[j] = element
// lane + 64 j.  The FWHT runs its widths in the reference's order (1, 2, 4, ...:
// lanes via shuffles, then within the lane), so the rotated values are those of
// turboquant_fwht_inplace_scalar (inference.rs:681-701) bit for bit (adds and
// subtracts only, then one scaling multiply).
#pragma once

#include "gr_common.hpp"

namespace gr {
namespace tq {

constexpr float kC0 = 0.45278f;    // TURBOQUANT_CENTROIDS, inference.rs:349
constexpr float kC1 = 1.510417f;
constexpr float kTh = 0.9815985f;  // TURBOQUANT_THRESHOLD_HI, inference.rs:351
constexpr float kFracPi2 = 1.5707964f;

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

// turboquant_transform_with_bits (inference.rs:596-605): signs, FWHT, signs
template <int D>
__device__ __forceinline__ void wave_transform(float (&x)[D / 64], const uint8_t* first, const uint8_t* second,
                                               int lane) {
    wave_signs<D>(x, first, lane);
    wave_fwht<D>(x, lane);
    wave_signs<D>(x, second, lane);
}

// Power of two 2^k with vmax * 2^k in [2^(top-1), 2^top); 1 for vmax <= 0.
__device__ __forceinline__ float pow2_for(float vmax, int top) {
    int ex;
    (void)frexpf(vmax, &ex);  // vmax = m 2^ex, m in [0.5, 1)
    return vmax > 0.0f ? ldexpf(1.0f, min(max(top - ex, -120), 120)) : 1.0f;
}

}  // namespace tq
}  // namespace gr
