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

// The value of lane l ^ W, by register moves: DPP within rows of 16 lanes (quad
// permutes, half-row and row mirrors: l ^ 4 = half_mirror(l ^ 3), l ^ 8 =
// row_mirror(l ^ 7)) and the row / half swaps across them.
template <int W>
__device__ __forceinline__ float lane_xor(float x) {
    const int v = __float_as_int(x);
    if constexpr (W == 1) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    } else if constexpr (W == 2) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    } else if constexpr (W == 4) {
        const int t = __builtin_amdgcn_mov_dpp(v, 0x1B, 0xF, 0xF, false);       // quad_perm [3,2,1,0]
        return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x141, 0xF, 0xF, false));  // row_half_mirror
    } else if constexpr (W == 8) {
        const int t = __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);      // row_half_mirror
        return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x140, 0xF, 0xF, false));  // row_mirror
    } else if constexpr (W == 16) {
        // rows (0, 1) and (2, 3) swap: r[0] holds the even rows twice, r[1] the odd ones
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
    } else {
        static_assert(W == 32, "lane_xor: 1, 2, 4, 8, 16 or 32");
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
    }
}

// LDS stores of this wave complete and visible to its own lanes (no workgroup barrier)
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

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
template <int D, int W>
__device__ __forceinline__ void wave_fwht_stage(float (&x)[D / 64], int lane) {
#pragma unroll
    for (int j = 0; j < D / 64; j++) {
        const float p = lane_xor<W>(x[j]);
        x[j] = (lane & W) ? p - x[j] : x[j] + p;  // lower a+b, upper a-b
    }
}

template <int D>
__device__ __forceinline__ void wave_fwht(float (&x)[D / 64], int lane) {
    wave_fwht_stage<D, 1>(x, lane);
    wave_fwht_stage<D, 2>(x, lane);
    wave_fwht_stage<D, 4>(x, lane);
    wave_fwht_stage<D, 8>(x, lane);
    wave_fwht_stage<D, 16>(x, lane);
    wave_fwht_stage<D, 32>(x, lane);
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
