// kvrt_device.h — device-side helpers shared by the kvrt HIP kernels (gfx950).
//
// bf16 is carried as raw uint16_t bits: widening is a 16-bit shift and
// narrowing is round-to-nearest-even on the bit pattern, so every bitwise
// cache operation is exact and reproducible on the CPU oracle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvrt {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// fp32 -> bf16, round to nearest even; NaN kept quiet.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Dot of two packed bf16 pairs accumulated in fp32 (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// ---- wave64 cross-lane exchange ------------------------------------------
// DPP controls: quad_perm xor1 = [1,0,3,2] = 0xB1, xor2 = [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141 (lane i <- 7-i within 8), row_mirror = 0x140
// (lane i <- 15-i within 16), row_ror:8 = 0x128 (lane i <- i^8 within 16).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Exact lane exchange with lane ^ MASK (MASK a power of two < 64).
template <int MASK>
__device__ __forceinline__ float xor_lane(float x) {
    if constexpr (MASK == 1) return dpp<0xB1>(x);
    else if constexpr (MASK == 2) return dpp<0x4E>(x);
    else if constexpr (MASK == 8) return dpp<0x128>(x);
    else if constexpr (MASK == 16)
        // ds_swizzle bit mode: and 0x1F, or 0, xor 0x10 (within 32 lanes).
        return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
    else
        return __shfl_xor(x, MASK, 64);
}

// Sum over aligned groups of G lanes (G in 1..64, power of two). Every lane
// of a group ends with the group total. Uses mirrors for 4 and 8/16, which
// pair the two halves of the group just as xor does.
template <int G>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (G >= 2) x += dpp<0xB1>(x);
    if constexpr (G >= 4) x += dpp<0x4E>(x);
    if constexpr (G >= 8) x += dpp<0x141>(x);
    if constexpr (G >= 16) x += dpp<0x140>(x);
    if constexpr (G >= 32) x += xor_lane<16>(x);
    if constexpr (G >= 64) x += xor_lane<32>(x);
    return x;
}

template <int G>
__device__ __forceinline__ float group_max(float x) {
    if constexpr (G >= 2) x = fmaxf(x, dpp<0xB1>(x));
    if constexpr (G >= 4) x = fmaxf(x, dpp<0x4E>(x));
    if constexpr (G >= 8) x = fmaxf(x, dpp<0x141>(x));
    if constexpr (G >= 16) x = fmaxf(x, dpp<0x140>(x));
    if constexpr (G >= 32) x = fmaxf(x, xor_lane<16>(x));
    if constexpr (G >= 64) x = fmaxf(x, xor_lane<32>(x));
    return x;
}

// Combine lanes that are STRIDE apart, for strides STRIDE, 2*STRIDE, ... < 64
// (the key sub-groups of one wave, which hold the same head dims).
template <int STRIDE>
__device__ __forceinline__ float strided_sum(float x) {
    if constexpr (STRIDE < 64) {
        x += xor_lane<STRIDE>(x);
        if constexpr (STRIDE * 2 < 64) x = strided_sum<STRIDE * 2>(x);
    }
    return x;
}
template <int STRIDE>
__device__ __forceinline__ float strided_max(float x) {
    if constexpr (STRIDE < 64) {
        x = fmaxf(x, xor_lane<STRIDE>(x));
        if constexpr (STRIDE * 2 < 64) x = strided_max<STRIDE * 2>(x);
    }
    return x;
}

}  // namespace kvrt
