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

// Two floats to packed bf16 (round to nearest even; v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2v_t));
}

// 16-byte load marked non-temporal (streamed once: K/V rows of a decode).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream16(const void *p) {
    const u32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(x[0], x[1], x[2], x[3]);
}

// Dot of two packed bf16 pairs accumulated in fp32 (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// ---- wave64 cross-lane reductions ------------------------------------------
// pair<OP, M>(x) combines x with the value of lane (lane ^ M), for every lane:
//   M = 1, 2: DPP quad_perm [1,0,3,2] (0xB1) / [2,3,0,1] (0x4E)
//   M = 8:    DPP row_ror:8 (0x128): lane i <- lane i ^ 8 within a row of 16
//   M = 16:   v_permlane16_swap: with both operands = x, the two results hold
//             the even-row and odd-row copies, i.e. x and its lane ^ 16 partner
//   M = 32:   v_permlane32_swap: the same for the two 32-lane halves
//   M = 4:    ds_swizzle xor 4 (rarely used: only group reductions over 8+
//             lanes pass through it, and those use the row mirrors instead)
// All are VALU data-path operations except M = 4.
struct OpSum {
    static __device__ __forceinline__ float f(float a, float b) { return a + b; }
};
struct OpMax {
    static __device__ __forceinline__ float f(float a, float b) { return fmaxf(a, b); }
};

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

template <class OP, int M>
__device__ __forceinline__ float pair(float x) {
    if constexpr (M == 1) return OP::f(x, dpp<0xB1>(x));
    else if constexpr (M == 2) return OP::f(x, dpp<0x4E>(x));
    else if constexpr (M == 8) return OP::f(x, dpp<0x128>(x));
    else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return OP::f(__uint_as_float(r[0]), __uint_as_float(r[1]));
    } else if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return OP::f(__uint_as_float(r[0]), __uint_as_float(r[1]));
    } else {
        static_assert(M == 4, "pair: M must be a power of two below 64");
        return OP::f(x, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x101F)));  // xor 4
    }
}

// Reduction over aligned groups of G lanes (G a power of two, 1..64); every
// lane of a group ends with the group result. Steps 4 and 8 use the row
// mirrors (lane i <- 7 - i within 8, i <- 15 - i within 16): once the
// smaller groups are uniform they pair the two halves exactly as xor does.
template <class OP, int G>
__device__ __forceinline__ float group_reduce(float x) {
    if constexpr (G >= 2) x = pair<OP, 1>(x);
    if constexpr (G >= 4) x = pair<OP, 2>(x);
    if constexpr (G >= 8) x = OP::f(x, dpp<0x141>(x));
    if constexpr (G >= 16) x = OP::f(x, dpp<0x140>(x));
    if constexpr (G >= 32) x = pair<OP, 16>(x);
    if constexpr (G >= 64) x = pair<OP, 32>(x);
    return x;
}
template <int G> __device__ __forceinline__ float group_sum(float x) { return group_reduce<OpSum, G>(x); }
template <int G> __device__ __forceinline__ float group_max(float x) { return group_reduce<OpMax, G>(x); }

// Reduction over the lanes STRIDE, 2*STRIDE, ... apart (the key sub-groups of
// one wave, which hold the same head dims); STRIDE is a power of two.
template <class OP, int STRIDE>
__device__ __forceinline__ float strided_reduce(float x) {
    if constexpr (STRIDE < 64) {
        x = pair<OP, STRIDE>(x);
        if constexpr (STRIDE * 2 < 64) x = strided_reduce<OP, STRIDE * 2>(x);
    }
    return x;
}
template <int S> __device__ __forceinline__ float strided_sum(float x) { return strided_reduce<OpSum, S>(x); }
template <int S> __device__ __forceinline__ float strided_max(float x) { return strided_reduce<OpMax, S>(x); }

// Agent-scope (cross-XCD) coherent accesses. On gfx950 a relaxed agent-scope
// store is written through the XCD's L2 (global_store ... sc1) and a relaxed
// agent-scope load reads past it (global_load ... sc1), so data exchanged
// only through them needs no L2 write-back or invalidate between workgroups,
// only the completion wait of the stores. The single-launch decode merge
// rests on exactly this lowering; the build compiles these helpers alone
// (kvrt_coherence_probe.hip) and refuses a compiler whose lowering differs.
__device__ __forceinline__ void store_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(float2 *p, float2 v) {
    const uint64_t b = (uint64_t)__float_as_uint(v.x) | ((uint64_t)__float_as_uint(v.y) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// N consecutive floats, as 8-byte stores where N is even (dst 8-byte aligned).
template <int N>
__device__ __forceinline__ void store_agent_n(float *dst, const float (&v)[N]) {
    if constexpr (N % 2 == 0) {
#pragma unroll
        for (int e = 0; e < N; e += 2) store_agent(reinterpret_cast<float2 *>(dst + e), make_float2(v[e], v[e + 1]));
    } else {
#pragma unroll
        for (int e = 0; e < N; ++e) store_agent(dst + e, v[e]);
    }
}
// 16 bytes as two 8-byte agent-scope stores: written through the XCD's L2
// instead of left dirty in it. The fused appends' rows use it: no later
// kernel of the step needs them in this L2, and a step of launches that
// leave fewer dirty lines measured shorter (two-model step 601.6 -> 593.3 us).
// Callers load every source first: loads after an atomic store are not moved
// above it, so a load-store-load-store order costs a round trip per row.
__device__ __forceinline__ void store_agent16(void *p, const uint4 &x) {
    uint64_t *d = static_cast<uint64_t *>(p);
    __hip_atomic_store(d, (uint64_t)x.x | ((uint64_t)x.y << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(d + 1, (uint64_t)x.z | ((uint64_t)x.w << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_agent(const float2 *p) {
    const uint64_t b = __hip_atomic_load(reinterpret_cast<uint64_t *>(const_cast<float2 *>(p)), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32)));
}
// Arrival counters of the single-launch merge: an L2 atomic add returning the
// count before it, and the reset by the last arrival.
__device__ __forceinline__ uint32_t arrive_agent(uint32_t *c) {
    return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void clear_agent(uint32_t *c) {
    __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace kvrt
