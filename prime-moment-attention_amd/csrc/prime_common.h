// Shared device helpers for the gfx950 PRIME kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "prime_mi355x.h"

namespace prime {

constexpr int kD = 64;      // head dim supported by the kernels
constexpr int kWave = 64;   // CDNA wavefront

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// round-to-nearest-even float -> bf16 bits (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// s = 2^e for a normal exponent: then round(round(x) * s) == round(x * s) for
// the fp32 and bf16 roundings (scaling by s is exact in both, whose exponent
// ranges are the same), so a scale can be folded into the operands before the
// one rounding
__device__ __forceinline__ bool pow2_scale(float s) {
    const uint32_t u = __float_as_uint(s) & 0x7FFFFFFFu;
    return (u & 0x007FFFFFu) == 0u && u >= 0x00800000u && u < 0x7F800000u;
}

__device__ __forceinline__ float h16_bits_to_f32(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

__device__ __forceinline__ uint16_t f32_to_h16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// load one element of dtype `dt` as fp32
__device__ __forceinline__ float load_elem(const void *p, int64_t idx, int dt) {
    if (dt == PRIME_BF16) return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[idx]);
    if (dt == PRIME_F16) return h16_bits_to_f32(static_cast<const uint16_t *>(p)[idx]);
    return static_cast<const float *>(p)[idx];
}

__device__ __forceinline__ void store_elem(void *p, int64_t idx, int dt, float x) {
    if (dt == PRIME_BF16) static_cast<uint16_t *>(p)[idx] = f32_to_bf16_bits(x);
    else if (dt == PRIME_F16) static_cast<uint16_t *>(p)[idx] = f32_to_h16_bits(x);
    else static_cast<float *>(p)[idx] = x;
}

// x of lane (lane ^ M), M = 8, 4, 2 or 1 (the partner within the lane's row of
// 16), by DPP moves on the VALU instead of a shuffle through the LDS unit.
// M = 8 and 4 combine row_shl:M (lanes whose partner is above) and row_shr:M
// (below) through bank masks (banks are groups of 4 lanes); M = 2 and 1 are
// quad permutations.
template <int M>
__device__ __forceinline__ float xor_lane(float x) {
    const int v = __float_as_int(x);
    if constexpr (M == 8) {
        int t = __builtin_amdgcn_update_dpp(0, v, 0x108, 0xF, 0x3, false);  // row_shl:8, lanes 0-7
        t = __builtin_amdgcn_update_dpp(t, v, 0x118, 0xF, 0xC, false);      // row_shr:8, lanes 8-15
        return __int_as_float(t);
    } else if constexpr (M == 4) {
        int t = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0x5, false);  // row_shl:4, lanes 0-3 / 8-11
        t = __builtin_amdgcn_update_dpp(t, v, 0x114, 0xF, 0xA, false);      // row_shr:4, lanes 4-7 / 12-15
        return __int_as_float(t);
    } else if constexpr (M == 2) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    } else {
        static_assert(M == 1, "partners at 8, 4, 2, 1");
        return __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    }
}

// x + x of lane (lane ^ 16), or (lane ^ 32), on the VALU: a v_permlane16_swap /
// v_permlane32_swap of x with itself leaves, in every lane, its own x in one
// result and its partner's in the other, so their sum is the pair's sum.
__device__ __forceinline__ float sum_lane16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_lane32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 64 lanes, in every lane: the butterfly x + x(lane ^ o) for
// o = 32, 16, 8, 4, 2, 1 (the order of a shuffle-based butterfly, so the
// result is the same), all on the VALU (permlane swaps and DPP) rather than
// through the LDS unit.
__device__ __forceinline__ float wave_sum(float x) {
    x = sum_lane32(x);
    x = sum_lane16(x);
    x += xor_lane<8>(x);
    x += xor_lane<4>(x);
    x += xor_lane<2>(x);
    x += xor_lane<1>(x);
    return x;
}

// Argmax candidate as one 64-bit key: an order-preserving image of the value in
// the high word (NaN -> all ones, -0 folded onto +0) and ~index in the low
// word, so the larger key is the larger value and, among equal values, the
// smaller index (torch.argmax's first maximal index, NaN counting as largest).
__device__ __forceinline__ uint64_t argmax_key(float f, uint32_t idx) {
    uint32_t k;
    if (f != f) {
        k = 0xffffffffu;
    } else {
        if (f == 0.f) f = 0.f;  // -0 and +0 compare equal
        const uint32_t b = __float_as_uint(f);
        k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    return (static_cast<uint64_t>(k) << 32) | static_cast<uint64_t>(~idx);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Element (r, k) of a bf16 matrix in the fragment layout of the decode step's
// projections: 16 x 32 blocks in row-block-major order (KS = K / 32 blocks per
// block row), each block the 64 lane slots of 8 elements of one MFMA operand
// (slot = r % 16 + 16 * ((k % 32) / 8)).
__device__ __forceinline__ int64_t frag_index(int r, int k, int KS) {
    return (static_cast<int64_t>(r >> 4) * KS + (k >> 5)) * 512 + ((r & 15) + 16 * ((k & 31) >> 3)) * 8 + (k & 7);
}

}  // namespace prime
