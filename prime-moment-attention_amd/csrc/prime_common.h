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

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, kWave);
    return x;
}

}  // namespace prime
