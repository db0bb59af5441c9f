// Shared pieces of the LDS-DMA GEMM kernels (gemm_rows.hip):
// direct-to-LDS loads of row tiles with a 16-byte-segment XOR swizzle, the
// matching operand reads, and small epilogue helpers.
#pragma once

#include "prefill_common.h"

namespace prime {

constexpr int kRK = 64;  // K block (elements): one 128-byte segment row of a stage

// Direct-to-LDS load of `rows` tile rows (a multiple of 8) starting at tile row
// t0: instruction i covers tile rows t0 + 8 i .. +7; lane l lands at LDS segment
// l % 8 of row l / 8 and loads the global segment that belongs there.
// Source rows past rmax re-read row rmax (never stored).
__device__ __forceinline__ void rows_dma(uint16_t *stage, const uint16_t *src, int64_t ld, int r0, int rmax, int t0,
                                         int n, int k0, int lane) {
    for (int i = 0; i < n; ++i) {
        const int rr = t0 + 8 * i + (lane >> 3);
        const int seg = (lane & 7) ^ (rr & 7);
        const int row = min(r0 + rr, rmax);
        const uint16_t *g = src + static_cast<int64_t>(row) * ld + k0 + 8 * seg;
        const uint32_t l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(stage + (t0 + 8 * i) * kRK));
        // asm: the compiler does not track these loads; the K loop's explicit
        // vmcnt waits are the only ones (see gemm_tile.hip).  M0 is set here
        // for each instruction; no compiler-generated code in this kernel uses it.
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(l) : "memory", "m0");
    }
}

__device__ __forceinline__ bf16x8 rfrag(const uint16_t *stage, int row, int seg) {
    return as_bf16x8(*reinterpret_cast<const u32x4 *>(stage + row * kRK + 8 * (seg ^ (row & 7))));
}

__device__ __forceinline__ float sumsq8(bf16x8 v) {
    const u32x4 u = __builtin_bit_cast(u32x4, v);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = __uint_as_float(u[i] << 16), hi = __uint_as_float(u[i] & 0xFFFF0000u);
        s = fmaf(lo, lo, s);
        s = fmaf(hi, hi, s);
    }
    return s;
}

__device__ __forceinline__ float gelu_erf_r(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

__device__ __forceinline__ float bf16r(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

}  // namespace prime
