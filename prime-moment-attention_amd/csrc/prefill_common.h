// Device helpers shared by the prefill kernels: chunk geometry, bf16 packing,
// the gfx950 MFMA and the LDS operand reads (row reads and ds_read_b64_tr_b16).
#pragma once

#include "prime_kernels.h"

namespace prime {

constexpr int kC = 64;          // tokens per chunk
constexpr int kF = 2 * kD;      // feature width
constexpr int kPW = kF + 8;     // pitch of 128-wide rows read 16 bytes per lane (68 dwords)
// Pitch of rows read with ds_read_b64_tr_b16.  A 16-lane group reads 4
// consecutive rows x 32 contiguous bytes and the next group the next 4 rows: a
// pitch of 72 dwords (8 mod 32 and mod 64) puts 8 consecutive rows' windows on
// disjoint banks.  The fp32 path (two planes per array) uses the tighter 68 /
// 44-dword pitches to fit in LDS.
constexpr int kPT = kF + 16;

typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 r) { return __builtin_bit_cast(bf16x8, r); }

// two floats -> packed bf16 pair (one v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ void unpack8(u32x4 r, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(r[i] << 16);
        f[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
    }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack2(f[2 * i], f[2 * i + 1]);
    return r;
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// An MFMA operand: hi part, plus the lo residual when split (S).
template <bool S>
struct Opnd {
    bf16x8 h, l;
};

template <bool S>
__device__ __forceinline__ f32x4 mma(const Opnd<S> &a, const Opnd<S> &b, f32x4 c) {
    c = mfma(a.h, b.h, c);
    if constexpr (S) {
        c = mfma(a.h, b.l, c);
        c = mfma(a.l, b.h, c);
    }
    return c;
}

// 8 floats -> bf16 hi (and lo residual) packed
template <bool S>
__device__ __forceinline__ void split_pack(const float (&f)[8], u32x4 &hi, u32x4 &lo) {
    hi = pack8(f);
    if constexpr (S) {
        float hf[8], r[8];
        unpack8(hi, hf);
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = f[i] - hf[i];
        lo = pack8(r);
    }
}

// Inclusive prefix sum of x over the 64 lanes on the VALU (DPP): Hillis-Steele
// within each row of 16 lanes (row_shr 1, 2, 4, 8, zero-filled), then the last
// lane of rows 0 and 2 added to rows 1 and 3 (row_bcast:15) and lane 31 added
// to rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ float wave_prefix_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xF, 0xF, true));  // row_shr:1
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xF, 0xF, true));  // row_shr:2
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xF, 0xF, true));  // row_shr:4
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xF, 0xF, true));  // row_shr:8
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xA, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xC, 0xF, false));
    return x;
}

// Sum of x over the 64 lanes, in every lane, on the VALU (DPP and permlane swaps).
__device__ __forceinline__ float wave_sum_valu(float x) {
    x += xor_lane<1>(x);
    x += xor_lane<2>(x);
    x += xor_lane<4>(x);
    x += xor_lane<8>(x);
    return sum_lane32(sum_lane16(x));
}

// 16-byte LDS read
__device__ __forceinline__ u32x4 lds128(const uint16_t *p) { return *reinterpret_cast<const u32x4 *>(p); }

// ds_read_b64_tr_b16 (see the header comment for the lane mapping)
__device__ __forceinline__ uint2 lds_tr(const uint16_t *p) {
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(const_cast<uint16_t *>(p)));
    return __builtin_bit_cast(uint2, v);
}

// operand of 8 consecutive tokens (two transposed 4-token reads) of one column
template <bool S>
__device__ __forceinline__ Opnd<S> tr_op(const uint16_t *p0, const uint16_t *p1, size_t plane) {
    Opnd<S> o;
    const uint2 a = lds_tr(p0), b = lds_tr(p1);
    o.h = as_bf16x8(u32x4{a.x, a.y, b.x, b.y});
    if constexpr (S) {
        const uint2 c = lds_tr(p0 + plane), d = lds_tr(p1 + plane);
        o.l = as_bf16x8(u32x4{c.x, c.y, d.x, d.y});
    }
    return o;
}

template <bool S>
__device__ __forceinline__ Opnd<S> row_op(const uint16_t *p, size_t plane) {
    Opnd<S> o;
    o.h = as_bf16x8(lds128(p));
    if constexpr (S) o.l = as_bf16x8(lds128(p + plane));
    return o;
}

}  // namespace prime
