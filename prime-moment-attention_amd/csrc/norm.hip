// Residual add + RMSNorm of the PRIME decoder blocks (model.py:47-56, 107-118):
//   x <- x + delta (rounded to x's dtype, as the block's residual add stores it)
//   out <- x * rsqrt(mean(x * x) + eps) * weight
// One wave per row, the row held in registers: lane l owns the 4-element
// groups l, l + 64, l + 128, ... (8-byte loads for 16-bit types, 16-byte for
// fp32).  All loads of a row are issued before the first store, so a row costs
// one memory round trip for x/delta/weight and one for the stores.

#include "prime_kernels.h"

namespace prime {

constexpr int kNormWaves = 4;

template <int DT> struct Group;  // 4 consecutive elements of a row

template <> struct Group<PRIME_F32> {
    typedef float4 raw;
    static __device__ __forceinline__ void unpack(const raw &r, float (&f)[4]) {
        f[0] = r.x; f[1] = r.y; f[2] = r.z; f[3] = r.w;
    }
    static __device__ __forceinline__ raw pack(const float (&f)[4]) { return make_float4(f[0], f[1], f[2], f[3]); }
    static __device__ __forceinline__ float round(float x) { return x; }
};

template <int DT> struct Group16 {  // bf16 / fp16, stored as 16-bit patterns
    typedef uint2 raw;
    static __device__ __forceinline__ float to_f(uint32_t b) {
        return DT == PRIME_BF16 ? bf16_bits_to_f32(static_cast<uint16_t>(b)) : h16_bits_to_f32(static_cast<uint16_t>(b));
    }
    static __device__ __forceinline__ uint32_t to_b(float x) {
        return DT == PRIME_BF16 ? f32_to_bf16_bits(x) : f32_to_h16_bits(x);
    }
    static __device__ __forceinline__ void unpack(const raw &r, float (&f)[4]) {
        f[0] = to_f(r.x & 0xffffu); f[1] = to_f(r.x >> 16); f[2] = to_f(r.y & 0xffffu); f[3] = to_f(r.y >> 16);
    }
    static __device__ __forceinline__ raw pack(const float (&f)[4]) {
        return make_uint2(to_b(f[0]) | (to_b(f[1]) << 16), to_b(f[2]) | (to_b(f[3]) << 16));
    }
    static __device__ __forceinline__ float round(float x) { return to_f(to_b(x)); }
};
template <> struct Group<PRIME_BF16> : Group16<PRIME_BF16> {};
template <> struct Group<PRIME_F16> : Group16<PRIME_F16> {};

template <int DT>
__global__ __launch_bounds__(kNormWaves * kWave) void add_rmsnorm_kernel(const RmsNormArgs a) {
    typedef Group<DT> G;
    typedef typename G::raw raw;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int row = blockIdx.x * kNormWaves + wave;
    if (row >= a.rows) return;  // whole wave leaves (no block-level barrier below)
    const int ng = a.hidden >> 2;  // groups per row
    const int64_t base = static_cast<int64_t>(row) * ng;
    raw *xr = static_cast<raw *>(a.x) + base;
    const raw *dr = a.delta ? static_cast<const raw *>(a.delta) + base : nullptr;
    const raw *wr = static_cast<const raw *>(a.weight);
    raw *orow = static_cast<raw *>(a.out) + base;
    raw xs[kNormMaxGroups], ds[kNormMaxGroups], ws[kNormMaxGroups];
#pragma unroll
    for (int i = 0; i < kNormMaxGroups; ++i) {
        const int g = lane + kWave * i;
        if (g < ng) {
            xs[i] = xr[g];
            ws[i] = wr[g];
            if (dr) ds[i] = dr[g];
        }
    }
    float v[kNormMaxGroups][4];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kNormMaxGroups; ++i) {
        const int g = lane + kWave * i;
        if (g < ng) {
            G::unpack(xs[i], v[i]);
            if (dr) {
                float d[4];
                G::unpack(ds[i], d);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[i][e] = G::round(v[i][e] + d[e]);  // the stored sum
                xr[g] = G::pack(v[i]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += v[i][e] * v[i][e];
        }
    }
    const float r = rsqrtf(wave_sum(ss) / static_cast<float>(a.hidden) + a.eps);
#pragma unroll
    for (int i = 0; i < kNormMaxGroups; ++i) {
        const int g = lane + kWave * i;
        if (g < ng) {
            float w[4], o[4];
            G::unpack(ws[i], w);
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = v[i][e] * r * w[e];
            orow[g] = G::pack(o);
        }
    }
}

// Per-head LayerNorm of the module's QK-norm (attention.py:96-101) over rows
// of 64: out = round(round(LN(x)) * scale), biased variance, each rounding to
// the tensor's dtype as the module's LayerNorm output and its scaled copy are
// stored.  Without LayerNorm parameters only the scale is applied.  16 lanes
// per row (4 elements each), 16 rows per 256-thread block; rows are visited
// in (b, l, h) order so that a block walks consecutive memory for the
// projection layout [B, L, H, D].
template <int DT>
__global__ __launch_bounds__(256) void head_layernorm_kernel(const HeadNormArgs a) {
    typedef Group<DT> G;
    typedef typename G::raw raw;
    const int64_t rows = static_cast<int64_t>(a.B) * a.L * a.H;
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    const bool live = r < rows;
    const int64_t rr = live ? r : 0;
    const int h = static_cast<int>(rr % a.H);
    const int64_t bl = rr / a.H;
    const int l = static_cast<int>(bl % a.L), b = static_cast<int>(bl / a.L);
    const raw *xp = reinterpret_cast<const raw *>(static_cast<const char *>(a.x) +
                                                  (b * a.x_sb + h * a.x_sh + l * a.x_sl) * (DT == PRIME_F32 ? 4 : 2));
    float v[4];
    G::unpack(xp[sub], v);
    if (a.weight) {
        float s = v[0] + v[1] + v[2] + v[3];
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, kWave);
        const float mean = s * (1.0f / kD);
        float d[4], q = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) { d[e] = v[e] - mean; q += d[e] * d[e]; }
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) q += __shfl_xor(q, o, kWave);
        const float rs = rsqrtf(q * (1.0f / kD) + a.ln_eps);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = 4 * sub + e;
            v[e] = G::round(d[e] * rs * load_elem(a.weight, c, a.dt_norm) + load_elem(a.bias, c, a.dt_norm));
        }
    }
    if (a.scale != 1.0f) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = G::round(v[e] * a.scale);
    }
    if (live) {
        raw *op = reinterpret_cast<raw *>(static_cast<char *>(a.out) +
                                          (b * a.o_sb + h * a.o_sh + l * a.o_sl) * (DT == PRIME_F32 ? 4 : 2));
        op[sub] = G::pack(v);
    }
}

hipError_t launch_head_layernorm(const HeadNormArgs &a, hipStream_t stream) {
    const int64_t rows = static_cast<int64_t>(a.B) * a.L * a.H;
    const dim3 grid(static_cast<unsigned>((rows + 15) / 16)), block(256);
    if (a.dt == PRIME_BF16) hipLaunchKernelGGL(head_layernorm_kernel<PRIME_BF16>, grid, block, 0, stream, a);
    else if (a.dt == PRIME_F16) hipLaunchKernelGGL(head_layernorm_kernel<PRIME_F16>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(head_layernorm_kernel<PRIME_F32>, grid, block, 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm(const RmsNormArgs &a, hipStream_t stream) {
    const dim3 grid((a.rows + kNormWaves - 1) / kNormWaves), block(kNormWaves * kWave);
    if (a.dt == PRIME_BF16) hipLaunchKernelGGL(add_rmsnorm_kernel<PRIME_BF16>, grid, block, 0, stream, a);
    else if (a.dt == PRIME_F16) hipLaunchKernelGGL(add_rmsnorm_kernel<PRIME_F16>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(add_rmsnorm_kernel<PRIME_F32>, grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace prime
