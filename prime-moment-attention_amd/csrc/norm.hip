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
// stored.  Without LayerNorm parameters only the scale is applied.
// A row is 128 B (16-bit types: 8 lanes x 16 B) or 256 B (fp32: 16 lanes x
// 16 B); a wave covers 8 or 4 rows per load and holds kHeadNormBatch such
// loads in flight; rows are visited in (b, l, h) order, so a wave walks
// consecutive memory for the projection layout [B, L, H, D].
constexpr int kHeadNormBatch = 4;

template <int DT>
__global__ __launch_bounds__(256) void head_layernorm_kernel(const HeadNormArgs a) {
    constexpr int es = DT == PRIME_F32 ? 4 : 2;
    constexpr int VE = 16 / es;             // elements per lane
    constexpr int LPR = kD / VE;            // lanes per row
    constexpr int RPW = kWave / LPR;        // rows per wave per load
    const uint32_t rows = static_cast<uint32_t>(a.B) * a.L * a.H;
    const int lane = threadIdx.x & 63, sub = lane % LPR;
    const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
    float w[VE], bb[VE];
    // a power-of-two scale folds into the weight and bias (pow2_scale): one
    // rounding, the same bits (fp16 keeps both: its exponent range is narrower)
    const bool fold = a.weight && DT != PRIME_F16 && pow2_scale(a.scale);
    const float scale = fold ? 1.0f : a.scale;
    if (a.weight) {
#pragma unroll
        for (int e = 0; e < VE; ++e) {
            w[e] = (fold ? a.scale : 1.0f) * load_elem(a.weight, VE * sub + e, a.dt_norm);
            bb[e] = (fold ? a.scale : 1.0f) * load_elem(a.bias, VE * sub + e, a.dt_norm);
        }
    }
    uint4 raw[kHeadNormBatch];
    int64_t oo[kHeadNormBatch];
    bool live[kHeadNormBatch];
#pragma unroll
    for (int i = 0; i < kHeadNormBatch; ++i) {
        const uint32_t r = (wave * kHeadNormBatch + i) * RPW + lane / LPR;
        live[i] = r < rows;
        const uint32_t rr = live[i] ? r : 0u;
        const uint32_t h = rr % static_cast<uint32_t>(a.H), bl = rr / static_cast<uint32_t>(a.H);
        const uint32_t l = bl % static_cast<uint32_t>(a.L), b = bl / static_cast<uint32_t>(a.L);
        const int64_t xo = b * a.x_sb + h * a.x_sh + l * a.x_sl + VE * sub;
        oo[i] = b * a.o_sb + h * a.o_sh + l * a.o_sl + VE * sub;
        raw[i] = *reinterpret_cast<const uint4 *>(static_cast<const char *>(a.x) + xo * es);
    }
#pragma unroll
    for (int i = 0; i < kHeadNormBatch; ++i) {
        float v[VE];
        const uint32_t wd[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
        for (int e = 0; e < VE; ++e) {
            if constexpr (DT == PRIME_F32) v[e] = __uint_as_float(wd[e]);
            else v[e] = Group<DT>::to_f(e & 1 ? wd[e >> 1] >> 16 : wd[e >> 1] & 0xffffu);
        }
        if (a.weight) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < VE; ++e) s += v[e];
#pragma unroll
            for (int o = LPR / 2; o >= 1; o >>= 1) s += __shfl_xor(s, o, kWave);
            const float mean = s * (1.0f / kD);
            float q = 0.f;
#pragma unroll
            for (int e = 0; e < VE; ++e) { v[e] -= mean; q += v[e] * v[e]; }
#pragma unroll
            for (int o = LPR / 2; o >= 1; o >>= 1) q += __shfl_xor(q, o, kWave);
            // v_rsq_f32 (as the prefill's QK-norm on load, which must give the same bits)
            const float rs = __builtin_amdgcn_rsqf(q * (1.0f / kD) + a.ln_eps);
#pragma unroll
            for (int e = 0; e < VE; ++e) v[e] = Group<DT>::round(fmaf(v[e] * rs, w[e], bb[e]));
        }
        if (scale != 1.0f) {
#pragma unroll
            for (int e = 0; e < VE; ++e) v[e] = Group<DT>::round(v[e] * scale);
        }
        uint4 o;
        if constexpr (DT == PRIME_F32) {
            o = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
        } else {
            uint32_t p[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) p[e] = Group<DT>::to_b(v[2 * e]) | (Group<DT>::to_b(v[2 * e + 1]) << 16);
            o = make_uint4(p[0], p[1], p[2], p[3]);
        }
        if (live[i]) *reinterpret_cast<uint4 *>(static_cast<char *>(a.out) + oo[i] * es) = o;
    }
}

// Exact (erf) GELU, y = x * 0.5 * (1 + erf(x / sqrt(2))) in fp32, rounded once to
// the dtype: the MLP activation of primelm_50m.py:64 (nn.GELU()).  Workgroup b
// owns the 16-byte groups [1024 b, 1024 (b + 1)), four per lane at a stride of
// 256 groups, all four loads issued before the first store (measured faster
// than a grid-stride loop over a capped grid); the elements past the last whole
// 16-byte group go to one lane each of workgroup 0.  y may be x.
constexpr int kGeluGroups = 4;  // 16-byte groups per lane
template <int DT>
__global__ __launch_bounds__(256) void gelu_kernel(const void *x, void *y, int64_t n) {
    constexpr int E = DT == PRIME_F32 ? 4 : 8;  // elements per 16 bytes
    const int64_t groups = n / E;
    auto act = [](float v) { return v * 0.5f * (1.0f + erff(v * 0.70710678118654752f)); };
    auto conv = [&](uint4 r) {
        if constexpr (DT == PRIME_F32) {
            return make_uint4(__float_as_uint(act(__uint_as_float(r.x))), __float_as_uint(act(__uint_as_float(r.y))),
                              __float_as_uint(act(__uint_as_float(r.z))), __float_as_uint(act(__uint_as_float(r.w))));
        } else {
            uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = Group<DT>::to_b(act(Group<DT>::to_f(w[e] & 0xffffu)));
                const uint32_t hi = Group<DT>::to_b(act(Group<DT>::to_f(w[e] >> 16)));
                w[e] = lo | (hi << 16);
            }
            return make_uint4(w[0], w[1], w[2], w[3]);
        }
    };
    const uint4 *xs = static_cast<const uint4 *>(x);
    uint4 *ys = static_cast<uint4 *>(y);
    const int64_t g0 = static_cast<int64_t>(blockIdx.x) * 256 * kGeluGroups + threadIdx.x;
    uint4 r[kGeluGroups];
#pragma unroll
    for (int u = 0; u < kGeluGroups; ++u)
        if (g0 + 256 * u < groups) r[u] = xs[g0 + 256 * u];
#pragma unroll
    for (int u = 0; u < kGeluGroups; ++u)
        if (g0 + 256 * u < groups) ys[g0 + 256 * u] = conv(r[u]);
    // the tail: fewer than E elements
    const int64_t t = groups * E + threadIdx.x;
    if (blockIdx.x == 0 && t < n) {
        if constexpr (DT == PRIME_F32) {
            static_cast<float *>(y)[t] = act(static_cast<const float *>(x)[t]);
        } else {
            const uint16_t b = static_cast<const uint16_t *>(x)[t];
            static_cast<uint16_t *>(y)[t] = static_cast<uint16_t>(Group<DT>::to_b(act(Group<DT>::to_f(b))));
        }
    }
}

hipError_t launch_gelu(const void *x, void *y, int64_t n, int dt, hipStream_t stream) {
    const int64_t groups = n / (dt == PRIME_F32 ? 4 : 8);
    const int64_t per = 256 * kGeluGroups;
    const int64_t blocks = (groups + per - 1) / per;
    if (blocks >= (int64_t(1) << 31)) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(blocks < 1 ? 1 : blocks)), block(256);
    if (dt == PRIME_BF16) hipLaunchKernelGGL(gelu_kernel<PRIME_BF16>, grid, block, 0, stream, x, y, n);
    else if (dt == PRIME_F16) hipLaunchKernelGGL(gelu_kernel<PRIME_F16>, grid, block, 0, stream, x, y, n);
    else hipLaunchKernelGGL(gelu_kernel<PRIME_F32>, grid, block, 0, stream, x, y, n);
    return hipGetLastError();
}

// Selective PRIME's per-token log decays from the step-size pre-activations
// s = delta_proj(x) (selective.py:368, 386): Delta = clamp(softplus(s)), each
// stage rounded to s's dtype as the module's tensors hold it, then
// log_decay[b, h, t] = -Delta / tau[h] in fp32.  One thread per (sequence,
// group of 4 heads, token), consecutive threads on consecutive tokens, so each
// head's stores are coalesced; the 4 loads carry no branch (an index past
// H - 1 re-reads head H - 1) and are all in flight before the first is used.
constexpr int kDecayHeads = 4;
template <int DT>
__global__ __launch_bounds__(256) void selective_log_decay_kernel(const void *__restrict__ step, int64_t sb,
                                                                  int64_t sl, const float *__restrict__ tau,
                                                                  float dmin, float dmax, int H, int L, int HG,
                                                                  int64_t n, float *__restrict__ out) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (r >= n) return;
    const int64_t bg = r / L, t = r - bg * L;
    const int64_t b = bg / HG;
    const int h0 = static_cast<int>(bg - b * HG) * kDecayHeads;
    auto rnd = [](float x) {
        if constexpr (DT == PRIME_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
        else if constexpr (DT == PRIME_F16) return h16_bits_to_f32(f32_to_h16_bits(x));
        else return x;
    };
    auto ld = [&](int64_t i) {
        if constexpr (DT == PRIME_F32) return static_cast<const float *>(step)[i];
        else if constexpr (DT == PRIME_BF16) return bf16_bits_to_f32(static_cast<const uint16_t *>(step)[i]);
        else return h16_bits_to_f32(static_cast<const uint16_t *>(step)[i]);
    };
    const int64_t src = b * sb + t * sl;
    float sv[kDecayHeads];
#pragma unroll
    for (int j = 0; j < kDecayHeads; ++j) sv[j] = ld(src + min(h0 + j, H - 1));
#pragma unroll
    for (int j = 0; j < kDecayHeads; ++j) {
        if (h0 + j < H) {
            const float s = sv[j];
            float d = rnd(s > 20.f ? s : log1pf(expf(s)));  // softplus (threshold 20, as torch)
            d = rnd(fminf(fmaxf(d, dmin), dmax));
            out[(b * H + h0 + j) * L + t] = -d / tau[h0 + j];
        }
    }
}

hipError_t launch_selective_log_decay(const void *step, int dt, int64_t sb, int64_t sl, const float *tau, float dmin,
                                      float dmax, int B, int H, int L, float *out, hipStream_t stream) {
    const int HG = (H + kDecayHeads - 1) / kDecayHeads;
    const int64_t n = static_cast<int64_t>(B) * HG * L;
    const int64_t blocks = (n + 255) / 256;
    if (blocks >= (int64_t(1) << 31)) return hipErrorInvalidValue;
    const dim3 g(static_cast<unsigned>(blocks)), blk(256);
    if (dt == PRIME_BF16)
        hipLaunchKernelGGL(selective_log_decay_kernel<PRIME_BF16>, g, blk, 0, stream, step, sb, sl, tau, dmin, dmax,
                           H, L, HG, n, out);
    else if (dt == PRIME_F16)
        hipLaunchKernelGGL(selective_log_decay_kernel<PRIME_F16>, g, blk, 0, stream, step, sb, sl, tau, dmin, dmax, H,
                           L, HG, n, out);
    else
        hipLaunchKernelGGL(selective_log_decay_kernel<PRIME_F32>, g, blk, 0, stream, step, sb, sl, tau, dmin, dmax, H,
                           L, HG, n, out);
    return hipGetLastError();
}

hipError_t launch_head_layernorm(const HeadNormArgs &a, hipStream_t stream) {
    const uint32_t rows = static_cast<uint32_t>(a.B) * a.L * a.H;
    const uint32_t per_block = 4u * kHeadNormBatch * (a.dt == PRIME_F32 ? 4u : 8u);  // 4 waves
    const dim3 grid((rows + per_block - 1) / per_block), block(256);
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
