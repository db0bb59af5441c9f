// Greedy token choice of the PRIME generate loop (model.py:230-231: argmax of
// the last position's logits at temperature 0).  One 1024-thread block per
// sequence row; lanes read 16-byte vectors of the row (8 bf16/fp16 or 4 fp32
// logits), a ragged tail element-wise.  The winner is the first index of the
// largest value, NaN counting as largest, as torch.argmax returns it.
//
// Each candidate is one 64-bit key: an order-preserving image of the value in
// the high word (NaN -> all ones, -0 folded onto +0) and ~index in the low word,
// so the larger key is the larger value and, among equal values, the smaller
// index.  Reductions are plain 64-bit max: lane -> wave (shuffles) -> block (LDS).

#include "prime_kernels.h"

namespace prime {

constexpr int kArgmaxThreads = 1024;

template <int DT>
__device__ __forceinline__ void scan_vector(const uint4 &r, uint32_t j0, uint64_t &best) {
    if constexpr (DT == PRIME_F32) {
        best = max_u64(best, argmax_key(__uint_as_float(r.x), j0));
        best = max_u64(best, argmax_key(__uint_as_float(r.y), j0 + 1));
        best = max_u64(best, argmax_key(__uint_as_float(r.z), j0 + 2));
        best = max_u64(best, argmax_key(__uint_as_float(r.w), j0 + 3));
    } else {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float lo = DT == PRIME_BF16 ? bf16_bits_to_f32(w[e] & 0xffffu) : h16_bits_to_f32(w[e] & 0xffffu);
            const float hi = DT == PRIME_BF16 ? bf16_bits_to_f32(w[e] >> 16) : h16_bits_to_f32(w[e] >> 16);
            best = max_u64(best, argmax_key(lo, j0 + 2 * e));
            best = max_u64(best, argmax_key(hi, j0 + 2 * e + 1));
        }
    }
}

template <int DT>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const ArgmaxArgs a) {
    __shared__ uint64_t red[kArgmaxThreads / kWave];
    constexpr int VE = DT == PRIME_F32 ? 4 : 8;  // elements per 16-byte vector
    constexpr int es = DT == PRIME_F32 ? 4 : 2;
    const int row = blockIdx.x;
    const char *base = static_cast<const char *>(a.logits) + static_cast<int64_t>(row) * a.stride_n * es;
    const int nvec = a.vector ? a.vocab / VE : 0;
    uint64_t best = 0;  // below every key
    const uint4 *vp = reinterpret_cast<const uint4 *>(base);
    constexpr int U = 4;  // vectors in flight per lane
    int i = threadIdx.x;
    for (; i + (U - 1) * kArgmaxThreads < nvec; i += U * kArgmaxThreads) {
        uint4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = vp[i + u * kArgmaxThreads];
#pragma unroll
        for (int u = 0; u < U; ++u) scan_vector<DT>(r[u], static_cast<uint32_t>((i + u * kArgmaxThreads) * VE), best);
    }
    for (; i < nvec; i += kArgmaxThreads) scan_vector<DT>(vp[i], static_cast<uint32_t>(i * VE), best);
    for (int j = nvec * VE + threadIdx.x; j < a.vocab; j += kArgmaxThreads)
        best = max_u64(best, argmax_key(load_elem(base, j, DT), static_cast<uint32_t>(j)));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(best), o, kWave);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(best >> 32), o, kWave);
        best = max_u64(best, (static_cast<uint64_t>(hi) << 32) | lo);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = red[0];
#pragma unroll
        for (int w = 1; w < kArgmaxThreads / kWave; ++w) b = max_u64(b, red[w]);
        a.out[row] = static_cast<int64_t>(~static_cast<uint32_t>(b));
    }
}

hipError_t launch_argmax_rows(const ArgmaxArgs &a, hipStream_t stream) {
    const dim3 grid(a.n), block(kArgmaxThreads);
    if (a.dt == PRIME_BF16) hipLaunchKernelGGL(argmax_rows_kernel<PRIME_BF16>, grid, block, 0, stream, a);
    else if (a.dt == PRIME_F16) hipLaunchKernelGGL(argmax_rows_kernel<PRIME_F16>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(argmax_rows_kernel<PRIME_F32>, grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace prime
