// Residual add + RMSNorm of the PRIME decoder blocks (model.py:47-56, 107-118):
//   x <- x + delta (rounded to x's dtype, as the block's residual add stores it)
//   out <- x * rsqrt(mean(x * x) + eps) * weight
// One wave per row; lane l handles elements 4l + 256i (four at a time).

#include "prime_kernels.h"

namespace prime {

constexpr int kNormWaves = 4;

__global__ __launch_bounds__(kNormWaves * kWave) void add_rmsnorm_kernel(const RmsNormArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * kNormWaves + wave;
    if (row >= a.rows) return;  // whole wave leaves (no block-level barrier below)
    const int64_t base = static_cast<int64_t>(row) * a.hidden;
    const int per = a.hidden / (4 * kWave);  // full passes of 256 elements
    float ss = 0.f;
    // pass 1: add, store x, sum of squares
    for (int i = 0; i <= per; ++i) {
        const int c = 4 * lane + 4 * kWave * i;
        if (c >= a.hidden) break;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float x = load_elem(a.x, base + c + e, a.dt);
            if (a.delta) {
                x += load_elem(a.delta, base + c + e, a.dt);
                store_elem(a.x, base + c + e, a.dt, x);
                x = load_elem(a.x, base + c + e, a.dt);  // the rounded sum
            }
            ss += x * x;
        }
    }
    const float r = rsqrtf(wave_sum(ss) / static_cast<float>(a.hidden) + a.eps);
    // pass 2: normalise (the row is re-read from L1/L2)
    for (int i = 0; i <= per; ++i) {
        const int c = 4 * lane + 4 * kWave * i;
        if (c >= a.hidden) break;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x = load_elem(a.x, base + c + e, a.dt);
            store_elem(a.out, base + c + e, a.dt, x * r * load_elem(a.weight, c + e, a.dt));
        }
    }
}

hipError_t launch_add_rmsnorm(const RmsNormArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((a.rows + kNormWaves - 1) / kNormWaves), dim3(kNormWaves * kWave), 0,
                       stream, a);
    return hipGetLastError();
}

}  // namespace prime
