// Skinny linear layers of the PRIME decode step on gfx950 (model.py:59-68,
// 101-118, 160: the q/k/v, o, MLP and lm_head projections at one token per
// sequence): y[M, N] = epilogue(x[M, K] . w[N, K]^T), bf16 in and out, fp32
// accumulation.  M is the number of sequences (a few hundred at most), so the
// problem is a weight stream with little reuse, and its cost is latency, not
// MFMA throughput.
//
// Mapping.  Each wave accumulates a 32 x 32 output quadrant over its share of
// the 64-wide K blocks with v_mfma_f32_16x16x32_bf16 (2 x 2 tiles); a
// workgroup holds TM x TN quadrants and KS wave groups that split K between
// them, and the partial tiles are summed through LDS before the epilogue.
// Operands go from global memory straight to registers in MFMA layout -- no
// LDS staging:
//   A operand, m-tile t: lane l holds x[m0 + 16t + l%16][k-slots], B operand,
//   n-tile t: w[n0 + 16t + l%16][k-slots], where a lane's eight k-slots of
//   sub-step s (0, 1) in block i are the elements g K/4 + 16 i + 8 s ... +7,
//   g = l/16: lane group g walks the g-th quarter of K, 32 contiguous bytes
//   per row and block.  A and B use the same k permutation, so the
//   contraction is exact.  Spreading one load instruction's 64 segments over
//   16 rows x 4 quarters of K spreads them over the L2 channels; 16 rows at
//   one column offset (a whole 64-wide block per row) would put rows whose
//   stride is a multiple of the channel interleave on a few channels.
// Two blocks are in flight per wave (the next block's loads are issued before
// the current block's MFMAs).  Rows past M or N are clamped on load and
// dropped on store.

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kGT = 32;     // output tile (rows and columns)
constexpr int kGK = 64;     // K block

struct Blk {  // one K block of one wave: 2 m-tiles and 2 n-tiles, 2 sub-steps each
    u32x4 a[2][2], b[2][2];
};

__device__ __forceinline__ void load_blk(Blk &o, const uint16_t *xr0, const uint16_t *xr1, const uint16_t *wr0,
                                         const uint16_t *wr1, int kb) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        o.a[0][s] = *reinterpret_cast<const u32x4 *>(xr0 + kb + 8 * s);
        o.a[1][s] = *reinterpret_cast<const u32x4 *>(xr1 + kb + 8 * s);
        o.b[0][s] = *reinterpret_cast<const u32x4 *>(wr0 + kb + 8 * s);
        o.b[1][s] = *reinterpret_cast<const u32x4 *>(wr1 + kb + 8 * s);
    }
}

__device__ __forceinline__ void mma_blk(f32x4 (&acc)[2][2], const Blk &o) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o.a[i][s]), as_bf16x8(o.b[j][s]),
                                                                    acc[i][j], 0, 0, 0);
}

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

}  // namespace

// TM x TN waves tile the output in 32 x 32 quadrants; KS groups of them split
// K (group g takes blocks g, g + KS, ...).  Waves of one group and one
// quadrant row read the same x rows, waves of one quadrant column the same w
// rows, at about the same time, so the second read of a line hits the CU's L1.
template <int TM, int TN, int KS>
__global__ __launch_bounds__(TM * TN * KS * kWave) void linear_skinny_kernel(const LinearArgs a) {
    constexpr int RM = TM * kGT, RN = TN * kGT;
    __shared__ float red[KS][RM][RN + 1];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int qn = wave % TN, qm = (wave / TN) % TM, ks = wave / (TM * TN);
    const int n0 = blockIdx.x * RN + qn * kGT, m0 = blockIdx.y * RM + qm * kGT;
    const int r16 = lane & 15, kq = (lane >> 4) * (a.K / 4);  // lane group g walks the g-th quarter of K
    // operand rows (clamped into range; their products are never stored)
    const uint16_t *x = static_cast<const uint16_t *>(a.x), *w = static_cast<const uint16_t *>(a.w);
    const uint16_t *xr0 = x + static_cast<int64_t>(min(m0 + r16, a.M - 1)) * a.ldx + kq;
    const uint16_t *xr1 = x + static_cast<int64_t>(min(m0 + 16 + r16, a.M - 1)) * a.ldx + kq;
    const uint16_t *wr0 = w + static_cast<int64_t>(min(n0 + r16, a.N - 1)) * a.ldw + kq;
    const uint16_t *wr1 = w + static_cast<int64_t>(min(n0 + 16 + r16, a.N - 1)) * a.ldw + kq;

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nblk = a.K / kGK;
    const int nb = ks < nblk ? (nblk - 1 - ks) / KS + 1 : 0;  // this wave's blocks: ks, ks + KS, ...
    if (nb > 0) {
        // Ping-pong register buffers: no copies, and every iteration issues
        // the same loads (the prefetch past the last block re-reads the last
        // block), so the compiler's load counters let a block's MFMAs wait
        // for that block's loads only.
        const int last = ks + (nb - 1) * KS;
        Blk b0, b1;
        int kb = ks;
        // (sched_barrier keeps the compiler from sinking a prefetch next to
        // its MFMAs, which would serialise the loads)
        load_blk(b0, xr0, xr1, wr0, wr1, kb * (kGK / 4));
        for (int i = 0;; i += 2) {
            load_blk(b1, xr0, xr1, wr0, wr1, min(kb + KS, last) * (kGK / 4));
            __builtin_amdgcn_sched_barrier(0);
            mma_blk(acc, b0);
            if (i + 1 >= nb) break;
            kb += KS;
            load_blk(b0, xr0, xr1, wr0, wr1, min(kb + KS, last) * (kGK / 4));
            __builtin_amdgcn_sched_barrier(0);
            mma_blk(acc, b1);
            if (i + 2 >= nb) break;
            kb += KS;
        }
    }
    // partial tiles -> LDS: accumulator row 4(l/16) + r, column l%16 of tile (i, j)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                red[ks][qm * kGT + 16 * i + 4 * (lane >> 4) + r][qn * kGT + 16 * j + r16] = acc[i][j][r];
    __syncthreads();
    // item t: row t / (RN / 4), columns 4 (t % (RN / 4)) .. +3
    for (int t = threadIdx.x; t < RM * RN / 4; t += TM * TN * KS * kWave) {
        const int row = t / (RN / 4), c4 = 4 * (t % (RN / 4));
        const int m = blockIdx.y * RM + row, n = blockIdx.x * RN + c4;
        if (m < a.M && n < a.N) {
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float s = 0.f;
#pragma unroll
                for (int v = 0; v < KS; ++v) s += red[v][row][c4 + e];
                o[e] = a.epilogue == PRIME_EPILOGUE_GELU ? gelu_erf(s) : s;
            }
            if (a.epilogue == PRIME_EPILOGUE_RESIDUAL) {  // the product rounded, then the residual add
                const uint2 rv = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(a.r) +
                                                                  static_cast<int64_t>(m) * a.ldr + n);
                o[0] = bf16_bits_to_f32(f32_to_bf16_bits(o[0])) + __uint_as_float(rv.x << 16);
                o[1] = bf16_bits_to_f32(f32_to_bf16_bits(o[1])) + __uint_as_float(rv.x & 0xFFFF0000u);
                o[2] = bf16_bits_to_f32(f32_to_bf16_bits(o[2])) + __uint_as_float(rv.y << 16);
                o[3] = bf16_bits_to_f32(f32_to_bf16_bits(o[3])) + __uint_as_float(rv.y & 0xFFFF0000u);
            }
            uint16_t *yp = static_cast<uint16_t *>(a.y) + static_cast<int64_t>(m) * a.ldy + n;
            *reinterpret_cast<uint2 *>(yp) = uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
        }
    }
}

template <int TM, int TN, int KS>
static void launch_cfg(const LinearArgs &a, hipStream_t stream) {
    const dim3 grid((a.N + TN * kGT - 1) / (TN * kGT), (a.M + TM * kGT - 1) / (TM * kGT)), block(TM * TN * KS * kWave);
    hipLaunchKernelGGL((linear_skinny_kernel<TM, TN, KS>), grid, block, 0, stream, a);
}

// 64 x 64 tiles (half the operand traffic of 32 x 32) when they still give
// enough workgroups; otherwise 32 x 32 tiles with K split over 4 or 16 waves.
hipError_t launch_linear(const LinearArgs &a, hipStream_t stream) {
    if (a.M >= 2048 && linear_tile_fits(a)) return launch_linear_tile(a, stream);
    const int64_t tiles64 = static_cast<int64_t>((a.M + 63) / 64) * ((a.N + 63) / 64);
    const int nblk = a.K / kGK;
    if (tiles64 >= 96) launch_cfg<2, 2, 2>(a, stream);
    else if (nblk > 16) launch_cfg<1, 1, 16>(a, stream);
    else launch_cfg<1, 1, 4>(a, stream);
    return hipGetLastError();
}

}  // namespace prime
