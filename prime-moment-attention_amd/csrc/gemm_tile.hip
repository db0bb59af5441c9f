// Large-M linear layers of the PRIME prefill on gfx950 (model.py:59-68,
// 101-118: the q/k/v, o and MLP projections over every token of the batch):
// y[M, N] = epilogue(x[M, K] . w[N, K]^T), bf16 in and out, fp32 accumulation,
// with the element-wise pass that follows each projection in the block folded
// into the store:
//   PRIME_EPILOGUE_GELU      y = gelu(x w^T)      (up projection; exact erf GELU)
//   PRIME_EPILOGUE_RESIDUAL  y = r + x w^T        (o / down projection and the
//                                                  block's residual add; r may be y)
// The product is rounded to bf16 before the epilogue, as the separate passes
// see it.
//
// Tiling.  One workgroup of 4 waves computes a 256 x 256 tile of y over K in
// blocks of 32; wave (wm, wn) owns the 128 x 128 quadrant (wm, wn) as 4 x 4
// v_mfma_f32_32x32x16_bf16 accumulators (256 fp32 registers per lane).  The
// operands pass through four LDS stages of 2 x 16 KB filled by
// global_load_lds_dwordx4 (HBM/L2 straight into LDS, no registers), three K
// blocks ahead of the MFMAs: one wave instruction moves 16 tile rows x 64
// bytes.  Rows are stored with their four 16-byte segments XOR-swizzled by
// (row >> 2) & 3, applied on the global side (lane -> source segment), so the
// ds_read_b128 operand reads of 16 consecutive rows at one segment hit
// distinct banks.  One barrier per K block: after it the loads of block k+3
// go into the stage block k-1 used, and block k is computed.
//
// The MFMA runs with w as its A operand and x as its B operand, so the
// accumulator holds y^T blocks: lane l, register t of block (i, j) is
// y[32 i + l % 32][32 j + 8 (t / 4) + 4 (l / 32) + t % 4] -- four consecutive
// columns of one row per register quad, stored as one 8-byte write.
//
// Workgroups are numbered so that each XCD (workgroup index mod 8) runs a
// contiguous range of tiles, n fastest: the tiles running together on one XCD
// share their x rows in its L2.

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kTM = 256, kTN = 256, kTK = 32, kNS = 4;  // tile, K block, LDS stages
constexpr int kStage = kTM * kTK;  // bf16 elements of one operand stage (16 KB)

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float gelu_exact(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

__device__ __forceinline__ float round_bf16(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

// swizzled segment position of 16-byte segment `seg` of tile row `row` (4 per row)
__device__ __forceinline__ int swz(int row, int seg) { return seg ^ ((row >> 2) & 3); }

// Direct-to-LDS loads of one K block: tile rows [r0, r0 + 256) of `src`
// (clamped to rmax: rows past the matrix re-read its last row and are never
// stored), columns [k0, k0 + 32).  Wave w, instruction i covers tile rows
// 16 (4 w + i) .. +15; lane l lands at LDS segment l % 4 of row l / 4 and loads
// the global segment that belongs there.
__device__ __forceinline__ void load_operand(uint16_t *stage, const uint16_t *src, int64_t ld, int r0, int rmax,
                                             int k0, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rr = 16 * (4 * wave + i) + (lane >> 2);
        const int seg = swz(rr, lane & 3);
        const int row = min(r0 + rr, rmax);
        const uint16_t *g = src + static_cast<int64_t>(row) * ld + k0 + 8 * seg;
        const uint32_t l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(stage + 16 * (4 * wave + i) * kTK));
        // written as asm: the compiler then does not track these loads, and
        // the explicit vmcnt waits of the K loop are the only ones (its own
        // tracking of loads into LDS would wait for all of them before every
        // LDS read it cannot separate from them).  M0 is set here for each
        // instruction; no compiler-generated code in this kernel uses it.
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(l) : "memory", "m0");
    }
}

// operand of tile row `row`, 16-byte segment `seg`
__device__ __forceinline__ bf16x8 frag(const uint16_t *stage, int row, int seg) {
    return as_bf16x8(*reinterpret_cast<const u32x4 *>(stage + row * kTK + 8 * swz(row, seg)));
}

}  // namespace

// One K block: wait until this thread's loads of block kt have landed (the
// loads of the two later blocks, 2 x 8, may still be in flight), barrier (every
// thread's have landed, and every wave is done with the stage of block kt - 1),
// issue block kt + 3 into that stage (cX / cW: the stage block kt - 1 used),
// then the MFMAs of block kt.  The barrier is written as an asm statement (a
// compiler memory barrier), not __syncthreads(), whose fence would make the
// compiler wait for every load into LDS, the ones just issued included; the
// stages are separate arrays so that it can tell the loads into one stage from
// the operand reads of another.
#define PRIME_TILE_STEP(kt, rX, rW, cX, cW)                                                       \
    if ((kt) < nk) {                                                                              \
        asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");                            \
        const int kb = min((kt) + kNS - 1, nk - 1) * kTK;                                         \
        load_operand(cX, x, a.ldx, m0, a.M - 1, kb, wave, lane);                                  \
        load_operand(cW, w, a.ldw, n0, a.N - 1, kb, wave, lane);                                  \
        bf16x8 fx[2][4], fw[2][4];                                                                \
        _Pragma("unroll") for (int s = 0; s < 2; ++s) {                                           \
            _Pragma("unroll") for (int i = 0; i < 4; ++i) fx[s][i] = frag(rX, 128 * wm + 32 * i + r32, 2 * s + h); \
            _Pragma("unroll") for (int j = 0; j < 4; ++j) fw[s][j] = frag(rW, 128 * wn + 32 * j + r32, 2 * s + h); \
        }                                                                                         \
        _Pragma("unroll") for (int s = 0; s < 2; ++s)                                             \
            _Pragma("unroll") for (int i = 0; i < 4; ++i)                                         \
                _Pragma("unroll") for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(fw[s][j], fx[s][i], acc[i][j]); \
    }

__global__ __launch_bounds__(256, 1) void linear_tile_kernel(const LinearArgs a) {
    __shared__ __attribute__((aligned(1024))) uint16_t sX0[kStage], sX1[kStage], sX2[kStage], sX3[kStage];
    __shared__ __attribute__((aligned(1024))) uint16_t sW0[kStage], sW1[kStage], sW2[kStage], sW3[kStage];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int NB = a.N / kTN, MB = (a.M + kTM - 1) / kTM;
    const int tiles = MB * NB;
    int t = blockIdx.x;
    if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);  // XCD-contiguous tile ranges
    const int m0 = (t / NB) * kTM, n0 = (t % NB) * kTN;
    const uint16_t *x = static_cast<const uint16_t *>(a.x), *w = static_cast<const uint16_t *>(a.w);

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int nk = a.K / kTK;
    // blocks 0, 1, 2 in flight before the loop; each step then issues block
    // kt + 3 (clamped to the last block: a copy into a stage that is never
    // read again, so that every step issues the same 8 loads per thread and
    // one wait count fits all)
    load_operand(sX0, x, a.ldx, m0, a.M - 1, 0, wave, lane);
    load_operand(sW0, w, a.ldw, n0, a.N - 1, 0, wave, lane);
    load_operand(sX1, x, a.ldx, m0, a.M - 1, min(1, nk - 1) * kTK, wave, lane);
    load_operand(sW1, w, a.ldw, n0, a.N - 1, min(1, nk - 1) * kTK, wave, lane);
    load_operand(sX2, x, a.ldx, m0, a.M - 1, min(2, nk - 1) * kTK, wave, lane);
    load_operand(sW2, w, a.ldw, n0, a.N - 1, min(2, nk - 1) * kTK, wave, lane);
    const int r32 = lane & 31, h = lane >> 5;
    for (int kt = 0; kt < nk; kt += kNS) {
        PRIME_TILE_STEP(kt, sX0, sW0, sX3, sW3)
        PRIME_TILE_STEP(kt + 1, sX1, sW1, sX0, sW0)
        PRIME_TILE_STEP(kt + 2, sX2, sW2, sX1, sW1)
        PRIME_TILE_STEP(kt + 3, sX3, sW3, sX2, sW2)
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the workgroup
#undef PRIME_TILE_STEP

    // ---- epilogue: lane holds y[m][n .. n+3] per register quad
    uint16_t *y = static_cast<uint16_t *>(a.y);
    const uint16_t *r = static_cast<const uint16_t *>(a.r);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 128 * wm + 32 * i + r32;
        if (m >= a.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int tq = 0; tq < 4; ++tq) {
                const int n = n0 + 128 * wn + 32 * j + 8 * tq + 4 * h;
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = round_bf16(acc[i][j][4 * tq + e]);
                if (a.epilogue == PRIME_EPILOGUE_GELU) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = gelu_exact(o[e]);
                } else if (a.epilogue == PRIME_EPILOGUE_RESIDUAL) {
                    const uint2 rv = *reinterpret_cast<const uint2 *>(r + static_cast<int64_t>(m) * a.ldr + n);
                    o[0] += __uint_as_float(rv.x << 16);
                    o[1] += __uint_as_float(rv.x & 0xFFFF0000u);
                    o[2] += __uint_as_float(rv.y << 16);
                    o[3] += __uint_as_float(rv.y & 0xFFFF0000u);
                }
                *reinterpret_cast<uint2 *>(y + static_cast<int64_t>(m) * a.ldy + n) =
                    uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
            }
    }
}

bool linear_tile_fits(const LinearArgs &a) {
    return a.M >= kTM && a.N % kTN == 0 && a.K % kTK == 0;
}

hipError_t launch_linear_tile(const LinearArgs &a, hipStream_t stream) {
    const int tiles = ((a.M + kTM - 1) / kTM) * (a.N / kTN);
    hipLaunchKernelGGL(linear_tile_kernel, dim3(tiles), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace prime
