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

__device__ __forceinline__ int nk_of(const LinearArgs &a) { return a.K / kTK; }


// The operand fragments of one K block for one wave: x rows of its four
// 32-row blocks and w rows of its four 32-column blocks, two 16-wide k-steps.
struct Frags {
    bf16x8 x[2][4], w[2][4];
};

__device__ __forceinline__ void read_frags(Frags &f, const uint16_t *sx, const uint16_t *sw, int wm, int wn, int r32,
                                           int h) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) f.x[s][i] = frag(sx, 128 * wm + 32 * i + r32, 2 * s + h);
#pragma unroll
        for (int j = 0; j < 4; ++j) f.w[s][j] = frag(sw, 128 * wn + 32 * j + r32, 2 * s + h);
    }
}

__device__ __forceinline__ void mma_frags(f32x16 (&acc)[4][4], const Frags &f) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(f.w[s][j], f.x[s][i], acc[i][j]);
}

// epilogue staging: a wave's 128 x 128 bf16 quadrant, rows of 16 16-byte
// granules stored at granule g ^ (row & 15)
__device__ __forceinline__ int ep_off(int row, int col) {
    return row * 128 + 8 * ((col >> 3) ^ (row & 15)) + (col & 7);
}

}  // namespace

// K loop.  Four LDS stages hold K blocks kt+1 .. kt+3 while block kt is
// multiplied from registers: the step of block kt waits for its own loads of
// block kt+1 and for its own LDS reads (block kt's fragments, issued one step
// earlier: they must have returned before another wave overwrites their
// stage), meets the barrier (after which every thread's loads of kt+1 have
// landed and kt's stage is free), issues block kt+4 into that stage, reads
// block kt+1's fragments into the other register set and runs block kt's
// MFMAs.  The barriers are asm
// statements (compiler memory barriers), not __syncthreads(), whose fence
// would make the compiler wait for loads it does not know about anyway.
__global__ __launch_bounds__(256, 1) void linear_tile_kernel(const LinearArgs a) {
    __shared__ __attribute__((aligned(1024))) uint16_t sbuf[kNS * 2 * kStage];  // stage s: x at 2s, w at 2s+1

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int NB = a.N / kTN, MB = (a.M + kTM - 1) / kTM;
    const int tiles = MB * NB;
    int t = blockIdx.x;
    if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);  // XCD-contiguous tile ranges
    const int m0 = (t / NB) * kTM, n0 = (t % NB) * kTN;
    const uint16_t *x = static_cast<const uint16_t *>(a.x), *w = static_cast<const uint16_t *>(a.w);
    auto sx = [&](int st) { return sbuf + (2 * st) * kStage; };
    auto sw = [&](int st) { return sbuf + (2 * st + 1) * kStage; };
    // block kb into stage st (kb clamped to the last block: such copies land in
    // a stage that is never read again, and keep the count of loads per step)
    auto issue = [&](int kb, int st) {
        const int k0 = min(kb, nk_of(a) - 1) * kTK;
        load_operand(sx(st), x, a.ldx, m0, a.M - 1, k0, wave, lane);
        load_operand(sw(st), w, a.ldw, n0, a.N - 1, k0, wave, lane);
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int nk = nk_of(a);
    const int r32 = lane & 31, h = lane >> 5;
#pragma unroll
    for (int b = 0; b < kNS; ++b) issue(b, b);
    asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    Frags fa, fb;
    read_frags(fa, sx(0), sw(0), wm, wn, r32, h);
    for (int kt = 0; kt < nk; kt += 2) {
        asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(kt + kNS, kt & (kNS - 1));
        read_frags(fb, sx((kt + 1) & (kNS - 1)), sw((kt + 1) & (kNS - 1)), wm, wn, r32, h);
        // (the scheduler would otherwise sink the reads next to their MFMAs)
        __builtin_amdgcn_sched_barrier(0);
        mma_frags(acc, fa);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(kt + 1 + kNS, (kt + 1) & (kNS - 1));
        read_frags(fa, sx((kt + 2) & (kNS - 1)), sw((kt + 2) & (kNS - 1)), wm, wn, r32, h);
        __builtin_amdgcn_sched_barrier(0);
        mma_frags(acc, fb);
        __builtin_amdgcn_sched_barrier(0);
    }
    // every load into LDS has landed and every wave is done with the stages
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- epilogue: the products, rounded to bf16, through LDS (the wave's
    // quadrant in 32 KB of the stages), then row segments of 8 columns per
    // lane: 4 rows x 256 contiguous bytes per store instruction
    uint16_t *ep = sbuf + wave * (128 * 128);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int tq = 0; tq < 4; ++tq) {
                const int row = 32 * i + r32, col = 32 * j + 8 * tq + 4 * h;
                *reinterpret_cast<uint2 *>(ep + ep_off(row, col)) =
                    uint2{pack2(acc[i][j][4 * tq], acc[i][j][4 * tq + 1]),
                          pack2(acc[i][j][4 * tq + 2], acc[i][j][4 * tq + 3])};
            }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave reads back only its own rows
    uint16_t *y = static_cast<uint16_t *>(a.y);
    const uint16_t *r = static_cast<const uint16_t *>(a.r);
    const int gcol = 8 * (lane & 15);
#pragma unroll 4
    for (int it = 0; it < 32; ++it) {
        const int row = 4 * it + (lane >> 4);
        const int m = m0 + 128 * wm + row, n = n0 + 128 * wn + gcol;
        if (m >= a.M) continue;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(ep + ep_off(row, gcol));
        u32x4 o = v;
        if (a.epilogue == PRIME_EPILOGUE_GELU) {
            float f[8];
            unpack8(v, f);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = gelu_exact(f[e]);
            o = pack8(f);
        } else if (a.epilogue == PRIME_EPILOGUE_RESIDUAL) {
            float f[8], g[8];
            unpack8(v, f);
            unpack8(*reinterpret_cast<const u32x4 *>(r + static_cast<int64_t>(m) * a.ldr + n), g);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] += g[e];
            o = pack8(f);
        }
        *reinterpret_cast<u32x4 *>(y + static_cast<int64_t>(m) * a.ldy + n) = o;
    }
}

bool linear_tile_fits(const LinearArgs &a) {
    return a.M >= kTM && a.N % kTN == 0 && a.K % (2 * kTK) == 0;  // K blocks in pairs
}

hipError_t launch_linear_tile(const LinearArgs &a, hipStream_t stream) {
    const int tiles = ((a.M + kTM - 1) / kTM) * (a.N / kTN);
    hipLaunchKernelGGL(linear_tile_kernel, dim3(tiles), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace prime
