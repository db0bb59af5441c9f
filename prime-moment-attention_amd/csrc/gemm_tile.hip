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
// blocks of 64 (a block row is one whole 128-byte line); wave (wm, wn) owns the
// 128 x 128 quadrant (wm, wn) as 4 x 4 v_mfma_f32_32x32x16_bf16 accumulators
// (256 fp32 registers per lane), a block as four substeps of 16 MFMAs.
//
// Operands reach LDS by global_load_lds_dwordx4 (no registers): one wave
// instruction moves 8 tile rows x 128 bytes.  The 160 KB of LDS hold three x
// slots and two w slots of 32 KB.  Rows keep their eight 16-byte segments
// XOR-swizzled by (row >> 1) & 7 (applied on the global side), so the
// ds_read_b128 operand reads, 16 lanes a cycle, hit distinct banks.
//
// Schedule of block g (measured on MI355X, one per-phase cycle count per
// change): every substep interleaves its 16 MFMAs with the 8 fragment reads of
// the next substep and at most one load instruction per two MFMAs -- a burst
// of load instructions stalls the issuing wave (and with it its MFMAs) for
// about 44 cycles an instruction, spread out they cost nothing.  The loads:
// substep 0 the second half of block g+1's w and two of block g+2's eight x
// instructions, substeps 1 and 2 the other six, substep 3 the first half of
// block g+2's w.  The one barrier per block sits before substep 3: it waits
// for block g+1 (its x was issued a whole block earlier, into the third x
// slot) and frees block g's slots, so substep 3 reads block g+1's first
// fragments and loads block g+2's w into block g's w slot.  Four load
// instructions share one M0 (the instruction offset steps both the LDS and the
// global address; the global offsets are pre-shifted back), with the global
// address as a 32-bit per-lane offset on a scalar base.
//
// The MFMA runs with w as its A operand and x as its B operand, so the
// accumulator holds y^T blocks: lane l, register t of block (i, j) is
// y[32 i + l % 32][32 j + 8 (t / 4) + 4 (l / 32) + t % 4].  The epilogue
// rounds to bf16, swaps halves between lanes l and l + 32 (v_permlane32_swap)
// so that each lane holds 8 consecutive columns, stages the wave's quadrant in
// LDS with one ds_write_b128 per 16 bytes, then writes rows as 4 x 256
// contiguous bytes per store instruction (nontemporal: the tile is not read
// again by this kernel).
//
// Workgroups are numbered so that each XCD (workgroup index mod 8) runs a
// contiguous range of tiles, n fastest: the tiles running together on one XCD
// share their x rows in its L2.

#include <type_traits>

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kTM = 256, kTN = 256, kTK = 64;
constexpr int kSlot = kTM * kTK;  // bf16 elements of one operand slot (32 KB)
constexpr int kXSlots = 3, kWSlots = 2;

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float gelu_exact(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

// swizzled position of 16-byte segment `seg` of slot row `row` (8 per row)
__device__ __forceinline__ int swz(int row, int seg) { return seg ^ ((row >> 1) & 7); }

// operand fragment of slot row `row`, 16-byte segment `seg`
__device__ __forceinline__ bf16x8 frag(const uint16_t *slot, int row, int seg) {
    return as_bf16x8(*reinterpret_cast<const u32x4 *>(slot + row * kTK + 8 * swz(row, seg)));
}

// The loads into LDS are asm: the compiler then does not track them, and the
// explicit vmcnt waits at the barriers are the only ones (its own tracking
// would wait for all of them before every LDS read it cannot separate from
// them).  M0 is set by this asm only; no compiler-generated code in the kernel
// uses it.
__device__ __forceinline__ void set_m0(uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0" ::"s"(lds_addr) : "memory", "m0");
}
template <int OFF>
__device__ __forceinline__ void load_lds(uint32_t voff, const void *base) {
    asm volatile("global_load_lds_dwordx4 %0, %1 offset:%2" ::"v"(voff - OFF), "s"(base), "i"(OFF) : "memory");
}

struct Frags {
    bf16x8 x[4], w[4];
};

// epilogue staging: a wave's 128 x 128 bf16 quadrant, rows of 16 16-byte
// granules stored at granule g ^ (row & 15)
__device__ __forceinline__ int ep_off(int row, int col) {
    return row * 128 + 8 * ((col >> 3) ^ (row & 15)) + (col & 7);
}

}  // namespace

template <int EPI>
__global__ __launch_bounds__(256, 1) void linear_tile_kernel(const LinearArgs a) {
    __shared__ __attribute__((aligned(1024))) uint16_t sbuf[(kXSlots + kWSlots) * kSlot];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1, r32 = lane & 31, h = lane >> 5;
    const int NB = a.N / kTN, MB = (a.M + kTM - 1) / kTM;
    const int tiles = MB * NB;
    int t = blockIdx.x;
    if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);  // XCD-contiguous tile ranges
    const int m0 = (t / NB) * kTM, n0 = (t % NB) * kTN;
    const int nk = a.K / kTK;
    auto xslot = [&](int s) __attribute__((always_inline)) { return sbuf + s * kSlot; };
    auto wslot = [&](int s) __attribute__((always_inline)) { return sbuf + (kXSlots + s) * kSlot; };

    // Load instruction i (0..7) of an operand covers slot rows 64 wave + 8 i ..
    // +7: lane l takes row + l / 8 and lands at segment position l % 8, which
    // holds logical segment (l % 8) ^ ((row >> 1) & 7) = (l % 8) ^ (l / 16) ^ 4 (i % 2).
    uint32_t vx[8], vw[8];  // byte offsets of this lane's source segment
    {
        const uint32_t so = 16 * ((lane & 7) ^ (lane >> 4));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int rr = 64 * wave + 8 * i + (lane >> 3);
            const uint32_t s = (i & 1) ? so ^ 64 : so;
            vx[i] = static_cast<uint32_t>(min(m0 + rr, a.M - 1)) * static_cast<uint32_t>(a.ldx * 2) + s;
            vw[i] = static_cast<uint32_t>(min(n0 + rr, a.N - 1)) * static_cast<uint32_t>(a.ldw * 2) + s;
        }
    }
    const uint32_t lds_wave =
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbuf)) + 64 * wave * kTK * static_cast<uint32_t>(sizeof(uint16_t));
    // load instruction i of block kb's x (or w) into slot s
    auto load = [&](bool isx, int s, int kb, int i) __attribute__((always_inline)) {
        const char *base = reinterpret_cast<const char *>(isx ? a.x : a.w) + static_cast<int64_t>(kb) * kTK * 2;
        set_m0(lds_wave + (isx ? s : kXSlots + s) * kSlot * 2 + 8 * (i & 4) * kTK * 2);
        const uint32_t v = isx ? vx[i] : vw[i];
        if ((i & 3) == 0) load_lds<0>(v, base);
        else if ((i & 3) == 1) load_lds<1024>(v, base);
        else if ((i & 3) == 2) load_lds<2048>(v, base);
        else load_lds<3072>(v, base);
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    // prologue: block 0 whole, block 1's x and the first half of its w
#pragma unroll
    for (int i = 0; i < 8; ++i) load(true, 0, 0, i);
#pragma unroll
    for (int i = 0; i < 8; ++i) load(false, 0, 0, i);
#pragma unroll
    for (int i = 0; i < 8; ++i) load(true, 1, 1, i);
#pragma unroll
    for (int i = 0; i < 4; ++i) load(false, 1, 1, i);
    asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");  // block 0 landed
    Frags f[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) f[0].w[j] = frag(wslot(0), 128 * wn + 32 * j + r32, h);
#pragma unroll
    for (int i = 0; i < 4; ++i) f[0].x[i] = frag(xslot(0), 128 * wm + 32 * i + r32, h);
    __builtin_amdgcn_sched_barrier(0);

    int xc = 0;  // x slot of block g
    // block g; MORE: block g+1 exists, MORE2: block g+2 exists
    auto step = [&](int g, auto more_c, auto more2_c) __attribute__((always_inline)) {
        constexpr bool more = decltype(more_c)::value, more2 = decltype(more2_c)::value;
        const int xn = xc == kXSlots - 1 ? 0 : xc + 1, xn2 = xn == kXSlots - 1 ? 0 : xn + 1;
        const int wc = g & 1, wnx = wc ^ 1;
#pragma unroll
        for (int ss = 0; ss < 4; ++ss) {
            const Frags &c = f[ss & 1];
            Frags &nx = f[(ss + 1) & 1];
            if (ss == 3) {
                // block g+1 landed (block g+2's eight x loads may still be in flight);
                // this wave's reads of block g returned: its slots are free after the barrier
                if constexpr (more2) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
            }
            const uint16_t *rx = ss < 3 ? xslot(xc) : xslot(xn);
            const uint16_t *rw = ss < 3 ? wslot(wc) : wslot(wnx);
            const int rseg = ss < 3 ? 2 * (ss + 1) + h : h;
            const bool do_rd = ss < 3 || more;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int xi = q >> 2, wj = q & 3;
                acc[xi][wj] = mfma32(c.w[wj], c.x[xi], acc[xi][wj]);
                __builtin_amdgcn_sched_barrier(0);
                if ((q & 1) == 0 && do_rd) {
                    const int r = q >> 1;  // w fragments first: the next substep's first MFMAs need w[0..3], x[0]
                    if (r < 4) nx.w[r] = frag(rw, 128 * wn + 32 * r + r32, rseg);
                    else nx.x[r - 4] = frag(rx, 128 * wm + 32 * (r - 4) + r32, rseg);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if ((q & 1) == 1) {
                    const int sl = q >> 1;
                    if (ss == 0) {
                        if (more && sl < 4) { load(false, wnx, g + 1, 4 + sl); __builtin_amdgcn_sched_barrier(0); }
                        if (more2 && (sl == 4 || sl == 5)) { load(true, xn2, g + 2, sl - 4); __builtin_amdgcn_sched_barrier(0); }
                    } else if (ss == 1) {
                        if (more2 && sl < 3) { load(true, xn2, g + 2, 2 + sl); __builtin_amdgcn_sched_barrier(0); }
                    } else if (ss == 2) {
                        if (more2 && sl < 3) { load(true, xn2, g + 2, 5 + sl); __builtin_amdgcn_sched_barrier(0); }
                    } else {
                        if (more2 && sl < 4) { load(false, wc, g + 2, sl); __builtin_amdgcn_sched_barrier(0); }
                    }
                }
            }
        }
        xc = xn;
    };
    using T_ = std::integral_constant<bool, true>;
    using F_ = std::integral_constant<bool, false>;
    for (int g = 0; g < nk - 2; ++g) step(g, T_{}, T_{});
    step(nk - 2, T_{}, F_{});
    step(nk - 1, F_{}, F_{});
    // every load into LDS has landed and every wave is done with the slots
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- epilogue: the products rounded to bf16; lanes l and l + 32 swap
    // halves so each holds 8 consecutive columns of its row; the wave's
    // quadrant through 32 KB of LDS, then 4 rows x 256 contiguous bytes per
    // store instruction
    uint16_t *ep = sbuf + wave * (128 * 128);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t P0 = pack2(acc[i][j][8 * p + 0], acc[i][j][8 * p + 1]);
                const uint32_t P1 = pack2(acc[i][j][8 * p + 2], acc[i][j][8 * p + 3]);
                const uint32_t Q0 = pack2(acc[i][j][8 * p + 4], acc[i][j][8 * p + 5]);
                const uint32_t Q1 = pack2(acc[i][j][8 * p + 6], acc[i][j][8 * p + 7]);
                // lane l < 32 keeps its columns c..c+3 and takes lane l+32's c+4..c+7; lane l+32
                // takes lane l's c+8..c+11 and keeps its c+12..c+15 (c = 32 j + 16 p)
                const auto s0 = __builtin_amdgcn_permlane32_swap(P0, Q0, false, false);
                const auto s1 = __builtin_amdgcn_permlane32_swap(P1, Q1, false, false);
                const int row = 32 * i + r32, col = 32 * j + 16 * p + 8 * h;
                *reinterpret_cast<u32x4 *>(ep + ep_off(row, col)) = u32x4{s0[0], s1[0], s0[1], s1[1]};
            }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave reads back only its own rows
    uint16_t *y = static_cast<uint16_t *>(a.y);
    const uint16_t *r = static_cast<const uint16_t *>(a.r);
    const int gcol = 8 * (lane & 15);
    const bool full = m0 + kTM <= a.M;
#pragma unroll
    for (int b8 = 0; b8 < 4; ++b8) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const u32x4 *>(ep + ep_off(4 * (8 * b8 + u) + (lane >> 4), gcol));
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int m = m0 + 128 * wm + 4 * (8 * b8 + u) + (lane >> 4), n = n0 + 128 * wn + gcol;
            if (!full && m >= a.M) continue;
            u32x4 o = v[u];
            if constexpr (EPI == PRIME_EPILOGUE_GELU) {
                float fv[8];
                unpack8(o, fv);
#pragma unroll
                for (int e = 0; e < 8; ++e) fv[e] = gelu_exact(fv[e]);
                o = pack8(fv);
            } else if constexpr (EPI == PRIME_EPILOGUE_RESIDUAL) {
                float fv[8], gv[8];
                unpack8(o, fv);
                unpack8(*reinterpret_cast<const u32x4 *>(r + static_cast<int64_t>(m) * a.ldr + n), gv);
#pragma unroll
                for (int e = 0; e < 8; ++e) fv[e] += gv[e];
                o = pack8(fv);
            }
            __builtin_nontemporal_store(o, reinterpret_cast<u32x4 *>(y + static_cast<int64_t>(m) * a.ldy + n));
        }
    }
}

bool linear_tile_fits(const LinearArgs &a) {
    // the load offsets are 32-bit per lane on a 64-bit base
    const int64_t xspan = (static_cast<int64_t>(a.M) - 1) * a.ldx * 2 + static_cast<int64_t>(a.K) * 2;
    const int64_t wspan = (static_cast<int64_t>(a.N) - 1) * a.ldw * 2 + static_cast<int64_t>(a.K) * 2;
    return a.M >= kTM && a.N % kTN == 0 && a.K % kTK == 0 && a.K >= 2 * kTK && xspan < (int64_t(1) << 32) &&
           wspan < (int64_t(1) << 32);
}

hipError_t launch_linear_tile(const LinearArgs &a, hipStream_t stream) {
    const int tiles = ((a.M + kTM - 1) / kTM) * (a.N / kTN);
    if (a.epilogue == PRIME_EPILOGUE_GELU)
        hipLaunchKernelGGL(linear_tile_kernel<PRIME_EPILOGUE_GELU>, dim3(tiles), dim3(256), 0, stream, a);
    else if (a.epilogue == PRIME_EPILOGUE_RESIDUAL)
        hipLaunchKernelGGL(linear_tile_kernel<PRIME_EPILOGUE_RESIDUAL>, dim3(tiles), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(linear_tile_kernel<PRIME_EPILOGUE_NONE>, dim3(tiles), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace prime
