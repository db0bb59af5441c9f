// Projections of the decode step on gfx950 (model.py:59-68, 101-118, 160 at one
// token per sequence): y[M, N] = epilogue(rowscale * x[M, K] . w[N, K]^T) for a
// few hundred rows, bf16 in and out, fp32 accumulation.  The element-wise
// passes around each projection of the block fold into it:
//   RMS (rms_eps > 0):       y = (x . w'^T) * rsqrt(mean_k x^2 + eps) per row --
//     the RMSNorm before the projection, with its weight pre-multiplied into
//     the columns of w (w' = w diag(g)); the norm's output is then never
//     rounded on its own;
//   PRIME_EPILOGUE_GELU:     the exact GELU of the rounded product;
//   PRIME_EPILOGUE_RESIDUAL: y = r + rounded product (r may be y).
//
// With M a few hundred the weights are the only large stream, read once per
// call from HBM, and the kernel is bound by memory latency.  One workgroup of
// 4 waves owns 64 rows x BN columns (BN = 64 or 32) over the whole of K;
// wave w owns rows 16w .. 16w+15 and all BN columns as BN / 16
// v_mfma_f32_16x16x32_bf16 tiles, with w as the A operand so that a lane's
// register quad holds four consecutive columns of one row (one 8-byte store).
// K runs in blocks of 64 through four LDS stages, three blocks ahead, filled
// by global_load_lds_dwordx4 (one wave instruction moves 8 rows x 128 bytes;
// 16-byte segments XOR-swizzled by row & 7 on the global side, so the
// ds_read_b128 operand reads of 8 consecutive rows are conflict-free).  The
// row sums of squares of the RMS prologue come from the x operands the wave
// reads anyway (lane group g holds k-slots 8g..8g+7 of every 32-wide step;
// the four groups are summed at the end).

#include "gemm_common.h"

namespace prime {

constexpr int kRM = 64;  // rows per workgroup


// NS stages (4 in use).  One
// K block per step: wait for this thread's loads of block kt+1 (the NS - 2
// later blocks' may still be in flight; once no block past nk is left to
// issue, for all of them) and for its LDS reads (block kt's fragments, read
// one step earlier, must have returned before another wave overwrites their
// stage), barrier, issue block kt+NS into kt's stage, read kt+1's fragments,
// run kt's MFMAs.
template <int BN, bool RMS, int EPI, int NS>
__global__ __launch_bounds__(256) void linear_rows_kernel(const LinearArgs a) {
    constexpr int NT = BN / 16;                         // n tiles per wave
    constexpr int XS = kRM * kRK, WS = BN * kRK;        // stage sizes (elements)
    constexpr int LPS = 2 + BN / 32;                    // loads per thread per stage
    static_assert((NS & (NS - 1)) == 0 && NS >= 4, "NS: a power of two");
    __shared__ __attribute__((aligned(1024))) uint16_t sbuf[NS * (XS + WS)];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int l16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * kRM;
    const uint16_t *x = static_cast<const uint16_t *>(a.x), *w = static_cast<const uint16_t *>(a.w);
    const int nk = a.K / kRK;
    auto sx = [&](int st) { return sbuf + st * (XS + WS); };
    auto sw = [&](int st) { return sbuf + st * (XS + WS) + XS; };
    auto issue = [&](int kb, int st) {  // (wave-uniform: no block past the last)
        if (kb >= nk) return;
        rows_dma(sx(st), x, a.ldx, m0, a.M - 1, 16 * wave, 2, kb * kRK, lane);
        rows_dma(sw(st), w, a.ldw, n0, a.N - 1, (BN / 4) * wave, BN / 32, kb * kRK, lane);
    };
    // block kb landed (this thread's loads, then everyone's): with the
    // pipeline full NS - 2 later blocks may be outstanding, else none
    auto wait_block = [&](int kb) {
        if (kb + NS - 1 <= nk)
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 2) * LPS) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    struct Fr {
        bf16x8 x[2], w[2][NT];
    };
    auto read = [&](Fr &f, int st) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            f.x[s] = rfrag(sx(st), 16 * wave + l16, g + 4 * s);
#pragma unroll
            for (int j = 0; j < NT; ++j) f.w[s][j] = rfrag(sw(st), 16 * j + l16, g + 4 * s);
        }
    };
    f32x4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
    auto mma = [&](const Fr &f) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[j] = mfma(f.w[s][j], f.x[s], acc[j]);
            if constexpr (RMS) ss += sumsq8(f.x[s]);
        }
    };

#pragma unroll
    for (int b = 0; b < NS; ++b) issue(b, b);
    // block 0 landed: with all NS issued, NS - 1 later blocks may be outstanding
    if (NS <= nk) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 1) * LPS) : "memory");
    else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    Fr fa, fb;
    read(fa, 0);
    for (int kt = 0; kt < nk; kt += 2) {
        // (nk is even: K a multiple of 128)
        wait_block(kt + 1);
        issue(kt + NS, kt & (NS - 1));
        read(fb, (kt + 1) & (NS - 1));
        __builtin_amdgcn_sched_barrier(0);
        mma(fa);
        __builtin_amdgcn_sched_barrier(0);
        wait_block(kt + 2);  // (past the last block: every load landed)
        issue(kt + 1 + NS, (kt + 1) & (NS - 1));
        read(fa, (kt + 2) & (NS - 1));
        __builtin_amdgcn_sched_barrier(0);
        mma(fb);
        __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the workgroup

    // ---- epilogue: lane holds y[m][n .. n+3], m = m0 + 16 wave + l16, n = n0 + 16 j + 4 g
    const int m = m0 + 16 * wave + l16;
    float rs = 1.0f;
    if constexpr (RMS) {
        ss += __shfl_xor(ss, 16, kWave);
        ss += __shfl_xor(ss, 32, kWave);
        rs = rsqrtf(ss / static_cast<float>(a.K) + a.rms_eps);
    }
    if (m >= a.M) return;
    uint16_t *y = static_cast<uint16_t *>(a.y);
    const uint16_t *r = static_cast<const uint16_t *>(a.r);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int n = n0 + 16 * j + 4 * g;
        if (n >= a.N) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = bf16r(acc[j][e] * rs);
        if constexpr (EPI == PRIME_EPILOGUE_GELU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = gelu_erf_r(o[e]);
        } else if constexpr (EPI == PRIME_EPILOGUE_RESIDUAL) {
            const uint2 rv = *reinterpret_cast<const uint2 *>(r + static_cast<int64_t>(m) * a.ldr + n);
            o[0] += __uint_as_float(rv.x << 16);
            o[1] += __uint_as_float(rv.x & 0xFFFF0000u);
            o[2] += __uint_as_float(rv.y << 16);
            o[3] += __uint_as_float(rv.y & 0xFFFF0000u);
        }
        *reinterpret_cast<uint2 *>(y + static_cast<int64_t>(m) * a.ldy + n) = uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
    }
}

// The same products for K <= 768 with every K block in flight at once: one
// workgroup owns 64 rows x 32 columns, all NK = K / 64 blocks of x and w sit in
// LDS together (NK x 12 KB, 144 KB at K = 768), so the workgroup waits for one
// memory latency instead of one per three blocks; the K loop then reads block
// kt once its loads have landed (vmcnt counts this thread's outstanding
// blocks, a barrier the other threads').  Products, sums and epilogues are
// those of linear_rows_kernel, in the same order: the results are identical.
template <int NK, bool RMS, int EPI>
__global__ __launch_bounds__(256) void linear_rows_wholek_kernel(const LinearArgs a) {
    constexpr int BN = 32, NT = 2;
    constexpr int XS = kRM * kRK, WS = BN * kRK;  // stage sizes (elements)
    __shared__ __attribute__((aligned(1024))) uint16_t sbuf[NK * (XS + WS)];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int l16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * kRM;
    const uint16_t *x = static_cast<const uint16_t *>(a.x), *w = static_cast<const uint16_t *>(a.w);
    auto sx = [&](int st) { return sbuf + st * (XS + WS); };
    auto sw = [&](int st) { return sbuf + st * (XS + WS) + XS; };
#pragma unroll
    for (int kb = 0; kb < NK; ++kb) {  // three loads per thread per block
        rows_dma(sx(kb), x, a.ldx, m0, a.M - 1, 16 * wave, 2, kb * kRK, lane);
        rows_dma(sw(kb), w, a.ldw, n0, a.N - 1, (BN / 4) * wave, 1, kb * kRK, lane);
    }
    f32x4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
#pragma unroll
    for (int kt = 0; kt < NK; ++kt) {
        // this thread's loads of blocks 0..kt have landed (3 per later block
        // may still be in flight), then everyone's
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(3 * (NK - 1 - kt)) : "memory");
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const bf16x8 xf = rfrag(sx(kt), 16 * wave + l16, g + 4 * s);
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[j] = mfma(rfrag(sw(kt), 16 * j + l16, g + 4 * s), xf, acc[j]);
            if constexpr (RMS) ss += sumsq8(xf);
        }
    }

    // ---- epilogue (as linear_rows_kernel): lane holds y[m][n .. n+3]
    const int m = m0 + 16 * wave + l16;
    float rs = 1.0f;
    if constexpr (RMS) {
        ss += __shfl_xor(ss, 16, kWave);
        ss += __shfl_xor(ss, 32, kWave);
        rs = rsqrtf(ss / static_cast<float>(a.K) + a.rms_eps);
    }
    if (m >= a.M) return;
    uint16_t *y = static_cast<uint16_t *>(a.y);
    const uint16_t *r = static_cast<const uint16_t *>(a.r);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int n = n0 + 16 * j + 4 * g;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = bf16r(acc[j][e] * rs);
        if constexpr (EPI == PRIME_EPILOGUE_GELU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = gelu_erf_r(o[e]);
        } else if constexpr (EPI == PRIME_EPILOGUE_RESIDUAL) {
            const uint2 rv = *reinterpret_cast<const uint2 *>(r + static_cast<int64_t>(m) * a.ldr + n);
            o[0] += __uint_as_float(rv.x << 16);
            o[1] += __uint_as_float(rv.x & 0xFFFF0000u);
            o[2] += __uint_as_float(rv.y << 16);
            o[3] += __uint_as_float(rv.y & 0xFFFF0000u);
        }
        *reinterpret_cast<uint2 *>(y + static_cast<int64_t>(m) * a.ldy + n) = uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
    }
}

bool linear_rows_fits(const LinearArgs &a) { return a.N % 32 == 0 && a.K % (2 * kRK) == 0; }

template <int BN, bool RMS, int NS>
static void launch_rows_epi(const LinearArgs &a, hipStream_t stream) {
    const dim3 grid(a.N / BN, (a.M + kRM - 1) / kRM), block(256);
    if (a.epilogue == PRIME_EPILOGUE_GELU)
        hipLaunchKernelGGL((linear_rows_kernel<BN, RMS, PRIME_EPILOGUE_GELU, NS>), grid, block, 0, stream, a);
    else if (a.epilogue == PRIME_EPILOGUE_RESIDUAL)
        hipLaunchKernelGGL((linear_rows_kernel<BN, RMS, PRIME_EPILOGUE_RESIDUAL, NS>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((linear_rows_kernel<BN, RMS, PRIME_EPILOGUE_NONE, NS>), grid, block, 0, stream, a);
}


template <int NK, bool RMS>
static void launch_wholek_epi(const LinearArgs &a, hipStream_t stream) {
    const dim3 grid(a.N / 32, (a.M + kRM - 1) / kRM), block(256);
    if (a.epilogue == PRIME_EPILOGUE_GELU)
        hipLaunchKernelGGL((linear_rows_wholek_kernel<NK, RMS, PRIME_EPILOGUE_GELU>), grid, block, 0, stream, a);
    else if (a.epilogue == PRIME_EPILOGUE_RESIDUAL)
        hipLaunchKernelGGL((linear_rows_wholek_kernel<NK, RMS, PRIME_EPILOGUE_RESIDUAL>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((linear_rows_wholek_kernel<NK, RMS, PRIME_EPILOGUE_NONE>), grid, block, 0, stream, a);
}

template <int NK>
static void launch_wholek(const LinearArgs &a, hipStream_t stream) {
    if (a.rms) launch_wholek_epi<NK, true>(a, stream);
    else launch_wholek_epi<NK, false>(a, stream);
}

// K <= 768 with 32-column tiles that fill the chip in one round at most:
// every K block in flight at once.  Otherwise 64-column tiles when they give
// at least 128 workgroups, else 32, four stages.  (Measured at 256 rows in
// HIP graphs, 1.7 us of each launch being the graph's floor: the one-round
// form 3.9 us against 4.3 us for 768 -> 768; for 768 -> 2304 / 3072 it needs
// two rounds and loses, 9.3 / 11.1 us against 6.9 / 8.7 us, and eight stages
// lose too, 7.3 / 9.2 us: the LDS operand reads, each wave reading the
// workgroup's whole weight tile, bound these more than the loads do.)
hipError_t launch_linear_rows(const LinearArgs &a, hipStream_t stream) {
    const int64_t rt = (a.M + kRM - 1) / kRM, cus = device_cus();
    if (rt * (a.N / 32) <= cus) {
        switch (a.K) {
            case 256: launch_wholek<4>(a, stream); return hipGetLastError();
            case 384: launch_wholek<6>(a, stream); return hipGetLastError();
            case 512: launch_wholek<8>(a, stream); return hipGetLastError();
            case 640: launch_wholek<10>(a, stream); return hipGetLastError();
            case 768: launch_wholek<12>(a, stream); return hipGetLastError();
            default: break;
        }
    }
    const bool wide = a.N % 64 == 0 && rt * (a.N / 64) >= 128;
    if (a.rms) {
        if (wide) launch_rows_epi<64, true, 4>(a, stream);
        else launch_rows_epi<32, true, 4>(a, stream);
    } else {
        if (wide) launch_rows_epi<64, false, 4>(a, stream);
        else launch_rows_epi<32, false, 4>(a, stream);
    }
    return hipGetLastError();
}

}  // namespace prime
