// Projections of the decode step on gfx950 in the fragment layout (model.py:
// 59-68, 101-118, 160 at one token per sequence).
//
// With a few hundred rows the projections of a decode step are bound by how
// fast each CU can pull its operands, not by HBM or the MFMA rate.  Two costs
// dominate a conventional kernel: LDS staging (every wave re-reads the
// workgroup's whole weight tile, ~480 KB of LDS reads per q/k/v workgroup),
// and, for operands loaded straight into registers, the MFMA operand layout
// (lane l holds row l%16, k 8(l/16)..+7 of a 16 x 32 block: one 16-byte load
// instruction touches 16 rows x 64 bytes, half of each cache line).
//
// Here the operands are STORED in that layout ("fragment layout"): a matrix
// X[R, K] (R padded to a multiple of 16, K a multiple of 32) is a sequence of
// 16 x 32 blocks, block (R/16, K/32) in row-block-major order, each block the
// 64 lane slots of 8 bf16 an MFMA operand load wants:
//   X(r, k) at ((r/16) K/32 + k/32) * 512 + ((r%16) + 16 ((k%32)/8)) * 8 + k%8.
// A wave-wide 16-byte load of one block is one contiguous 1 KB access that
// lands in operand registers with no LDS and no shuffles.  The weights are
// packed once (prime_pack_frag); the decode step keeps its activations (the
// residual stream, the attention output, the MLP's hidden layer) in this
// layout: every producer writes it and every consumer reads it.
//
// One workgroup of NW = 8 waves owns an output tile of 16 MT rows x 16 NT
// columns over the whole of K; wave w owns the K range [w K/NW, (w+1) K/NW)
// and issues every load of that range before its first MFMA (one memory round
// trip per wave, the workgroup's operands all in flight at once).  The eight
// partial tiles meet in LDS; each thread then sums the eight partials of a
// 4-column strip and applies the epilogue:
//   RMS:      * rsqrt(mean_k x^2 + eps) per row (the RMSNorm before the
//             projection with its weight pre-multiplied into w's columns; the
//             sums of squares come from the x operands the waves load anyway);
//   bias:     + bias[n] (fp32), before the one rounding to bf16;
//   GELU:     exact-erf GELU of the rounded product, rounded again;
//   RESIDUAL: y = r + rounded product (r in y's layout; r == y in place);
//   keys:     argmax candidates of the rounded products (the greedy token of
//             the lm_head): per row, the largest key of the tile, written to
//             keys[row][tile column]; prime_linear_frag's second kernel reduces
//             them per row.
// The output is row-major [M, ldy] or, for the activations, fragment layout.
// Workgroups are numbered so that the row tiles sharing a weight tile run on
// one XCD (dispatch is round-robin over the 8 XCDs): the tile is fetched into
// that XCD's L2 once.

#include <algorithm>

#include "gemm_common.h"

namespace prime {

constexpr int kFragNW = 8;  // waves per workgroup (K split eight ways)

// MT x NT blocks of 16 x 16 outputs per workgroup, KPW 32-wide k-steps per wave
template <int MT, int NT, int NW, int KPW>
__global__ __launch_bounds__(NW * kWave) void linear_frag_kernel(const FragArgs a) {
    constexpr int NTILE = MT * NT;
    __shared__ f32x4 red[NW][NTILE][kWave];
    __shared__ float ssp[NW][16 * MT];
    __shared__ uint64_t rowkey[16 * MT];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;

    // workgroup -> (column tile, row tile): consecutive indices of one XCD
    // (i, i + 8, i + 16, ...) take the row tiles of one column tile
    const int G = gridDim.x, bi = blockIdx.x;
    const int L = (G & 7) == 0 ? (bi & 7) * (G >> 3) + (bi >> 3) : bi;
    const int tn = L / a.gm, tm = L - tn * a.gm;
    const int mb0 = tm * MT, nb0 = tn * NT;  // first 16-row block of x, of w
    if (a.keys && threadIdx.x < 16 * MT) rowkey[threadIdx.x] = 0;

    // ---- loads: every operand block of this wave's K range
    const u32x4 *xf = reinterpret_cast<const u32x4 *>(a.x) + lane;
    const u32x4 *wf = reinterpret_cast<const u32x4 *>(a.w) + lane;
    const int KS = a.KS, ks0 = wave * KPW;
    u32x4 xa[KPW][MT], wa[KPW][NT];
#pragma unroll
    for (int kk = 0; kk < KPW; ++kk) {
#pragma unroll
        for (int j = 0; j < NT; ++j)
            wa[kk][j] = wf[(static_cast<int64_t>(nb0 + j) * KS + ks0 + kk) * 64];
#pragma unroll
        for (int i = 0; i < MT; ++i) xa[kk][i] = xf[(static_cast<int64_t>(mb0 + i) * KS + ks0 + kk) * 64];
    }
    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) ss[i] = 0.f;
    const bool rms = a.rms != 0;
#pragma unroll
    for (int kk = 0; kk < KPW; ++kk) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const bf16x8 xb = as_bf16x8(xa[kk][i]);
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[i][j] = mfma(as_bf16x8(wa[kk][j]), xb, acc[i][j]);
            if (rms) ss[i] += sumsq8(xb);
        }
    }

    // ---- partial tiles and row sums of squares through LDS
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) red[wave][i * NT + j][lane] = acc[i][j];
    if (rms) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            float s = ss[i];
            s += __shfl_xor(s, 16, kWave);
            s += __shfl_xor(s, 32, kWave);
            if (lane < 16) ssp[wave][16 * i + lane] = s;
        }
    }
    __syncthreads();

    // ---- epilogue: unit u = (block ti, lane slot l) holds rows m, columns n..n+3
    const float inv_k = 1.0f / static_cast<float>(a.K);
    const int KSo = a.N >> 5;  // fragment-layout output: 32-wide steps per row
    for (int u = threadIdx.x; u < NTILE * kWave; u += NW * kWave) {
        const int ti = u >> 6, l = u & 63;
        const int i = ti / NT, j = ti - (ti / NT) * NT;
        f32x4 s = red[0][ti][l];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const f32x4 p = red[w][ti][l];
#pragma unroll
            for (int e = 0; e < 4; ++e) s[e] += p[e];
        }
        const int rl = 16 * i + (l & 15);
        const int m = 16 * mb0 + rl;
        const int n = 16 * (nb0 + j) + 4 * (l >> 4);
        float rs = 1.0f;
        if (rms) {
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) t += ssp[w][rl];
            rs = rsqrtf(t * inv_k + a.rms_eps);
        }
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = bf16r(s[e] * rs + (a.bias ? a.bias[n + e] : 0.0f));
        if (a.epilogue == PRIME_EPILOGUE_GELU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = bf16r(gelu_erf_r(o[e]));
        }
        int64_t yo;
        if (a.out_frag) yo = frag_index(m, n, KSo);
        else yo = static_cast<int64_t>(m) * a.ldy + n;
        const bool live = a.out_frag || m < a.M;  // (row-major y and r hold M rows)
        if (a.epilogue == PRIME_EPILOGUE_RESIDUAL && live) {
            const uint2 rv = *reinterpret_cast<const uint2 *>(a.r + yo);
            o[0] += __uint_as_float(rv.x << 16);
            o[1] += __uint_as_float(rv.x & 0xFFFF0000u);
            o[2] += __uint_as_float(rv.y << 16);
            o[3] += __uint_as_float(rv.y & 0xFFFF0000u);
        }
        if (a.y && live)
            *reinterpret_cast<uint2 *>(a.y + yo) = uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
        if (a.keys) {
            uint64_t best = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) best = max_u64(best, argmax_key(bf16r(o[e]), static_cast<uint32_t>(n + e)));
            atomicMax(reinterpret_cast<unsigned long long *>(&rowkey[rl]), static_cast<unsigned long long>(best));
        }
    }
    if (a.keys) {
        __syncthreads();
        if (threadIdx.x < 16 * MT) a.keys[static_cast<int64_t>(16 * mb0 + threadIdx.x) * a.gn + tn] = rowkey[threadIdx.x];
    }
}

// The lm_head (N in the tens of thousands) as a persistent kernel: one
// workgroup per CU, 4 K-quarter waves x RHN row halves; a workgroup owns a
// row tile of 16 MB RHN rows (its x operands stay in registers: MB blocks x
// KPW k-steps per wave) and a contiguous range of 16-column tiles, whose
// weight blocks stream through a ring of NBUF register sets (NBUF - 1 tiles
// in flight while one is multiplied, reduced and stored; the register budget
// is set so that nothing spills: a scratch reload would wait for every
// outstanding load).  Per column tile the four K-quarter partials meet in LDS
// (two buffers, one LDS-only barrier per tile: __syncthreads() would also
// wait for the prefetched loads); wave (kq, rh) then finishes the tile's
// 16-row block kq of its half (MB = 4) or half of one (MB = 2, the waves
// kq and kq ^ 1 sharing rows), so its argmax candidates are a running maximum
// in registers, folded per row through LDS at the end and written once to
// keys[row][workgroup slot].
template <int MB, int RHN, int KPW>
__global__ __launch_bounds__(4 * RHN * kWave) void lm_head_frag_kernel(const FragArgs a) {
    constexpr int KQ = 4, NBUF = 4;
    static_assert(MB == 4 || MB == 2, "row blocks per half");
    __shared__ f32x4 red[2][KQ][RHN][MB][kWave];
    __shared__ float ssp[KQ][RHN][16 * MB];
    __shared__ unsigned long long rowkey[16 * MB * RHN];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int kq = wave & (KQ - 1), rh = wave / KQ;
    const int G = gridDim.x, bi = blockIdx.x;
    // workgroup -> (row tile, column-tile range): the row tiles of one range on one XCD
    const int L = (G & 7) == 0 ? (bi & 7) * (G >> 3) + (bi >> 3) : bi;
    const int rt = L % a.gm, slot = L / a.gm, nslot = G / a.gm;
    const int ntiles = a.N / 16;
    const int j0 = static_cast<int>(static_cast<int64_t>(ntiles) * slot / nslot);
    const int j1 = static_cast<int>(static_cast<int64_t>(ntiles) * (slot + 1) / nslot);
    const int KS = a.KS, ks0 = kq * KPW;
    const int mb0 = rt * MB * RHN + rh * MB;  // first 16-row block of this wave's half
    // the row block this wave finishes: MB = 4, block kq; MB = 2, block kq / 2 (column
    // lanes 32 (kq & 1) .. +31 of it: each lane group g covers 4 columns, and the
    // two waves split the lane groups g = 0, 1 and 2, 3)
    const int fb = MB == 4 ? kq : kq >> 1;
    const bool half_mine = MB == 4 || ((lane >> 5) == (kq & 1));
    if (threadIdx.x < 16 * MB * RHN) rowkey[threadIdx.x] = 0ull;
    const u32x4 *xf = reinterpret_cast<const u32x4 *>(a.x) + lane;
    const u32x4 *wf = reinterpret_cast<const u32x4 *>(a.w) + lane;

    u32x4 xr[KPW][MB];
#pragma unroll
    for (int kk = 0; kk < KPW; ++kk)
#pragma unroll
        for (int i = 0; i < MB; ++i) xr[kk][i] = xf[(static_cast<int64_t>(mb0 + i) * KS + ks0 + kk) * 64];
    // row sums of squares over the wave's K quarter, then over the quarters (LDS)
    float rs = 1.0f;
    {
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            float ss = 0.f;
#pragma unroll
            for (int kk = 0; kk < KPW; ++kk) ss += sumsq8(as_bf16x8(xr[kk][i]));
            ss += __shfl_xor(ss, 16, kWave);
            ss += __shfl_xor(ss, 32, kWave);
            if (lane < 16) ssp[kq][rh][16 * i + lane] = ss;
        }
        __syncthreads();
        float tt = 0.f;
#pragma unroll
        for (int q = 0; q < KQ; ++q) tt += ssp[q][rh][16 * fb + (lane & 15)];
        if (a.rms) rs = rsqrtf(tt / static_cast<float>(a.K) + a.rms_eps);
    }

    u32x4 w[NBUF][KPW];
    auto loadw = [&](u32x4(&ws)[KPW], int j) {
#pragma unroll
        for (int kk = 0; kk < KPW; ++kk) ws[kk] = wf[(static_cast<int64_t>(j) * KS + ks0 + kk) * 64];
    };
    uint64_t best = 0;
    const int m = 16 * (mb0 + fb) + (lane & 15);
    auto tile = [&](const u32x4(&ws)[KPW], int j) {
        const int buf = j & 1;
        f32x4 acc[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KPW; ++kk)
#pragma unroll
            for (int i = 0; i < MB; ++i) acc[i] = mfma(as_bf16x8(ws[kk]), as_bf16x8(xr[kk][i]), acc[i]);
#pragma unroll
        for (int i = 0; i < MB; ++i) red[buf][kq][rh][i][lane] = acc[i];
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        f32x4 sum = red[buf][0][rh][fb][lane];
#pragma unroll
        for (int q = 1; q < KQ; ++q) {
            const f32x4 p = red[buf][q][rh][fb][lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[e] += p[e];
        }
        if (half_mine) {
            const int col = 16 * j + 4 * (lane >> 4);
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = bf16r(sum[e] * rs);
            if (a.y && m < a.M)
                *reinterpret_cast<uint2 *>(a.y + static_cast<int64_t>(m) * a.ldy + col) =
                    uint2{pack2(o[0], o[1]), pack2(o[2], o[3])};
#pragma unroll
            for (int e = 0; e < 4; ++e) best = max_u64(best, argmax_key(o[e], static_cast<uint32_t>(col + e)));
        }
    };
    // ring of NBUF weight sets: set (b - 1) mod NBUF, free once tile j + b - 1
    // was multiplied, takes tile j + b + NBUF - 1
#pragma unroll
    for (int b = 0; b < NBUF - 1; ++b)
        if (j0 + b < j1) loadw(w[b], j0 + b);
    for (int j = j0; j < j1; j += NBUF) {
#pragma unroll
        for (int b = 0; b < NBUF; ++b) {
            if (j + b < j1) {
                if (j + b + NBUF - 1 < j1) loadw(w[(b + NBUF - 1) % NBUF], j + b + NBUF - 1);
                tile(w[b], j + b);
            }
        }
    }
    if (a.keys) {
        // per row: the lane groups of a wave, then the waves sharing rows (LDS max)
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {
            const uint32_t lo = __shfl_xor(static_cast<uint32_t>(best), o, kWave);
            const uint32_t hi = __shfl_xor(static_cast<uint32_t>(best >> 32), o, kWave);
            best = max_u64(best, (static_cast<uint64_t>(hi) << 32) | lo);
        }
        if (lane < 16) atomicMax(&rowkey[16 * (rh * MB + fb) + lane], static_cast<unsigned long long>(best));
        __syncthreads();
        if (threadIdx.x < 16 * MB * RHN)
            a.keys[static_cast<int64_t>(16 * rt * MB * RHN + threadIdx.x) * a.gn + slot] = rowkey[threadIdx.x];
    }
}

// the greedy token per row: the largest of the row's gn tile keys (one wave per row)
__global__ __launch_bounds__(256) void frag_argmax_reduce_kernel(const uint64_t *__restrict__ keys, int gn, int M,
                                                                int64_t *__restrict__ tokens) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;
    uint64_t best = 0;
    for (int t = lane; t < gn; t += kWave) best = max_u64(best, keys[static_cast<int64_t>(row) * gn + t]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(best), o, kWave);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(best >> 32), o, kWave);
        best = max_u64(best, (static_cast<uint64_t>(hi) << 32) | lo);
    }
    if (lane == 0) tokens[row] = static_cast<int64_t>(~static_cast<uint32_t>(best));
}

// out (fragment layout, Mp rows) <- rows of a row-major bf16 matrix, row r
// taken from src row idx[r] (or r), rows M .. Mp-1 zero; one 16-byte lane slot
// per thread
__global__ __launch_bounds__(256) void pack_frag_kernel(const uint16_t *__restrict__ src, int64_t ld,
                                                       const int64_t *__restrict__ idx, int M, int Mp, int K,
                                                       int64_t nrows_src, uint16_t *__restrict__ out) {
    const int KS = K >> 5;
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // (block, lane)
    const int64_t nslots = static_cast<int64_t>(Mp >> 4) * KS * 64;
    if (slot >= nslots) return;
    const int64_t blk = slot >> 6;
    const int l = static_cast<int>(slot & 63);
    const int rb = static_cast<int>(blk / KS), ks = static_cast<int>(blk - static_cast<int64_t>(rb) * KS);
    const int r = 16 * rb + (l & 15), k = 32 * ks + 8 * (l >> 4);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < M) {
        int64_t sr = idx ? idx[r] : r;
        if (sr >= 0 && sr < nrows_src) v = *reinterpret_cast<const u32x4 *>(src + sr * ld + k);
    }
    *reinterpret_cast<u32x4 *>(out + slot * 8) = v;
}

namespace {

template <int MT, int NT, int KPW>
void launch_tile(const FragArgs &a, hipStream_t s) {
    hipLaunchKernelGGL((linear_frag_kernel<MT, NT, kFragNW, KPW>), dim3(a.gm * a.gn), dim3(kFragNW * kWave), 0, s, a);
}

template <int MT, int NT>
bool launch_kpw(const FragArgs &a, hipStream_t s) {
    switch (a.KS / kFragNW) {
        case 1: launch_tile<MT, NT, 1>(a, s); return true;
        case 2: launch_tile<MT, NT, 2>(a, s); return true;
        case 3: launch_tile<MT, NT, 3>(a, s); return true;
        case 4: launch_tile<MT, NT, 4>(a, s); return true;
        case 6: launch_tile<MT, NT, 6>(a, s); return true;
        case 12: launch_tile<MT, NT, 12>(a, s); return true;
        default: return false;
    }
}

}  // namespace

// Tile of the workgroup: 32 x 32 outputs where that gives at least half a
// workgroup per CU (the decode step's projections at 256 rows: 192 to 768
// workgroups, several resident per CU), 32 x 16 where that does, 16 x 16
// otherwise (the o and down projections at 32 rows: 96 workgroups instead of
// 48; the B = 32 step 0.350 -> 0.336 ms).  (Measured at 256 rows: 64 x 64
// tiles, one workgroup per CU, are no faster for the q/k/v projection and
// slower for the up projection.)
void frag_tile(int Mp, int N, int K, int *MT, int *NT) {
    (void)K;
    const int64_t cus = device_cus();
    if (Mp % 32 == 0 && N % 32 == 0 && static_cast<int64_t>(Mp / 32) * (N / 32) >= cus / 2) {
        *MT = 2; *NT = 2;
    } else if (Mp % 32 == 0 && static_cast<int64_t>(Mp / 32) * (N / 16) >= cus / 2) {
        *MT = 2; *NT = 1;
    } else {
        *MT = 1; *NT = 1;
    }
}

bool frag_k_supported(int K) {
    if (K % (32 * kFragNW)) return false;
    const int kpw = K / (32 * kFragNW);
    return kpw == 1 || kpw == 2 || kpw == 3 || kpw == 4 || kpw == 6 || kpw == 12;
}

namespace {

template <int MB, int RHN>
bool launch_lm(const FragArgs &a, hipStream_t s) {
    const dim3 g(a.gm * a.gn), b(4 * RHN * kWave);
    switch (a.KS / 4) {
        case 2: hipLaunchKernelGGL((lm_head_frag_kernel<MB, RHN, 2>), g, b, 0, s, a); return true;
        case 4: hipLaunchKernelGGL((lm_head_frag_kernel<MB, RHN, 4>), g, b, 0, s, a); return true;
        case 6: hipLaunchKernelGGL((lm_head_frag_kernel<MB, RHN, 6>), g, b, 0, s, a); return true;
        default: return false;
    }
}

}  // namespace

// Plan of a call: the persistent lm_head kernel for wide outputs (N >= 8192;
// K = 256, 512 or 768): row tiles of 128 rows (32 when
// the padded rows are not a multiple of 128) x the column-tile ranges of one
// workgroup per CU; otherwise the tile kernel.
void frag_plan(FragArgs &a) {
    const int KS = a.K / 32;
    a.persistent = a.N >= 8192 && KS % 4 == 0 && (KS / 4 == 2 || KS / 4 == 4 || KS / 4 == 6);
    if (a.persistent) {
        const bool wide = a.Mp % 128 == 0;
        a.mt = wide ? 4 : 2;  // m-blocks per row half
        a.nt = wide ? 2 : 1;  // row halves
        a.gm = a.Mp / (wide ? 128 : 32);
        int G = static_cast<int>(device_cus());
        G -= G % (8 * a.gm);
        if (G < 8 * a.gm) G = 8 * a.gm;
        a.gn = std::min(G / a.gm, a.N / 16);  // column-tile ranges (workgroups per row tile)
        return;
    }
    frag_tile(a.Mp, a.N, a.K, &a.mt, &a.nt);
    a.gm = a.Mp / (16 * a.mt);
    a.gn = a.N / (16 * a.nt);
}

hipError_t launch_linear_frag(const FragArgs &a, hipStream_t s) {
    bool ok;
    if (a.persistent) ok = a.mt == 4 ? launch_lm<4, 2>(a, s) : launch_lm<2, 1>(a, s);
    else if (a.mt == 2 && a.nt == 2) ok = launch_kpw<2, 2>(a, s);
    else if (a.mt == 2 && a.nt == 1) ok = launch_kpw<2, 1>(a, s);
    else if (a.mt == 1 && a.nt == 1) ok = launch_kpw<1, 1>(a, s);
    else ok = false;
    if (!ok) return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !a.tokens) return e;
    hipLaunchKernelGGL(frag_argmax_reduce_kernel, dim3((a.M + 3) / 4), dim3(256), 0, s, a.keys, a.gn, a.M, a.tokens);
    return hipGetLastError();
}

hipError_t launch_pack_frag(const uint16_t *src, int64_t ld, const int64_t *idx, int M, int Mp, int K,
                            int64_t nrows_src, uint16_t *out, hipStream_t s) {
    const int64_t nslots = static_cast<int64_t>(Mp / 16) * (K / 32) * 64;
    hipLaunchKernelGGL(pack_frag_kernel, dim3(static_cast<unsigned>((nslots + 255) / 256)), dim3(256), 0, s, src, ld,
                       idx, M, Mp, K, nrows_src, out);
    return hipGetLastError();
}

}  // namespace prime
