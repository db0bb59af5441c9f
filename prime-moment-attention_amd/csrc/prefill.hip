// Chunked PRIME prefill on bf16 MFMA (gfx950).
//
// Semantics: chunked_prime_ssd_core (chunked_ssd.py:48-184) of the reference,
// and with PRIME_FLAG_DENSE_CLAMP the module's dense branch
// (attention.py:160-202).  Per (b,h), tokens are processed in 64-token chunks.
// With query/key features Fq_i = [q_i, q_i*q_i], Fk_j = [k_j, k_j*k_j/2]
// (128 wide) and the state kept as M = [S1; S2/2] (128 x 64) plus the K state
// [K1; K2/2]:
//   A_ij  = l^(i-j) [i>=j] (1 + Fq_i . Fk_j)                        (intra block)
//   num_i = sum_j A_ij v_j + l^(i+1) (S0 + Fq_i M)
//   den_i = sum_j A_ij     + l^(i+1) (K0 + Fq_i . [K1; K2/2])
//   y_i   = num_i / max(den_i, eps)
//   M    <- l^n M + sum_j Fk_j^T (w_j v_j),  w_j = l^(n-1-j)  (n valid tokens)
// The reference's O(Nc^2) inter-chunk matrix (chunked_ssd.py:113-126) is the
// closed form of this carried scan; padding is exact because decays use the
// number of valid tokens, which equals the reference's l^(-pad) correction
// (chunked_ssd.py:171-178).
//
// Layout and mapping.  One workgroup per (sequence, segment) with two roles:
//   readout waves 0..3 own query rows [16w, 16w+16): score block S^T = Fk Fq^T,
//     y^T = V^T A^T + M^T Fq^T (computed transposed so each lane holds its own
//     query row and four consecutive value columns), y stores;
//   update waves 4..7 own feature rows [32u, 32u+32) of M in fp32 MFMA
//     accumulators and add each chunk's Fk^T (w v).
// q/k/v tiles stay row-major in LDS (16-byte stores).  Operands contracted over
// the token index are read with ds_read_b64_tr_b16: in a 16-lane group, lane s
// addresses X[r0 + s/4][c0 + 4(s%4)] and lane i receives X[r0 + e][c0 + i],
// e = 0..3, i.e. four consecutive tokens of one column.  A 16-column block
// whose first column is 1 (w in the update) rides along every product and
// yields the intra denominator, the K state and its readout on MFMA.
// Per chunk: barrier; both roles issue the next chunk's HBM loads (readout: q
// and k, update: v; 8 whole 128-byte rows per wave load), then compute;
// barrier; the update role publishes the bf16 state copy while both roles
// write the next chunk's tiles to LDS.
//
// Precision: bf16 inputs enter the MFMA exactly; derived operands (squares,
// the score block, the state copy, w v) are rounded to bf16 once.  fp32 inputs
// (F32IN) keep every LDS array as a bf16 hi plane plus a lo residual plane and
// accumulate hi*hi + hi*lo + lo*hi (three MFMAs per product, ~2^-16 relative).

#include <algorithm>
#include <functional>
#include <mutex>
#include <vector>

#include "prefill_common.h"

namespace prime {

// one 8-element row segment of a q/k/v tile, kept packed until it is stored
template <bool F32IN>
struct Seg8;
template <>
struct Seg8<false> {
    u32x4 r;
};
template <>
struct Seg8<true> {
    f32x4 a, b;
};

// Unconditional load of an in-bounds row (rows past L are clamped to row L-1
// by the caller).  Rows that are not part of the chunk are zeroed when the
// tile is stored to LDS, not here: a select on the loaded value right after
// the load would make the wave wait for the load before its chunk's compute,
// and a conditional load lets the optimiser merge the stores into a pointer
// select and keep the prefetch registers in scratch memory.
template <bool F32IN>
__device__ __forceinline__ Seg8<F32IN> load_seg(const void *base, int64_t off) {
    Seg8<F32IN> s;
    if constexpr (!F32IN) {
        s.r = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(base) + off);
    } else {
        const f32x4 *p = reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + off);
        s.a = p[0];
        s.b = p[1];
    }
    return s;
}

__device__ __forceinline__ void seg_f32(const Seg8<false> &s, float (&f)[8]) { unpack8(s.r, f); }
__device__ __forceinline__ void seg_f32(const Seg8<true> &s, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = s.a[i];
        f[4 + i] = s.b[i];
    }
}

// store 8 fp32 as bf16 (hi plane, lo plane when S) at p
template <bool S>
__device__ __forceinline__ void put8(uint16_t *p, size_t plane, const float (&f)[8]) {
    u32x4 hi, lo;
    split_pack<S>(f, hi, lo);
    *reinterpret_cast<u32x4 *>(p) = hi;
    if constexpr (S) *reinterpret_cast<u32x4 *>(p + plane) = lo;
}

template <bool S>
__device__ __forceinline__ void put1(uint16_t *p, size_t plane, float x) {
    const uint16_t hb = f32_to_bf16_bits(x);
    *p = hb;
    if constexpr (S) p[plane] = f32_to_bf16_bits(x - bf16_bits_to_f32(hb));
}

// Registers holding the next chunk's tiles (kept packed until stored).  Each
// role's 256 threads read rows rt/8 and rt/8 + 32, 16-byte segment rt%8, so a
// wave's load covers 8 whole 128-byte rows.  Both roles fill the same four
// slots -- readout: q -> r0,r1 and k -> r2,r3; update: v -> r0,r1 and k
// (state-only launch) or zero -> r2,r3 -- so that no role branch leaves a slot
// unwritten (which makes the optimiser keep the slots in scratch memory behind
// a pointer select).
template <bool F32IN>
struct TileRegs {
    Seg8<F32IN> r0, r1, r2, r3;
};

template <bool F32IN, bool STATE_ONLY>
__device__ __forceinline__ void load_tiles_fn(const PrefillArgs &a, TileRegs<F32IN> &R, int c, int rt, bool is_u,
                                              int64_t qb, int64_t kb, int64_t vb) {
    const int col = 8 * (rt & 7);
    const int ta = c * kC + (rt >> 3), tb = ta + 32;
    const int sa = min(ta, a.L - 1), sb = min(tb, a.L - 1);  // in-bounds rows
    const void *x = is_u ? a.v : a.q;
    const int64_t xb = is_u ? vb : qb, xl = is_u ? a.v_sl : a.q_sl;
    R.r0 = load_seg<F32IN>(x, xb + sa * xl + col);
    R.r1 = load_seg<F32IN>(x, xb + sb * xl + col);
    // update waves of the fused kernel need no k: they re-read their v rows (L1
    // hits) into the k slots, which they never store
    const bool want_k = !is_u || STATE_ONLY;
    const void *kx = want_k ? a.k : x;
    const int64_t kbb = want_k ? kb : xb, kl = want_k ? a.k_sl : xl;
    R.r2 = load_seg<F32IN>(kx, kbb + sa * kl + col);
    R.r3 = load_seg<F32IN>(kx, kbb + sb * kl + col);
}

// One 8-column segment of one token row: q -> [q | q*q], k -> [k | k*k/2],
// v -> v and w v (plus w itself in column 64 from the segment-0 thread).
template <bool F32IN>
__device__ __forceinline__ void seg_f32_masked(const Seg8<F32IN> &s, bool valid, float (&f)[8]) {
    seg_f32(s, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = valid ? f[e] : 0.f;
}

// Rows past the chunk's valid tokens (valid == false) are stored as zeros.
template <bool F32IN, bool STATE_ONLY>
__device__ __forceinline__ void store_seg_fn(const Seg8<F32IN> &x01, const Seg8<F32IN> &k, int row, int col,
                                             bool valid, bool is_u, float w, uint16_t *sQf, size_t plQ,
                                             uint16_t *sKf, size_t plK, int kPK, uint16_t *sV, size_t plV,
                                             uint16_t *sVw, size_t plVw, int kPV) {
    constexpr bool S = F32IN;
    float x[8], y2[8];
    if (!is_u || STATE_ONLY) {
        if (!is_u) {
            seg_f32_masked(x01, valid, x);
            put8<S>(sQf + row * kPW + col, plQ, x);
#pragma unroll
            for (int e = 0; e < 8; ++e) y2[e] = x[e] * x[e];
            put8<S>(sQf + row * kPW + kD + col, plQ, y2);
        }
        seg_f32_masked(k, valid, x);
        put8<S>(sKf + row * kPK + col, plK, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) y2[e] = 0.5f * x[e] * x[e];
        put8<S>(sKf + row * kPK + kD + col, plK, y2);
    }
    if (is_u) {
        seg_f32_masked(x01, valid, x);
        if constexpr (!STATE_ONLY) put8<S>(sV + row * kPV + col, plV, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) y2[e] = w * x[e];
        put8<S>(sVw + row * kPV + col, plVw, y2);
        if (col == 0) put1<S>(sVw + row * kPV + kD, plVw, w);
    }
}

template <bool F32IN, bool STATE_ONLY>
__device__ __forceinline__ void store_tiles_fn(const TileRegs<F32IN> &R, int rt, bool is_u, const float *sPw,
                                               int nvalid, uint16_t *sQf, size_t plQ, uint16_t *sKf, size_t plK,
                                               int kPK, uint16_t *sV, size_t plV, uint16_t *sVw, size_t plVw,
                                               int kPV) {
    const int col = 8 * (rt & 7);
    const int ra = rt >> 3, rb = ra + 32;
    const float wa = ra < nvalid ? sPw[nvalid - 1 - ra] : 0.f;
    const float wb = rb < nvalid ? sPw[nvalid - 1 - rb] : 0.f;
    store_seg_fn<F32IN, STATE_ONLY>(R.r0, R.r2, ra, col, ra < nvalid, is_u, wa, sQf, plQ, sKf, plK, kPK, sV, plV,
                                    sVw, plVw, kPV);
    store_seg_fn<F32IN, STATE_ONLY>(R.r1, R.r3, rb, col, rb < nvalid, is_u, wb, sQf, plQ, sKf, plK, kPK, sV, plV,
                                    sVw, plVw, kPV);
}

// Segment plan.  Without a workspace (or for the dense branch, whose clamp
// needs the incoming state apart from the tokens of this call) every sequence
// is one segment.  Otherwise choose the number of segments G minimising a
// simple cost in chunk-steps: the fused kernel runs one workgroup per CU, in
// ceil(S*G / CUs) rounds of cps chunks each; the state-only pass (about half
// the cost per chunk, several workgroups per CU) and the scan add the rest,
// and every workspace slot costs ~4 x 33.8 KB of HBM traffic (~0.03 chunk-steps).
constexpr int kMinCps = 4;

int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

void plan_segments(int S, int L, bool dense_clamp, size_t ws_bytes, int *G, int *cps) {
    const int NC = (L + kC - 1) / kC;
    int best_g = 1, best_c = NC;
    if (!dense_clamp && NC >= 2 * kMinCps) {
        const int cu = device_cus();
        const int gmax = NC / kMinCps < 64 ? NC / kMinCps : 64;
        double best = 1e300;
        for (int g0 = 1; g0 <= gmax; ++g0) {
            const int c = (NC + g0 - 1) / g0;
            const int g = (NC + c - 1) / c;  // no empty segments
            if (g > 1 && static_cast<size_t>(S) * g * kWsStride * sizeof(float) > ws_bytes) continue;
            const double rounds = static_cast<double>((static_cast<int64_t>(S) * g + cu - 1) / cu);
            double cost = rounds * c;
            if (g > 1)
                cost += 0.5 * static_cast<double>((static_cast<int64_t>(S) * (g - 1) + 4 * cu - 1) / (4 * cu)) * c +
                        1.0 + 0.03 * S * g;
            if (cost < best - 1e-9) {
                best = cost;
                best_g = g;
                best_c = c;
            }
        }
    }
    *G = best_g;
    *cps = best_c;
}

// Paired split.  With more sequences S than CUs the fused kernel (one
// workgroup per CU) runs ceil(S / CUs) rounds of whole sequences, the last one
// partly empty (384 sequences on 256 CUs: two rounds of work for 1.5).  Cutting
// K sequences into a first part of pcs chunks and a second part, launched
// [K first parts][S - K whole][K second parts], lets the in-order dispatch
// pack them (at 1.5 x CUs: half the CUs run a first part and then a whole
// sequence, the other half a whole sequence and then a second part, whose
// first part ended long before).  The plan comes from simulating that
// dispatch (each unit to the CU that frees first; a second part starts no
// earlier than its first part's end) in chunk-steps, with half a chunk-step
// per workgroup for its prologue and state I/O; a plan must beat whole
// sequences by 3 %.  Plans are cached per (S, chunks, CUs).
namespace {

double simulate_pairs(int S, int NC, int cu, int K, int pcs) {
    constexpr double kUnit = 0.5;
    std::vector<double> cpu(static_cast<size_t>(cu), 0.0);  // min-heap of CU free times
    std::vector<double> first_end(static_cast<size_t>(K), 0.0);
    auto run = [&](double len, double ready) {
        std::pop_heap(cpu.begin(), cpu.end(), std::greater<double>());
        const double end = std::max(cpu.back(), ready) + len + kUnit;
        cpu.back() = end;
        std::push_heap(cpu.begin(), cpu.end(), std::greater<double>());
        return end;
    };
    double span = 0.0;
    for (int i = 0; i < K; ++i) span = std::max(span, first_end[static_cast<size_t>(i)] = run(pcs, 0.0));
    for (int i = K; i < S; ++i) span = std::max(span, run(NC, 0.0));
    for (int i = 0; i < K; ++i) span = std::max(span, run(NC - pcs, first_end[static_cast<size_t>(i)]));
    return span;
}

struct PairPlan {
    int S, NC, cu, K, pcs;
};
std::mutex g_pair_mu;
std::vector<PairPlan> g_pair_cache;

}  // namespace

void plan_pairs(int S, int L, int *K, int *pcs) {
    const int NC = (L + kC - 1) / kC;
    const int cu = device_cus();
    *K = 0;
    *pcs = NC;
    if (S <= cu || NC < 2) return;
    std::lock_guard<std::mutex> lock(g_pair_mu);
    for (const PairPlan &p : g_pair_cache)
        if (p.S == S && p.NC == NC && p.cu == cu) {
            *K = p.K;
            *pcs = p.pcs;
            return;
        }
    const double whole = simulate_pairs(S, NC, cu, 0, NC);
    double best = 0.97 * whole;
    int best_k = 0, best_p = NC;
    const int kmax = std::min(S, cu), step = std::max(1, cu / 64);
    const int cand[5] = {NC / 2, NC / 3, (2 * NC) / 3, NC / 4, (3 * NC) / 4};
    for (int k = step; k <= kmax; k += step)
        for (int p : cand) {
            if (p < 1 || p >= NC) continue;
            const double t = simulate_pairs(S, NC, cu, k, p);
            if (t < best - 1e-9) {
                best = t;
                best_k = k;
                best_p = p;
            }
        }
    if (g_pair_cache.size() >= 64) g_pair_cache.clear();
    g_pair_cache.push_back(PairPlan{S, NC, cu, best_k, best_p});
    *K = best_k;
    *pcs = best_p;
}

// One workgroup = (sequence, segment); see the header comment.  STATE_ONLY
// launches the update role alone (4 waves, which also write the k tile) from
// a zero state and stores the segment's contribution in its workspace slot.
template <bool F32IN, bool STATE_ONLY>
__global__ __launch_bounds__(512, 1) void prefill_kernel(const PrefillArgs a) {
    constexpr bool S = F32IN;        // split operands
    constexpr int NP = S ? 2 : 1;    // LDS planes (hi, lo)
    constexpr int NB = kD / 16;      // value blocks
    constexpr int NBX = NB + 1;      // + the ones / K block
    constexpr int QR = STATE_ONLY ? 1 : kC;
    constexpr int SR = STATE_ONLY ? 1 : kD + 1;  // state copy rows: 64 value columns + K
    constexpr int kPK = F32IN ? kPW : kPT;       // sKf pitch (16-byte rows and transposed reads)
    constexpr int kPV = F32IN ? kD + 24 : kPT;   // v pitch: 64 values + the 16-wide ones block

    __shared__ __attribute__((aligned(16))) uint16_t sQf[NP][QR][kPW];   // [q | q*q]
    __shared__ __attribute__((aligned(16))) uint16_t sKf[NP][kC][kPK];   // [k | k*k/2]
    __shared__ __attribute__((aligned(16))) uint16_t sV[NP][QR][kPV];    // [v | 1 0..0]
    __shared__ __attribute__((aligned(16))) uint16_t sVw[NP][kC][kPV];   // [w v | w 0..0]
    __shared__ __attribute__((aligned(16))) uint16_t sSt[NP][SR][kPW];   // bf16 [S1; S2/2 | K]^T
    __shared__ float sPw[kC + 2];                                         // l^n, n = 0..65
    __shared__ float sPs[kC + 2];                                         // sum_{m<n} l^m
    __shared__ __attribute__((aligned(16))) float sS0[kD];
    __shared__ float sKi[kF];                                             // incoming [K1; K2/2] (dense)
    __shared__ float sK0[2];                                              // K0 of the call / incoming
    constexpr size_t plQ = static_cast<size_t>(QR) * kPW, plK = static_cast<size_t>(kC) * kPK;
    constexpr size_t plV = static_cast<size_t>(QR) * kPV, plVw = static_cast<size_t>(kC) * kPV;
    constexpr size_t plS = static_cast<size_t>(SR) * kPW;

    const int tid = threadIdx.x;
    // wave index in a scalar register: every role / wave test below is then a
    // scalar branch, so no MFMA runs under a partial or empty EXEC mask
    // (MFMAs write their whole destination regardless of EXEC)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const bool is_u = STATE_ONLY || wave >= 4;
    const int u = STATE_ONLY ? wave : wave - 4;  // update-wave index
    const int utid = 64 * u + lane;              // thread index within the update role
    const int tr_r = c16 >> 2, tr_c = 4 * (c16 & 3);  // ds_read_tr address offsets of this lane

    const int Sq = a.B * a.H;
    const int unit = blockIdx.x;
    if (unit >= Sq * a.nseg_launch) return;  // whole workgroup leaves before any barrier
    const int seq = unit / a.nseg_launch, seg = unit - seq * a.nseg_launch;
    const int b = seq / a.H, h = seq - b * a.H, hk = h / a.group;
    const float lam = a.decay[h];
    const int NC = (a.L + kC - 1) / kC;
    const int c_begin = seg * a.cps;
    const int c_end = min(c_begin + a.cps, NC);
    const bool from_ws = !STATE_ONLY && a.G > 1;
    const bool has_in = !STATE_ONLY && !from_ws && a.s1i != nullptr;
    const bool dense = !STATE_ONLY && a.dense_clamp;
    float *wslot = a.ws ? a.ws + (static_cast<size_t>(seq) * a.G + seg) * kWsStride : nullptr;

    if (tid < kC + 2) {
        const double ld = static_cast<double>(lam);
        sPw[tid] = static_cast<float>(pow(ld, static_cast<double>(tid)));
        double ps = 0.0, pm = 1.0;  // prefix sum of powers in fp64 (1 - l is tiny near l = 1)
        for (int m = 0; m < tid; ++m, pm *= ld) ps += pm;
        sPs[tid] = static_cast<float>(ps);
    }
    __syncthreads();  // the power tables are read by the first store_tiles below

    // ---- initial state (update role): M = [S1; S2/2], K block = [K1; K2/2]
    const size_t so1 = static_cast<size_t>(seq) * kD * kD;
    const size_t so0 = static_cast<size_t>(seq) * kD;
    f32x4 st[2][NBX];  // feature blocks 2u+fi (rows 4g+r), value blocks nb (column c16)
    if (is_u) {
#pragma unroll
        for (int fi = 0; fi < 2; ++fi)
#pragma unroll
            for (int nb = 0; nb < NBX; ++nb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int f = 16 * (2 * u + fi) + 4 * g + r, fr = f & (kD - 1);
                    const int n = 16 * nb + c16;
                    float x = 0.f;
                    if (n < kD) {
                        if (from_ws) x = wslot[(f < kD ? kWsS1 : kWsS2) + fr * kD + n];
                        else if (has_in) x = (f < kD ? a.s1i : a.s2i)[so1 + fr * kD + n];
                    } else if (n == kD && !dense) {  // dense: K of the call only, incoming in sKi
                        if (from_ws) x = wslot[(f < kD ? kWsK1 : kWsK2) + fr];
                        else if (has_in) x = (f < kD ? a.k1i : a.k2i)[so0 + fr];
                    }
                    st[fi][nb][r] = f < kD ? x : 0.5f * x;
                }
        if (utid < kD) {
            sS0[utid] = from_ws ? wslot[kWsS0 + utid] : (has_in ? a.s0i[so0 + utid] : 0.f);
        } else if (utid < kD + kF) {
            const int f = utid - kD, fr = f & (kD - 1);
            float x = 0.f;
            if (dense && has_in) x = (f < kD ? a.k1i : a.k2i)[so0 + fr];
            sKi[f] = f < kD ? x : 0.5f * x;
        } else if (utid == kD + kF) {
            const float x = from_ws ? wslot[kWsK0] : (has_in ? a.k0i[seq] : 0.f);
            sK0[0] = dense ? 0.f : x;
            sK0[1] = dense ? x : 0.f;
        }
        // constant columns 64..79 of v (1, 0, ...) and 65..79 of w v (column 64,
        // w, is written with every chunk's tile, racing nothing here)
        for (int idx = utid; idx < kC * 16; idx += 256) {
            const int row = idx >> 4, col = kD + (idx & 15);
            for (int p = 0; p < NP; ++p) {
                if constexpr (!STATE_ONLY) sV[p][row][col] = (col == kD && p == 0) ? 0x3F80u : 0u;
                if (col != kD) sVw[p][row][col] = 0u;
            }
        }
    }
    // bf16 (hi[, lo]) copy of the state for the readout (rows 0..64)
    auto write_state_copy = [&]() {
        if constexpr (!STATE_ONLY) {
#pragma unroll
            for (int fi = 0; fi < 2; ++fi) {
                const int f = 16 * (2 * u + fi) + 4 * g;
#pragma unroll
                for (int nb = 0; nb < NBX; ++nb) {
                    const int n = 16 * nb + c16;
                    if (n > kD) continue;  // columns 65..79 of the ones block are zero
                    const f32x4 x = st[fi][nb];
                    const uint32_t h0 = pack2(x[0], x[1]), h1 = pack2(x[2], x[3]);
                    *reinterpret_cast<uint2 *>(&sSt[0][n][f]) = uint2{h0, h1};
                    if constexpr (S) {
                        float lo[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) lo[r] = x[r] - bf16_bits_to_f32(f32_to_bf16_bits(x[r]));
                        *reinterpret_cast<uint2 *>(&sSt[NP - 1][n][f]) = uint2{pack2(lo[0], lo[1]), pack2(lo[2], lo[3])};
                    }
                }
            }
        }
    };
    if (is_u) write_state_copy();

    // ---- readout-role constants (query row of the lane: iw)
    const int iw = 16 * wave + c16;
    float mask[4][4];  // l^(i-j) [i >= j] for S^T[j = 16jb + 4g + r][i = iw]
    float pin = 0.f;   // l^(iw+1)
    if (!is_u) {  // from the power table (sPw[n]: l^n rounded from fp64)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = iw - (16 * jb + 4 * g + r);
                mask[jb][r] = (jb <= wave && d >= 0) ? sPw[max(d, 0)] : 0.f;
            }
        pin = sPw[iw + 1];
    }

    // ---- tiles: readout waves load q, k; update waves load v (and k when STATE_ONLY).
    const int64_t qb = b * a.q_sb + h * a.q_sh, kb = b * a.k_sb + hk * a.k_sh, vb = b * a.v_sb + hk * a.v_sh;
    const int rt = tid & 255;  // thread index within the role
    TileRegs<F32IN> R;
#define PRIME_LOAD_TILES(c) load_tiles_fn<F32IN, STATE_ONLY>(a, R, (c), rt, is_u, qb, kb, vb)
#define PRIME_STORE_TILES(c)                                                                                       \
    store_tiles_fn<F32IN, STATE_ONLY>(R, rt, is_u, sPw, min(kC, a.L - (c) * kC), &sQf[0][0][0], plQ, &sKf[0][0][0], \
                                      plK, kPK, &sV[0][0][0], plV, &sVw[0][0][0], plVw, kPV)

    PRIME_LOAD_TILES(c_begin);
    PRIME_STORE_TILES(c_begin);
    __syncthreads();

    for (int c = c_begin; c < c_end; ++c) {
        const int nvalid = min(kC, a.L - c * kC);
        // unconditional (past the last chunk the rows clamp to L-1 and the
        // registers are never stored): no branch around the loads means no
        // register copies, and no wait for the loads, at the join
        PRIME_LOAD_TILES(c + 1);

        float ds0 = 0.f;  // update role: sum_j w_j v[j][16u + c16] over this lane's tokens
        if (!is_u) {
            if constexpr (!STATE_ONLY) {
                // ---- query features of row iw (B operand of S^T and of the readout)
                Opnd<S> fq[4];
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) fq[ks] = row_op<S>(&sQf[0][iw][32 * ks + 8 * g], plQ);
                // ---- transposed score block S^T[j][i] for j-blocks jb <= wave
                f32x4 sT[4];
#pragma unroll
                for (int jb = 0; jb < 4; ++jb) {
                    sT[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
                    if (jb > wave) continue;
                    Opnd<S> ak[4];
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) ak[ks] = row_op<S>(&sKf[0][16 * jb + c16][32 * ks + 8 * g], plK);
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) sT[jb] = mma<S>(ak[ks], fq[ks], sT[jb]);
                }
                // ---- A = decay mask * (1 + S) as packed bf16 (hi[, lo])
                uint32_t Ah[4][2], Al[4][2];
#pragma unroll
                for (int jb = 0; jb < 4; ++jb) {
                    float x[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) x[r] = mask[jb][r] * (1.0f + sT[jb][r]);
                    Ah[jb][0] = pack2(x[0], x[1]);
                    Ah[jb][1] = pack2(x[2], x[3]);
                    if constexpr (S) {
                        float lo[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) lo[r] = x[r] - bf16_bits_to_f32(f32_to_bf16_bits(x[r]));
                        Al[jb][0] = pack2(lo[0], lo[1]);
                        Al[jb][1] = pack2(lo[2], lo[3]);
                    }
                }
                // ---- y^T = V^T A^T: accumulator row = value column 16nb + 4g + r,
                // column = query row iw; register t of A^T <-> token 32kk + 16(t/4) + 4g + t%4
                f32x4 acc_av[NBX], acc_ro[NBX];
#pragma unroll
                for (int nb = 0; nb < NBX; ++nb) {
                    acc_av[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
                    acc_ro[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    if (2 * kk > wave) continue;
                    const bool second = 2 * kk + 1 <= wave;  // second j-block unmasked
                    Opnd<S> aop;
                    aop.h = as_bf16x8(u32x4{Ah[2 * kk][0], Ah[2 * kk][1], second ? Ah[2 * kk + 1][0] : 0u,
                                            second ? Ah[2 * kk + 1][1] : 0u});
                    if constexpr (S)
                        aop.l = as_bf16x8(u32x4{Al[2 * kk][0], Al[2 * kk][1], second ? Al[2 * kk + 1][0] : 0u,
                                                second ? Al[2 * kk + 1][1] : 0u});
                    Opnd<S> vop[NBX];
#pragma unroll
                    for (int nb = 0; nb < NBX; ++nb) {
                        const uint16_t *p0 = &sV[0][32 * kk + 4 * g + tr_r][16 * nb + tr_c];
                        vop[nb] = tr_op<S>(p0, p0 + 16 * kPV, plV);
                    }
#pragma unroll
                    for (int nb = 0; nb < NBX; ++nb) acc_av[nb] = mma<S>(vop[nb], aop, acc_av[nb]);
                }
                // ---- y^T += [S1; S2/2 | K]^T Fq^T  (the state entering the chunk)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh) {
                    Opnd<S> sop[2][NBX];
#pragma unroll
                    for (int kq = 0; kq < 2; ++kq)
#pragma unroll
                        for (int nb = 0; nb < NBX; ++nb) {
                            const int n = nb == NB ? kD : 16 * nb + c16;  // ones block: only row 64 (K)
                            sop[kq][nb] = row_op<S>(&sSt[0][n][32 * (2 * kh + kq) + 8 * g], plS);
                            if (nb == NB && c16 != 0) {
                                sop[kq][nb].h = as_bf16x8(u32x4{0u, 0u, 0u, 0u});
                                if constexpr (S) sop[kq][nb].l = sop[kq][nb].h;
                            }
                        }
#pragma unroll
                    for (int kq = 0; kq < 2; ++kq)
#pragma unroll
                        for (int nb = 0; nb < NBX; ++nb) acc_ro[nb] = mma<S>(sop[kq][nb], fq[2 * kh + kq], acc_ro[nb]);
                }
                // ---- denominator of row iw: column 64 of both products (lane g = 0, r = 0)
                float den_call = acc_av[NB][0] + pin * (sK0[0] + acc_ro[NB][0]);
                den_call = __shfl(den_call, c16, kWave);
                float den;
                if (dense) {
                    // incoming K state, decayed to this chunk, read out on the VALU
                    float ki = 0.f;
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) {
                        float qf[8];
                        unpack8(__builtin_bit_cast(u32x4, fq[ks].h), qf);
                        if constexpr (S) {
                            float ql[8];
                            unpack8(__builtin_bit_cast(u32x4, fq[ks].l), ql);
#pragma unroll
                            for (int t = 0; t < 8; ++t) qf[t] += ql[t];
                        }
#pragma unroll
                        for (int t = 0; t < 8; ++t) ki += qf[t] * sKi[32 * ks + 8 * g + t];
                    }
                    ki += __shfl_xor(ki, 16, kWave);
                    ki += __shfl_xor(ki, 32, kWave);
                    const float den_init = pin * (sK0[1] + ki * static_cast<float>(pow(static_cast<double>(lam), 64.0 * c)));
                    den = fmaxf(fmaxf(den_call, a.eps) + den_init, a.eps);
                } else {
                    den = fmaxf(den_call, a.eps);
                }
                const float inv = 1.0f / den;
                // ---- y[iw][16nb + 4g .. +4] straight from the accumulators
                const int t = c * kC + iw;
                if (t < a.L) {
                    const int64_t yo = b * a.y_sb + h * a.y_sh + t * a.y_sl + 4 * g;
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        const f32x4 s0 = *reinterpret_cast<const f32x4 *>(&sS0[16 * nb + 4 * g]);
                        f32x4 yv;
#pragma unroll
                        for (int r = 0; r < 4; ++r) yv[r] = (acc_av[nb][r] + pin * (s0[r] + acc_ro[nb][r])) * inv;
                        const int64_t o = yo + 16 * nb;
                        if (a.dt_y == PRIME_BF16) {
                            *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(a.y) + o) =
                                uint2{pack2(yv[0], yv[1]), pack2(yv[2], yv[3])};
                        } else if (a.dt_y == PRIME_F32) {
                            *reinterpret_cast<f32x4 *>(static_cast<float *>(a.y) + o) = yv;
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r) store_elem(a.y, o + r, a.dt_y, yv[r]);
                        }
                    }
                }
            }
        } else {
            // ---- state update: st = l^n st + [k; k*k/2]^T [w v | w]
            const float ln = sPw[nvalid];
#pragma unroll
            for (int fi = 0; fi < 2; ++fi)
#pragma unroll
                for (int nb = 0; nb < NBX; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) st[fi][nb][r] *= ln;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                // register t of both operands <-> token 32ks + 16(t/4) + 4g + t%4, so
                // the lane groups of one transposed read cover consecutive rows
                const int j0 = 32 * ks + 4 * g + tr_r;
                Opnd<S> ak[2], vop[NBX];
#pragma unroll
                for (int fi = 0; fi < 2; ++fi) {
                    const uint16_t *p0 = &sKf[0][j0][16 * (2 * u + fi) + tr_c];
                    ak[fi] = tr_op<S>(p0, p0 + 16 * kPK, plK);
                }
#pragma unroll
                for (int nb = 0; nb < NBX; ++nb) {
                    const uint16_t *p0 = &sVw[0][j0][16 * nb + tr_c];
                    vop[nb] = tr_op<S>(p0, p0 + 16 * kPV, plVw);
                }
                {  // S0 contribution of value block u: the w v operand summed over its
                   // tokens (selected with compile-time indices: a runtime index into
                   // a register array would send it to scratch memory)
                    u32x4 sh = __builtin_bit_cast(u32x4, vop[0].h), sl = {0u, 0u, 0u, 0u};
                    if constexpr (S) sl = __builtin_bit_cast(u32x4, vop[0].l);
#pragma unroll
                    for (int nb = 1; nb < NB; ++nb)
                        if (u == nb) {
                            sh = __builtin_bit_cast(u32x4, vop[nb].h);
                            if constexpr (S) sl = __builtin_bit_cast(u32x4, vop[nb].l);
                        }
                    float vf[8];
                    unpack8(sh, vf);
#pragma unroll
                    for (int e = 0; e < 8; ++e) ds0 += vf[e];
                    if constexpr (S) {
                        unpack8(sl, vf);
#pragma unroll
                        for (int e = 0; e < 8; ++e) ds0 += vf[e];
                    }
                }
#pragma unroll
                for (int fi = 0; fi < 2; ++fi)
#pragma unroll
                    for (int nb = 0; nb < NBX; ++nb) st[fi][nb] = mma<S>(ak[fi], vop[nb], st[fi][nb]);
            }
            ds0 += __shfl_xor(ds0, 16, kWave);
            ds0 += __shfl_xor(ds0, 32, kWave);
        }
        __syncthreads();  // B: every read of chunk c's tiles, the state copy and S0/K0 done

        if (is_u) {
            const float ln = sPw[nvalid];
            write_state_copy();
            if (g == 0) sS0[16 * u + c16] = ln * sS0[16 * u + c16] + ds0;
            if (utid == 0) {
                sK0[0] = ln * sK0[0] + sPs[nvalid];
                sK0[1] = ln * sK0[1];
            }
        }
        if (c + 1 < c_end) PRIME_STORE_TILES(c + 1);
        __syncthreads();  // A: chunk c+1 tiles, state copy and S0/K0 visible
    }

#undef PRIME_LOAD_TILES
#undef PRIME_STORE_TILES

    // ---- segment / final state (decays used the valid counts: no pad correction)
    if (!is_u) return;
    float *o_s1, *o_s2, *o_s0, *o_k1, *o_k2, *o_k0;
    size_t off1, off0, offk0;
    if (STATE_ONLY) {
        o_s1 = wslot + kWsS1; o_s2 = wslot + kWsS2; o_s0 = wslot + kWsS0;
        o_k1 = wslot + kWsK1; o_k2 = wslot + kWsK2; o_k0 = wslot + kWsK0;
        off1 = 0; off0 = 0; offk0 = 0;
    } else {
        if (seg != a.G - 1 || a.s1o == nullptr) return;
        o_s1 = a.s1o; o_s2 = a.s2o; o_s0 = a.s0o; o_k1 = a.k1o; o_k2 = a.k2o; o_k0 = a.k0o;
        off1 = so1; off0 = so0; offk0 = seq;
    }
    // dense clamp: the incoming K state decays separately (l^L over the call)
    const float linit = dense ? static_cast<float>(pow(static_cast<double>(lam), static_cast<double>(a.L))) : 0.f;
#pragma unroll
    for (int fi = 0; fi < 2; ++fi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int f = 16 * (2 * u + fi) + 4 * g + r;
            const int fr = f & (kD - 1);
            const float sc = f < kD ? 1.0f : 2.0f;  // rows 64.. hold S2/2 and K2/2
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                (f < kD ? o_s1 : o_s2)[off1 + fr * kD + 16 * nb + c16] = sc * st[fi][nb][r];
            if (c16 == 0) {
                float kv = st[fi][NB][r];
                if (dense) kv += linit * sKi[f];
                (f < kD ? o_k1 : o_k2)[off0 + fr] = sc * kv;
            }
        }
    if (utid < kD) o_s0[off0 + utid] = sS0[utid];
    if (utid == kD) o_k0[offk0] = sK0[0] + sK0[1];
}

// Scan over segments, elementwise: slot s <- state entering segment s.
// One thread per (sequence, state element); the initial state (or zero) enters
// segment 0 and each full segment of T tokens maps X -> l^T X + delta.
__global__ __launch_bounds__(256) void segment_scan_kernel(const PrefillArgs a) {
    const int Sq = a.B * a.H;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= static_cast<int64_t>(Sq) * kWsElems) return;
    const int seq = static_cast<int>(gid / kWsElems), e = static_cast<int>(gid % kWsElems);
    const int h = seq % a.H;
    const bool sel = a.log_decay != nullptr;
    const float lT = sel ? 0.f : static_cast<float>(pow(static_cast<double>(a.decay[h]), static_cast<double>(a.cps) * kC));
    float carry = 0.f;
    if (a.s1i != nullptr) {
        const size_t so1 = static_cast<size_t>(seq) * kD * kD, so0 = static_cast<size_t>(seq) * kD;
        if (e < kWsS2) carry = a.s1i[so1 + e];
        else if (e < kWsS0) carry = a.s2i[so1 + e - kWsS2];
        else if (e < kWsK1) carry = a.s0i[so0 + e - kWsS0];
        else if (e < kWsK2) carry = a.k1i[so0 + e - kWsK1];
        else if (e < kWsK0) carry = a.k2i[so0 + e - kWsK2];
        else carry = a.k0i[seq];
    }
    float *slot = a.ws + static_cast<size_t>(seq) * a.G * kWsStride + e;
    // accumulate: all G segments (the last one may be short), the total out;
    // otherwise: exclusive prefixes for the chunk loop, in place
    const int ns = a.accumulate ? a.G : a.G - 1;
    const float lLast = (a.accumulate && !sel)
        ? static_cast<float>(pow(static_cast<double>(a.decay[h]),
                                 static_cast<double>(a.L - (a.G - 1) * a.cps * kC)))
        : 0.f;
    // eight slots' loads in flight at a time, then their dependent updates
    for (int s0 = 0; s0 < ns; s0 += 8) {
        float d[8], f[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int s = s0 + t < ns ? s0 + t : ns - 1;  // clamped (unused past ns)
            d[t] = slot[static_cast<size_t>(s) * kWsStride];
            // selective: segment s's own decay, stored beside its slot's state
            f[t] = sel ? exp2f(slot[static_cast<size_t>(s) * kWsStride + kWsDecay - e])
                       : (s == a.G - 1 ? lLast : lT);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            if (s0 + t >= ns) break;
            if (!a.accumulate) slot[static_cast<size_t>(s0 + t) * kWsStride] = carry;
            carry = f[t] * carry + d[t];
        }
    }
    if (!a.accumulate) {
        slot[static_cast<size_t>(a.G - 1) * kWsStride] = carry;
        return;
    }
    const size_t so1 = static_cast<size_t>(seq) * kD * kD, so0 = static_cast<size_t>(seq) * kD;
    if (e < kWsS2) a.s1o[so1 + e] = carry;
    else if (e < kWsS0) a.s2o[so1 + e - kWsS2] = carry;
    else if (e < kWsK1) a.s0o[so0 + e - kWsS0] = carry;
    else if (e < kWsK2) a.k1o[so0 + e - kWsK1] = carry;
    else if (e < kWsK0) a.k2o[so0 + e - kWsK2] = carry;
    else a.k0o[seq] = carry;
}

hipError_t launch_segment_scan(const PrefillArgs &a, hipStream_t stream) {
    const int64_t n = static_cast<int64_t>(a.B) * a.H * kWsElems;
    const TimerEvents tb = timer_events(PRIME_KERNEL_SEGMENT_SCAN);
    hipExtLaunchKernelGGL(segment_scan_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                          tb.start, tb.stop, 0, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) timer_drop(tb);
    return e;
}

template <bool F32IN>
static hipError_t launch_variant(PrefillArgs a, hipStream_t stream) {
    const int Sq = a.B * a.H;
    hipError_t e;
    if (a.accumulate) {
        // every segment's contribution, then the inclusive scan into the state
        a.nseg_launch = a.G;
        const TimerEvents ta = timer_events(PRIME_KERNEL_PREFILL_SEGMENTS);
        if constexpr (F32IN)
            hipExtLaunchKernelGGL((prefill_kernel<true, true>), dim3(Sq * a.G), dim3(256), 0, stream, ta.start,
                                  ta.stop, 0, a);
        else launch_prefill_bf16(a, true, Sq * a.G, stream, ta);
        if ((e = hipGetLastError()) != hipSuccess) return timer_drop(ta), e;
        const int64_t n = static_cast<int64_t>(Sq) * kWsElems;
        const TimerEvents tb = timer_events(PRIME_KERNEL_SEGMENT_SCAN);
        hipExtLaunchKernelGGL(segment_scan_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                              tb.start, tb.stop, 0, a);
        if ((e = hipGetLastError()) != hipSuccess) timer_drop(tb);
        return e;
    }
    if (a.G > 1) {
        // A: state contribution of every segment but the last, from zero
        a.nseg_launch = a.G - 1;
        const TimerEvents ta = timer_events(PRIME_KERNEL_PREFILL_SEGMENTS);
        if constexpr (F32IN)
            hipExtLaunchKernelGGL((prefill_kernel<true, true>), dim3(Sq * (a.G - 1)), dim3(256), 0, stream, ta.start,
                                  ta.stop, 0, a);
        else launch_prefill_bf16(a, true, Sq * (a.G - 1), stream, ta);
        if ((e = hipGetLastError()) != hipSuccess) return timer_drop(ta), e;
        // B: exclusive scan over segments (incoming state first)
        const int64_t n = static_cast<int64_t>(Sq) * kWsElems;
        const TimerEvents tb = timer_events(PRIME_KERNEL_SEGMENT_SCAN);
        hipExtLaunchKernelGGL(segment_scan_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                              tb.start, tb.stop, 0, a);
        if ((e = hipGetLastError()) != hipSuccess) return timer_drop(tb), e;
        if (a.states_only) return hipSuccess;
    }
    a.nseg_launch = a.G;
    const TimerEvents tc = timer_events(PRIME_KERNEL_PREFILL_CHUNKS);
    if constexpr (F32IN)
        hipExtLaunchKernelGGL((prefill_kernel<true, false>), dim3(Sq * a.G), dim3(512), 0, stream, tc.start, tc.stop, 0,
                              a);
    else launch_prefill_bf16(a, false, Sq * a.G + a.npair, stream, tc);
    if ((e = hipGetLastError()) != hipSuccess) timer_drop(tc);
    return e;
}

hipError_t launch_prefill(PrefillArgs a, hipStream_t stream) {
    if (a.log_decay != nullptr && a.dt_in == PRIME_F32 && !a.accumulate && !a.states_only)
        return launch_selective_f32(a, stream);
    return a.dt_in == PRIME_F32 ? launch_variant<true>(a, stream) : launch_variant<false>(a, stream);
}

}  // namespace prime
