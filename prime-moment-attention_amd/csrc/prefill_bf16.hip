// Chunked PRIME prefill for bf16 inputs on gfx950: double-buffered chunk
// tiles and state copy, one workgroup barrier per chunk.
//
// Same algorithm and semantics as the generic kernel in prefill.hip (see its
// header comment for the chunk equations and the operand layouts); this kernel
// differs in its schedule.  The fused pass runs 16 waves (base and selective
// forms):
//   readout waves 0..7 only compute, each for one query block and half of the
//     value columns: score block, AV, state readout, y;
//   update waves 8..15 own the state M = [S1; S2/2 | K] in MFMA accumulators,
//     one feature block each, and, in the step of chunk c, (a) convert and
//     store chunk c+1's tiles (loaded from HBM one chunk earlier) into the other
//     tile buffer, (b) issue the HBM loads of chunk c+2, (c) add chunk c's
//     contribution and (d) publish the bf16 state copy entering chunk c+1 into
//     the other state buffer.  (Timestamps per phase show the update waves as
//     the critical path -- the readout waves wait at the barrier -- and (a)
//     first lets the conversion overlap the readout waves' first phase.)
// Chunk c reads tile buffer c&1 and state buffer c&1 while chunk c+1's are
// written, so one barrier per chunk orders every hazard.  S0 also accumulates
// on MFMA: update wave u multiplies value block u of [w v] by an A operand whose
// row 0 is all ones (other rows zero), which sums w_j v_j over the chunk's
// tokens; K0 is a scalar recurrence with the exact fp32 power sums.
//
// The state-only launch (segment contributions from a zero state) runs the
// update role alone: 4 waves, k and v tiles only, one tile buffer and two
// barriers per chunk (a third of the LDS: three workgroups fit on a CU).

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kPV8 = kD + 16;  // sV / sVw pitch in bf16 (40 dwords, conflict-free transposed reads)
constexpr int kSR = kD + 2;    // state copy rows: 64 value columns, the K column, a zero row
// Pitch of the feature tiles and the state copy: 72 dwords.  On gfx950 a
// ds_read_b128 serves 16 lanes a cycle, lane octets {0,3}, {1,2}, {4,7}, {5,6}
// together (measured with SQ_LDS_BANK_CONFLICT), so a row read (lane = row
// c16, 16-byte granule g) meets rows r and r+8 at granules g and g+1 in one
// cycle: a pitch of 68 dwords puts them on the same banks (2-way conflicts on
// every readout row read), 72 dwords on disjoint ones; ds_read_b64_tr_b16 (32
// consecutive lanes, 8 rows) and the tile stores are conflict-free at 72 too.
constexpr int kPS = kPT;

__device__ __forceinline__ u32x4 ld16(const uint16_t *p) { return *reinterpret_cast<const u32x4 *>(p); }

__device__ __forceinline__ void st16(uint16_t *p, u32x4 x) { *reinterpret_cast<u32x4 *>(p) = x; }

__device__ __forceinline__ u32x4 and4(u32x4 x, uint32_t m) { return u32x4{x[0] & m, x[1] & m, x[2] & m, x[3] & m}; }

// s * x * x of 8 packed bf16, repacked (round to nearest even)
__device__ __forceinline__ u32x4 sq8(u32x4 x, float s) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = __uint_as_float(x[i] << 16), hi = __uint_as_float(x[i] & 0xFFFF0000u);
        r[i] = pack2(s * lo * lo, s * hi * hi);
    }
    return r;
}

// w * x of 8 packed bf16, repacked
__device__ __forceinline__ u32x4 scale8(u32x4 x, float w) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack2(w * __uint_as_float(x[i] << 16), w * __uint_as_float(x[i] & 0xFFFF0000u));
    return r;
}

// QK LayerNorm of one 64-element row held as 8 bf16 by each of 8 consecutive
// lanes (this lane: columns col..col+7): the same arithmetic, summation order
// and roundings as head_layernorm_kernel, so the result is bit-identical to
// normalising the projections first.  affine false: no LayerNorm, the scale only.
// With the LayerNorm and scale == 1 the FMA results are packed (rounded) once;
// a power-of-two scale reaches here folded into w and b (pow2_scale).
// Every lane of the wave takes part (the sums are lane shuffles).
// (w, b: LDS rows of the parameters, read at columns col..col+7)
__device__ __forceinline__ u32x4 norm_row8(u32x4 x, bool affine, const float *w, const float *b, int col, float eps,
                                          float scale) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(x[i] << 16);
        v[2 * i + 1] = __uint_as_float(x[i] & 0xFFFF0000u);
    }
    if (affine) {
        float sm = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sm += v[e];
        sm += xor_lane<4>(sm);
        sm += xor_lane<2>(sm);
        sm += xor_lane<1>(sm);
        const float mean = sm * (1.0f / kD);
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[e] -= mean;
            sq += v[e] * v[e];
        }
        sq += xor_lane<4>(sq);
        sq += xor_lane<2>(sq);
        sq += xor_lane<1>(sq);
        // v_rsq_f32 itself: rsqrtf adds a denormal guard (compare, two scalings,
        // selects) that an argument of at least eps never takes; head_layernorm
        // uses the same instruction, so both give the same bits
        const float rs = __builtin_amdgcn_rsqf(sq * (1.0f / kD) + eps);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = fmaf(v[e] * rs, w[col + e], b[col + e]);
        if (scale == 1.0f) return pack8(v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = bf16_bits_to_f32(f32_to_bf16_bits(v[e]));
    }
    if (scale != 1.0f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = bf16_bits_to_f32(f32_to_bf16_bits(v[e] * scale));
    }
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = f32_to_bf16_bits(v[2 * i]) | (static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i + 1])) << 16);
    return r;
}

// The next chunk's rows ra and ra + 32, one 16-byte segment each, per update thread.
struct Tiles {
    u32x4 q0, q1, k0, k1, v0, v1;
    float ld;  // selective: log2 decay of token `lane` of the chunk (0 past L)
};

// Unconditional loads; rows past L clamp to row L-1 (zeroed when stored).
// ONE_ROW: the thread owns row ra only (512 update threads).
template <bool STATE_ONLY, bool SEL, bool ONE_ROW = false>
__device__ __forceinline__ void load_tiles(Tiles &T, const PrefillArgs &a, const uint16_t *qp, const uint16_t *kp,
                                           const uint16_t *vp, const float *ldp, int c, int ra, int lane) {
    const int64_t ta = min(c * kC + ra, a.L - 1), tb = min(c * kC + ra + 32, a.L - 1);
    if constexpr (SEL) T.ld = ldp[min(c * kC + lane, a.L - 1)];  // scaled and masked when used
    if constexpr (!STATE_ONLY) {
        T.q0 = ld16(qp + ta * a.q_sl);
        if constexpr (!ONE_ROW) T.q1 = ld16(qp + tb * a.q_sl);
    }
    T.k0 = ld16(kp + ta * a.k_sl);
    T.v0 = ld16(vp + ta * a.v_sl);
    if constexpr (!ONE_ROW) {
        T.k1 = ld16(kp + tb * a.k_sl);
        T.v1 = ld16(vp + tb * a.v_sl);
    }
}

// One row segment into the tile buffers: [q | q*q], [k | k*k/2], [v], [w v | w].
// Invalid rows (past the chunk's tokens) are stored as zeros.
template <bool STATE_ONLY, bool SEL>
__device__ __forceinline__ void store_row(u32x4 q, u32x4 k, u32x4 v, int row, int col, bool ragged, bool valid,
                                          float w, float ks, uint16_t *sQf, uint16_t *sKf, uint16_t *sV,
                                          uint16_t *sVw) {
    if (ragged) {  // wave-uniform: only a chunk with rows past the end masks them
        const uint32_t m = valid ? 0xFFFFFFFFu : 0u;
        k = and4(k, m);
        v = and4(v, m);
        if constexpr (!STATE_ONLY) q = and4(q, m);
    }
    if constexpr (!STATE_ONLY) {
        st16(sQf + row * kPS + col, q);
        st16(sQf + row * kPS + kD + col, sq8(q, 1.0f));
        st16(sV + row * kPV8 + col, v);
    }
    // selective: k enters as beta k, its square feature as beta^2 k^2 / 2 (from the
    // unrounded product), i.e. the module's beta and beta^2 / 2 weights
    st16(sKf + row * kPS + col, SEL ? scale8(k, ks) : k);
    st16(sKf + row * kPS + kD + col, sq8(k, SEL ? 0.5f * ks * ks : 0.5f));
    st16(sVw + row * kPV8 + col, scale8(v, w));
    if (col == 0) sVw[row * kPV8 + kD] = f32_to_bf16_bits(w);
}

}  // namespace

// Wave layouts of the fused pass: UW8 = 8 update waves (one feature block each,
// one tile row per thread) instead of 4; RH = 8 readout waves (query block x
// half of the value columns) instead of 4.  QKN: the QK LayerNorm on load.
template <bool STATE_ONLY, bool SEL, bool UW8 = false, bool RH = false, bool QKN = false>
__global__ __launch_bounds__(64 * ((STATE_ONLY ? 0 : (RH ? 8 : 4)) + (UW8 ? 8 : 4)), STATE_ONLY ? 3 : 1) void prefill_bf16_kernel(
    const PrefillArgs a) {
    constexpr int NB = kD / 16;    // value blocks
    constexpr int NBX = NB + 1;    // + the ones / K block
    constexpr int NRW = STATE_ONLY ? 0 : (RH ? 8 : 4);  // readout waves
    constexpr int NUW = UW8 ? 8 : 4;                     // update waves
    constexpr int FI = UW8 ? 1 : 2;                      // feature blocks per update wave
    constexpr int NVB = RH ? 3 : NBX;                    // value blocks per readout wave (incl. the K block)
    constexpr int QB = STATE_ONLY ? 1 : 2;   // buffers of the readout-only arrays
    constexpr int QR = STATE_ONLY ? 1 : kC;
    constexpr int SR = STATE_ONLY ? 1 : kSR;
    constexpr int KI = STATE_ONLY ? 1 : kF;
    constexpr int XB = STATE_ONLY ? 1 : 2;   // tile buffers

    __shared__ __attribute__((aligned(16))) uint16_t sQf[QB][QR][kPS];   // [q | q*q]
    __shared__ __attribute__((aligned(16))) uint16_t sKf[XB][kC][kPS];   // [k | k*k/2]
    __shared__ __attribute__((aligned(16))) uint16_t sV[QB][QR][kPV8];   // [v | 1 0..0]
    __shared__ __attribute__((aligned(16))) uint16_t sVw[XB][kC][kPV8];  // [w v | w 0..0]
    __shared__ __attribute__((aligned(16))) uint16_t sSt[QB][SR][kPS];   // bf16 [S1; S2/2 | K]^T entering the chunk
    __shared__ __attribute__((aligned(16))) float sS0[QB][kD];           // S0 entering the chunk
    __shared__ float sK0[QB];                                             // K0 entering the chunk
    __shared__ float sPw[kC + 2];                                         // l^n, n = 0..65
    __shared__ float sPs[kC + 2];                                         // sum_{m<n} l^m
    __shared__ float sPm[RH ? 2 * kC : 1];                                // RH: [63 + d] = l^d (d >= 0), 0 (d < 0)
    __shared__ float sKi[KI];                                             // incoming [K1; K2/2] (dense)
    __shared__ float sKi0;                                                // incoming K0 (dense)
    __shared__ float sCum[SEL && !STATE_ONLY ? 2 : 1][kC];                // selective: log2 decay to token i
    __shared__ float sLn[QKN ? 4 : 1][kD];                                // QKN: q weight, q bias, k weight, k bias

    const int tid = threadIdx.x;
    // wave index in a scalar register: every role / wave test below is then a
    // scalar branch, so no MFMA runs under a partial or empty EXEC mask
    // (MFMAs write their whole destination regardless of EXEC)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const bool is_u = STATE_ONLY || wave >= NRW;
    const int u = wave - NRW;                          // update-wave index
    const int ut = tid - 64 * NRW;                     // thread index within the update role
    const int tr_r = c16 >> 2, tr_c = 4 * (c16 & 3);  // ds_read_tr address offsets of this lane

    const int Sq = a.B * a.H;
    const int unit = blockIdx.x;
    const int NC = (a.L + kC - 1) / kC;
    // part: -1 a whole segment; 0 / 1 the first / second part of a paired sequence
    int seq, seg, c_begin, c_end, part = -1;
    if (!STATE_ONLY && a.npair > 0) {
        if (unit >= Sq + a.npair) return;  // whole workgroup leaves before any barrier
        seg = 0;
        if (unit < Sq) {
            seq = unit;
            if (unit < a.npair) part = 0;
        } else {
            seq = unit - Sq;
            part = 1;
        }
        c_begin = part == 1 ? a.pcs : 0;
        c_end = part == 0 ? a.pcs : NC;
    } else {
        if (unit >= Sq * a.nseg_launch) return;  // whole workgroup leaves before any barrier
        seq = unit / a.nseg_launch;
        seg = unit - seq * a.nseg_launch;
        c_begin = seg * a.cps;
        c_end = min(c_begin + a.cps, NC);
    }
    const int b = seq / a.H, h = seq - b * a.H, hk = h / a.group;
    const float lam = SEL ? 1.0f : a.decay[h];
    const float kscale = SEL ? a.k_scale[h] : 1.0f;
    // selective: per-token natural-log decays, read as log2 (exp2 on the VALU)
    const float *ldp = SEL ? a.log_decay + static_cast<size_t>(b * a.H + h) * a.L : nullptr;
    const bool from_ws = !STATE_ONLY && (a.G > 1 || part == 1);
    const bool has_in = !STATE_ONLY && !from_ws && a.s1i != nullptr;
    const bool dense = !STATE_ONLY && a.dense_clamp;
    float *wslot = a.ws ? a.ws + (static_cast<size_t>(seq) * a.G + seg) * kWsStride : nullptr;

    // second part of a paired sequence: wait for the first part's end state.
    // The first part has the lower workgroup index, so it was dispatched
    // earlier and finishes without waiting; the bound only guards against a
    // broken launch (the state then reads as NaN, so the outputs show it).
    __shared__ int sPairBad;
    if (part == 1 && tid == 0) {
        unsigned long long *f = a.pflag + seq;
        int n = 0, bad = 0;
        while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != a.epoch) {
            if (++n > kPairSpin) {
                bad = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(8);
        }
        // one acquire for the workgroup: it invalidates this CU's and this
        // XCD's caches, so the other waves' slot reads after the barrier miss
        // any line of the slot cached before the first part wrote it
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        __hip_atomic_store(f, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sPairBad = bad;
    }

    if (tid < kC + 2) {
        const double ld = static_cast<double>(lam);
        sPw[tid] = static_cast<float>(pow(ld, static_cast<double>(tid)));
        double ps = 0.0, pm = 1.0;  // prefix sum of powers in fp64 (1 - l is tiny near l = 1)
        for (int m = 0; m < tid; ++m, pm *= ld) ps += pm;
        sPs[tid] = static_cast<float>(ps);
    }
    if constexpr (RH) {
        if (tid < 2 * kC)
            sPm[tid] = tid >= kC - 1 ? static_cast<float>(pow(static_cast<double>(lam), static_cast<double>(tid - (kC - 1))))
                                     : 0.f;
    }
    if constexpr (QKN) {
        if (tid < 4 * kD) {
            const int t = tid >> 6, e = tid & (kD - 1);
            const void *src = t == 0 ? a.qn_w : t == 1 ? a.qn_b : t == 2 ? a.kn_w : a.kn_b;
            // a power-of-two q scale folds into q's weight and bias (pow2_scale)
            const float fold = t < 2 && a.qn_w && pow2_scale(a.q_scale) ? a.q_scale : 1.0f;
            sLn[t][e] = src ? fold * load_elem(src, e, a.dt_norm) : 0.f;
        }
    }
    __syncthreads();  // the power tables (and QKN's parameters) are read by the first tile stores below
    // second part: every wave's slot reads below come after the first part's release
    const bool pair_bad = part == 1 && sPairBad != 0;
    auto ws_at = [&](int i) { return pair_bad ? __builtin_nanf("") : wslot[i]; };

    // ---- update role: state registers, tile pointers, first tiles
    const size_t so1 = static_cast<size_t>(seq) * kD * kD;
    const size_t so0 = static_cast<size_t>(seq) * kD;
    f32x4 st[FI][NBX];  // feature blocks FI u + fi (rows 4g+r), value blocks nb (column c16)
    f32x4 s0t;          // row 0 (lanes 0..15, element 0) = S0[16u + c16] (update waves u < 4)
    float k0 = 0.f;    // K0 (same value in every lane and update wave)
    Tiles T;
    if constexpr (STATE_ONLY) T.q0 = T.q1 = u32x4{0u, 0u, 0u, 0u};
    const int ra = ut >> 3, col = 8 * (ut & 7);
    const uint16_t *qp = static_cast<const uint16_t *>(a.q) + (b * a.q_sb + h * a.q_sh + col);
    const uint16_t *kp = static_cast<const uint16_t *>(a.k) + (b * a.k_sb + hk * a.k_sh + col);
    const uint16_t *vp = static_cast<const uint16_t *>(a.v) + (b * a.v_sb + hk * a.v_sh + col);
    // selective: log2 decay of the stored chunk (l^n) and its weight sum
    // sum_j w_j (the K0 increment), for the update of that chunk; and the
    // segment's total log2 decay (state-only pass)
    float sel_ln = 1.f, sel_sw = 0.f, seg_ld = 0.f;
    auto store_tiles = [&](int c, int xb) {
        const int nv = min(kC, a.L - c * kC);
        const bool va = ra < nv, vb = ra + 32 < nv;
        float wa, wb;
        if constexpr (SEL) {
            // inclusive scan of the chunk's log2 decays over the lanes (lane = token),
            // on the VALU; every lane takes part (the cross-lane moves read all lanes)
            const float x = wave_prefix_sum(lane < nv ? T.ld * 1.4426950408889634f : 0.f);
            const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), nv - 1));
            const float xra = __shfl(x, ra, kWave);
            wa = va ? exp2f(tot - xra) : 0.f;
            if constexpr (!UW8) {
                const float xrb = __shfl(x, ra + 32, kWave);
                wb = vb ? exp2f(tot - xrb) : 0.f;
            } else {
                wb = 0.f;
            }
            sel_ln = exp2f(tot);
            sel_sw = wave_sum_valu(lane < nv ? exp2f(tot - x) : 0.f);
            seg_ld += tot;
            if constexpr (!STATE_ONLY) {
                if (u == 0) sCum[xb][lane] = x;
            }
        } else {
            wa = va ? sPw[nv - 1 - ra] : 0.f;
            wb = vb ? sPw[nv - 1 - (ra + 32)] : 0.f;
        }
        if constexpr (QKN) {
            // the module's QK LayerNorm (and q's scale) on the raw projections
            const bool qa = a.qn_w != nullptr, ka = a.kn_w != nullptr;
            if constexpr (!STATE_ONLY) {
                const float qs = qa && pow2_scale(a.q_scale) ? 1.0f : a.q_scale;  // (folded into sLn)
                T.q0 = norm_row8(T.q0, qa, sLn[0], sLn[1], col, a.ln_eps, qs);
                if constexpr (!UW8) T.q1 = norm_row8(T.q1, qa, sLn[0], sLn[1], col, a.ln_eps, qs);
            }
            __builtin_amdgcn_sched_barrier(0);  // one row's temporaries at a time
            T.k0 = norm_row8(T.k0, ka, sLn[2], sLn[3], col, a.ln_eps, 1.0f);
            if constexpr (!UW8) T.k1 = norm_row8(T.k1, ka, sLn[2], sLn[3], col, a.ln_eps, 1.0f);
        }
        uint16_t *pq = &sQf[STATE_ONLY ? 0 : xb][0][0], *pv = &sV[STATE_ONLY ? 0 : xb][0][0];
        const bool ragged = nv < kC;
        store_row<STATE_ONLY, SEL>(T.q0, T.k0, T.v0, ra, col, ragged, va, wa, kscale, pq, &sKf[xb][0][0], pv,
                                   &sVw[xb][0][0]);
        if constexpr (!UW8)
            store_row<STATE_ONLY, SEL>(T.q1, T.k1, T.v1, ra + 32, col, ragged, vb, wb, kscale, pq, &sKf[xb][0][0], pv,
                                       &sVw[xb][0][0]);
    };
    // bf16 copy of the state entering the next chunk, into state buffer xb
    auto publish_state = [&](int xb) {
        if constexpr (!STATE_ONLY) {
#pragma unroll
            for (int fi = 0; fi < FI; ++fi) {
                const int f = 16 * (FI * u + fi) + 4 * g;
#pragma unroll
                for (int nb = 0; nb < NBX; ++nb) {
                    const int n = 16 * nb + c16;
                    if (n > kD) continue;  // columns 65..79 of the ones block are zero
                    *reinterpret_cast<uint2 *>(&sSt[xb][n][f]) =
                        uint2{pack2(st[fi][nb][0], st[fi][nb][1]), pack2(st[fi][nb][2], st[fi][nb][3])};
                }
            }
            if (g == 0 && u < 4) sS0[xb][16 * u + c16] = s0t[0];
            if (u == 0 && lane == 0) sK0[xb] = k0;
        }
    };
    if (is_u) {
        load_tiles<STATE_ONLY, SEL, UW8>(T, a, qp, kp, vp, ldp, c_begin, ra, lane);
#pragma unroll
        for (int fi = 0; fi < FI; ++fi)
#pragma unroll
            for (int nb = 0; nb < NBX; ++nb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int f = 16 * (FI * u + fi) + 4 * g + r, fr = f & (kD - 1);
                    const int n = 16 * nb + c16;
                    float x = 0.f;
                    if (n < kD) {
                        if (from_ws) x = ws_at((f < kD ? kWsS1 : kWsS2) + fr * kD + n);
                        else if (has_in) x = (f < kD ? a.s1i : a.s2i)[so1 + fr * kD + n];
                    } else if (n == kD && !dense) {  // dense: K of the call only, incoming in sKi
                        if (from_ws) x = ws_at((f < kD ? kWsK1 : kWsK2) + fr);
                        else if (has_in) x = (f < kD ? a.k1i : a.k2i)[so0 + fr];
                    }
                    st[fi][nb][r] = (f < kD || SEL) ? x : 0.5f * x;  // selective states carry the 1/2
                }
        {
            float x = 0.f;
            if (g == 0 && u < 4) x = from_ws ? ws_at(kWsS0 + 16 * u + c16) : (has_in ? a.s0i[so0 + 16 * u + c16] : 0.f);
            s0t = f32x4{x, 0.f, 0.f, 0.f};
        }
        {
            const float x = from_ws ? ws_at(kWsK0) : (has_in ? a.k0i[seq] : 0.f);
            k0 = dense ? 0.f : x;
            if (!STATE_ONLY && ut == 0) sKi0 = dense ? x : 0.f;
        }
        if constexpr (!STATE_ONLY) {
            if (ut < kF) {
                const int fr = ut & (kD - 1);
                float x = 0.f;
                if (dense && has_in) x = (ut < kD ? a.k1i : a.k2i)[so0 + fr];
                sKi[ut] = ut < kD ? x : 0.5f * x;
            }
        }
        // the zero row of both state copies (read as the K block's other columns)
        if constexpr (!STATE_ONLY) {
            for (int idx = ut; idx < 2 * (kF / 2); idx += 64 * NUW)
                reinterpret_cast<uint32_t *>(&sSt[idx / (kF / 2)][kD + 1][0])[idx % (kF / 2)] = 0u;
        }
        // constant columns: 64..79 of v (1, 0, ...) and 65..79 of w v (column 64
        // holds w and is written with every chunk's tile)
        for (int idx = ut; idx < XB * kC * 16; idx += 64 * NUW) {
            const int xb = idx / (kC * 16), row = (idx >> 4) & (kC - 1), cc = kD + (idx & 15);
            if constexpr (!STATE_ONLY) sV[xb][row][cc] = cc == kD ? 0x3F80u : 0u;
            if (cc != kD) sVw[xb][row][cc] = 0u;
        }
        publish_state(c_begin & 1);
        store_tiles(c_begin, STATE_ONLY ? 0 : c_begin & 1);
        load_tiles<STATE_ONLY, SEL, UW8>(T, a, qp, kp, vp, ldp, c_begin + 1, ra, lane);
    }

    __syncthreads();

    // each role runs its own copy of the chunk loop (the same barriers, one per
    // chunk), so that only its own loop-carried registers are live in it
    if (!is_u) {
        // ---- readout-role constants (query row of the lane: iw)
        // query block rb of this readout wave (RH: the two halves of a block sit on
        // different SIMDs) and, for RH, its half hh of the value columns
        const int rb = RH ? (wave < 4 ? wave : ((wave + 2) & 3)) : wave;
        const int hh = RH ? (wave >> 2) : 0;
        auto vblk = [&](int i) { return RH ? (i < 2 ? 2 * hh + i : NB) : i; };
        const int iw = 16 * rb + c16;
        float mask[4][4];  // l^(i-j) [i >= j] for S^T[j = 16jb + 4g + r][i = iw]
        float pin = 0.f;   // l^(iw+1)
        if (!is_u && !SEL) {
            if constexpr (!RH) {
    #pragma unroll
                for (int jb = 0; jb < 4; ++jb)
    #pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int d = iw - (16 * jb + 4 * g + r);
                        mask[jb][r] = (jb <= rb && d >= 0) ? sPw[max(d, 0)] : 0.f;
                    }
            }
            pin = sPw[iw + 1];  // the power tables: sPw[n] is l^n rounded from fp64
        }
        // dense: l^(64 c) of the chunk, advanced by one chunk decay per step
        float dcr = dense ? static_cast<float>(pow(static_cast<double>(lam), 64.0 * c_begin)) : 0.f;
        for (int c = c_begin; c < c_end; ++c) {
            const int p = STATE_ONLY ? 0 : c & 1;
            const int nvalid = min(kC, a.L - c * kC);
            (void)nvalid;
            if constexpr (!STATE_ONLY) {
                if constexpr (SEL) {
                    // decays within the chunk: l(i <- j) = 2^(cum_i - cum_j), and from
                    // the chunk start to row iw: 2^cum_iw
                    const float ci = sCum[p][iw];
                    pin = exp2f(ci);
#pragma unroll
                    for (int jb = 0; jb < 4; ++jb) {
                        const f32x4 cj = *reinterpret_cast<const f32x4 *>(&sCum[p][16 * jb + 4 * g]);
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            mask[jb][r] = (jb <= rb && 16 * jb + 4 * g + r <= iw) ? exp2f(ci - cj[r]) : 0.f;
                    }
                }
                // ---- phases: score block, A, y^T += V^T A^T, then the state readout
                // y^T += [S1; S2/2 | K]^T Fq^T last (its operand reads then miss the
                // burst of LDS reads that follows the barrier); the query features of
                // row iw are read once, and the phases are kept apart so that few
                // operands are live at once
                f32x4 acc_av[NVB], acc_ro[NVB];
#pragma unroll
                for (int i = 0; i < NVB; ++i) {
                    acc_av[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                    acc_ro[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
                Opnd<false> fq[4];  // query features of row iw, read once per chunk
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) fq[ks] = row_op<false>(&sQf[p][iw][32 * ks + 8 * g], 0);
                __builtin_amdgcn_sched_barrier(0);
                // ---- transposed score block S^T[j][i] for j-blocks jb <= rb
                f32x4 sT[4];
#pragma unroll
                for (int jb = 0; jb < 4; ++jb) {
                    sT[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
                    if (jb > rb) continue;
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks)
                        sT[jb] = mma<false>(row_op<false>(&sKf[p][16 * jb + c16][32 * ks + 8 * g], 0), fq[ks], sT[jb]);
                }
                // ---- A = decay mask * (1 + S) as packed bf16
                uint32_t Ah[4][2];
#pragma unroll
                for (int jb = 0; jb < 4; ++jb) {
                    float x[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        // RH: the decay mask from the power table (registers are short)
                        const int d = iw - (16 * jb + 4 * g + r);
                        // RH: one base address, immediate offsets: index 63 + iw - j
                        const float mk = (RH && !SEL) ? (&sPm[RH ? iw - 4 * g + 12 : 0])[51 - 16 * jb - r] : mask[jb][r];
                        (void)d;
                        x[r] = fmaf(mk, sT[jb][r], mk);  // mk (1 + s)
                    }
                    Ah[jb][0] = pack2(x[0], x[1]);
                    Ah[jb][1] = pack2(x[2], x[3]);
                }
                __builtin_amdgcn_sched_barrier(0);
                // ---- y^T += V^T A^T: accumulator row = value column 16nb + 4g + r,
                // column = query row iw; register t of A^T <-> token 32kk + 16(t/4) + 4g + t%4
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    if (2 * kk > rb) continue;
                    const bool second = 2 * kk + 1 <= rb;  // second j-block unmasked
                    Opnd<false> aop;
                    aop.h = as_bf16x8(u32x4{Ah[2 * kk][0], Ah[2 * kk][1], second ? Ah[2 * kk + 1][0] : 0u,
                                            second ? Ah[2 * kk + 1][1] : 0u});
                    Opnd<false> vop[NVB];
#pragma unroll
                    for (int i = 0; i < NVB; ++i) {
                        const uint16_t *p0 = &sV[p][32 * kk + 4 * g + tr_r][16 * vblk(i) + tr_c];
                        vop[i] = tr_op<false>(p0, p0 + 16 * kPV8, 0);
                    }
#pragma unroll
                    for (int i = 0; i < NVB; ++i) acc_av[i] = mma<false>(vop[i], aop, acc_av[i]);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const Opnd<false> &fqk = fq[ks];
                    Opnd<false> sop[NVB];
#pragma unroll
                    for (int i = 0; i < NVB; ++i) {
                        const int nb = vblk(i);
                        // ones block: row 64 (K) in lane 0 of each row group, the zero row elsewhere
                        const int n = nb == NB ? (c16 == 0 ? kD : kD + 1) : 16 * nb + c16;
                        sop[i] = row_op<false>(&sSt[p][n][32 * ks + 8 * g], 0);
                    }
#pragma unroll
                    for (int i = 0; i < NVB; ++i) acc_ro[i] = mma<false>(sop[i], fqk, acc_ro[i]);
                }
                // ---- denominator of row iw: column 64 of both products (lane g = 0, r = 0)
                float den_call = acc_av[NVB - 1][0] + pin * (sK0[p] + acc_ro[NVB - 1][0]);
                den_call = __shfl(den_call, c16, kWave);
                float den;
                if (dense) {
                    // incoming K state, decayed to this chunk, read out on the VALU
                    float ki = 0.f;
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) {
                        float qf[8];
                        unpack8(lds128(&sQf[p][iw][32 * ks + 8 * g]), qf);
#pragma unroll
                        for (int t = 0; t < 8; ++t) ki += qf[t] * sKi[32 * ks + 8 * g + t];
                    }
                    ki += __shfl_xor(ki, 16, kWave);
                    ki += __shfl_xor(ki, 32, kWave);
                    const float dc = dcr;
                    dcr *= sPw[kC];
                    den = fmaxf(fmaxf(den_call, a.eps) + pin * dc * (sKi0 + ki), a.eps);
                } else {
                    den = fmaxf(den_call, a.eps);
                }
                const float inv = __builtin_amdgcn_rcpf(den);  // 1 ulp
                // ---- y[iw][16nb + 4g .. +4] straight from the accumulators
                const int t = c * kC + iw;
                if (t < a.L) {
                    const int64_t yo = b * a.y_sb + h * a.y_sh + t * a.y_sl + 4 * g;
#pragma unroll
                    for (int i = 0; i < NVB - 1; ++i) {
                        const int nb = vblk(i);
                        const f32x4 s0 = *reinterpret_cast<const f32x4 *>(&sS0[p][16 * nb + 4 * g]);
                        f32x4 yv;
#pragma unroll
                        for (int r = 0; r < 4; ++r) yv[r] = (acc_av[i][r] + pin * (s0[r] + acc_ro[i][r])) * inv;
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
            __syncthreads();
        }
        if (part == 0) __syncthreads();  // the update waves' hand-off barrier below
        return;
    }
    // row 0 of the ones operand: lanes of A-row 0 hold eight 1.0s
    const bf16x8 ones = as_bf16x8(c16 == 0 ? u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u}
                                           : u32x4{0u, 0u, 0u, 0u});
    for (int c = c_begin; c < c_end; ++c) {
        const int p = STATE_ONLY ? 0 : c & 1, xq = STATE_ONLY ? 0 : p ^ 1;
        const int nvalid = min(kC, a.L - c * kC);
        {
            // ---- state update: st = l^n st + [k; k*k/2]^T [w v | w];  S0 on the ones row
            const float ln = SEL ? sel_ln : sPw[nvalid];  // selective: set when chunk c was stored
            const float sw = SEL ? sel_sw : sPs[nvalid];
            const bool more = c + 1 < c_end;
            if constexpr (!STATE_ONLY) {
                // chunk c+1's tiles first (into the other buffer, which no wave
                // reads in this step): this conversion and its LDS stores then
                // overlap the readout waves' first phase instead of following
                // the update's MFMAs, and the HBM loads of chunk c+2 go out early
                if (more) store_tiles(c + 1, xq);
                load_tiles<STATE_ONLY, SEL, UW8>(T, a, qp, kp, vp, ldp, c + 2, ra, lane);
            }
#pragma unroll
            for (int fi = 0; fi < FI; ++fi)
#pragma unroll
                for (int nb = 0; nb < NBX; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) st[fi][nb][r] *= ln;
            s0t[0] *= ln;
            k0 = ln * k0 + sw;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                // register t of both operands <-> token 32ks + 16(t/4) + 4g + t%4
                const int j0 = 32 * ks + 4 * g + tr_r;
                Opnd<false> ak[FI], vop[NBX];
#pragma unroll
                for (int fi = 0; fi < FI; ++fi) {
                    const uint16_t *p0 = &sKf[p][j0][16 * (FI * u + fi) + tr_c];
                    ak[fi] = tr_op<false>(p0, p0 + 16 * kPS, 0);
                }
#pragma unroll
                for (int nb = 0; nb < NBX; ++nb) {
                    const uint16_t *p0 = &sVw[p][j0][16 * nb + tr_c];
                    vop[nb] = tr_op<false>(p0, p0 + 16 * kPV8, 0);
                }
#pragma unroll
                for (int fi = 0; fi < FI; ++fi)
#pragma unroll
                    for (int nb = 0; nb < NBX; ++nb) st[fi][nb] = mma<false>(ak[fi], vop[nb], st[fi][nb]);
                // value block u of [w v] on the ones row (a wave-uniform switch, so
                // that the operand is selected without a register-indexed access)
                if (u < 4) switch (u) {
                    case 0: s0t = mfma(ones, vop[0].h, s0t); break;
                    case 1: s0t = mfma(ones, vop[1].h, s0t); break;
                    case 2: s0t = mfma(ones, vop[2].h, s0t); break;
                    default: s0t = mfma(ones, vop[3].h, s0t); break;
                }
            }
            if constexpr (STATE_ONLY) {
                __syncthreads();  // every wave has read the single tile buffer
                if (more) store_tiles(c + 1, xq);
                load_tiles<STATE_ONLY, SEL, UW8>(T, a, qp, kp, vp, ldp, c + 2, ra, lane);
            }
            if (more) publish_state(xq);
        }
        __syncthreads();
    }

    // ---- segment / final state (decays used the valid counts: no pad correction)
    float *o_s1, *o_s2, *o_s0, *o_k1, *o_k2, *o_k0;
    size_t off1, off0, offk0;
    if (STATE_ONLY || part == 0) {  // a segment's contribution / a first part's end state
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
    for (int fi = 0; fi < FI; ++fi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int f = 16 * (FI * u + fi) + 4 * g + r;
            const int fr = f & (kD - 1);
            const float sc = (f < kD || SEL) ? 1.0f : 2.0f;  // rows 64.. hold S2/2 and K2/2
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                (f < kD ? o_s1 : o_s2)[off1 + fr * kD + 16 * nb + c16] = sc * st[fi][nb][r];
            if (c16 == 0) {
                float kv = st[fi][NB][r];
                if constexpr (!STATE_ONLY) {
                    if (dense) kv += linit * sKi[f];
                }
                (f < kD ? o_k1 : o_k2)[off0 + fr] = sc * kv;
            }
        }
    if (g == 0 && u < 4) o_s0[off0 + 16 * u + c16] = s0t[0];
    if (u == 0 && lane == 0) o_k0[offk0] = k0 + (STATE_ONLY ? 0.f : linit * sKi0);
    // selective: the segment's own log2 decay, for the scan over segments
    if (SEL && STATE_ONLY && u == 0 && lane == 0) wslot[kWsDecay] = seg_ld;
    if (!STATE_ONLY && part == 0) {
        // hand-off: every update thread waits until its slot stores have
        // reached this XCD's L2; after the barrier (which the readout waves also
        // meet) one release writes the L2 back and publishes the flag.  (A
        // device-scope fence in every thread would write the L2 back once per
        // wave, and those write-backs stall the whole XCD.)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (ut == 0) __hip_atomic_store(a.pflag + seq, a.epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <bool QKN>
static void launch_variant_bf16(const PrefillArgs &a, bool state_only, int grid, hipStream_t stream, TimerEvents t) {
    const bool sel = a.log_decay != nullptr;
    const dim3 g(grid), blk(state_only ? 256 : 1024);
    if (state_only && sel)
        hipExtLaunchKernelGGL((prefill_bf16_kernel<true, true, false, false, QKN>), g, blk, 0, stream, t.start, t.stop, 0, a);
    else if (state_only)
        hipExtLaunchKernelGGL((prefill_bf16_kernel<true, false, false, false, QKN>), g, blk, 0, stream, t.start, t.stop, 0, a);
    else if (sel)
        hipExtLaunchKernelGGL((prefill_bf16_kernel<false, true, true, true, QKN>), g, blk, 0, stream, t.start, t.stop, 0, a);
    else
        hipExtLaunchKernelGGL((prefill_bf16_kernel<false, false, true, true, QKN>), g, blk, 0, stream, t.start, t.stop, 0, a);
}

void launch_prefill_bf16(const PrefillArgs &a, bool state_only, int grid, hipStream_t stream, TimerEvents t) {
    if (a.qk_norm) launch_variant_bf16<true>(a, state_only, grid, stream, t);
    else launch_variant_bf16<false>(a, state_only, grid, stream, t);
}

}  // namespace prime
