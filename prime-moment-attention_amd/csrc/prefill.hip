// Chunked PRIME prefill on bf16 MFMA (gfx950).
//
// Semantics: chunked_prime_ssd_core (chunked_ssd.py:48-184) of the reference,
// and with PRIME_FLAG_DENSE_CLAMP the module's dense branch
// (attention.py:160-202).  For each (b,h) the tokens are processed in 64-token
// chunks.  With features Fq_i = [q_i, q_i*q_i/2], Fk_j = [k_j, k_j*k_j]
// (128 wide) and the state packed as Sst = [S1; S2] (128 x D), Kst = [K1; K2]:
//   A_ij   = l^(i-j) [i>=j] (1 + Fq_i . Fk_j)                      (intra block)
//   num_i  = sum_j A_ij v_j + l^(i+1) (S0 + Fq_i Sst)
//   den_i  = sum_j A_ij     + l^(i+1) (K0 + Fq_i . Kst)
//   y_i    = num_i / max(den_i, eps)
//   Sst   <- l^n Sst + sum_j l^(n-1-j) Fk_j^T v_j   (n = valid tokens in chunk)
// The reference's O(Nc^2) inter-chunk matrix (chunked_ssd.py:113-126) is the
// closed form of this carried scan; padding is handled exactly by decaying with
// the number of valid tokens, which equals the reference's l^(-pad) correction
// (chunked_ssd.py:171-178).
//
// Mapping: one workgroup (4 wavefronts) per (sequence, value-column slice of
// NV columns).  The state slice lives in MFMA accumulators across all chunks
// (fp32); a bf16 copy in LDS feeds the readout.  Wave w owns query rows
// [16w, 16w+16) for the score block, the intra product and the readout, and
// feature rows [32w, 32w+32) of the state.  The score block is computed
// transposed (S^T = Fk Fq^T) so its accumulator layout is directly the A
// operand of the A.V product (the token index is permuted consistently in the
// V operand), without an LDS round trip.  q/k/v tiles for chunk c+1 are loaded
// into registers while chunk c computes.  Workgroups that share a sequence are
// placed on the same XCD (blockIdx % 8) so their q/k reads share its L2.
//
// Precision: bf16 inputs are exact in the MFMA operands; derived operands
// (squares, decay-scaled features, the score block, the state copy) are rounded
// to bf16 once.  fp32 inputs (F32IN) keep fp32 tiles in LDS and split every
// operand x into bf16 hi + lo, accumulating hi*hi + hi*lo + lo*hi (three MFMAs
// per product, ~2^-16 relative), with a hi/lo copy of the state.

#include "prime_kernels.h"

namespace prime {

constexpr int kC = 64;          // tokens per chunk
constexpr int kF = 2 * kD;      // feature width
constexpr int kPF = kF + 8;     // LDS pitch for the 128-wide transposed state

typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 r) { return __builtin_bit_cast(bf16x8, r); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}

__device__ __forceinline__ void unpack8(u32x4 r, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(r[i] << 16);
        f[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
    }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack2(f[2 * i], f[2 * i + 1]);
    return r;
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// An MFMA operand: hi part, plus the lo residual when split (S).
template <bool S>
struct Opnd {
    bf16x8 h, l;
};

template <bool S>
__device__ __forceinline__ Opnd<S> split8(const float (&f)[8]) {
    Opnd<S> o;
    const u32x4 hr = pack8(f);
    o.h = as_bf16x8(hr);
    if constexpr (S) {
        float hf[8], r[8];
        unpack8(hr, hf);
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = f[i] - hf[i];
        o.l = as_bf16x8(pack8(r));
    }
    return o;
}

template <bool S>
__device__ __forceinline__ f32x4 mma(const Opnd<S> &a, const Opnd<S> &b, f32x4 c) {
    c = mfma(a.h, b.h, c);
    if constexpr (S) {
        c = mfma(a.h, b.l, c);
        c = mfma(a.l, b.h, c);
    }
    return c;
}

// 8 consecutive LDS elements as fp32
__device__ __forceinline__ void lds8(const uint16_t *p, float (&f)[8]) {
    unpack8(*reinterpret_cast<const u32x4 *>(p), f);
}
__device__ __forceinline__ void lds8(const float *p, float (&f)[8]) {
    const f32x4 a = reinterpret_cast<const f32x4 *>(p)[0], b = reinterpret_cast<const f32x4 *>(p)[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = a[i];
        f[4 + i] = b[i];
    }
}
__device__ __forceinline__ float ldsf(const uint16_t *p) { return bf16_bits_to_f32(*p); }
__device__ __forceinline__ float ldsf(const float *p) { return *p; }

// identity features: a bf16 row is already an operand
template <bool S, typename T>
__device__ __forceinline__ Opnd<S> raw_op(const T *p) {
    if constexpr (!S) {
        Opnd<S> o;
        o.h = as_bf16x8(*reinterpret_cast<const u32x4 *>(p));
        return o;
    } else {
        float f[8];
        lds8(p, f);
        return split8<S>(f);
    }
}

// s*x or s*x*x features
template <bool S, typename T>
__device__ __forceinline__ Opnd<S> xform_op(const T *p, bool square, float s) {
    float f[8];
    lds8(p, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = square ? s * f[i] * f[i] : s * f[i];
    return split8<S>(f);
}

// Registers holding one 8-element row segment of the next chunk.
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

template <bool F32IN>
__device__ __forceinline__ Seg8<F32IN> load_seg(const void *base, int64_t off, bool valid) {
    Seg8<F32IN> s;
    if constexpr (!F32IN) {
        s.r = u32x4{0u, 0u, 0u, 0u};
        if (valid) s.r = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(base) + off);
    } else {
        s.a = f32x4{0.f, 0.f, 0.f, 0.f};
        s.b = s.a;
        if (valid) {
            const f32x4 *p = reinterpret_cast<const f32x4 *>(static_cast<const float *>(base) + off);
            s.a = p[0];
            s.b = p[1];
        }
    }
    return s;
}

// row-major store of a segment (8 elements at p)
__device__ __forceinline__ void store_row(uint16_t *p, const Seg8<false> &s) {
    *reinterpret_cast<u32x4 *>(p) = s.r;
}
__device__ __forceinline__ void store_row(float *p, const Seg8<true> &s) {
    reinterpret_cast<f32x4 *>(p)[0] = s.a;
    reinterpret_cast<f32x4 *>(p)[1] = s.b;
}
// element e of a segment in storage format
__device__ __forceinline__ uint16_t seg_elem(const Seg8<false> &s, int e) {
    return static_cast<uint16_t>((e & 1) ? (s.r[e >> 1] >> 16) : (s.r[e >> 1] & 0xFFFFu));
}
__device__ __forceinline__ float seg_elem(const Seg8<true> &s, int e) { return e < 4 ? s.a[e] : s.b[e - 4]; }

// Segment plan.  Without a workspace (or for the dense branch, whose clamp
// needs the incoming state separate from the tokens of this call) every
// sequence is one segment.  Otherwise sequences are cut into segments of whole
// chunks so that about kTargetUnits workgroups run, each segment >= kMinCps
// chunks long.
constexpr int kTargetUnits = 768;
constexpr int kMinCps = 4;

void plan_segments(int S, int L, bool dense_clamp, size_t ws_bytes, int *G, int *cps) {
    const int NC = (L + kC - 1) / kC;
    int g = 1;
    if (!dense_clamp && S < kTargetUnits) {
        g = (kTargetUnits + S - 1) / S;
        const int gmax = NC / kMinCps;
        if (g > gmax) g = gmax;
        if (g < 1) g = 1;
    }
    int c = (NC + g - 1) / g;
    g = (NC + c - 1) / c;  // no empty segments
    while (g > 1 && static_cast<size_t>(S) * g * kWsStride * sizeof(float) > ws_bytes) {
        c = c * 2;
        g = (NC + c - 1) / c;
    }
    if (g <= 1) {
        g = 1;
        c = NC;
    }
    *G = g;
    *cps = c;
}

// One workgroup = (sequence, segment[, value slice]).  STATE_ONLY: only the
// segment's state contribution from a zero state (no q, no output) -> ws slot.
template <int NV, bool F32IN, bool STATE_ONLY>
__global__ __launch_bounds__(256, 2) void prefill_kernel(const PrefillArgs a) {
    using T = typename std::conditional<F32IN, float, uint16_t>::type;  // tile storage
    constexpr bool S = F32IN;                    // split operands
    constexpr int NP = S ? 2 : 1;                // state planes (hi, lo)
    constexpr int kP = F32IN ? kD + 4 : kD + 8;  // tile row pitch (elements; 16-byte multiple)
    constexpr int NB = NV / 16;                  // 16-wide value blocks per workgroup
    constexpr int NVL = NV / 32;                 // v segments per thread
    constexpr int QR = STATE_ONLY ? 1 : kC;      // q / bf16-state buffers unused when STATE_ONLY
    constexpr int SR = STATE_ONLY ? 1 : NV;

    __shared__ __attribute__((aligned(16))) T sQ[QR][kP];               // q rows (pre-scaled)
    __shared__ __attribute__((aligned(16))) T sK[QR][kP];               // k rows
    __shared__ __attribute__((aligned(16))) T sKt[kD][kP];              // k transposed [f][j]
    __shared__ __attribute__((aligned(16))) T sVt[NV][kP];              // v transposed [n][j]
    __shared__ __attribute__((aligned(16))) uint16_t sSt[NP][SR][kPF];  // bf16 state [n][f]
    __shared__ __attribute__((aligned(16))) float sW[kC];               // token weights of the chunk
    __shared__ float sPw[kC + 2];                                       // l^n, n = 0..65
    __shared__ float sPs[kC + 2];                                       // sum_{m<n} l^m
    __shared__ __attribute__((aligned(16))) float sKc[kF], sKi[kF];     // K state (call / init part)
    __shared__ float sS0[NV], sK0[2];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;

    // ---- workgroup -> (sequence, segment, value slice); with two slices the
    // pair shares an XCD (blockIdx % 8) so its q/k reads share that L2
    const int Sq = a.B * a.H;
    int unit, split;
    if (a.nsplit == 1) {
        unit = blockIdx.x;
        split = 0;
    } else {
        split = (blockIdx.x >> 3) & 1;
        unit = ((blockIdx.x >> 4) << 3) + (blockIdx.x & 7);
    }
    if (unit >= Sq * a.nseg_launch) return;  // whole workgroup leaves before any barrier
    const int seq = unit / a.nseg_launch, seg = unit - seq * a.nseg_launch;
    const int b = seq / a.H, h = seq - b * a.H, hk = h / a.group;
    const int n0 = split * NV;
    const float lam = a.decay[h];
    const int NC = (a.L + kC - 1) / kC;
    const int c_begin = seg * a.cps;
    const int c_end = min(c_begin + a.cps, NC);
    const bool from_ws = !STATE_ONLY && a.G > 1;
    const bool has_in = !STATE_ONLY && !from_ws && a.s1i != nullptr;
    const bool last_seg = seg == a.G - 1;
    float *wslot = a.ws ? a.ws + (static_cast<size_t>(seq) * a.G + seg) * kWsStride : nullptr;

    if (tid < kC + 2) {
        const double ld = static_cast<double>(lam);
        sPw[tid] = static_cast<float>(pow(ld, static_cast<double>(tid)));
        double ps = 0.0, pm = 1.0;  // prefix sum of powers in fp64 (1 - l is tiny near l = 1)
        for (int m = 0; m < tid; ++m, pm *= ld) ps += pm;
        sPs[tid] = static_cast<float>(ps);
    }
    if (tid < kC) sW[tid] = static_cast<float>(pow(static_cast<double>(lam), static_cast<double>(kC - 1 - tid)));

    // ---- initial state
    const size_t so1 = static_cast<size_t>(seq) * kD * kD;
    const size_t so0 = static_cast<size_t>(seq) * kD;
    f32x4 st[2][NB];  // feature blocks 2*wave+fi, value blocks nb
#pragma unroll
    for (int fi = 0; fi < 2; ++fi)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = 16 * (2 * wave + fi) + 4 * g + r;
                const int n = n0 + 16 * nb + c16;
                const int fr = f & (kD - 1);
                float x = 0.f;
                if (from_ws) x = wslot[(f < kD ? kWsS1 : kWsS2) + fr * kD + n];
                else if (has_in) x = (f < kD ? a.s1i : a.s2i)[so1 + fr * kD + n];
                st[fi][nb][r] = x;
            }
    if (tid < kF) {
        const int fr = tid & (kD - 1);
        float x = 0.f;
        if (from_ws) x = wslot[(tid < kD ? kWsK1 : kWsK2) + fr];
        else if (has_in) x = (tid < kD ? a.k1i : a.k2i)[so0 + fr];
        sKc[tid] = a.dense_clamp ? 0.f : x;
        sKi[tid] = a.dense_clamp ? x : 0.f;
    } else if (tid < kF + NV) {
        const int n = n0 + tid - kF;
        sS0[tid - kF] = from_ws ? wslot[kWsS0 + n] : (has_in ? a.s0i[so0 + n] : 0.f);
    } else if (tid == kF + NV) {
        const float x = from_ws ? wslot[kWsK0] : (has_in ? a.k0i[seq] : 0.f);
        sK0[0] = a.dense_clamp ? 0.f : x;
        sK0[1] = a.dense_clamp ? x : 0.f;
    }
    // bf16 (hi[, lo]) copy of the state for the readout
    auto write_state_copy = [&]() {
        if constexpr (!STATE_ONLY) {
#pragma unroll
            for (int fi = 0; fi < 2; ++fi)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int f = 16 * (2 * wave + fi) + 4 * g;
                    const int n = 16 * nb + c16;
                    uint2 w2;
                    w2.x = pack2(st[fi][nb][0], st[fi][nb][1]);
                    w2.y = pack2(st[fi][nb][2], st[fi][nb][3]);
                    *reinterpret_cast<uint2 *>(&sSt[0][n][f]) = w2;
                    if constexpr (S) {
                        float lo[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            lo[r] = st[fi][nb][r] - bf16_bits_to_f32(f32_to_bf16_bits(st[fi][nb][r]));
                        w2.x = pack2(lo[0], lo[1]);
                        w2.y = pack2(lo[2], lo[3]);
                        *reinterpret_cast<uint2 *>(&sSt[NP - 1][n][f]) = w2;
                    }
                }
        }
    };
    write_state_copy();

    // ---- per-lane constants of the chunk layout (full chunks)
    const int iw = 16 * wave + c16;  // query row of this lane in the score/readout operands
    float mask[4][4];                // l^(i-j) [i >= j] for S^T[j = 16jb + 4g + r][i = iw]
    float prow[4];                   // l^(i+1) for accumulator rows i = 16 wave + 4g + r
    if constexpr (!STATE_ONLY) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = iw - (16 * jb + 4 * g + r);
                mask[jb][r] = (jb <= wave && d >= 0) ? static_cast<float>(pow(static_cast<double>(lam), static_cast<double>(d))) : 0.f;
            }
#pragma unroll
        for (int r = 0; r < 4; ++r)
            prow[r] = static_cast<float>(pow(static_cast<double>(lam), static_cast<double>(16 * wave + 4 * g + r + 1)));
    }
    const float pin = STATE_ONLY ? 0.f : static_cast<float>(pow(static_cast<double>(lam), static_cast<double>(iw + 1)));

    // ---- tile loads.  q: row = tid/8 (+32), segment = tid%8 (row-major, coalesced).
    // k, v: token = lane and the 8-wide segments spread over the waves, so each
    // transposed LDS write of a wave covers 64 consecutive tokens of one row.
    const int64_t qb = b * a.q_sb + h * a.q_sh, kb = b * a.k_sb + hk * a.k_sh, vb = b * a.v_sb + hk * a.v_sh;
    Seg8<F32IN> Rq[2], Rk[2], Rv[NVL];
    auto load_tiles = [&](int c) {
        if constexpr (!STATE_ONLY) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int row = (tid >> 3) + 32 * p, sgm = tid & 7;
                const int t = c * kC + row;
                Rq[p] = load_seg<F32IN>(a.q, qb + t * a.q_sl + 8 * sgm, t < a.L);
            }
        }
        const int t = c * kC + lane;
        const bool ok = t < a.L;
#pragma unroll
        for (int p = 0; p < 2; ++p) Rk[p] = load_seg<F32IN>(a.k, kb + t * a.k_sl + 8 * (2 * wave + p), ok);
#pragma unroll
        for (int p = 0; p < NVL; ++p)
            Rv[p] = load_seg<F32IN>(a.v, vb + t * a.v_sl + n0 + 8 * (NVL * wave + p), ok);
    };
    auto store_tiles = [&]() {
        if constexpr (!STATE_ONLY) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int row = (tid >> 3) + 32 * p, sgm = tid & 7;
                store_row(&sQ[row][8 * sgm], Rq[p]);
            }
        }
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int sgm = 2 * wave + p;
            if constexpr (!STATE_ONLY) store_row(&sK[lane][8 * sgm], Rk[p]);
#pragma unroll
            for (int e = 0; e < 8; ++e) sKt[8 * sgm + e][lane] = seg_elem(Rk[p], e);
        }
#pragma unroll
        for (int p = 0; p < NVL; ++p) {
            const int sgm = NVL * wave + p;
#pragma unroll
            for (int e = 0; e < 8; ++e) sVt[8 * sgm + e][lane] = seg_elem(Rv[p], e);
        }
    };

    load_tiles(c_begin);

    for (int c = c_begin; c < c_end; ++c) {
        const int nvalid = min(kC, a.L - c * kC);
        store_tiles();
        if (nvalid < kC && tid < kC) sW[tid] = tid < nvalid ? sPw[nvalid - 1 - tid] : 0.f;
        __syncthreads();  // A: tiles of chunk c and state^(c) visible
        if (c + 1 < c_end) load_tiles(c + 1);

        if constexpr (!STATE_ONLY) {
            // ---- query features of row iw: B operand of the score block and A
            // operand of the readout (k index f = 32 ks + 8g + t in both)
            Opnd<S> fq[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const T *qr = &sQ[iw][(ks & 1) * 32 + 8 * g];
                fq[ks] = ks >= 2 ? xform_op<S>(qr, true, 0.5f) : raw_op<S>(qr);
            }
            // ---- transposed score block S^T[j][i] for j-blocks jb <= wave
            f32x4 sT[4];
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) sT[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                if (jb > wave) continue;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const T *kr = &sK[16 * jb + c16][(ks & 1) * 32 + 8 * g];
                    const Opnd<S> ak = ks >= 2 ? xform_op<S>(kr, true, 1.0f) : raw_op<S>(kr);
                    sT[jb] = mma<S>(ak, fq[ks], sT[jb]);
                }
            }
            // ---- decay mask -> A and the intra denominator (lane: S^T[16jb+4g+r][iw])
            uint32_t Ah[4][2], Al[4][2];
            float denp = 0.f;
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                float av[4], lo[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float x = mask[jb][r] * (1.0f + sT[jb][r]);
                    const float xh = bf16_bits_to_f32(f32_to_bf16_bits(x));
                    av[r] = xh;
                    lo[r] = S ? x - xh : 0.f;
                    denp += S ? x : xh;  // unsplit: numerator and denominator use the same weight
                }
                Ah[jb][0] = pack2(av[0], av[1]);
                Ah[jb][1] = pack2(av[2], av[3]);
                Al[jb][0] = pack2(lo[0], lo[1]);
                Al[jb][1] = pack2(lo[2], lo[3]);
            }
            // ---- acc_av = A.V (register t <-> j = 32kk + 16(t/4) + 4g + t%4)
            f32x4 acc_av[NB], acc_ro[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                acc_av[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
                acc_ro[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                if (2 * kk > wave) continue;
                Opnd<S> aop;
                aop.h = as_bf16x8(u32x4{Ah[2 * kk][0], Ah[2 * kk][1], Ah[2 * kk + 1][0], Ah[2 * kk + 1][1]});
                if constexpr (S) aop.l = as_bf16x8(u32x4{Al[2 * kk][0], Al[2 * kk][1], Al[2 * kk + 1][0], Al[2 * kk + 1][1]});
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const T *vr = &sVt[16 * nb + c16][32 * kk + 4 * g];
                    Opnd<S> bop;
                    if constexpr (!S) {
                        const uint2 lo = *reinterpret_cast<const uint2 *>(vr);
                        const uint2 hi = *reinterpret_cast<const uint2 *>(vr + 16);
                        bop.h = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
                    } else {
                        const f32x4 lo = *reinterpret_cast<const f32x4 *>(vr);
                        const f32x4 hi = *reinterpret_cast<const f32x4 *>(vr + 16);
                        const float f[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        bop = split8<S>(f);
                    }
                    acc_av[nb] = mma<S>(aop, bop, acc_av[nb]);
                }
            }
            // ---- acc_ro = Fq . Sst  (readout of the state entering the chunk)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    Opnd<S> sop;
                    sop.h = as_bf16x8(*reinterpret_cast<const u32x4 *>(&sSt[0][16 * nb + c16][32 * ks + 8 * g]));
                    if constexpr (S)
                        sop.l = as_bf16x8(*reinterpret_cast<const u32x4 *>(&sSt[NP - 1][16 * nb + c16][32 * ks + 8 * g]));
                    acc_ro[nb] = mma<S>(fq[ks], sop, acc_ro[nb]);
                }
            // ---- denominator of row iw: intra + l^(i+1) (K0 + Fq . Kst), call and init parts
            float kc = 0.f, ki = 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int f = 32 * ks + 8 * g;
                float qf[8];
                unpack8(__builtin_bit_cast(u32x4, fq[ks].h), qf);
                if constexpr (S) {
                    float ql[8];
                    unpack8(__builtin_bit_cast(u32x4, fq[ks].l), ql);
#pragma unroll
                    for (int t = 0; t < 8; ++t) qf[t] += ql[t];
                }
                const f32x4 c0 = *reinterpret_cast<const f32x4 *>(&sKc[f]);
                const f32x4 c1 = *reinterpret_cast<const f32x4 *>(&sKc[f + 4]);
                const f32x4 i0 = *reinterpret_cast<const f32x4 *>(&sKi[f]);
                const f32x4 i1 = *reinterpret_cast<const f32x4 *>(&sKi[f + 4]);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    kc += qf[t] * c0[t] + qf[4 + t] * c1[t];
                    ki += qf[t] * i0[t] + qf[4 + t] * i1[t];
                }
            }
            denp += __shfl_xor(denp, 16, kWave);
            denp += __shfl_xor(denp, 32, kWave);
            kc += __shfl_xor(kc, 16, kWave);
            kc += __shfl_xor(kc, 32, kWave);
            ki += __shfl_xor(ki, 16, kWave);
            ki += __shfl_xor(ki, 32, kWave);
            const float den_call = denp + pin * (sK0[0] + kc);
            const float den_init = pin * (sK0[1] + ki);
            const float den = a.dense_clamp ? fmaxf(fmaxf(den_call, a.eps) + den_init, a.eps)
                                            : fmaxf(den_call + den_init, a.eps);
            // ---- y rows 16w + 4g + r straight from the accumulators
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * wave + 4 * g + r;
                const float inv = 1.0f / __shfl(den, 4 * g + r, kWave);
                const int t = c * kC + row;
                if (t < a.L) {
                    const int64_t yo = b * a.y_sb + h * a.y_sh + t * a.y_sl + n0 + c16;
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        const float yv = (acc_av[nb][r] + prow[r] * (sS0[16 * nb + c16] + acc_ro[nb][r])) * inv;
                        store_elem(a.y, yo + 16 * nb, a.dt_y, yv);
                    }
                }
            }
            __syncthreads();  // B: readout of state^(c) finished everywhere
        }

        // ---- state update with this chunk (exact for a partial last chunk)
        const float ln = sPw[nvalid];
#pragma unroll
        for (int fi = 0; fi < 2; ++fi)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int r = 0; r < 4; ++r) st[fi][nb][r] *= ln;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int j0 = 32 * ks + 8 * g;
            const f32x4 w0 = *reinterpret_cast<const f32x4 *>(&sW[j0]);
            const f32x4 w1 = *reinterpret_cast<const f32x4 *>(&sW[j0 + 4]);
            Opnd<S> vop[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) vop[nb] = raw_op<S>(&sVt[16 * nb + c16][j0]);
#pragma unroll
            for (int fi = 0; fi < 2; ++fi) {
                const int f = 16 * (2 * wave + fi) + c16;  // A-operand row (feature)
                const bool sq = f >= kD;
                float kf[8];
                lds8(&sKt[f & (kD - 1)][j0], kf);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const float w = t < 4 ? w0[t] : w1[t - 4];
                    kf[t] = sq ? w * kf[t] * kf[t] : w * kf[t];
                }
                const Opnd<S> ak = split8<S>(kf);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) st[fi][nb] = mma<S>(ak, vop[nb], st[fi][nb]);
            }
        }
        write_state_copy();
        // ---- small moments (fp32 VALU): lanes split the token range, butterflies combine
        {
            const int f = 32 * wave + (lane & 31), fr = f & (kD - 1);
            const int jh = 32 * (lane >> 5);
            float s = 0.f;
#pragma unroll
            for (int jj = 0; jj < 32; jj += 8) {
                float kf[8];
                lds8(&sKt[fr][jh + jj], kf);
                const f32x4 w0 = *reinterpret_cast<const f32x4 *>(&sW[jh + jj]);
                const f32x4 w1 = *reinterpret_cast<const f32x4 *>(&sW[jh + jj + 4]);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const float w = t < 4 ? w0[t] : w1[t - 4];
                    s += w * (f < kD ? kf[t] : kf[t] * kf[t]);
                }
            }
            s += __shfl_xor(s, 32, kWave);
            constexpr int NPW = NV / 4, NPART = 64 / NPW, JL = kC / NPART;
            const int n = NPW * wave + lane % NPW, jp = (lane / NPW) * JL;
            float s0 = 0.f;
#pragma unroll
            for (int jj = 0; jj < JL; jj += 8) {
                float vf[8];
                lds8(&sVt[n][jp + jj], vf);
                const f32x4 w0 = *reinterpret_cast<const f32x4 *>(&sW[jp + jj]);
                const f32x4 w1 = *reinterpret_cast<const f32x4 *>(&sW[jp + jj + 4]);
#pragma unroll
                for (int t = 0; t < 4; ++t) s0 += w0[t] * vf[t] + w1[t] * vf[4 + t];
            }
#pragma unroll
            for (int o = NPW; o < kWave; o <<= 1) s0 += __shfl_xor(s0, o, kWave);
            if (lane < 32) {
                sKc[f] = ln * sKc[f] + s;
                sKi[f] = ln * sKi[f];
            }
            if (lane < NPW) sS0[n] = ln * sS0[n] + s0;
            if (tid == 0) {
                sK0[0] = ln * sK0[0] + sPs[nvalid];
                sK0[1] = ln * sK0[1];
            }
        }
        __syncthreads();  // C: tiles free for the next chunk, small state visible
    }

    // ---- segment / final state (decays used the valid counts: no pad correction)
    float *o_s1, *o_s2, *o_s0, *o_k1, *o_k2, *o_k0;
    size_t off1, off0, offk0;
    if (STATE_ONLY) {
        o_s1 = wslot + kWsS1; o_s2 = wslot + kWsS2; o_s0 = wslot + kWsS0;
        o_k1 = wslot + kWsK1; o_k2 = wslot + kWsK2; o_k0 = wslot + kWsK0;
        off1 = 0; off0 = 0; offk0 = 0;
    } else {
        if (!last_seg || a.s1o == nullptr) return;
        o_s1 = a.s1o; o_s2 = a.s2o; o_s0 = a.s0o; o_k1 = a.k1o; o_k2 = a.k2o; o_k0 = a.k0o;
        off1 = so1; off0 = so0; offk0 = seq;
    }
#pragma unroll
    for (int fi = 0; fi < 2; ++fi)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = 16 * (2 * wave + fi) + 4 * g + r;
                const int n = n0 + 16 * nb + c16;
                (f < kD ? o_s1 : o_s2)[off1 + (f & (kD - 1)) * kD + n] = st[fi][nb][r];
            }
    if (tid < NV) o_s0[off0 + n0 + tid] = sS0[tid];
    if (split == 0) {
        if (tid < kF) (tid < kD ? o_k1 : o_k2)[off0 + (tid & (kD - 1))] = sKc[tid] + sKi[tid];
        if (tid == kF) o_k0[offk0] = sK0[0] + sK0[1];
    }
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
    const float lT = static_cast<float>(pow(static_cast<double>(a.decay[h]), static_cast<double>(a.cps) * kC));
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
    for (int s = 0; s + 1 < a.G; ++s) {
        const float d = slot[static_cast<size_t>(s) * kWsStride];
        slot[static_cast<size_t>(s) * kWsStride] = carry;
        carry = lT * carry + d;
    }
    slot[static_cast<size_t>(a.G - 1) * kWsStride] = carry;
}

template <bool F32IN>
static void launch_variant(PrefillArgs a, hipStream_t stream) {
    const int Sq = a.B * a.H;
    if (a.G > 1) {
        // A: state contribution of every segment but the last, from zero
        a.nsplit = 1;
        a.nseg_launch = a.G - 1;
        hipLaunchKernelGGL((prefill_kernel<64, F32IN, true>), dim3(Sq * (a.G - 1)), dim3(256), 0, stream, a);
        // B: exclusive scan over segments (incoming state first)
        const int64_t n = static_cast<int64_t>(Sq) * kWsElems;
        hipLaunchKernelGGL(segment_scan_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, a);
    }
    a.nseg_launch = a.G;
    if (a.nsplit == 2) {
        const int U8 = (Sq * a.G + 7) / 8 * 8;
        hipLaunchKernelGGL((prefill_kernel<32, F32IN, false>), dim3(U8 * 2), dim3(256), 0, stream, a);
    } else {
        a.nsplit = 1;
        hipLaunchKernelGGL((prefill_kernel<64, F32IN, false>), dim3(Sq * a.G), dim3(256), 0, stream, a);
    }
}

hipError_t launch_prefill(PrefillArgs a, hipStream_t stream) {
    if (a.dt_in == PRIME_F32) launch_variant<true>(a, stream);
    else launch_variant<false>(a, stream);
    return hipGetLastError();
}

}  // namespace prime
