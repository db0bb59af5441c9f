// Backward of the chunked PRIME prefill for fp32 inputs, in fp32 throughout:
// the reverse-mode derivative of attention.py:119-143 (the recurrence the
// reference's prefill computes, chunked_ssd.py:48-184) that torch autograd
// takes when it trains in fp32 (tests/test_attention.py:50-62).
//
// Forward, per 64-token chunk with Fq_i = [q_i, q_i*q_i], Fk_j = [k_j, k_j*k_j/2],
// the state M = [S1; S2/2] (128 x 64), Kf = [K1; K2/2], and l^(i-j) written
// e^(cum_i - cum_j) (cum_i = (i+1) log l for the chunk's valid tokens, flat past L):
//   a_ij  = [j <= i] e^(cum_i - cum_j) (1 + Fq_i . Fk_j)
//   num_i = sum_j a_ij v_j + e^cum_i (S0 + Fq_i M),  den_i = sum_j a_ij + e^cum_i (K0 + Fq_i . Kf)
//   y_i   = num_i / D_i,  D_i = max(den_i, eps)
//   M <- e^cum_63 M + Fk^T diag(w) V, w_j = e^(cum_63 - cum_j) (likewise S0, K0, Kf)
// Backward, with g_i = dy_i / D_i and h_i = -[den_i >= eps] (dy_i . num_i) / D_i^2:
//   da_ij  = e^(cum_i - cum_j) (g_i . v_j + h_i)                 (j <= i)
//   dFq_i  = sum_j da_ij Fk_j + e^cum_i (M g_i + h_i Kf)           (state entering the chunk)
//   dv_j   = sum_i a_ij g_i + w_j (Fk_j dM + dS0)                  (adjoint dM, dS0, dKf of the
//   dFk_j  = sum_i da_ij Fq_i + w_j (dM v_j + dKf)                  state leaving the chunk)
//   dM    <- e^cum_63 dM + Fq^T diag(e^cum) G   (likewise dS0 from g, dK0 and dKf from h)
//   dq = dFq[:64] + 2 q * dFq[64:],  dk = dFk[:64] + k * dFk[64:]
// Two kernels, one workgroup of 8 waves per (sequence, head): the dq pass runs
// the chunks in order, carrying the forward state, and leaves 1/D_i and h_i
// per token in the workspace; the dk/dv pass runs them in reverse, carrying
// the adjoint, and ends with the adjoint of the incoming state.  Every
// product is an fp32 MFMA (v_mfma_f32_16x16x4_f32: lane l holds A[l%16][l/16]
// and B[l/16][l%16], the accumulator D[4(l/16) + r][l%16]).

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kFP = 2 * kD;   // features
constexpr int kPQ = kFP + 4;  // Fq / Fk rows: 16-byte reads of 16 rows fall on distinct bank quads
constexpr int kPR = kC + 4;   // 64-wide rows (v, dy / g, a, da) and M rows
constexpr int kBW = 8;        // waves

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }
__device__ __forceinline__ void st4(float *p, f32x4 v) { *reinterpret_cast<f32x4 *>(p) = v; }

__device__ __forceinline__ void store4(void *p, int dt, int64_t idx, f32x4 v) {
    if (dt == PRIME_F32) {
        st4(static_cast<float *>(p) + idx, v);
    } else if (dt == PRIME_BF16) {
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p) + idx) = uint2{pack2(v[0], v[1]), pack2(v[2], v[3])};
    } else {
        uint16_t *h = static_cast<uint16_t *>(p) + idx;
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = f32_to_h16_bits(v[r]);
    }
}

// lower 16x16 tile t (0..9) -> (row block, column block)
__device__ __forceinline__ void lower_tile(int t, int &ib, int &jb) {
    ib = t < 1 ? 0 : t < 3 ? 1 : t < 6 ? 2 : 3;
    jb = t - ib * (ib + 1) / 2;
}

// The chunk's tiles: Fq, Fk (fp32 inputs), v, dy (dtype dt_dy), one token per
// 8 threads; tokens past L are zero.  Wave 0 forms cum, e^cum and w.
// SEL: per-token log decays (logd) and k scaled by kscale[h] as it is loaded.
template <bool SEL>
__device__ __forceinline__ void load_chunk(const BwdArgs &a, int b, int h, int c, int tid, int w, int lane,
                                           float (*sFq)[kPQ], float (*sFk)[kPQ], float (*sV)[kPR],
                                           float (*sDY)[kPR], float *sCum, float *sEc, float *sW, float logl) {
    const int i = tid >> 3, d0 = 8 * (tid & 7);
    const int t = c * kC + i;
    const bool valid = t < a.L;
    const int64_t tc = valid ? t : a.L - 1;
    const float *qp = static_cast<const float *>(a.q) + b * a.q_sb + h * a.q_sh + tc * a.q_sl + d0;
    const float *kp = static_cast<const float *>(a.k) + b * a.k_sb + h * a.k_sh + tc * a.k_sl + d0;
    const float *vp = static_cast<const float *>(a.v) + b * a.v_sb + h * a.v_sh + tc * a.v_sl + d0;
    const int64_t yo = b * a.dy_sb + h * a.dy_sh + tc * a.dy_sl + d0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        const f32x4 q = valid ? ld4(qp + 4 * j) : z, v = valid ? ld4(vp + 4 * j) : z;
        f32x4 k = valid ? ld4(kp + 4 * j) : z;
        if constexpr (SEL) k *= a.kscale[h];
        f32x4 q2, k2, dy;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            q2[r] = q[r] * q[r];
            k2[r] = 0.5f * (k[r] * k[r]);
            dy[r] = valid ? load_elem(a.dy, yo + 4 * j + r, a.dt_dy) : 0.f;
        }
        st4(&sFq[i][d0 + 4 * j], q);
        st4(&sFq[i][kD + d0 + 4 * j], q2);
        st4(&sFk[i][d0 + 4 * j], k);
        st4(&sFk[i][kD + d0 + 4 * j], k2);
        st4(&sV[i][d0 + 4 * j], v);
        st4(&sDY[i][d0 + 4 * j], dy);
    }
    if (w == 0) {
        const bool vl = c * kC + lane < a.L;
        float cum = 0.f;
        if (vl) cum = SEL ? a.logd[static_cast<size_t>(b * a.H + h) * a.L + c * kC + lane] : logl;
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) {
            const float x = __shfl_up(cum, s, kWave);
            if (lane >= s) cum += x;
        }
        const float cend = __shfl(cum, 63, kWave);
        sCum[lane] = cum;
        sEc[lane] = expf(cum);
        sW[lane] = vl ? expf(cend - cum) : 0.f;
    }
}

// A on the 10 lower tiles (feature k-slot g of k-step s: 32g + s), masked to
// valid columns; wave w takes tiles w and w + 8
__device__ __forceinline__ void scores(const BwdArgs &a, int c, int w, int g, int c16, const float (*sFq)[kPQ],
                                       const float (*sFk)[kPQ], const float *sCum, float (*sA)[kPR]) {
    for (int ti = w; ti < 10; ti += kBW) {
        int ib, jb;
        lower_tile(ti, ib, jb);
        const float *pa = &sFq[16 * ib + c16][32 * g];
        const float *pb = &sFk[16 * jb + c16][32 * g];
        f32x4 p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q4 = 0; q4 < 8; ++q4) {
            const f32x4 x = ld4(pa + 4 * q4), z = ld4(pb + 4 * q4);
#pragma unroll
            for (int r = 0; r < 4; ++r) p = mfma4(x[r], z[r], p);
        }
        const int j = 16 * jb + c16;
        const bool vj = c * kC + j < a.L;
        const float cj = sCum[j];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * ib + 4 * g + r;
            sA[i][j] = (i >= j && vj) ? expf(sCum[i] - cj) * (1.0f + p[r]) : 0.f;
        }
    }
}

// da on the lower tiles: e^(cum_i - cum_j) (G_i . v_j + h_i), masked like A
__device__ __forceinline__ void dscores(const BwdArgs &a, int c, int w, int g, int c16, const float (*sG)[kPR],
                                        const float (*sV)[kPR], const float *sCum, const float *sH,
                                        float (*sDA)[kPR]) {
    for (int ti = w; ti < 10; ti += kBW) {
        int ib, jb;
        lower_tile(ti, ib, jb);
        f32x4 p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (int s = 0; s < 16; ++s) p = mfma4(sG[16 * ib + c16][4 * s + g], sV[16 * jb + c16][4 * s + g], p);
        const int j = 16 * jb + c16;
        const bool vj = c * kC + j < a.L;
        const float cj = sCum[j];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * ib + 4 * g + r;
            sDA[i][j] = (i >= j && vj) ? expf(sCum[i] - cj) * (p[r] + sH[i]) : 0.f;
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// dq pass: chunks in order, the forward state carried (M tiles of feature
// block w in wave w's accumulators, Kf / S0 / K0 by threads 0..192).
// ---------------------------------------------------------------------------
// DIN: the dense double clamp with an incoming state (BwdArgs::dense_in);
// SEL: the selective form (BwdArgs::logd), which also leaves per token
// phi_q'(i) . dphi_q'(i) (the query side of the log decays' adjoint, phi_q'
// = [1, q, q*q]) and per sequence <dstate_out, state_out>
template <bool DIN, bool SEL>
__global__ __launch_bounds__(kBW * kWave, 1) void prefill_bwd_dq_f32_kernel(const BwdArgs a) {
    __shared__ __attribute__((aligned(16))) float sFq[kC][kPQ];
    __shared__ __attribute__((aligned(16))) float sFk[kC][kPQ];
    __shared__ __attribute__((aligned(16))) float sV[kC][kPR];
    __shared__ __attribute__((aligned(16))) float sG[kC][kPR];   // dy, then g = dy / D
    __shared__ __attribute__((aligned(16))) float sA[kC][kPR];   // a, then da
    __shared__ __attribute__((aligned(16))) float sM[kFP][kPR];
    __shared__ float sKf[kFP], sS0[kD], sCum[kC], sEc[kC], sW[kC], sD[kC], sH[kC], sDen[kC], sK0[1];
    __shared__ float sPart[kBW][16];
    // dense double clamp with an incoming state: the incoming Kf and K0 (sKf, sK0
    // then carry the call's own), per token max(den, eps) + the incoming term
    // (sD1), l^(64c) times the outer clamp's adjoint (sHc), and l^(t+1) times the
    // part of it the inner clamp withholds from the call's tokens (sDh)
    __shared__ float sKin[kFP], sK0in[1], sD1[kC], sHc[kC], sDh[kC];
    __shared__ float sFin[kBW];  // SEL: the waves' shares of <dstate_out, state_out>

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    // one unit per (sequence, segment of a.cps chunks); G > 1 only for the base
    // form without the dense clamp's incoming-state split
    const int unit = blockIdx.x;
    if (unit >= a.B * a.H * a.G) return;
    const int seq = unit / a.G, seg = unit - seq * a.G;
    const int b = seq / a.H, h = seq - b * a.H;
    const float logl = logf(a.decay[h]);
    const size_t so1 = static_cast<size_t>(seq) * kD * kD, so0 = static_cast<size_t>(seq) * kD;
    // the state entering the segment: state_in, or the segment's slot (the
    // forward's state-only pass; the same components and conventions)
    const float *S0p = a.s0i ? a.s0i + so0 : nullptr, *S1p = a.s1i ? a.s1i + so1 : nullptr;
    const float *S2p = a.s2i ? a.s2i + so1 : nullptr, *K0p = a.k0i ? a.k0i + seq : nullptr;
    const float *K1p = a.k1i ? a.k1i + so0 : nullptr, *K2p = a.k2i ? a.k2i + so0 : nullptr;
    if (a.G > 1) {
        const float *slot = a.ws + static_cast<size_t>(unit) * kWsStride;
        S1p = slot + kWsS1; S2p = slot + kWsS2; S0p = slot + kWsS0;
        K1p = slot + kWsK1; K2p = slot + kWsK2; K0p = slot + kWsK0;
    }

    // incoming state: M = [S1; S2/2], Kf = [K1; K2/2]
    f32x4 mt[4];
#pragma unroll
    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int f = 16 * w + 4 * g + r, col = 16 * dv + c16;
            float x = 0.f;
            // rows 64.. of M: S2/2 (S2 in the selective convention, whose S2 carries the 1/2)
            if (S1p) x = f < kD ? S1p[f * kD + col] : (SEL ? 1.0f : 0.5f) * S2p[(f - kD) * kD + col];
            mt[dv][r] = x;
            sM[f][col] = x;
        }
    float kreg = 0.f;
    if (S1p) {
        if (tid < kD) kreg = K1p[tid];
        else if (tid < kFP) kreg = (SEL ? 1.0f : 0.5f) * K2p[tid - kD];
        else if (tid < kFP + kD) kreg = S0p[tid - kFP];
        else if (tid == kFP + kD) kreg = K0p[0];
    }
    constexpr bool din = DIN;
    const bool kthr = tid < kFP || tid == kFP + kD;  // threads that carry Kf or K0
    if (din && kthr) {
        if (tid < kFP) sKin[tid] = kreg;
        else sK0in[0] = kreg;
        kreg = 0.f;  // the call's own K moments from zero
    }
    if (tid < kFP) sKf[tid] = kreg;
    else if (tid < kFP + kD) sS0[tid - kFP] = kreg;
    else if (tid == kFP + kD) sK0[0] = kreg;
    float corr = 0.f;  // (din) this thread's feature (tid < 128) or K0 (tid == 192) of the correction

    const int NC = (a.L + kC - 1) / kC;
    const int c_begin = seg * a.cps, c_end = min(c_begin + a.cps, NC);
    const int64_t gbase = b * a.g_sb + h * a.g_sh;
    for (int c = c_begin; c < c_end; ++c) {
        // (din) l^(64 c): the incoming state's decay to the chunk's start
        const float lc = din ? static_cast<float>(pow(static_cast<double>(a.decay[h]), 64.0 * c)) : 0.f;
        load_chunk<SEL>(a, b, h, c, tid, w, lane, sFq, sFk, sV, sG, sCum, sEc, sW, logl);
        __syncthreads();
        scores(a, c, w, g, c16, sFq, sFk, sCum, sA);
        __syncthreads();
        // ---- denominators (four threads per token; only A's lower tiles exist)
        if (tid < 4 * kC) {
            const int i = tid >> 2, qt = tid & 3;
            float part = 0.f;
            if (qt <= (i >> 4)) {
#pragma unroll
                for (int e = 0; e < 16; ++e) part += sA[i][16 * qt + e];
            }
            float rd = qt == 0 ? sK0[0] : 0.f, ri = qt == 0 && din ? sK0in[0] : 0.f;
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                rd += sFq[i][32 * qt + e] * sKf[32 * qt + e];
                if (din) ri += sFq[i][32 * qt + e] * sKin[32 * qt + e];
            }
            part += sEc[i] * rd;
            part += xor_lane<1>(part);
            part += xor_lane<2>(part);
            if (din) {
                ri += xor_lane<1>(ri);
                ri += xor_lane<2>(ri);
            }
            if (qt == 0) {
                // single clamp max(den, eps), or the double clamp max(max(den, eps) + cr, eps)
                const float d1 = din ? fmaxf(part, a.eps) + lc * sEc[i] * ri : part;
                sDen[i] = part;
                sD1[i] = d1;
                sD[i] = fmaxf(d1, a.eps);
            }
        }
        __syncthreads();
        // ---- num^T tiles (token block w/2, value blocks 2(w&1)+jj) and their dot with dy
        {
            const int ib = w >> 1, tok = 16 * ib + c16;
            const float ec = sEc[tok];
            float dot = 0.f;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int dv = 2 * (w & 1) + jj;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                for (int s = 0; s < 4 * (ib + 1); ++s)
                    acc = mfma4(sV[4 * s + g][16 * dv + c16], sA[tok][4 * s + g], acc);
#pragma unroll 8
                for (int s = 0; s < 32; ++s)
                    acc = mfma4(sM[4 * s + g][16 * dv + c16], ec * sFq[tok][4 * s + g], acc);
                const f32x4 dy = ld4(&sG[tok][16 * dv + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; ++r) dot += dy[r] * (acc[r] + ec * sS0[16 * dv + 4 * g + r]);
            }
            dot = sum_lane16(dot);
            dot = sum_lane32(dot);
            if (g == 0) sPart[w][c16] = dot;
        }
        __syncthreads();
        // ---- g = dy / D, h = -[den >= eps] (dy . num) / D^2; 1/D and h to the workspace
        if (tid < kC) {
            const int i = tid, ib = i >> 4, cc = i & 15;
            const float dot = sPart[2 * ib][cc] + sPart[2 * ib + 1][cc];
            const float D = sD[i];
            // the outer clamp's adjoint, and the call's share of it (inner clamp)
            const float hout = sD1[i] >= a.eps ? -dot / (D * D) : 0.f;
            const float hh = sDen[i] >= a.eps ? hout : 0.f;
            sH[i] = hh;
            if (din) {
                sHc[i] = lc * hout;
                sDh[i] = lc * sEc[i] * (hout - hh);
            }
            const int64_t t = static_cast<int64_t>(c) * kC + i;
            if (t < a.L) {
                a.inv_den[static_cast<size_t>(seq) * a.L + t] = 1.0f / D;
                a.g_den[static_cast<size_t>(seq) * a.L + t] = hh;
                // SEL: phi_q'(i) . dphi_q'(i) = (num . dy) / D + den h.  e^cum_i scales num and
                // den alike, so this is exactly 0 while den >= eps (h = -(num . dy) / den^2)
                // and (num . dy) / eps where the clamp holds (h = 0): formed here without
                // the cancellation of summing it over the features
                if constexpr (SEL) a.pq[static_cast<size_t>(seq) * a.L + t] = sDen[i] >= a.eps ? 0.f : dot / D;
            }
        }
        for (int e = tid; e < kC * kD; e += kBW * kWave) {
            const int i = e >> 6, d = e & 63;
            sG[i][d] = sG[i][d] / sD[i];
        }
        __syncthreads();
        dscores(a, c, w, g, c16, sG, sV, sCum, sH, sA);
        __syncthreads();
        // ---- dFq (token block w/2; feature blocks db and 4 + db for db = 2(w&1) + jj) -> dq
        {
            const int ib = w >> 1, tok = 16 * ib + c16;
            const float ec = sEc[tok];
            const int64_t t = static_cast<int64_t>(c) * kC;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int db = 2 * (w & 1) + jj;
                f32x4 d2[2];
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int fb = db + 4 * hf;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    // dFq^T tile: rows f, columns tokens
                    for (int s = 0; s < 4 * (ib + 1); ++s)
                        acc = mfma4(sFk[4 * s + g][16 * fb + c16], sA[tok][4 * s + g], acc);
#pragma unroll 8
                    for (int s = 0; s < 16; ++s)
                        acc = mfma4(sM[16 * fb + c16][4 * s + g], ec * sG[tok][4 * s + g], acc);
                    const float hh = ec * sH[tok];
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[r] += hh * sKf[16 * fb + 4 * g + r];
                    if (din) {  // the incoming K's denominator term, under the outer clamp only
                        const float hc = ec * sHc[tok];
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[r] += hc * sKin[16 * fb + 4 * g + r];
                    }
                    d2[hf] = acc;
                }
                // lane: features 16 db + 4g + r of token tok; dq = dFq1 + 2 q dFq2
                if (t + tok < a.L) {
                    const f32x4 q = ld4(&sFq[tok][16 * db + 4 * g]);
                    f32x4 dq;
#pragma unroll
                    for (int r = 0; r < 4; ++r) dq[r] = d2[0][r] + 2.0f * q[r] * d2[1][r];
                    store4(a.dq, a.dt_g, gbase + (t + tok) * a.g_sl + 16 * db + 4 * g, dq);
                }
            }
        }
        // ---- forward state update: M tiles of feature block w; Kf, S0, K0 by their threads
        {
            const float e63 = sEc[kC - 1];
#pragma unroll
            for (int dv = 0; dv < 4; ++dv) {
                f32x4 x;
#pragma unroll
                for (int r = 0; r < 4; ++r) x[r] = e63 * mt[dv][r];
#pragma unroll 8
                for (int s = 0; s < 16; ++s) {
                    const int j = 4 * s + g;
                    x = mfma4(sFk[j][16 * w + c16], sW[j] * sV[j][16 * dv + c16], x);
                }
                mt[dv] = x;
            }
            if (tid < kFP) {
                float acc = e63 * kreg;
                for (int j = 0; j < kC; ++j) acc += sW[j] * sFk[j][tid];
                kreg = acc;
                if (din) {  // correction: sum over the chunk of sDh_t Fq(t)
                    float sacc = 0.f;
                    for (int i = 0; i < kC; ++i) sacc += sDh[i] * sFq[i][tid];
                    corr += sacc;
                }
            } else if (tid < kFP + kD) {
                float acc = e63 * kreg;
                for (int j = 0; j < kC; ++j) acc += sW[j] * sV[j][tid - kFP];
                kreg = acc;
            } else if (tid == kFP + kD) {
                float acc = e63 * kreg;
                for (int j = 0; j < kC; ++j) acc += sW[j];
                kreg = acc;
                if (din) {
                    float sacc = 0.f;
                    for (int i = 0; i < kC; ++i) sacc += sDh[i];
                    corr += sacc;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int dv = 0; dv < 4; ++dv)
#pragma unroll
            for (int r = 0; r < 4; ++r) sM[16 * w + 4 * g + r][16 * dv + c16] = mt[dv][r];
        if (tid < kFP) sKf[tid] = kreg;
        else if (tid < kFP + kD) sS0[tid - kFP] = kreg;
        else if (tid == kFP + kD) sK0[0] = kreg;
    }
    if (din && kthr) a.kcorr[static_cast<size_t>(seq) * kBwdCorr + (tid < kFP ? tid : kFP)] = corr;
    if constexpr (SEL) {
        // <dstate_out, state_out> in the selective convention (M rows 64.. hold S2
        // itself, Kf rows 64.. K2): the final state's share of the log decays' adjoint
        float fp = 0.f;
        if (a.ds1o) {
#pragma unroll
            for (int dv = 0; dv < 4; ++dv)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int f = 16 * w + 4 * g + r, col = 16 * dv + c16;
                    fp += mt[dv][r] * (f < kD ? a.ds1o[so1 + f * kD + col] : a.ds2o[so1 + (f - kD) * kD + col]);
                }
            if (tid < kD) fp += kreg * a.dk1o[so0 + tid];
            else if (tid < kFP) fp += kreg * a.dk2o[so0 + tid - kD];
            else if (tid < kFP + kD) fp += kreg * a.ds0o[so0 + tid - kFP];
            else if (tid == kFP + kD) fp += kreg * a.dk0o[seq];
        }
        fp = wave_sum(fp);
        if (lane == 0) sFin[w] = fp;
        __syncthreads();
        if (tid == 0) {
            float tot = 0.f;
            for (int i = 0; i < kBW; ++i) tot += sFin[i];
            a.fin[seq] = tot;
        }
    }
}

// ---------------------------------------------------------------------------
// dk/dv pass: chunks in reverse, the adjoint of the state leaving each chunk
// carried (dM tiles of feature block w in wave w's accumulators, dKf / dS0 /
// dK0 by threads 0..192); it ends as the adjoint of the incoming state.
// ---------------------------------------------------------------------------
// SEL: the selective form; also forms per token phi_k'(j) . dphi_k'(j), turns
// the dq pass's query-side terms into the log decays' adjoint (a suffix sum
// over the tokens, carried from the last chunk back) and the key scale's
// adjoint per sequence
// DUAL: the dual-state pass of a segment (G > 1) -- from a zero adjoint, no dk /
// dv, the adjoint reached at the segment's start (its contribution) written to
// its slot for the reverse scan over segments.
template <bool SEL, bool DUAL>
__global__ __launch_bounds__(kBW * kWave, 1) void prefill_bwd_dkv_f32_kernel(const BwdArgs a) {
    __shared__ __attribute__((aligned(16))) float sFq[kC][kPQ];
    __shared__ __attribute__((aligned(16))) float sFk[kC][kPQ];
    __shared__ __attribute__((aligned(16))) float sV[kC][kPR];
    __shared__ __attribute__((aligned(16))) float sG[kC][kPR];   // dy, then g
    __shared__ __attribute__((aligned(16))) float sA[kC][kPR];   // a, then da
    __shared__ __attribute__((aligned(16))) float sM[kFP][kPR];  // dM
    __shared__ float sKf[kFP], sS0[kD], sCum[kC], sEc[kC], sW[kC], sH[kC], sK0[1];
    __shared__ float sPp[2][kC], sPc[kC];  // SEL: the two waves' feature parts, the constant feature's part

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int unit = blockIdx.x;
    if (unit >= a.B * a.H * a.G) return;
    const int seq = unit / a.G, seg = unit - seq * a.G;
    const int b = seq / a.H, h = seq - b * a.H;
    const float logl = logf(a.decay[h]);
    const size_t so1 = static_cast<size_t>(seq) * kD * kD, so0 = static_cast<size_t>(seq) * kD;
    float *slot = a.G > 1 ? a.ws + static_cast<size_t>(unit) * kWsStride : nullptr;

    // adjoint of the state leaving the last chunk: dM = [dS1; 2 dS2], dKf = [dK1;
    // 2 dK2] of the final state; with segments the dual state at the segment's
    // end, which the reverse scan left in its slot in this convention; zero for
    // the dual pass
    f32x4 mt[4];
#pragma unroll
    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int f = 16 * w + 4 * g + r, col = 16 * dv + c16;
            float x = 0.f;
            if (DUAL) x = 0.f;
            else if (slot) x = f < kD ? slot[kWsS1 + f * kD + col] : slot[kWsS2 + (f - kD) * kD + col];
            else if (f < kD) x = a.ds1o ? a.ds1o[so1 + f * kD + col] : 0.f;
            else x = a.ds2o ? (SEL ? 1.0f : 2.0f) * a.ds2o[so1 + (f - kD) * kD + col] : 0.f;
            mt[dv][r] = x;
            sM[f][col] = x;
        }
    float kreg = 0.f;
    if (DUAL) {
        kreg = 0.f;
    } else if (slot) {
        if (tid < kD) kreg = slot[kWsK1 + tid];
        else if (tid < kFP) kreg = slot[kWsK2 + tid - kD];
        else if (tid < kFP + kD) kreg = slot[kWsS0 + tid - kFP];
        else if (tid == kFP + kD) kreg = slot[kWsK0];
    } else {
        if (tid < kD) kreg = a.dk1o ? a.dk1o[so0 + tid] : 0.f;
        else if (tid < kFP) kreg = a.dk2o ? (SEL ? 1.0f : 2.0f) * a.dk2o[so0 + tid - kD] : 0.f;
        else if (tid < kFP + kD) kreg = a.ds0o ? a.ds0o[so0 + tid - kFP] : 0.f;
        else if (tid == kFP + kD) kreg = a.dk0o ? a.dk0o[seq] : 0.f;
    }
    if (tid < kFP) sKf[tid] = kreg;
    else if (tid < kFP + kD) sS0[tid - kFP] = kreg;
    else if (tid == kFP + kD) sK0[0] = kreg;

    const int NC = (a.L + kC - 1) / kC;
    const int64_t gbase = b * a.g_sb + h * a.g_sh;
    // SEL: the suffix sum of the log decays' adjoint, carried from the last
    // chunk back (every lane of wave 0 holds it), starting with the final
    // state's share; and this thread's part of the key scale's adjoint
    float dl_carry = SEL ? a.fin[seq] : 0.f, dks = 0.f;
    const int c_begin = seg * a.cps, c_end = min(c_begin + a.cps, NC);
    for (int c = c_end - 1; c >= c_begin; --c) {
        load_chunk<SEL>(a, b, h, c, tid, w, lane, sFq, sFk, sV, sG, sCum, sEc, sW, logl);
        __syncthreads();
        if (!DUAL) scores(a, c, w, g, c16, sFq, sFk, sCum, sA);
        if (tid < kC) {
            const int64_t t = static_cast<int64_t>(c) * kC + tid;
            sH[tid] = t < a.L ? a.g_den[static_cast<size_t>(seq) * a.L + t] : 0.f;
        }
        for (int e = tid; e < kC * kD; e += kBW * kWave) {
            const int i = e >> 6, d = e & 63;
            const int64_t t = static_cast<int64_t>(c) * kC + i;
            sG[i][d] = t < a.L ? sG[i][d] * a.inv_den[static_cast<size_t>(seq) * a.L + t] : 0.f;
        }
        __syncthreads();
        const int jb = w >> 1;  // this wave's token block (as the column j of a and da)
        const int64_t t0 = static_cast<int64_t>(c) * kC;
        if constexpr (!DUAL) {
        // ---- dv^T tiles (value blocks 2(w&1)+jj, tokens of block jb):
        //      sum_i a_ij g_i + w_j (Fk_j dM + dS0)
        {
            const int tok = 16 * jb + c16;
            const float wj = sW[tok];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int dv = 2 * (w & 1) + jj;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                for (int s = 4 * jb; s < 16; ++s)  // a_ij = 0 for i < j
                    acc = mfma4(sG[4 * s + g][16 * dv + c16], sA[4 * s + g][tok], acc);
#pragma unroll 8
                for (int s = 0; s < 32; ++s)
                    acc = mfma4(sM[4 * s + g][16 * dv + c16], wj * sFk[tok][4 * s + g], acc);
                if (t0 + tok < a.L) {
                    f32x4 o;
#pragma unroll
                    for (int r = 0; r < 4; ++r) o[r] = acc[r] + wj * sS0[16 * dv + 4 * g + r];
                    store4(a.dv, a.dt_g, gbase + (t0 + tok) * a.g_sl + 16 * dv + 4 * g, o);
                }
            }
        }
        __syncthreads();
        dscores(a, c, w, g, c16, sG, sV, sCum, sH, sA);
        __syncthreads();
        // ---- dFk^T tiles (feature blocks db, 4 + db; tokens of block jb) -> dk:
        //      sum_i da_ij Fq_i + w_j (dM v_j + dKf)
        {
            const int tok = 16 * jb + c16;
            const float wj = sW[tok];
            float pkp = 0.f;  // SEL: sum over this lane's features of Fk . dFk
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int db = 2 * (w & 1) + jj;
                f32x4 d2[2];
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int fb = db + 4 * hf;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    for (int s = 4 * jb; s < 16; ++s)
                        acc = mfma4(sFq[4 * s + g][16 * fb + c16], sA[4 * s + g][tok], acc);
#pragma unroll 8
                    for (int s = 0; s < 16; ++s)
                        acc = mfma4(sM[16 * fb + c16][4 * s + g], wj * sV[tok][4 * s + g], acc);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[r] += wj * sKf[16 * fb + 4 * g + r];
                    d2[hf] = acc;
                }
                if (t0 + tok < a.L) {
                    const f32x4 k = ld4(&sFk[tok][16 * db + 4 * g]);
                    f32x4 dk;
#pragma unroll
                    for (int r = 0; r < 4; ++r) dk[r] = d2[0][r] + k[r] * d2[1][r];
                    if constexpr (SEL) {
                        // Fk holds kscale k: dk above is the adjoint of the scaled key; the
                        // key's is kscale times it, the scale's the sum of k times it
                        const f32x4 kraw = ld4(static_cast<const float *>(a.k) + b * a.k_sb + h * a.k_sh +
                                               (t0 + tok) * a.k_sl + 16 * db + 4 * g);
                        const float ks = a.kscale[h];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            dks += kraw[r] * dk[r];
                            dk[r] *= ks;
                        }
                    }
                    store4(a.dk, a.dt_g, gbase + (t0 + tok) * a.g_sl + 16 * db + 4 * g, dk);
                }
                if constexpr (SEL) {
                    const f32x4 k = ld4(&sFk[tok][16 * db + 4 * g]), k2 = ld4(&sFk[tok][kD + 16 * db + 4 * g]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) pkp += k[r] * d2[0][r] + k2[r] * d2[1][r];
                }
            }
            if constexpr (SEL) {
                // the token's four lane groups, then (after the barrier) the two waves of its token block
                pkp += __shfl_xor(pkp, 16, kWave);
                pkp += __shfl_xor(pkp, 32, kWave);
                if (g == 0) sPp[w & 1][tok] = pkp;
                // the constant feature: sum_i da_ij + w_j (dS0 . v_j + dK0), dS0 and dK0 the
                // adjoint of the state leaving the chunk
                if (tid < kC) {
                    float cs = 0.f, vs = 0.f;
                    for (int i = 16 * (tid >> 4); i < kC; ++i) cs += sA[i][tid];  // (da's lower tiles)
                    for (int d = 0; d < kD; ++d) vs += sS0[d] * sV[tid][d];
                    sPc[tid] = cs + sW[tid] * (vs + sK0[0]);
                }
            }
        }
        }  // !DUAL
        // ---- adjoint to the chunk's start: dM = e^cum_63 dM + Fq^T diag(e^cum) G, and the vectors
        {
            const float e63 = sEc[kC - 1];
#pragma unroll
            for (int dv = 0; dv < 4; ++dv) {
                f32x4 x;
#pragma unroll
                for (int r = 0; r < 4; ++r) x[r] = e63 * mt[dv][r];
#pragma unroll 8
                for (int s = 0; s < 16; ++s) {
                    const int i = 4 * s + g;
                    x = mfma4(sFq[i][16 * w + c16], sEc[i] * sG[i][16 * dv + c16], x);
                }
                mt[dv] = x;
            }
            if (tid < kFP) {
                float acc = e63 * kreg;
                for (int i = 0; i < kC; ++i) acc += sEc[i] * sH[i] * sFq[i][tid];
                kreg = acc;
            } else if (tid < kFP + kD) {
                float acc = e63 * kreg;
                for (int i = 0; i < kC; ++i) acc += sEc[i] * sG[i][tid - kFP];
                kreg = acc;
            } else if (tid == kFP + kD) {
                float acc = e63 * kreg;
                for (int i = 0; i < kC; ++i) acc += sEc[i] * sH[i];
                kreg = acc;
            }
        }
        __syncthreads();
        if constexpr (SEL) {
            // the log decays' adjoint: per token dc = phi_q' . dphi_q' - phi_k' . dphi_k',
            // summed over every later token (a suffix sum over the chunk, plus the carry)
            if (w == 0) {
                const int64_t t = t0 + lane;
                float x = 0.f;
                if (t < a.L) x = a.pq[static_cast<size_t>(seq) * a.L + t] - (sPc[lane] + sPp[0][lane] + sPp[1][lane]);
#pragma unroll
                for (int o = 1; o < kWave; o <<= 1) {
                    const float y = __shfl_down(x, o, kWave);
                    if (lane + o < kWave) x += y;
                }
                if (t < a.L) a.dlogd[static_cast<size_t>(seq) * a.L + t] = x + dl_carry;
                dl_carry += __shfl(x, 0, kWave);
            }
        }
#pragma unroll
        for (int dv = 0; dv < 4; ++dv)
#pragma unroll
            for (int r = 0; r < 4; ++r) sM[16 * w + 4 * g + r][16 * dv + c16] = mt[dv][r];
        if (tid < kFP) sKf[tid] = kreg;
        else if (tid < kFP + kD) sS0[tid - kFP] = kreg;
        else if (tid == kFP + kD) sK0[0] = kreg;
    }
    if constexpr (SEL) {  // the key scale's adjoint, this sequence's share
        const float v = wave_sum(dks);
        __syncthreads();  // (sPp: its last readers passed the loop's barriers)
        if (lane == 0) sPp[0][w] = v;
        __syncthreads();
        if (tid == 0) {
            float tot = 0.f;
            for (int i = 0; i < kBW; ++i) tot += sPp[0][i];
            a.dkscale[seq] = tot;
        }
    }

    if constexpr (DUAL) {
        // the segment's contribution to the dual state at its start, this kernel's convention
#pragma unroll
        for (int dv = 0; dv < 4; ++dv)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = 16 * w + 4 * g + r, col = 16 * dv + c16;
                if (f < kD) slot[kWsS1 + f * kD + col] = mt[dv][r];
                else slot[kWsS2 + (f - kD) * kD + col] = mt[dv][r];
            }
        if (tid < kD) slot[kWsK1 + tid] = kreg;
        else if (tid < kFP) slot[kWsK2 + tid - kD] = kreg;
        else if (tid < kFP + kD) slot[kWsS0 + tid - kFP] = kreg;
        else if (tid == kFP + kD) slot[kWsK0] = kreg;
        return;
    }
    // ---- adjoint of the incoming state: dS1 = dM[:64], dS2 = dM[64:] / 2, dK1, dK2 = dKf[64:] / 2
    // (with segments the reverse scan over them writes it)
    if (a.ds1i && a.G == 1) {
#pragma unroll
        for (int dv = 0; dv < 4; ++dv)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = 16 * w + 4 * g + r, col = 16 * dv + c16;
                if (f < kD) a.ds1i[so1 + f * kD + col] = mt[dv][r];
                else a.ds2i[so1 + (f - kD) * kD + col] = (SEL ? 1.0f : 0.5f) * mt[dv][r];
            }
        // (dense double clamp with a state: plus the dq pass's correction)
        const float* kc = a.dense_in ? a.kcorr + static_cast<size_t>(seq) * kBwdCorr : nullptr;
        if (tid < kD) a.dk1i[so0 + tid] = kreg + (kc ? kc[tid] : 0.f);
        else if (tid < kFP) a.dk2i[so0 + tid - kD] = (SEL ? 1.0f : 0.5f) * (kreg + (kc ? kc[tid] : 0.f));
        else if (tid < kFP + kD) a.ds0i[so0 + tid - kFP] = kreg;
        else if (tid == kFP + kD) a.dk0i[seq] = kreg + (kc ? kc[kFP] : 0.f);
    }
}

hipError_t launch_prefill_backward_f32(const BwdArgs &a, hipStream_t stream) {
    // (with segments the forward's state-only pass has filled the slots)
    const dim3 grid(a.B * a.H * a.G), block(kBW * kWave);
    const TimerEvents t1 = timer_events(PRIME_KERNEL_BWD_DQ);
    const bool sel = a.logd != nullptr;  // (the selective form has no dense clamp and one segment)
    if (sel)
        hipExtLaunchKernelGGL((prefill_bwd_dq_f32_kernel<false, true>), grid, block, 0, stream, t1.start, t1.stop, 0, a);
    else if (a.dense_in)
        hipExtLaunchKernelGGL((prefill_bwd_dq_f32_kernel<true, false>), grid, block, 0, stream, t1.start, t1.stop, 0, a);
    else
        hipExtLaunchKernelGGL((prefill_bwd_dq_f32_kernel<false, false>), grid, block, 0, stream, t1.start, t1.stop, 0, a);
    hipError_t e;
    if ((e = hipGetLastError()) != hipSuccess) return timer_drop(t1), e;
    if (a.G > 1 && !sel) {
        // each segment's dual contribution, then the reverse scan (slots now hold dual states)
        const TimerEvents td = timer_events(PRIME_KERNEL_BWD_DUAL);
        hipExtLaunchKernelGGL((prefill_bwd_dkv_f32_kernel<false, true>), grid, block, 0, stream, td.start, td.stop, 0,
                              a);
        if ((e = hipGetLastError()) != hipSuccess) return timer_drop(td), e;
        if ((e = launch_bwd_dual_scan(a, stream)) != hipSuccess) return e;
    }
    const TimerEvents t2 = timer_events(PRIME_KERNEL_BWD_DKV);
    if (sel)
        hipExtLaunchKernelGGL((prefill_bwd_dkv_f32_kernel<true, false>), grid, block, 0, stream, t2.start, t2.stop, 0,
                              a);
    else
        hipExtLaunchKernelGGL((prefill_bwd_dkv_f32_kernel<false, false>), grid, block, 0, stream, t2.start, t2.stop,
                              0, a);
    if ((e = hipGetLastError()) != hipSuccess) timer_drop(t2);
    return e;
}

}  // namespace prime
