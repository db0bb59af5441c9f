// Selective PRIME prefill for fp32 inputs, in fp32 throughout
// (PrimeSelectiveMomentAttention computes in fp32, selective.py:363-365,
// 414-440).
//
// The recurrence (selective.py:394-408) with per-token decays l_t = e^ld_t,
// key features Fk_j = [beta k_j, beta^2/2 (k_j*k_j)] and query features
// Fq_i = [q_i, q_i*q_i], in 64-token chunks with cum_i = sum_{s<=i} ld_s:
//   A_ij  = [j <= i] e^(cum_i - cum_j) (1 + Fq_i . Fk_j)
//   num_i = sum_j A_ij v_j + e^cum_i (S0 + Fq_i M),   M = [S1; S2]  (128 x 64)
//   den_i = sum_j A_ij     + e^cum_i (K0 + Fq_i . Kf), Kf = [K1; K2]
//   y_i   = num_i / max(den_i, eps)
//   M <- e^cum_63 M + Fk^T diag(w) V,  w_j = e^(cum_63 - cum_j)  (likewise S0, K0, Kf)
// Tokens past L carry no weight and no decay, so the final state is the state
// after token L-1.
//
// One workgroup of 8 waves per (sequence, head), chunks in order; every
// product is an fp32 MFMA (v_mfma_f32_16x16x4_f32: lane l holds A[l%16][l/16]
// and B[l/16][l%16], the accumulator D[4(l/16) + r][l%16]).  Per chunk:
//   load the chunk's features | A (10 lower tiles) | denominators |
//   y^T tiles (value block x token block: V^T A^T + M^T (e^cum Fq)^T) and the
//   state update (wave w owns M's feature rows 16w..16w+15 in accumulators) |
//   publish the state to LDS for the next chunk's readout.
// Few long sequences run in segments of a.cps chunks, as the bf16 path does:
// a state-only pass (STATE_ONLY: no readout) forms every segment's state from
// zero and its total log decay, the scan over segments turns them into the
// state entering each segment, and the main pass runs one workgroup per
// (sequence, segment) from that state.

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kFP = 2 * kD;   // features
constexpr int kPQ = kFP + 4;  // Fq / Fk rows: 16-byte reads of 16 rows fall on distinct bank quads
constexpr int kPV = kD + 16;  // V rows: scalar reads of 4 rows x 16 columns meet no bank twice
constexpr int kPA = kC + 4;   // A rows
constexpr int kPM = kD + 16;  // M rows (as V)
constexpr int kSelWaves = 8;

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }
__device__ __forceinline__ void st4(float *p, f32x4 v) { *reinterpret_cast<f32x4 *>(p) = v; }

__device__ __forceinline__ void store_y4(void *y, int dt, int64_t idx, f32x4 v) {
    if (dt == PRIME_F32) {
        st4(static_cast<float *>(y) + idx, v);
    } else if (dt == PRIME_BF16) {
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + idx) = uint2{pack2(v[0], v[1]), pack2(v[2], v[3])};
    } else {
        uint16_t *p = static_cast<uint16_t *>(y) + idx;
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = f32_to_h16_bits(v[r]);
    }
}

}  // namespace

template <bool STATE_ONLY>
__global__ __launch_bounds__(kSelWaves * kWave, 1) void selective_prefill_f32_kernel(const PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) float sFq[kC][kPQ];
    __shared__ __attribute__((aligned(16))) float sFk[kC][kPQ];
    __shared__ __attribute__((aligned(16))) float sV[kC][kPV];
    __shared__ __attribute__((aligned(16))) float sA[kC][kPA];
    __shared__ __attribute__((aligned(16))) float sM[kFP][kPM];
    __shared__ float sKf[kFP], sS0[kD], sCum[kC], sEc[kC], sW[kC], sDen[kC], sK0[1];

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    // units: (sequence, segment); the state-only pass takes segments 0 .. G-2
    const int nseg = STATE_ONLY ? a.G - 1 : a.G;
    const int unit = blockIdx.x;
    if (unit >= a.B * a.H * nseg) return;
    const int seq = unit / nseg, seg = unit - seq * nseg;
    float *slot = a.G > 1 ? a.ws + (static_cast<size_t>(seq) * a.G + seg) * kWsStride : nullptr;
    const int b = seq / a.H, h = seq - b * a.H, hk = h / a.group;
    const float beta = a.k_scale[h], hb2 = 0.5f * beta * beta;
    const float *ldp = a.log_decay + static_cast<size_t>(seq) * a.L;
    const float *qf = static_cast<const float *>(a.q);
    const float *kf = static_cast<const float *>(a.k);
    const float *vf = static_cast<const float *>(a.v);
    const size_t so1 = static_cast<size_t>(seq) * kD * kD, so0 = static_cast<size_t>(seq) * kD;

    // ---- incoming state: M tiles of feature block w in accumulators (and in
    // LDS for the readout); thread t < 128 holds Kf[t], 128..191 S0, 192 K0
    f32x4 mt[4];
#pragma unroll
    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int f = 16 * w + 4 * g + r, col = 16 * dv + c16;
            float x = 0.f;
            if (STATE_ONLY) x = 0.f;
            else if (slot) x = f < kD ? slot[kWsS1 + f * kD + col] : slot[kWsS2 + (f - kD) * kD + col];
            else if (a.s1i) x = f < kD ? a.s1i[so1 + f * kD + col] : a.s2i[so1 + (f - kD) * kD + col];
            mt[dv][r] = x;
            sM[f][col] = x;
        }
    float kreg = 0.f;
    if (STATE_ONLY) {
        kreg = 0.f;
    } else if (slot) {
        if (tid < kD) kreg = slot[kWsK1 + tid];
        else if (tid < kFP) kreg = slot[kWsK2 + tid - kD];
        else if (tid < kFP + kD) kreg = slot[kWsS0 + tid - kFP];
        else if (tid == kFP + kD) kreg = slot[kWsK0];
    } else if (a.s1i) {
        if (tid < kD) kreg = a.k1i[so0 + tid];
        else if (tid < kFP) kreg = a.k2i[so0 + tid - kD];
        else if (tid < kFP + kD) kreg = a.s0i[so0 + tid - kFP];
        else if (tid == kFP + kD) kreg = a.k0i[seq];
    }
    if (tid < kFP) sKf[tid] = kreg;
    else if (tid < kFP + kD) sS0[tid - kFP] = kreg;
    else if (tid == kFP + kD) sK0[0] = kreg;

    const int NC = (a.L + kC - 1) / kC;
    const int c_begin = seg * a.cps, c_end = min(c_begin + a.cps, NC);
    const int64_t ybase = b * a.y_sb + h * a.y_sh;
    float seg_ld = 0.f;  // (state-only, wave 0) the segment's total natural-log decay
    for (int c = c_begin; c < c_end; ++c) {
        // ---- the chunk's features: thread = (token tid/8, 8 dims)
        {
            const int i = tid >> 3, d0 = 8 * (tid & 7);
            const int t = c * kC + i;
            const bool valid = t < a.L;
            const int64_t tc = valid ? t : a.L - 1;
            const float *qp = qf + b * a.q_sb + h * a.q_sh + tc * a.q_sl + d0;
            const float *kp = kf + b * a.k_sb + hk * a.k_sh + tc * a.k_sl + d0;
            const float *vp = vf + b * a.v_sb + hk * a.v_sh + tc * a.v_sl + d0;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                const f32x4 q = valid ? ld4(qp + 4 * j) : z, k = valid ? ld4(kp + 4 * j) : z,
                            v = valid ? ld4(vp + 4 * j) : z;
                f32x4 q2, k1, k2;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    q2[r] = q[r] * q[r];
                    k1[r] = beta * k[r];
                    k2[r] = hb2 * (k[r] * k[r]);
                }
                st4(&sFq[i][d0 + 4 * j], q);
                st4(&sFq[i][kD + d0 + 4 * j], q2);
                st4(&sFk[i][d0 + 4 * j], k1);
                st4(&sFk[i][kD + d0 + 4 * j], k2);
                st4(&sV[i][d0 + 4 * j], v);
            }
        }
        if (w == 0) {
            const int t = c * kC + lane;
            const bool valid = t < a.L;
            float cum = valid ? ldp[t] : 0.f;
#pragma unroll
            for (int s = 1; s < 64; s <<= 1) {
                const float x = __shfl_up(cum, s, kWave);
                if (lane >= s) cum += x;
            }
            const float cend = __shfl(cum, 63, kWave);
            seg_ld += cend;
            sCum[lane] = cum;
            sEc[lane] = expf(cum);
            sW[lane] = valid ? expf(cend - cum) : 0.f;
        }
        __syncthreads();

        if constexpr (!STATE_ONLY) {
        // ---- A on the 10 lower 16x16 tiles (feature k-slot g of k-step s: 32g + s)
        for (int ti = w; ti < 10; ti += kSelWaves) {
            const int ib = ti < 1 ? 0 : ti < 3 ? 1 : ti < 6 ? 2 : 3;
            const int jb = ti - ib * (ib + 1) / 2;
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
        __syncthreads();

        // ---- denominators, four threads per token (thread qt sums A's column
        // block qt, written only for qt <= i/16: the upper tiles are never formed)
        if (tid < 4 * kC) {
            const int i = tid >> 2, qt = tid & 3;
            float part = 0.f;
            if (qt <= (i >> 4)) {
#pragma unroll
                for (int e = 0; e < 16; ++e) part += sA[i][16 * qt + e];
            }
            float rd = qt == 0 ? sK0[0] : 0.f;
#pragma unroll
            for (int e = 0; e < 32; ++e) rd += sFq[i][32 * qt + e] * sKf[32 * qt + e];
            part += sEc[i] * rd;
            part += xor_lane<1>(part);
            part += xor_lane<2>(part);
            if (qt == 0) sDen[i] = fmaxf(part, a.eps);
        }
        __syncthreads();

        // ---- y^T tiles: token block w/2, value blocks 2(w&1) and 2(w&1)+1
        {
            const int ib = w >> 1;
            const int tok = 16 * ib + c16;
            const float ec = sEc[tok];
            const int64_t t = static_cast<int64_t>(c) * kC + tok;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int dv = 2 * (w & 1) + jj;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                for (int s = 0; s < 4 * (ib + 1); ++s)  // A is zero above token 16 ib + 15
                    acc = mfma4(sV[4 * s + g][16 * dv + c16], sA[tok][4 * s + g], acc);
#pragma unroll 8
                for (int s = 0; s < 32; ++s) acc = mfma4(sM[4 * s + g][16 * dv + c16], ec * sFq[tok][4 * s + g], acc);
                if (t < a.L) {
                    const float rden = 1.0f / sDen[tok];
                    f32x4 yv;
#pragma unroll
                    for (int r = 0; r < 4; ++r) yv[r] = (acc[r] + ec * sS0[16 * dv + 4 * g + r]) * rden;
                    store_y4(a.y, a.dt_y, ybase + t * a.y_sl + 16 * dv + 4 * g, yv);
                }
            }
        }
        }  // !STATE_ONLY
        // ---- state update: M tiles of feature block w; Kf, S0, K0 by their threads
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
            } else if (tid < kFP + kD) {
                float acc = e63 * kreg;
                for (int j = 0; j < kC; ++j) acc += sW[j] * sV[j][tid - kFP];
                kreg = acc;
            } else if (tid == kFP + kD) {
                float acc = e63 * kreg;
                for (int j = 0; j < kC; ++j) acc += sW[j];
                kreg = acc;
            }
        }
        __syncthreads();
        // ---- publish the state for the next chunk's readout (ordered before
        // its use by the barrier after the next chunk's loads)
#pragma unroll
        for (int dv = 0; dv < 4; ++dv)
#pragma unroll
            for (int r = 0; r < 4; ++r) sM[16 * w + 4 * g + r][16 * dv + c16] = mt[dv][r];
        if (tid < kFP) sKf[tid] = kreg;
        else if (tid < kFP + kD) sS0[tid - kFP] = kreg;
        else if (tid == kFP + kD) sK0[0] = kreg;
    }

    if constexpr (STATE_ONLY) {
        // the segment's state from zero and its log2 decay, for the scan over segments
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
        if (tid == 0) slot[kWsDecay] = seg_ld * 1.44269504088896341f;  // log2
        return;
    }
    // ---- final state, in the selective convention (S2, K2 carry the 1/2)
    if (a.s1o && seg == a.G - 1) {
#pragma unroll
        for (int dv = 0; dv < 4; ++dv)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = 16 * w + 4 * g + r, col = 16 * dv + c16;
                if (f < kD) a.s1o[so1 + f * kD + col] = mt[dv][r];
                else a.s2o[so1 + (f - kD) * kD + col] = mt[dv][r];
            }
        if (tid < kD) a.k1o[so0 + tid] = kreg;
        else if (tid < kFP) a.k2o[so0 + tid - kD] = kreg;
        else if (tid < kFP + kD) a.s0o[so0 + tid - kFP] = kreg;
        else if (tid == kFP + kD) a.k0o[seq] = kreg;
    }
}

hipError_t launch_selective_f32(const PrefillArgs &a, hipStream_t stream) {
    const int S = a.B * a.H;
    hipError_t e;
    if (a.G > 1) {
        const TimerEvents ta = timer_events(PRIME_KERNEL_PREFILL_SEGMENTS);
        hipExtLaunchKernelGGL(selective_prefill_f32_kernel<true>, dim3(S * (a.G - 1)), dim3(kSelWaves * kWave), 0,
                              stream, ta.start, ta.stop, 0, a);
        if ((e = hipGetLastError()) != hipSuccess) return timer_drop(ta), e;
        if ((e = launch_segment_scan(a, stream)) != hipSuccess) return e;
    }
    const TimerEvents t = timer_events(PRIME_KERNEL_PREFILL_CHUNKS);
    hipExtLaunchKernelGGL(selective_prefill_f32_kernel<false>, dim3(S * a.G), dim3(kSelWaves * kWave), 0, stream,
                          t.start, t.stop, 0, a);
    e = hipGetLastError();
    if (e != hipSuccess) timer_drop(t);
    return e;
}

}  // namespace prime
