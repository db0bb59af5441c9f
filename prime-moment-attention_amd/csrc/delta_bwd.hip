// Backward of the chunked gated delta-rule PRIME prefill
// (ChunkedGatedDeltaPrimeAttention, chunked_delta_prime.py:177-283), gfx950.
//
// Per (sequence, head), chunk c of C = 64 tokens with features psi_i, phi_i
// (chunked_delta_prime.py:73-87: psi = [q, q^2/sqrt2], phi = [k/|k|,
// (k^2/|k^2|)/sqrt2]), values v_i, write rates beta_i, cumulative log-decays
// g_i = sum_{m<=i} log clamp(alpha_m, 1e-5, 1), entering state S (D x 2D):
//   d_i = e^{g_i},  b_j = e^{g_63 - g_j},  a = e^{g_63},  L_ij = e^{g_i - g_j} (i >= j)
//   T   = I + [i>j] beta_j L_ij (phi_i . phi_j)            (unit lower triangular)
//   U   = V - diag(d) Phi S^T,   E = T^-1 U,   W = diag(beta) E
//   y   = M W + diag(d) Psi S^T,  M_ij = [i>=j] L_ij (psi_i . phi_j)
//   S'  = a S + W^T diag(b) Phi,  S'' = S' min(1, B / (|S'|_F + 1e-6)).
// The backward walks the chunks in reverse with the adjoint dS of the state
// leaving the chunk:
//   clamp:  dS' = s dS'' - [s < 1 or = 1] (B / (n+1e-6)^2) <dS'', S'> / n  S'
//   state:  dS_in = a dS' + (diag(d) dY)^T Psi - (diag(d) dU)^T Phi
//           dW = diag(b) Phi dS'^T + M^T dY,  dE = diag(beta) dW,
//           dU = T^-T dE,  dT = -dU E^T (strictly lower),  dV = dU
//   features: dPsi = (dM o L) Phi + diag(d) dY S,   dM = dY W^T (masked)
//           dPhi = diag(b) W dS' + (dM o L)^T Psi + (dG + dG^T) Phi - diag(d) dU S,
//           dG_ij = dT_ij beta_j L_ij
//   beta:   dbeta = rowdot(E, dW) + colsum(dT o L o G)
//   decays: dg from a, b, d, L in T and M; dlog alpha = reverse cumulative sum
//           of dg over the chunk; dalpha = dlog alpha / alpha inside the clamp
// and q, k through the feature maps (F.normalize's backward for the k
// features, eps = feat_eps).  The state entering every chunk comes from a
// forward recompute pass (delta_chunk_kernel<false>) into the workspace.
//
// Everything is fp32 on the VALU: one workgroup of 4 waves per (sequence,
// head), the chunk's q, k, v, dy and the C x C / C x D work arrays in LDS, the
// D x 2D state, its adjoint and the C x 2D feature adjoints in registers
// (thread t owns row t/4, columns 32 (t%4) .. +31), the triangular solves
// column-parallel with the substitution terms in registers (four lanes per
// column, shuffles only).  Features are formed from q and k as they are read.

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kDC = 64, kDD = 64, kDF = 128;
constexpr int kDP = kDD + 4;   // pitch of the C x D / C x C arrays (floats)
constexpr int kDPF = kDF + 4;  // pitch of the D x 2D operand array
constexpr float kInvSqrt2 = 0.70710678118654752f;

__device__ __forceinline__ float red4(float x) {
    x += __shfl_xor(x, 1, kWave);
    x += __shfl_xor(x, 2, kWave);
    return x;
}

// 16 consecutive inputs of one row as fp32 (bf16 or fp32 storage), zero when !valid
__device__ __forceinline__ void load_row16(const void *p, int64_t off, int dt, bool valid, float *o) {
    if (!valid) {
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] = 0.f;
        return;
    }
    if (dt == PRIME_BF16) {
        const u32x4 *s = reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p) + off);
        const u32x4 x = s[0], y = s[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(x[i] << 16);
            o[2 * i + 1] = __uint_as_float(x[i] & 0xFFFF0000u);
            o[8 + 2 * i] = __uint_as_float(y[i] << 16);
            o[8 + 2 * i + 1] = __uint_as_float(y[i] & 0xFFFF0000u);
        }
    } else {
        const f32x4 *s = reinterpret_cast<const f32x4 *>(static_cast<const float *>(p) + off);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 v = s[i];
#pragma unroll
            for (int r = 0; r < 4; ++r) o[4 * i + r] = v[r];
        }
    }
}

}  // namespace

// BWD false: the forward recompute (the state entering every chunk into the
// workspace); true: the reverse scan.
template <bool BWD>
__global__ __launch_bounds__(256) void delta_chunk_kernel(const DeltaBwdArgs a) {
    __shared__ float sQ[kDC][kDP], sK[kDC][kDP], sT[kDC][kDP], sM[kDC][kDP], sE[kDC][kDP], sW[kDC][kDP];
    __shared__ float sY[BWD ? kDC : 1][kDP];
    __shared__ float sOp[BWD ? kDD : 1][kDPF];
    __shared__ float sG[kDC], sBeta[kDC], sAl[kDC], sDi[kDC], sBj[kDC], sR1[kDC], sR2[kDC], sDg[kDC], sDb[kDC];
    __shared__ float sRed[8];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bh = blockIdx.x, b = bh / a.H, h = bh - b * a.H, hk = h / a.group;
    const int NC = (a.L + kDC - 1) / kDC;
    // row-owner mapping of D x 2D and C x 2D arrays: row ro, columns 32 fq .. +31,
    // i.e. half h2 of the features (0: k or q, 1: the squares), elements e0 .. e0+31
    const int ro = tid >> 2, fq = tid & 3, h2 = fq >> 1, e0 = 32 * (fq & 1);
    // 4 x 4 block mapping of C x C and C x D arrays
    const int bi0 = 4 * (tid >> 4), bj0 = 4 * (tid & 15);
    float *wsbh = a.ws + static_cast<size_t>(bh) * NC * kDD * kDF;
    const float bound = a.bound;

    auto block_sum = [&](float x) {
        x = wave_sum(x);
        __syncthreads();
        if (lane == 0) sRed[wave] = x;
        __syncthreads();
        return sRed[0] + sRed[1] + sRed[2] + sRed[3];
    };

    float S[32];  // state entering the chunk (row ro)
    if constexpr (!BWD) {
#pragma unroll
        for (int u = 0; u < 32; ++u)
            S[u] = a.state_in ? a.state_in[static_cast<size_t>(bh) * kDD * kDF + ro * kDF + 32 * fq + u] : 0.f;
    }
    float dS[32];  // BWD: adjoint of the state leaving the chunk
    if constexpr (BWD) {
#pragma unroll
        for (int u = 0; u < 32; ++u)
            dS[u] = a.dstate_out ? a.dstate_out[static_cast<size_t>(bh) * kDD * kDF + ro * kDF + 32 * fq + u] : 0.f;
    }

    for (int it = 0; it < NC; ++it) {
        const int c = BWD ? NC - 1 - it : it;
        const int t0 = c * kDC, nv = min(kDC, a.L - t0);
        float *wsc = wsbh + static_cast<size_t>(c) * kDD * kDF;
        if constexpr (!BWD) {
#pragma unroll
            for (int u = 0; u < 32; ++u) wsc[ro * kDF + 32 * fq + u] = S[u];
        } else {
#pragma unroll
            for (int u = 0; u < 32; ++u) S[u] = wsc[ro * kDF + 32 * fq + u];
        }
        // ---- chunk inputs: rows r = tid / 4, 16 columns each
        {
            const int r = tid >> 2, c0 = 16 * (tid & 3);
            const bool valid = r < nv;
            const int64_t tok = t0 + (valid ? r : 0);
            float tmp[16];
            load_row16(a.q, b * a.q_sb + h * a.q_sh + tok * a.q_sl + c0, a.dt_in, valid, tmp);
#pragma unroll
            for (int e = 0; e < 16; ++e) sQ[r][c0 + e] = tmp[e];
            load_row16(a.k, b * a.k_sb + hk * a.k_sh + tok * a.k_sl + c0, a.dt_in, valid, tmp);
#pragma unroll
            for (int e = 0; e < 16; ++e) sK[r][c0 + e] = tmp[e];
            load_row16(a.v, b * a.v_sb + hk * a.v_sh + tok * a.v_sl + c0, a.dt_in, valid, tmp);
#pragma unroll
            for (int e = 0; e < 16; ++e) sW[r][c0 + e] = tmp[e];
            if constexpr (BWD) {
                load_row16(a.dy, b * a.dy_sb + h * a.dy_sh + tok * a.dy_sl + c0, a.dt_dy, valid, tmp);
#pragma unroll
                for (int e = 0; e < 16; ++e) sY[r][c0 + e] = tmp[e];
            }
            if (tid < kDC) {
                const size_t gi = static_cast<size_t>(bh) * a.L + t0 + tid;
                sBeta[tid] = tid < nv ? a.beta[gi] : 0.f;
                sAl[tid] = tid < nv ? a.alpha[gi] : a.decay_pad;
                sDg[tid] = 0.f;
                sDb[tid] = 0.f;
            }
        }
        __syncthreads();
        {
            // k feature norms: 1 / max(|k|, eps), 1 / max(|k^2|, eps)
            const int r = tid >> 2, c0 = 16 * (tid & 3);
            float s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float x = sK[r][c0 + e], x2 = x * x;
                s1 += x2;
                s2 += x2 * x2;
            }
            s1 = red4(s1);
            s2 = red4(s2);
            if ((tid & 3) == 0) {
                sR1[r] = 1.0f / fmaxf(sqrtf(s1), a.feat_eps);
                sR2[r] = 1.0f / fmaxf(sqrtf(s2), a.feat_eps);
            }
            if (wave == 0) {
                const float lg = logf(fminf(fmaxf(sAl[lane], 1e-5f), 1.0f));
                const float g = wave_prefix_sum(lg);
                const float g63 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), 63));
                sG[lane] = g;
                sDi[lane] = expf(g);
                sBj[lane] = expf(g63 - g);
                if (lane == 0) sRed[4] = expf(g63);
            }
        }
        __syncthreads();
        const float aC = sRed[4];

        // ---- T (and L o G kept for the backward), 4 x 4 block per thread
        float LG[4][4];
        {
            float d1[4][4], d2[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) d1[i][j] = d2[i][j] = 0.f;
            for (int e = 0; e < kDD; ++e) {
                float ki[4], kj[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) ki[i] = sK[bi0 + i][e];
#pragma unroll
                for (int j = 0; j < 4; ++j) kj[j] = sK[bj0 + j][e];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        d1[i][j] = fmaf(ki[i], kj[j], d1[i][j]);
                        d2[i][j] = fmaf(ki[i] * ki[i], kj[j] * kj[j], d2[i][j]);
                    }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int ii = bi0 + i, jj = bj0 + j;
                    const float G = sR1[ii] * sR1[jj] * d1[i][j] + 0.5f * sR2[ii] * sR2[jj] * d2[i][j];
                    LG[i][j] = ii > jj ? expf(sG[ii] - sG[jj]) * G : 0.f;
                    sT[ii][jj] = ii > jj ? sBeta[jj] * LG[i][j] : (ii == jj ? 1.f : 0.f);
                }
        }
        // ---- U = V - diag(d) Phi S^T  (row-owner over d = ro; sW holds V)
        for (int i = 0; i < kDC; ++i) {
            float p = 0.f;
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const float kx = sK[i][e0 + u];
                p = fmaf(h2 ? kx * kx : kx, S[u], p);
            }
            p *= h2 ? sR2[i] * kInvSqrt2 : sR1[i];
            p = red4(p);
            if (fq == 0) sW[i][ro] -= sDi[i] * p;
        }
        __syncthreads();
        // ---- E = T^-1 U: column d = tid / 4, lanes q = tid % 4 hold e_j, j = q mod 4
        {
            const int d = tid >> 2, q = tid & 3;
            float er[16];
#pragma unroll
            for (int i = 0; i < kDC; ++i) {
                float p = 0.f;
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) {
                    const int j = 4 * jj + q;
                    if (j < i) p = fmaf(sT[i][j], er[jj], p);
                }
                p = red4(p);
                const float e = sW[i][d] - p;
                if ((i & 3) == q) er[i >> 2] = e;
                if (q == 0) sE[i][d] = e;
            }
        }
        __syncthreads();
        // ---- S' = a S + W^T diag(b) Phi and its Frobenius norm
        float Sp[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) Sp[u] = aC * S[u];
        for (int j = 0; j < kDC; ++j) {
            const float coef = sBj[j] * sBeta[j] * sE[j][ro] * (h2 ? sR2[j] * kInvSqrt2 : sR1[j]);
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const float kx = sK[j][e0 + u];
                Sp[u] = fmaf(coef, h2 ? kx * kx : kx, Sp[u]);
            }
        }
        float n2 = 0.f;
#pragma unroll
        for (int u = 0; u < 32; ++u) n2 = fmaf(Sp[u], Sp[u], n2);
        n2 = block_sum(n2);
        const float nrm = sqrtf(n2);
        const float x = bound / (nrm + 1e-6f);
        const bool clamp = bound > 0.f && x <= 1.0f;
        if constexpr (!BWD) {
            const float s = clamp ? x : 1.0f;
#pragma unroll
            for (int u = 0; u < 32; ++u) S[u] = s * Sp[u];
            __syncthreads();  // the next chunk's inputs overwrite the LDS arrays
        } else {
        // ================================================================ backward
        // ---- clamp
        float dSp[32];
        if (clamp) {
            float c1 = 0.f;
#pragma unroll
            for (int u = 0; u < 32; ++u) c1 = fmaf(dS[u], Sp[u], c1);
            c1 = block_sum(c1);
            const float den = nrm + 1e-6f;
            const float coef = -bound / (den * den) * c1 / nrm;
#pragma unroll
            for (int u = 0; u < 32; ++u) dSp[u] = x * dS[u] + coef * Sp[u];
        } else {
#pragma unroll
            for (int u = 0; u < 32; ++u) dSp[u] = dS[u];
        }
        float dSin[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) dSin[u] = aC * dSp[u];
        float dg63 = 0.f;  // (every thread holds the same value)
        {
            float t = 0.f;
#pragma unroll
            for (int u = 0; u < 32; ++u) t = fmaf(dSp[u], S[u], t);
            dg63 += aC * block_sum(t);
        }
#pragma unroll
        for (int u = 0; u < 32; ++u) sOp[ro][32 * fq + u] = dSp[u];
        __syncthreads();
        // ---- dW (state) = diag(b) Phi dS'^T into sW (U is no longer needed)
        for (int j = 0; j < kDC; ++j) {
            float p = 0.f;
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const float kx = sK[j][e0 + u];
                p = fmaf(h2 ? kx * kx : kx, dSp[u], p);
            }
            p *= h2 ? sR2[j] * kInvSqrt2 : sR1[j];
            p = red4(p);
            if (fq == 0) sW[j][ro] = sBj[j] * p;
        }
        __syncthreads();
        // z_j = E_j . dW_j: dg_63 += sum_j beta_j z_j, dg_j -= beta_j z_j
        {
            const int j = ro;
            float z = 0.f;
#pragma unroll
            for (int u = 0; u < 16; ++u) z = fmaf(sE[j][16 * fq + u], sW[j][16 * fq + u], z);
            z = red4(z) * sBeta[j];
            if (fq == 0) sDg[j] -= z;
            dg63 += block_sum(fq == 0 ? z : 0.f);
        }
        // dPhi (state) = diag(b beta) E dS'  (row-owner over j = ro)
        float dPhi[32], dPsi[32];
        {
            const float w = sBj[ro] * sBeta[ro];
#pragma unroll
            for (int u = 0; u < 32; ++u) dPhi[u] = 0.f;
            for (int d = 0; d < kDD; ++d) {
                const float e = sE[ro][d];
#pragma unroll
                for (int u = 0; u < 32; ++u) dPhi[u] = fmaf(e, sOp[d][32 * fq + u], dPhi[u]);
            }
#pragma unroll
            for (int u = 0; u < 32; ++u) dPhi[u] *= w;
        }
        // ---- M (block), dW += M^T dY, dM = dY W^T (masked)
        float Mb[4][4], dMb[4][4];
        {
            float d1[4][4], d2[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) d1[i][j] = d2[i][j] = 0.f;
            for (int e = 0; e < kDD; ++e) {
                float qi[4], kj[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) qi[i] = sQ[bi0 + i][e];
#pragma unroll
                for (int j = 0; j < 4; ++j) kj[j] = sK[bj0 + j][e];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        d1[i][j] = fmaf(qi[i], kj[j], d1[i][j]);
                        d2[i][j] = fmaf(qi[i] * qi[i], kj[j] * kj[j], d2[i][j]);
                    }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int ii = bi0 + i, jj = bj0 + j;
                    Mb[i][j] = ii >= jj ? expf(sG[ii] - sG[jj]) * (sR1[jj] * d1[i][j] + 0.5f * sR2[jj] * d2[i][j]) : 0.f;
                }
        }
        __syncthreads();  // (z reads of sW done)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) sM[bi0 + i][bj0 + j] = Mb[i][j];
        __syncthreads();
        {
            // dW[j][d] += sum_i M_ij dY[i][d]  (block: j = bi0.., d = bj0..)
            float o[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) o[i][j] = 0.f, dMb[i][j] = 0.f;
            for (int r = 0; r < kDC; ++r) {
                float m[4], y[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) m[i] = sM[r][bi0 + i];
#pragma unroll
                for (int j = 0; j < 4; ++j) y[j] = sY[r][bj0 + j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) o[i][j] = fmaf(m[i], y[j], o[i][j]);
            }
            // dM_ij = beta_j (dY_i . E_j)  (block: i = bi0.., j = bj0..)
            for (int d = 0; d < kDD; ++d) {
                float y[4], e[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = sY[bi0 + i][d];
#pragma unroll
                for (int j = 0; j < 4; ++j) e[j] = sE[bj0 + j][d];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) dMb[i][j] = fmaf(y[i], e[j], dMb[i][j]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sW[bi0 + i][bj0 + j] += o[i][j];
                    const int ii = bi0 + i, jj = bj0 + j;
                    dMb[i][j] = ii >= jj ? dMb[i][j] * sBeta[jj] : 0.f;
                }
        }
        __syncthreads();
        // dg from L in M: dg_i += sum_j dM_ij M_ij, dg_j -= sum_i dM_ij M_ij
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) sM[bi0 + i][bj0 + j] = dMb[i][j] * Mb[i][j];
        __syncthreads();
        if (tid < kDC) {
            float rs = 0.f, cs = 0.f;
            for (int j = 0; j < kDC; ++j) {
                rs += sM[tid][j];
                cs += sM[j][tid];
            }
            sDg[tid] += rs - cs;
        }
        __syncthreads();
        // dM o L into sM; dPsi = (dM o L) Phi, dPhi += (dM o L)^T Psi
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ii = bi0 + i, jj = bj0 + j;
                sM[ii][jj] = ii >= jj ? dMb[i][j] * expf(sG[ii] - sG[jj]) : 0.f;
            }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 32; ++u) dPsi[u] = 0.f;
        for (int j = 0; j < kDC; ++j) {
            const float cpsi = sM[ro][j] * (h2 ? sR2[j] * kInvSqrt2 : sR1[j]);  // (dM o L)_{ro, j} phi_j
            const float cphi = sM[j][ro] * (h2 ? kInvSqrt2 : 1.0f);              // (dM o L)_{j, ro} psi_j
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const float kx = sK[j][e0 + u], qx = sQ[j][e0 + u];
                dPsi[u] = fmaf(cpsi, h2 ? kx * kx : kx, dPsi[u]);
                dPhi[u] = fmaf(cphi, h2 ? qx * qx : qx, dPhi[u]);
            }
        }
        __syncthreads();
        // ---- S_in as the LDS operand: the inter-chunk readout's terms
#pragma unroll
        for (int u = 0; u < 32; ++u) sOp[ro][32 * fq + u] = S[u];
        __syncthreads();
        {
            // dPsi_i += d_i S^T dy_i; dg_i += psi_i . (that term)
            float tmp[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) tmp[u] = 0.f;
            for (int d = 0; d < kDD; ++d) {
                const float y = sY[ro][d];
#pragma unroll
                for (int u = 0; u < 32; ++u) tmp[u] = fmaf(y, sOp[d][32 * fq + u], tmp[u]);
            }
            const float di = sDi[ro];
            float dot = 0.f;
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                tmp[u] *= di;
                dPsi[u] += tmp[u];
                const float qx = sQ[ro][e0 + u];
                dot = fmaf(h2 ? qx * qx * kInvSqrt2 : qx, tmp[u], dot);
            }
            dot = red4(dot);
            if (fq == 0) sDg[ro] += dot;
            // dS_in += sum_i d_i dy_i psi_i^T  (row-owner over d = ro)
            for (int i = 0; i < kDC; ++i) {
                const float y = sDi[i] * sY[i][ro] * (h2 ? kInvSqrt2 : 1.0f);
#pragma unroll
                for (int u = 0; u < 32; ++u) {
                    const float qx = sQ[i][e0 + u];
                    dSin[u] = fmaf(y, h2 ? qx * qx : qx, dSin[u]);
                }
            }
        }
        // ---- dbeta_i += E_i . dW_i, dE = beta dW (in place)
        {
            const int i = ro;
            float z = 0.f;
#pragma unroll
            for (int u = 0; u < 16; ++u) z = fmaf(sE[i][16 * fq + u], sW[i][16 * fq + u], z);
            z = red4(z);
            if (fq == 0) sDb[i] += z;
            const float bi = sBeta[i];
#pragma unroll
            for (int u = 0; u < 16; ++u) sW[i][16 * fq + u] *= bi;
        }
        __syncthreads();
        // ---- dU = T^-T dE (backward substitution, in place in sW)
        {
            const int d = tid >> 2, q = tid & 3;
            float ur[16];
#pragma unroll
            for (int i = kDC - 1; i >= 0; --i) {
                float p = 0.f;
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) {
                    const int j = 4 * jj + q;
                    if (j > i) p = fmaf(sT[j][i], ur[jj], p);
                }
                p = red4(p);
                const float du = sW[i][d] - p;
                if ((i & 3) == q) ur[i >> 2] = du;
                if (q == 0) sW[i][d] = du;
            }
        }
        __syncthreads();
        // ---- dT = -dU E^T (i > j): dg, dbeta, dG
        float dT[4][4];
        {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) dT[i][j] = 0.f;
            for (int d = 0; d < kDD; ++d) {
                float u_[4], e[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) u_[i] = sW[bi0 + i][d];
#pragma unroll
                for (int j = 0; j < 4; ++j) e[j] = sE[bj0 + j][d];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) dT[i][j] = fmaf(-u_[i], e[j], dT[i][j]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (bi0 + i <= bj0 + j) dT[i][j] = 0.f;
        }
        // dg_i += dT_ij T_ij, dg_j -= dT_ij T_ij  (T_ij = beta_j L_ij G_ij)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) sM[bi0 + i][bj0 + j] = dT[i][j] * sBeta[bj0 + j] * LG[i][j];
        __syncthreads();
        if (tid < kDC) {
            float rs = 0.f, cs = 0.f;
            for (int j = 0; j < kDC; ++j) {
                rs += sM[tid][j];
                cs += sM[j][tid];
            }
            sDg[tid] += rs - cs;
        }
        __syncthreads();
        // dbeta_j += sum_i dT_ij L_ij G_ij
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) sM[bi0 + i][bj0 + j] = dT[i][j] * LG[i][j];
        __syncthreads();
        if (tid < kDC) {
            float cs = 0.f;
            for (int i = 0; i < kDC; ++i) cs += sM[i][tid];
            sDb[tid] += cs;
        }
        __syncthreads();
        // dG_ij = dT_ij beta_j L_ij; dPhi += (dG + dG^T) Phi
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ii = bi0 + i, jj = bj0 + j;
                sM[ii][jj] = ii > jj ? dT[i][j] * sBeta[jj] * expf(sG[ii] - sG[jj]) : 0.f;
            }
        __syncthreads();
        for (int j = 0; j < kDC; ++j) {
            const float cg = (sM[ro][j] + sM[j][ro]) * (h2 ? sR2[j] * kInvSqrt2 : sR1[j]);
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const float kx = sK[j][e0 + u];
                dPhi[u] = fmaf(cg, h2 ? kx * kx : kx, dPhi[u]);
            }
        }
        // ---- dV = dU; dPhi_i -= d_i S^T du_i (dg_i += phi_i . that); dS_in -= sum_i d_i du_i phi_i^T
        {
            const int r = tid >> 2, c0 = 16 * (tid & 3);
            if (r < nv) {
                float *dv = a.dv + (static_cast<size_t>(bh) * a.L + t0 + r) * kDD + c0;
#pragma unroll
                for (int e = 0; e < 16; ++e) dv[e] = sW[r][c0 + e];
            }
            float tmp[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) tmp[u] = 0.f;
            for (int d = 0; d < kDD; ++d) {
                const float du = sW[ro][d];
#pragma unroll
                for (int u = 0; u < 32; ++u) tmp[u] = fmaf(du, sOp[d][32 * fq + u], tmp[u]);
            }
            const float di = -sDi[ro];
            float dot = 0.f;
            const float rk = h2 ? sR2[ro] * kInvSqrt2 : sR1[ro];
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                tmp[u] *= di;
                dPhi[u] += tmp[u];
                const float kx = sK[ro][e0 + u];
                dot = fmaf((h2 ? kx * kx : kx) * rk, tmp[u], dot);
            }
            dot = red4(dot);
            if (fq == 0) sDg[ro] += dot;
            for (int i = 0; i < kDC; ++i) {
                const float w = -sDi[i] * sW[i][ro] * (h2 ? sR2[i] * kInvSqrt2 : sR1[i]);
#pragma unroll
                for (int u = 0; u < 32; ++u) {
                    const float kx = sK[i][e0 + u];
                    dSin[u] = fmaf(w, h2 ? kx * kx : kx, dSin[u]);
                }
            }
        }
        __syncthreads();
        // ---- decays and write rates of the chunk's tokens
        if (wave == 0) {
            float dg = sDg[lane] + (lane == kDC - 1 ? dg63 : 0.f);
            const float pre = wave_prefix_sum(dg);
            const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pre), 63));
            const float dlog = tot - pre + dg;  // sum over i >= lane
            if (lane < nv) {
                const float al = sAl[lane];
                const size_t gi = static_cast<size_t>(bh) * a.L + t0 + lane;
                a.dalpha[gi] = (al >= 1e-5f && al <= 1.0f) ? dlog / al : 0.f;
                a.dbeta[gi] = sDb[lane];
            }
        }
        // ---- q and k through the feature maps (row-owner over tokens i = ro)
        {
            const int i = ro;
            float oth[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) oth[u] = __shfl_xor(dPsi[u], 2, kWave);
            if (fq < 2 && i < nv) {
                float *dq = a.dq + (static_cast<size_t>(bh) * a.L + t0 + i) * kDD + e0;
#pragma unroll
                for (int u = 0; u < 32; ++u) dq[u] = dPsi[u] + 2.0f * kInvSqrt2 * sQ[i][e0 + u] * oth[u];
            }
            // normalize backward: k/|k| (first half), (k^2/|k^2|)/sqrt2 (second half)
            const float r = h2 ? sR2[i] : sR1[i];
            const bool proj = r * a.feat_eps < 1.0f;  // |x| > eps
            float dot = 0.f;
            float g[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const float kx = sK[i][e0 + u];
                const float xh = (h2 ? kx * kx : kx) * r;  // x / |x|
                g[u] = h2 ? dPhi[u] * kInvSqrt2 : dPhi[u];
                dot = fmaf(xh, g[u], dot);
            }
            dot += __shfl_xor(dot, 1, kWave);  // the row's other 32 elements of this half
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const float kx = sK[i][e0 + u];
                const float xh = (h2 ? kx * kx : kx) * r;
                g[u] = r * (proj ? g[u] - xh * dot : g[u]);  // d x
            }
#pragma unroll
            for (int u = 0; u < 32; ++u) oth[u] = __shfl_xor(g[u], 2, kWave);
            if (fq < 2 && i < nv) {
                float *dk = a.dk + (static_cast<size_t>(bh) * a.L + t0 + i) * kDD + e0;
#pragma unroll
                for (int u = 0; u < 32; ++u) dk[u] = g[u] + 2.0f * sK[i][e0 + u] * oth[u];
            }
        }
#pragma unroll
        for (int u = 0; u < 32; ++u) dS[u] = dSin[u];
        __syncthreads();
        }
    }
    if constexpr (BWD) {
        if (a.dstate_in) {
#pragma unroll
            for (int u = 0; u < 32; ++u) a.dstate_in[static_cast<size_t>(bh) * kDD * kDF + ro * kDF + 32 * fq + u] = dS[u];
        }
    }
}

hipError_t launch_delta_backward(const DeltaBwdArgs &a, hipStream_t stream) {
    const dim3 grid(a.B * a.H), block(256);
    hipLaunchKernelGGL(delta_chunk_kernel<false>, grid, block, 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(delta_chunk_kernel<true>, grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace prime
