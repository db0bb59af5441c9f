// The gated delta-rule PRIME at any head dim D <= 64 and any chunk size: the
// chunked prefill (chunked_delta_prime.py:177-283), its decode step (:140-176)
// and the prefill's backward -- for the shapes the MFMA kernels (D = 64,
// chunk 64) do not take, as the reference's own test runs them (head_dim 32,
// chunk_size 32, tests/test_chunked_delta_prime.py:9-27).
//
// The chunk form's solve is the token recurrence written for a block: with
// a_t = clamp(alpha_t, 1e-5, 1) (the decays exp(cum_i - cum_j) of the chunk are
// products of these), unrolling
//   S <- a_t S;  E_t = v_t - S phi_t;  S <- S + beta_t E_t phi_t^T;  y_t = S psi_t
// gives the chunk's u, T E = u, y and S update, and the Lyapunov clamp
// S <- S min(1, bound / (|S|_F + 1e-6)) follows the last token of every chunk
// of `chunk` tokens; the last chunk's padding (tokens with alpha = decay_pad
// and nothing else, :181-188) decays the state by a_pad^pad before its clamp.
// The step branch predicts with the undecayed state and clamps before its
// readout: E = v - S phi, S <- alpha S + beta E phi^T, clamp, y = S psi.
// Features: psi = [q, q*q/sqrt2], phi = [k/max(|k|, eps), (k*k)/max(|k*k|, eps)/sqrt2]
// (:73-87).
//
// One wavefront per (sequence, head); lane j < D owns value row j of the
// state S [D, 2D] (2D registers); tokens are staged through LDS 64 at a time,
// lane t forming token t's features.
//
// Backward (the derivative torch autograd takes through the reference): the
// state entering every chunk is recorded by a forward pass; then, chunk by
// chunk from the last, the chunk's token states are recomputed into a
// per-(sequence, head) scratch and the tokens are run in reverse with the
// state's adjoint G (per token: G += dy psi^T; g = G phi; dv = beta g;
// dbeta = g.E; dphi = beta (G^T E - P^T g) with P = a S_prev; dpsi = S^T dy;
// G <- a (G - beta g phi^T); dalpha = <G - beta g phi^T, S_prev> inside the
// clamp's range), and the feature maps' derivatives (F.normalize's) give dq
// and dk.  The clamp's derivative at a chunk end: with X the state before it
// and s = bound / (|X| + 1e-6) <= 1, dX = s G - bound <G, X> X / ((|X| +
// 1e-6)^2 |X|); for s > 1 the clamp is the identity.  fp32 throughout.

#include "prime_kernels.h"

namespace prime {
namespace {

constexpr int kGW = 64;          // lanes (value rows)
constexpr int kGT = 64;          // tokens per LDS stage
constexpr int kFP = 2 * kGW + 1; // feature row pitch (2D <= 128 features)
constexpr int kVP = kGW + 1;     // value row pitch
constexpr float kRsqrt2Div = 1.41421356237309504880f;  // the reference divides by sqrt(2)

__device__ __forceinline__ float clamp_alpha(float a) { return fminf(fmaxf(a, 1e-5f), 1.0f); }

// Stage tokens t0 .. t0+nv-1 of (b, head h / kv head hk): raw q into ps[t][i],
// raw k into pf[t][i], v (and dy) rows, beta / alpha; then lane t expands
// token t into its features (psi in ps, phi in pf) and keeps |k| and |k*k|.
__device__ void delta_gen_stage(const DeltaGenArgs &a, int b, int h, int hk, int t0, int nv, float (*ps)[kFP],
                                float (*pf)[kFP], float (*sv)[kVP], float (*sdy)[kVP], float *sb, float *sa,
                                float *sn1, float *sn2, int lane) {
    const int D = a.D;
    const int64_t bh = static_cast<int64_t>(b) * a.H + h;
    for (int t = 0; t < nv; ++t) {
        const int64_t tok = t0 + t;
        if (lane < D) {
            ps[t][lane] = load_elem(a.q, b * a.q_sb + h * a.q_sh + tok * a.q_sl + lane, a.dt_q);
            pf[t][lane] = load_elem(a.k, b * a.k_sb + hk * a.k_sh + tok * a.k_sl + lane, a.dt_k);
            sv[t][lane] = load_elem(a.v, b * a.v_sb + hk * a.v_sh + tok * a.v_sl + lane, a.dt_v);
            if (sdy) sdy[t][lane] = load_elem(a.dy, b * a.dy_sb + h * a.dy_sh + tok * a.dy_sl + lane, a.dt_dy);
        } else {
            sv[t][lane] = 0.f;
            if (sdy) sdy[t][lane] = 0.f;
        }
    }
    if (lane < nv) {
        sb[lane] = a.beta[bh * a.L + t0 + lane];
        sa[lane] = a.alpha[bh * a.L + t0 + lane];
    }
    __syncthreads();
    if (lane < nv) {
        float *q = ps[lane], *k = pf[lane];
        float s1 = 0.f, s2 = 0.f;
        for (int i = 0; i < D; ++i) {
            const float k2 = k[i] * k[i];
            s1 = fmaf(k[i], k[i], s1);
            s2 = fmaf(k2, k2, s2);
        }
        const float n1 = sqrtf(s1), n2 = sqrtf(s2);
        const float m1 = fmaxf(n1, a.feat_eps), m2 = fmaxf(n2, a.feat_eps);
        for (int i = 0; i < D; ++i) {
            q[D + i] = q[i] * q[i] / kRsqrt2Div;
            const float ki = k[i];
            k[D + i] = ki * ki / m2 / kRsqrt2Div;
            k[i] = ki / m1;
        }
        sn1[lane] = n1;
        sn2[lane] = n2;
    }
    __syncthreads();
}

}  // namespace

// Forward: the chunked prefill (a.step == 0) or the decode step (a.step == 1,
// L == 1).  With a.ws (backward's first pass) the state entering every chunk
// is recorded there and y is not written.
template <int MD>
__global__ __launch_bounds__(kGW) void delta_gen_forward_kernel(const DeltaGenArgs a) {
    __shared__ float ps[kGT][kFP], pf[kGT][kFP], sv[kGT][kVP];
    __shared__ float sb[kGT], sa[kGT], sn1[kGT], sn2[kGT];
    const int lane = threadIdx.x, bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H, hk = h / a.group, D = a.D, P = 2 * D;
    const bool row = lane < D;
    const size_t so = static_cast<size_t>(bh) * D * P + static_cast<size_t>(lane) * P;
    const int NC = (a.L + a.chunk - 1) / a.chunk;
    float *rec = a.ws ? a.ws + static_cast<size_t>(bh) * NC * D * P : nullptr;
    float S[2 * MD];
#pragma unroll
    for (int f = 0; f < 2 * MD; ++f) S[f] = (f < P && row && a.state_in) ? a.state_in[so + f] : 0.f;
    auto clamp_state = [&]() {
        float n2 = 0.f;
#pragma unroll
        for (int f = 0; f < 2 * MD; ++f) n2 = fmaf(S[f], S[f], n2);
        const float sc = fminf(a.bound / (sqrtf(wave_sum(n2)) + 1e-6f), 1.0f);
#pragma unroll
        for (int f = 0; f < 2 * MD; ++f) S[f] *= sc;
    };
    for (int t0 = 0; t0 < a.L; t0 += kGT) {
        const int nv = min(kGT, a.L - t0);
        __syncthreads();  // the previous stage's reads are done
        delta_gen_stage(a, b, h, hk, t0, nv, ps, pf, sv, nullptr, sb, sa, sn1, sn2, lane);
        for (int t = 0; t < nv; ++t) {
            const int g = t0 + t;
            if (rec && g % a.chunk == 0 && row) {
                float *r = rec + static_cast<size_t>(g / a.chunk) * D * P + static_cast<size_t>(lane) * P;
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) r[f] = S[f];
            }
            const float vj = row ? sv[t][lane] : 0.f;
            float pred = 0.f;
            if (a.step) {
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) pred = fmaf(S[f], pf[t][f], pred);
                const float w = sb[t] * (vj - pred), al = sa[t];
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) S[f] = fmaf(w, pf[t][f], al * S[f]);
                if (a.bound > 0.f) clamp_state();
            } else {
                const float al = clamp_alpha(sa[t]);
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) {
                        S[f] *= al;
                        pred = fmaf(S[f], pf[t][f], pred);
                    }
                const float w = sb[t] * (vj - pred);
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) S[f] = fmaf(w, pf[t][f], S[f]);
            }
            if (!rec) {
                float yv = 0.f;
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) yv = fmaf(S[f], ps[t][f], yv);
                if (row) store_elem(a.y, b * a.y_sb + h * a.y_sh + static_cast<int64_t>(g) * a.y_sl + lane, a.dt_y, yv);
            }
            if (!a.step && (g + 1) % a.chunk == 0 && a.bound > 0.f) clamp_state();
        }
    }
    if (rec) return;
    const int rem = a.L % a.chunk;
    if (!a.step && rem) {
        // the padding of the last chunk: (chunk - rem) tokens of decay only, then its clamp
        const float pd = expf(static_cast<float>(a.chunk - rem) * logf(clamp_alpha(a.decay_pad)));
#pragma unroll
        for (int f = 0; f < 2 * MD; ++f) S[f] *= pd;
        if (a.bound > 0.f) clamp_state();
    }
    if (a.state_out && row) {
#pragma unroll
        for (int f = 0; f < 2 * MD; ++f)
            if (f < P) a.state_out[so + f] = S[f];
    }
}

// Backward: chunks from the last to the first; each chunk's token states are
// recomputed from the recorded entry state into the scratch, then its tokens
// run in reverse.  The state's adjoint waits in its own scratch slot while a
// chunk is recomputed (the two 2D-register rows would not fit together).
template <int MD>
__global__ __launch_bounds__(kGW) void delta_gen_backward_kernel(const DeltaGenArgs a) {
    __shared__ float ps[kGT][kFP], pf[kGT][kFP], sv[kGT][kVP], sdy[kGT][kVP];
    __shared__ float red[kGW][kFP];   // per-lane contributions to a feature-wide sum
    __shared__ float rdp[2][2 * kGW]; // reduced dpsi, dphi of the current token
    __shared__ float sb[kGT], sa[kGT], sn1[kGT], sn2[kGT];
    const int lane = threadIdx.x, bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H, hk = h / a.group, D = a.D, P = 2 * D, C = a.chunk;
    const bool row = lane < D;
    const int NC = (a.L + C - 1) / C;
    const size_t DP = static_cast<size_t>(D) * P, BH = static_cast<size_t>(a.B) * a.H;
    // workspace: entry states [BH][NC][D][2D] | token states [BH][C][D][2D] |
    //            E [BH][C][64] | the adjoint [BH][D][2D]
    const float *rec = a.ws + static_cast<size_t>(bh) * NC * DP;
    float *scr = a.ws + BH * NC * DP + static_cast<size_t>(bh) * C * DP;
    float *scrE = a.ws + BH * (NC + C) * DP + static_cast<size_t>(bh) * C * kGW;
    float *gsv = a.ws + BH * (NC + C) * DP + BH * C * kGW + static_cast<size_t>(bh) * DP;
    const size_t lo = static_cast<size_t>(lane) * P;
    const int64_t tb = static_cast<int64_t>(bh) * a.L;

    if (row) {
#pragma unroll
        for (int f = 0; f < 2 * MD; ++f)
            if (f < P) gsv[lo + f] = a.dstate_out ? a.dstate_out[bh * DP + lo + f] : 0.f;
    }

    for (int c = NC - 1; c >= 0; --c) {
        const int c0 = c * C, c1 = min(a.L, c0 + C), n = c1 - c0;
        // ---- recompute: S_t of every token of the chunk into the scratch (slot t - c0), E_t beside it
        float S[2 * MD];
#pragma unroll
        for (int f = 0; f < 2 * MD; ++f) S[f] = (f < P && row) ? rec[c * DP + lo + f] : 0.f;
        for (int s0 = 0; s0 < n; s0 += kGT) {
            const int nv = min(kGT, n - s0);
            __syncthreads();
            delta_gen_stage(a, b, h, hk, c0 + s0, nv, ps, pf, sv, nullptr, sb, sa, sn1, sn2, lane);
            for (int t = 0; t < nv; ++t) {
                const float al = clamp_alpha(sa[t]);
                float pred = 0.f;
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) {
                        S[f] *= al;
                        pred = fmaf(S[f], pf[t][f], pred);
                    }
                const float e = (row ? sv[t][lane] : 0.f) - pred, w = sb[t] * e;
                float *dst = scr + static_cast<size_t>(s0 + t) * DP + lo;
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) {
                        S[f] = fmaf(w, pf[t][f], S[f]);
                        if (row) dst[f] = S[f];
                    }
                scrE[static_cast<size_t>(s0 + t) * kGW + lane] = e;
            }
        }
        // ---- the chunk's end: padding decay and the clamp (the scratch's last
        // slot holds the state after the chunk's last token)
        float G[2 * MD];
        {
            const float *last = scr + static_cast<size_t>(n - 1) * DP + lo;
#pragma unroll
            for (int f = 0; f < 2 * MD; ++f) {
                G[f] = (f < P && row) ? gsv[lo + f] : 0.f;
                S[f] = (f < P && row) ? last[f] : 0.f;
            }
            const float pd = (c == NC - 1 && a.L % C)
                                 ? expf(static_cast<float>(C - a.L % C) * logf(clamp_alpha(a.decay_pad)))
                                 : 1.0f;
            if (a.bound > 0.f) {
                float n2 = 0.f, gx = 0.f;
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f) {
                    const float x = pd * S[f];
                    n2 = fmaf(x, x, n2);
                    gx = fmaf(G[f], x, gx);
                }
                const float nrm = sqrtf(wave_sum(n2)), den = nrm + 1e-6f;
                const float sc = a.bound / den;
                if (sc <= 1.0f) {
                    const float kx = nrm > 0.f ? a.bound * wave_sum(gx) / (den * den * nrm) : 0.f;
#pragma unroll
                    for (int f = 0; f < 2 * MD; ++f) G[f] = sc * G[f] - kx * pd * S[f];
                }
            }
#pragma unroll
            for (int f = 0; f < 2 * MD; ++f) G[f] *= pd;
        }
        // ---- tokens in reverse
        const int nst = (n + kGT - 1) / kGT;
        for (int si = nst - 1; si >= 0; --si) {
            const int s0 = si * kGT, nv = min(kGT, n - s0);
            __syncthreads();
            delta_gen_stage(a, b, h, hk, c0 + s0, nv, ps, pf, sv, sdy, sb, sa, sn1, sn2, lane);
            for (int t = nv - 1; t >= 0; --t) {
                const int lt = s0 + t;           // token within the chunk
                const int64_t g = c0 + lt;       // token within the sequence
                const float *cur = scr + static_cast<size_t>(lt) * DP + lo;
                const float *prv = lt ? scr + static_cast<size_t>(lt - 1) * DP + lo : rec + c * DP + lo;
                const float dyj = row ? sdy[t][lane] : 0.f;
                const float e = scrE[static_cast<size_t>(lt) * kGW + lane];
                const float be = sb[t], al = clamp_alpha(sa[t]);
                // G += dy psi^T; dpsi contributions S_t^T dy; g = G phi
                float gj = 0.f;
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) {
                        const float st = row ? cur[f] : 0.f;
                        G[f] = fmaf(dyj, ps[t][f], G[f]);
                        gj = fmaf(G[f], pf[t][f], gj);
                        red[lane][f] = st * dyj;
                    }
                __syncthreads();
                for (int f = lane; f < P; f += kGW) {
                    float s = 0.f;
                    for (int j = 0; j < D; ++j) s += red[j][f];
                    rdp[0][f] = s;
                }
                __syncthreads();
                // dphi contributions beta (G E - g P); the adjoint through the decay
                const float w = be * e;
                float da = 0.f;
#pragma unroll
                for (int f = 0; f < 2 * MD; ++f)
                    if (f < P) {
                        const float sp = row ? prv[f] : 0.f;                    // S_prev
                        const float pv = row ? (cur[f] - w * pf[t][f]) : 0.f;   // P = a S_prev
                        red[lane][f] = be * (G[f] * e - gj * pv);
                        const float dp = fmaf(-be * gj, pf[t][f], G[f]);
                        da = fmaf(dp, sp, da);
                        G[f] = al * dp;
                    }
                __syncthreads();
                for (int f = lane; f < P; f += kGW) {
                    float s = 0.f;
                    for (int j = 0; j < D; ++j) s += red[j][f];
                    rdp[1][f] = s;
                }
                __syncthreads();
                const float dbeta = wave_sum(row ? gj * e : 0.f);
                const float dal = wave_sum(da);
                const float araw = sa[t];
                if (lane == 0) {
                    a.dbeta[tb + g] = dbeta;
                    a.dalpha[tb + g] = (araw >= 1e-5f && araw <= 1.0f) ? dal : 0.f;
                }
                const size_t go = (static_cast<size_t>(bh) * a.L + g) * D;
                if (row) a.dv[go + lane] = be * gj;
                // features: dq from dpsi, dk through the two normalisations
                float ki = 0.f, u1 = 0.f, u2 = 0.f, f1 = 0.f, f2 = 0.f;
                const float n1 = sn1[t], n2 = sn2[t];
                const float m1 = fmaxf(n1, a.feat_eps), m2 = fmaxf(n2, a.feat_eps);
                if (row) {
                    const float qi = ps[t][lane];
                    ki = load_elem(a.k, b * a.k_sb + hk * a.k_sh + g * a.k_sl + lane, a.dt_k);
                    u1 = rdp[1][lane];
                    u2 = rdp[1][D + lane] / kRsqrt2Div;
                    f1 = ki / m1;
                    f2 = ki * ki / m2;
                    a.dq[go + lane] = rdp[0][lane] + kRsqrt2Div * qi * rdp[0][D + lane];
                }
                const float dot1 = wave_sum(f1 * u1), dot2 = wave_sum(f2 * u2);
                if (row) {
                    const float dk1 = n1 >= a.feat_eps ? (u1 - f1 * dot1) / n1 : u1 / a.feat_eps;
                    const float dx2 = n2 >= a.feat_eps ? (u2 - f2 * dot2) / n2 : u2 / a.feat_eps;
                    a.dk[go + lane] = dk1 + 2.0f * ki * dx2;
                }
            }
        }
        if (row) {
#pragma unroll
            for (int f = 0; f < 2 * MD; ++f)
                if (f < P) gsv[lo + f] = G[f];
        }
    }
    if (a.dstate_in && row) {
#pragma unroll
        for (int f = 0; f < 2 * MD; ++f)
            if (f < P) a.dstate_in[bh * DP + lo + f] = gsv[lo + f];
    }
}

// Backward of the decode step's form (one token, L == 1; chunked_delta_prime.py:
// 140-176): with E = v - S phi, X = alpha S + beta E phi^T, S' = s X (s the
// Lyapunov scale min(1, bound / (|X|_F + 1e-6))) and y = S' psi, given dy and
// dS' (the next state's adjoint):
//   G = dS' + dy psi^T;  dpsi = S'^T dy;  dX = s G - [s <= 1] bound <G, X> X /
//   ((|X| + 1e-6)^2 |X|);  g = dX phi;  dv = beta g;  dbeta = g . E;
//   dalpha = <dX, S> (the step uses alpha unclamped);  dphi = dX^T (beta E) -
//   S^T (beta g);  dS = alpha dX - (beta g) phi^T;
// then dq and dk through the feature maps as in the prefill's backward.  One
// wavefront per (sequence, head), lane j < D owning row j; fp32 throughout.
template <int MD>
__global__ __launch_bounds__(kGW) void delta_gen_step_backward_kernel(const DeltaGenArgs a) {
    __shared__ float ps[1][kFP], pf[1][kFP], sv[1][kVP], sdy[1][kVP];
    __shared__ float red[kGW][kFP];    // per-lane contributions to a feature-wide sum
    __shared__ float rdp[2][2 * kGW];  // reduced dpsi, dphi
    __shared__ float sb[1], sa[1], sn1[1], sn2[1];
    const int lane = threadIdx.x, bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H, hk = h / a.group, D = a.D, P = 2 * D;
    const bool row = lane < D;
    const size_t so = static_cast<size_t>(bh) * D * P + static_cast<size_t>(lane) * P;
    delta_gen_stage(a, b, h, hk, 0, 1, ps, pf, sv, sdy, sb, sa, sn1, sn2, lane);
    float S[2 * MD], X[2 * MD], G[2 * MD];
#pragma unroll
    for (int f = 0; f < 2 * MD; ++f) S[f] = (f < P && row && a.state_in) ? a.state_in[so + f] : 0.f;
    // the forward: E, X and the scale
    float pred = 0.f;
#pragma unroll
    for (int f = 0; f < 2 * MD; ++f)
        if (f < P) pred = fmaf(S[f], pf[0][f], pred);
    const float e = row ? sv[0][lane] - pred : 0.f;
    const float be = sb[0], al = sa[0], w = be * e;
    float n2 = 0.f;
#pragma unroll
    for (int f = 0; f < 2 * MD; ++f) {
        X[f] = f < P ? fmaf(w, pf[0][f], al * S[f]) : 0.f;
        n2 = fmaf(X[f], X[f], n2);
    }
    float sc = 1.f, nrm = 0.f, den = 1.f;
    if (a.bound > 0.f) {
        nrm = sqrtf(wave_sum(n2));
        den = nrm + 1e-6f;
        sc = fminf(a.bound / den, 1.0f);
    }
    // the adjoint of S' with the readout's term; dpsi
    const float dyj = row ? sdy[0][lane] : 0.f;
    float gx = 0.f;
#pragma unroll
    for (int f = 0; f < 2 * MD; ++f)
        if (f < P) {
            G[f] = ((a.dstate_out && row) ? a.dstate_out[so + f] : 0.f) + dyj * ps[0][f];
            red[lane][f] = sc * X[f] * dyj;
            gx = fmaf(G[f], X[f], gx);
        } else {
            G[f] = 0.f;
        }
    __syncthreads();
    for (int f = lane; f < P; f += kGW) {
        float t = 0.f;
        for (int j = 0; j < D; ++j) t += red[j][f];
        rdp[0][f] = t;
    }
    __syncthreads();
    // through the clamp (the identity where bound / (|X| + 1e-6) > 1)
    if (a.bound > 0.f && a.bound / den <= 1.0f) {
        const float kx = nrm > 0.f ? a.bound * wave_sum(gx) / (den * den * nrm) : 0.f;
#pragma unroll
        for (int f = 0; f < 2 * MD; ++f) G[f] = sc * G[f] - kx * X[f];
    }
    // through X = alpha S + (beta E) phi^T and E = v - S phi
    float gj = 0.f, da = 0.f;
#pragma unroll
    for (int f = 0; f < 2 * MD; ++f)
        if (f < P) {
            gj = fmaf(G[f], pf[0][f], gj);
            da = fmaf(G[f], S[f], da);
        }
    const float de = row ? be * gj : 0.f;
#pragma unroll
    for (int f = 0; f < 2 * MD; ++f)
        if (f < P) red[lane][f] = G[f] * w - de * S[f];
    __syncthreads();
    for (int f = lane; f < P; f += kGW) {
        float t = 0.f;
        for (int j = 0; j < D; ++j) t += red[j][f];
        rdp[1][f] = t;
    }
    __syncthreads();
    const float dbeta = wave_sum(row ? gj * e : 0.f);
    const float dal = wave_sum(row ? da : 0.f);
    if (lane == 0) {
        a.dbeta[bh] = dbeta;
        a.dalpha[bh] = dal;
    }
    const size_t go = static_cast<size_t>(bh) * D;
    if (row) {
        a.dv[go + lane] = de;
        if (a.dstate_in) {
#pragma unroll
            for (int f = 0; f < 2 * MD; ++f)
                if (f < P) a.dstate_in[so + f] = fmaf(-de, pf[0][f], al * G[f]);
        }
    }
    // features: dq from dpsi, dk through the two normalisations
    float ki = 0.f, u1 = 0.f, u2 = 0.f, f1 = 0.f, f2 = 0.f;
    const float n1 = sn1[0], nn2 = sn2[0];
    const float m1 = fmaxf(n1, a.feat_eps), m2 = fmaxf(nn2, a.feat_eps);
    if (row) {
        const float qi = ps[0][lane];
        ki = load_elem(a.k, b * a.k_sb + hk * a.k_sh + lane, a.dt_k);
        u1 = rdp[1][lane];
        u2 = rdp[1][D + lane] / kRsqrt2Div;
        f1 = ki / m1;
        f2 = ki * ki / m2;
        a.dq[go + lane] = rdp[0][lane] + kRsqrt2Div * qi * rdp[0][D + lane];
    }
    const float dot1 = wave_sum(f1 * u1), dot2 = wave_sum(f2 * u2);
    if (row) {
        const float dk1 = n1 >= a.feat_eps ? (u1 - f1 * dot1) / n1 : u1 / a.feat_eps;
        const float dx2 = nn2 >= a.feat_eps ? (u2 - f2 * dot2) / nn2 : u2 / a.feat_eps;
        a.dk[go + lane] = dk1 + 2.0f * ki * dx2;
    }
}

hipError_t launch_delta_gen_step_backward(const DeltaGenArgs &a, hipStream_t stream) {
    if (a.D <= 32) hipLaunchKernelGGL(delta_gen_step_backward_kernel<32>, dim3(a.B * a.H), dim3(kGW), 0, stream, a);
    else hipLaunchKernelGGL(delta_gen_step_backward_kernel<64>, dim3(a.B * a.H), dim3(kGW), 0, stream, a);
    return hipGetLastError();
}

size_t delta_gen_backward_ws_bytes(int B, int H, int L, int D, int chunk) {
    const size_t NC = (static_cast<size_t>(L) + chunk - 1) / chunk;
    const size_t DP = static_cast<size_t>(D) * 2 * D;
    const size_t floats = static_cast<size_t>(B) * H * ((NC + chunk + 1) * DP + static_cast<size_t>(chunk) * kGW);
    return (floats * sizeof(float) + 255) / 256 * 256;
}

hipError_t launch_delta_gen_forward(const DeltaGenArgs &a, hipStream_t stream) {
    if (a.D <= 32) hipLaunchKernelGGL(delta_gen_forward_kernel<32>, dim3(a.B * a.H), dim3(kGW), 0, stream, a);
    else hipLaunchKernelGGL(delta_gen_forward_kernel<64>, dim3(a.B * a.H), dim3(kGW), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_delta_gen_backward(const DeltaGenArgs &a, hipStream_t stream) {
    DeltaGenArgs f = a;
    f.y = nullptr;
    f.state_out = nullptr;
    if (a.D <= 32) {
        hipLaunchKernelGGL(delta_gen_forward_kernel<32>, dim3(a.B * a.H), dim3(kGW), 0, stream, f);
        hipLaunchKernelGGL(delta_gen_backward_kernel<32>, dim3(a.B * a.H), dim3(kGW), 0, stream, a);
    } else {
        hipLaunchKernelGGL(delta_gen_forward_kernel<64>, dim3(a.B * a.H), dim3(kGW), 0, stream, f);
        hipLaunchKernelGGL(delta_gen_backward_kernel<64>, dim3(a.B * a.H), dim3(kGW), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace prime
