// PRIME moment attention for head dims other than 64 (D < 64): the chunked
// prefill, the decode step and the prefill's backward (attention.py:77-210,
// chunked_ssd.py:48-184 at any head_dim, as the reference's own tests run
// them at head_dim 32, tests/test_attention.py:7-14).
//
// One wavefront per (sequence, head) runs the recurrence token by token:
// lane j < D owns value column j of the state -- S0[j], S1[:, j], S2[:, j] in
// registers -- and lane D the "ones" column that carries the normaliser
// K0, K1, K2 (the moments of a value that is always 1), so one readout gives
// every lane its numerator and lane D the denominator:
//   S <- l S + k v^T (v_D = 1),  num_j = S0_j + q . S1[:, j] + 1/2 q^2 . S2[:, j]
//   y_j = num_j / max(num_D, eps)
// (the update before the readout, attention.py:126-143).  Lanes read q_t and
// k_t from LDS, where each 64-token chunk is staged (and, with a QK
// LayerNorm, normalised on load: lane t normalises token t of the chunk).
// The dense branch's double clamp (attention.py:177-185, with an incoming
// state) splits the denominator into the call's part and the incoming
// state's l^(t+1) readout of its K moments (held in LDS).
//
// Backward (the derivative the reference obtains from autograd):
//   pass 1, tokens in order: the forward again; g_j = dy_j / den_c, the ones
//     column's adjoint h (the clamp's gradient where den >= eps, as torch's
//     clamp); dq_t = sum_j g_j (S1[:, j] + q o S2[:, j]) reduced over the
//     lanes through LDS; (den_c, h) of every token into the workspace;
//   pass 2, tokens in reverse: the adjoint of the state dS += q g^T (and
//     1/2 q^2 g^T, g), dv_t[j] = dS0[j] + k . dS1[:, j] + k^2 . dS2[:, j],
//     dk_t = sum_j v_j (dS1[:, j] + 2 k o dS2[:, j]) over the lanes, dS <- l dS;
//     what is left is the adjoint of the incoming state.
// fp32 arithmetic; bf16 / fp16 / fp32 storage.

#include "prime_kernels.h"

namespace prime {
namespace {

constexpr int kGD = 64;     // lanes: value columns 0 .. D-1 and the ones column D (D < 64)
constexpr int kGC = 64;     // tokens per staged chunk
constexpr int kGP = kGD + 1;

__device__ __forceinline__ float ld_any(const void *p, int64_t i, int dt) { return load_elem(p, i, dt); }

// round to storage dtype dt (to nearest even), as a module's tensor of that dtype holds it
__device__ __forceinline__ float round_dt(float x, int dt) {
    if (dt == PRIME_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
    if (dt == PRIME_F16) return h16_bits_to_f32(f32_to_h16_bits(x));
    return x;
}

}  // namespace

// One head row of D values in place: LayerNorm over D (biased variance;
// weight w / bias bb, or none when w is null), rounded to the storage dtype
// dt as the module's LayerNorm returns it, then the scale (rounded again).
// The prefill's QK-norm on load and prime_head_layernorm share it, so both
// give the same bits.
__device__ __forceinline__ void generic_ln_row(float *row, int D, const void *w, const void *bb, int dt_norm,
                                               float ln_eps, float scale, int dt) {
    if (w) {
        float m = 0.f;
        for (int i = 0; i < D; ++i) m += row[i];
        m /= static_cast<float>(D);
        float var = 0.f;
        for (int i = 0; i < D; ++i) var += (row[i] - m) * (row[i] - m);
        const float rs = rsqrtf(var / static_cast<float>(D) + ln_eps);
        for (int i = 0; i < D; ++i) row[i] = round_dt((row[i] - m) * rs * ld_any(w, i, dt_norm) + ld_any(bb, i, dt_norm), dt);
    }
    if (scale != 1.0f)
        for (int i = 0; i < D; ++i) row[i] = round_dt(row[i] * scale, dt);
}

// Stage tokens t0 .. t0+nv-1 of q, k, v (and dy) into LDS, normalising q and k
// when the args carry a QK LayerNorm; rows past nv are zero.
__device__ __forceinline__ void generic_stage(const GenericArgs &a, int b, int h, int hk, int t0, int nv,
                                              float (*sq)[kGP], float (*sk)[kGP], float (*sv)[kGP],
                                              float (*sdy)[kGP], float *sdec, int lane) {
    const int D = a.D;
    for (int t = 0; t < kGC; ++t) {
        const bool ok = t < nv && lane < D;
        const int64_t tok = t0 + t;
        sq[t][lane] = ok ? ld_any(a.q, b * a.q_sb + h * a.q_sh + tok * a.q_sl + lane, a.dt_q) : 0.f;
        sk[t][lane] = ok ? ld_any(a.k, b * a.k_sb + hk * a.k_sh + tok * a.k_sl + lane, a.dt_k) : 0.f;
        sv[t][lane] = ok ? ld_any(a.v, b * a.v_sb + hk * a.v_sh + tok * a.v_sl + lane, a.dt_v) : 0.f;
        if (sdy) sdy[t][lane] = ok ? ld_any(a.dy, b * a.dy_sb + h * a.dy_sh + tok * a.dy_sl + lane, a.dt_dy) : 0.f;
    }
    __syncthreads();
    if (a.qk_norm) {
        // lane t normalises token t
        const int t = lane;
        if (t < nv) {
            generic_ln_row(sq[t], D, a.qn_w, a.qn_b, a.dt_norm, a.ln_eps, a.q_scale, a.dt_q);
            generic_ln_row(sk[t], D, a.kn_w, a.kn_b, a.dt_norm, a.ln_eps, 1.0f, a.dt_k);
        }
        __syncthreads();
    }
    if (a.selective) {
        // beta k (the kernels then weight k*k by 1/2 and q*q by 1); the token's decay
        const float beta = a.k_scale[h];
        for (int t = 0; t < nv; ++t) sk[t][lane] *= beta;
        if (lane < nv) {
            const int64_t bh = static_cast<int64_t>(b) * a.H + h;
            float lam_t;
            if (a.log_decay) {
                lam_t = expf(a.log_decay[bh * a.L + t0 + lane]);
            } else if (a.decay_bh) {
                lam_t = a.decay_bh[bh];
            } else {
                // selective.py:368, 386: Delta = clamp(softplus(s)), each stage
                // rounded to the step's dtype as the module's tensors are
                const float sv0 = ld_any(a.step, b * a.step_sb + h, a.dt_step);
                float d = sv0 > 20.f ? sv0 : log1pf(expf(sv0));
                d = round_dt(d, a.dt_step);
                d = round_dt(fminf(fmaxf(d, a.step_min), a.step_max), a.dt_step);
                lam_t = expf(-d / a.tau[h]);
            }
            sdec[lane] = lam_t;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(kGD) void generic_prefill_kernel(const GenericArgs a) {
    __shared__ float sq[kGC][kGP], sk[kGC][kGP], sv[kGC][kGP], sdec[kGC];
    __shared__ float sKin[3][kGP];  // incoming K1, K2 (dense clamp), K0 at [2][0]
    const int lane = threadIdx.x, bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H, hk = h / a.group, D = a.D;
    const bool col = lane <= D;
    const bool sel = a.selective != 0;
    const float lam = sel ? 1.0f : a.decay[h];
    // the second-order weights: k*k and q*q/2 (base), (beta k)*(beta k)/2 and q*q (selective)
    const float ck2 = sel ? 0.5f : 1.0f, cq2 = sel ? 1.0f : 0.5f;
    const size_t o1 = static_cast<size_t>(bh) * D * D, o0 = static_cast<size_t>(bh) * D;
    float S0 = 0.f, S1[kGD - 1], S2[kGD - 1];
#pragma unroll
    for (int i = 0; i < kGD - 1; ++i) {
        S1[i] = S2[i] = 0.f;
        if (i < D && col && a.s1i) {
            S1[i] = lane < D ? a.s1i[o1 + i * D + lane] : a.k1i[o0 + i];
            S2[i] = lane < D ? a.s2i[o1 + i * D + lane] : a.k2i[o0 + i];
        }
    }
    if (col && a.s1i) S0 = lane < D ? a.s0i[o0 + lane] : a.k0i[bh];
    const bool dense = a.dense_clamp && a.s1i;
    if (dense) {
        if (lane < D) {
            sKin[0][lane] = a.k1i[o0 + lane];
            sKin[1][lane] = a.k2i[o0 + lane];
        }
        if (lane == 0) sKin[2][0] = a.k0i[bh];
    }
    const int NC = (a.L + kGC - 1) / kGC;
    for (int c = 0; c < NC; ++c) {
        const int t0 = c * kGC, nv = min(kGC, a.L - t0);
        __syncthreads();  // the previous chunk's reads are done
        generic_stage(a, b, h, hk, t0, nv, sq, sk, sv, nullptr, sdec, lane);
        float pin = dense ? static_cast<float>(pow(static_cast<double>(lam), static_cast<double>(t0 + 1))) : 0.f;
        for (int t = 0; t < nv; ++t) {
            const float vj = lane < D ? sv[t][lane] : (lane == D ? 1.0f : 0.0f);
            const float lt = sel ? sdec[t] : lam;
            S0 = lt * S0 + vj;
            float num = S0;
#pragma unroll
            for (int i = 0; i < kGD - 1; ++i) {
                if (i < D) {
                    const float ki = sk[t][i], qi = sq[t][i];
                    S1[i] = fmaf(lt, S1[i], ki * vj);
                    S2[i] = fmaf(lt, S2[i], ck2 * ki * ki * vj);
                    num = fmaf(qi, S1[i], num);
                    num = fmaf(cq2 * qi * qi, S2[i], num);
                }
            }
            const float den = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(num), D));
            float den_c;
            if (dense) {
                float di = sKin[2][0];
                for (int i = 0; i < D; ++i) {
                    const float qi = sq[t][i];
                    di = fmaf(qi, sKin[0][i], di);
                    di = fmaf(0.5f * qi * qi, sKin[1][i], di);
                }
                di *= pin;
                den_c = fmaxf(fmaxf(den - di, a.eps) + di, a.eps);
                pin *= lam;
            } else {
                den_c = fmaxf(den, a.eps);
            }
            if (lane < D && a.y)
                store_elem(a.y, b * a.y_sb + h * a.y_sh + static_cast<int64_t>(t0 + t) * a.y_sl + lane, a.dt_y,
                           num / den_c);
        }
    }
    if (a.s1o && col) {
#pragma unroll
        for (int i = 0; i < kGD - 1; ++i) {
            if (i < D) {
                if (lane < D) {
                    a.s1o[o1 + i * D + lane] = S1[i];
                    a.s2o[o1 + i * D + lane] = S2[i];
                } else {
                    a.k1o[o0 + i] = S1[i];
                    a.k2o[o0 + i] = S2[i];
                }
            }
        }
        if (lane < D) a.s0o[o0 + lane] = S0;
        else a.k0o[bh] = S0;
    }
}

__global__ __launch_bounds__(kGD) void generic_backward_kernel(const GenericArgs a) {
    __shared__ float sq[kGC][kGP], sk[kGC][kGP], sv[kGC][kGP], sdy[kGC][kGP], sdec[kGC];
    __shared__ float sred[kGP][kGP];
    __shared__ float sKin[3][kGP];
    const int lane = threadIdx.x, bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H, hk = h / a.group, D = a.D;
    const bool col = lane <= D;
    const bool sel = a.selective != 0;
    const float lam = sel ? 1.0f : a.decay[h];
    const float ck2 = sel ? 0.5f : 1.0f, cq2 = sel ? 1.0f : 0.5f;
    const size_t o1 = static_cast<size_t>(bh) * D * D, o0 = static_cast<size_t>(bh) * D;
    float *ws = a.ws + static_cast<size_t>(bh) * a.L * 2;
    // selective: <dstate_out, state_out> (the final state's share of every log
    // decay's adjoint), formed at the end of the forward pass
    float fin = 0.f;
    const int NC = (a.L + kGC - 1) / kGC;
    const bool dense = a.dense_clamp && a.s1i;
    if (dense) {
        if (lane < D) {
            sKin[0][lane] = a.k1i[o0 + lane];
            sKin[1][lane] = a.k2i[o0 + lane];
        }
        if (lane == 0) sKin[2][0] = a.k0i[bh];
    }
    // incoming-K adjoints of the dense clamp: lane i holds dK1[i], dK2[i]; dK0 in every lane
    float dkin1 = 0.f, dkin2 = 0.f, dkin0 = 0.f;

    // ---------------- pass 1: forward, dq, (den_c, h) per token
    {
        float S0 = 0.f, S1[kGD - 1], S2[kGD - 1];
#pragma unroll
        for (int i = 0; i < kGD - 1; ++i) {
            S1[i] = S2[i] = 0.f;
            if (i < D && col && a.s1i) {
                S1[i] = lane < D ? a.s1i[o1 + i * D + lane] : a.k1i[o0 + i];
                S2[i] = lane < D ? a.s2i[o1 + i * D + lane] : a.k2i[o0 + i];
            }
        }
        if (col && a.s1i) S0 = lane < D ? a.s0i[o0 + lane] : a.k0i[bh];
        for (int c = 0; c < NC; ++c) {
            const int t0 = c * kGC, nv = min(kGC, a.L - t0);
            __syncthreads();
            generic_stage(a, b, h, hk, t0, nv, sq, sk, sv, sdy, sdec, lane);
            float pin = dense ? static_cast<float>(pow(static_cast<double>(lam), static_cast<double>(t0 + 1))) : 0.f;
            for (int t = 0; t < nv; ++t) {
                const float vj = lane < D ? sv[t][lane] : (lane == D ? 1.0f : 0.0f);
                const float lt = sel ? sdec[t] : lam;
                S0 = lt * S0 + vj;
                float num = S0;
#pragma unroll
                for (int i = 0; i < kGD - 1; ++i) {
                    if (i < D) {
                        const float ki = sk[t][i], qi = sq[t][i];
                        S1[i] = fmaf(lt, S1[i], ki * vj);
                        S2[i] = fmaf(lt, S2[i], ck2 * ki * ki * vj);
                        num = fmaf(qi, S1[i], num);
                        num = fmaf(cq2 * qi * qi, S2[i], num);
                    }
                }
                const float den = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(num), D));
                float den_c, di = 0.f, A = 0.f;
                if (dense) {
                    di = sKin[2][0];
                    for (int i = 0; i < D; ++i) {
                        const float qi = sq[t][i];
                        di = fmaf(qi, sKin[0][i], di);
                        di = fmaf(0.5f * qi * qi, sKin[1][i], di);
                    }
                    di *= pin;
                    A = fmaxf(den - di, a.eps);
                    den_c = fmaxf(A + di, a.eps);
                } else {
                    den_c = fmaxf(den, a.eps);
                }
                const float dyj = lane < D ? sdy[t][lane] : 0.f;
                const float yj = lane < D ? num / den_c : 0.f;
                const float dD = -wave_sum(dyj * yj) / den_c;
                float hcol, hdi = 0.f;  // adjoint of the ones column (den_total), of di beyond it
                if (dense) {
                    const float dA = A + di >= a.eps ? dD : 0.f;
                    const float ddc = den - di >= a.eps ? dA : 0.f;
                    hcol = ddc;
                    hdi = dA - ddc;
                } else {
                    hcol = den >= a.eps ? dD : 0.f;
                }
                const float g = lane < D ? dyj / den_c : (lane == D ? hcol : 0.f);
                // selective: phi_q . dphi_q = sum_j g_j num_j (the ones column: hcol den)
                if (sel) {
                    const float pqt = wave_sum(col ? g * num : 0.f);
                    if (lane == 0) a.pq[static_cast<size_t>(bh) * a.L + t0 + t] = pqt;
                }
                // dq_t[i] = sum_j g_j (S1[i][j] + 2 cq2 q_i S2[i][j]) (+ the incoming-K term)
#pragma unroll
                for (int i = 0; i < kGD - 1; ++i)
                    if (i < D) sred[lane][i] = g * (S1[i] + (2.0f * cq2) * sq[t][i] * S2[i]);
                __syncthreads();
                if (lane < D) {
                    float s = 0.f;
                    for (int jj = 0; jj <= D; ++jj) s += sred[jj][lane];
                    const float qi = sq[t][lane];
                    if (dense) {
                        s += hdi * pin * (sKin[0][lane] + qi * sKin[1][lane]);
                        dkin1 += hdi * pin * qi;
                        dkin2 += 0.5f * hdi * pin * qi * qi;
                    }
                    store_elem(a.dq, b * a.g_sb + h * a.g_sh + static_cast<int64_t>(t0 + t) * a.g_sl + lane, a.dt_g, s);
                }
                if (dense) {
                    dkin0 += hdi * pin;
                    pin *= lam;
                }
                if (lane == 0) {
                    ws[2 * (t0 + t)] = den_c;
                    ws[2 * (t0 + t) + 1] = hcol;
                }
                __syncthreads();
            }
        }
        if (sel && a.ds1 && col) {
            float f = lane < D ? a.ds0[o0 + lane] * S0 : a.dk0[bh] * S0;
#pragma unroll
            for (int i = 0; i < kGD - 1; ++i)
                if (i < D)
                    f += lane < D ? a.ds1[o1 + i * D + lane] * S1[i] + a.ds2[o1 + i * D + lane] * S2[i]
                                  : a.dk1[o0 + i] * S1[i] + a.dk2[o0 + i] * S2[i];
            fin = f;
        }
        if (sel) fin = wave_sum(col ? fin : 0.f);
    }
    // ---------------- pass 2: reverse, dk, dv, the incoming state's adjoint
    float dl_acc = 0.f, dks = 0.f;  // selective: suffix sum of the log decays' adjoint; beta's
    float dS0 = 0.f, dS1[kGD - 1], dS2[kGD - 1];
#pragma unroll
    for (int i = 0; i < kGD - 1; ++i) {
        dS1[i] = dS2[i] = 0.f;
        if (i < D && col && a.ds1) {
            dS1[i] = lane < D ? a.ds1[o1 + i * D + lane] : a.dk1[o0 + i];
            dS2[i] = lane < D ? a.ds2[o1 + i * D + lane] : a.dk2[o0 + i];
        }
    }
    if (col && a.ds1) dS0 = lane < D ? a.ds0[o0 + lane] : a.dk0[bh];
    for (int c = NC - 1; c >= 0; --c) {
        const int t0 = c * kGC, nv = min(kGC, a.L - t0);
        __syncthreads();
        generic_stage(a, b, h, hk, t0, nv, sq, sk, sv, sdy, sdec, lane);
        for (int t = nv - 1; t >= 0; --t) {
            const float den_c = ws[2 * (t0 + t)], hcol = ws[2 * (t0 + t) + 1];
            const float g = lane < D ? sdy[t][lane] / den_c : (lane == D ? hcol : 0.f);
            const float vj = lane < D ? sv[t][lane] : (lane == D ? 1.0f : 0.0f);
            const float lt = sel ? sdec[t] : lam;
            dS0 += g;
            float dvj = dS0;
#pragma unroll
            for (int i = 0; i < kGD - 1; ++i) {
                if (i < D) {
                    const float qi = sq[t][i], ki = sk[t][i];
                    dS1[i] = fmaf(qi, g, dS1[i]);
                    dS2[i] = fmaf(cq2 * qi * qi, g, dS2[i]);
                    dvj = fmaf(ki, dS1[i], dvj);
                    dvj = fmaf(ck2 * ki * ki, dS2[i], dvj);
                    sred[lane][i] = vj * (dS1[i] + (2.0f * ck2) * ki * dS2[i]);
                }
            }
            if (lane < D) store_elem(a.dv, b * a.g_sb + h * a.g_sh + static_cast<int64_t>(t0 + t) * a.g_sl + lane, a.dt_g, dvj);
            if (sel) {
                // the log decays' adjoint: sum over the tokens m >= t of
                // phi_q(m).dphi_q(m) - phi_k(m).dphi_k(m), plus the final state's share
                const float pkt = wave_sum(col ? vj * dvj : 0.f);
                dl_acc += a.pq[static_cast<size_t>(bh) * a.L + t0 + t] - pkt;
                if (lane == 0) a.dlogd[static_cast<size_t>(bh) * a.L + t0 + t] = dl_acc + fin;
            }
            __syncthreads();
            if (lane < D) {
                float s = 0.f;
                for (int jj = 0; jj <= D; ++jj) s += sred[jj][lane];
                // (selective: s is the scaled key's adjoint; the raw key's is beta s,
                // beta's the sum of k s = (beta k) s / beta)
                if (sel) dks = fmaf(sk[t][lane], s, dks);
                store_elem(a.dk, b * a.g_sb + h * a.g_sh + static_cast<int64_t>(t0 + t) * a.g_sl + lane, a.dt_g,
                           sel ? a.k_scale[h] * s : s);
            }
            __syncthreads();
            dS0 *= lt;
#pragma unroll
            for (int i = 0; i < kGD - 1; ++i) {
                dS1[i] *= lt;
                dS2[i] *= lt;
            }
        }
    }
    if (sel) {
        const float tot = wave_sum(dks);
        if (lane == 0) a.dkscale[bh] = tot / a.k_scale[h];
    }
    if (a.dsi1) {
        // the ones column's K1 / K2 adjoint collects the dense clamp's direct
        // incoming-K term too (lane i holds dkin1[i], dkin2[i]; every lane reads them)
#pragma unroll
        for (int i = 0; i < kGD - 1; ++i) {
            if (i < D) {
                const float e1 = __shfl(dkin1, i, kWave), e2 = __shfl(dkin2, i, kWave);
                if (lane < D) {
                    a.dsi1[o1 + i * D + lane] = dS1[i];
                    a.dsi2[o1 + i * D + lane] = dS2[i];
                } else if (lane == D) {
                    a.dki1[o0 + i] = dS1[i] + e1;
                    a.dki2[o0 + i] = dS2[i] + e2;
                }
            }
        }
        if (lane < D) a.dsi0[o0 + lane] = dS0;
        else if (lane == D) a.dki0[bh] = dS0 + dkin0;
    }
}

hipError_t launch_generic_prefill(const GenericArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(generic_prefill_kernel, dim3(a.B * a.H), dim3(kGD), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_generic_backward(const GenericArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(generic_backward_kernel, dim3(a.B * a.H), dim3(kGD), 0, stream, a);
    return hipGetLastError();
}

// prime_head_layernorm for head dims below 64: 64 rows per wavefront, staged
// through LDS with coalesced loads, lane r normalising row r.
__global__ __launch_bounds__(kGD) void generic_head_layernorm_kernel(const HeadNormArgs a) {
    __shared__ float rows[kGC][kGP];
    const int lane = threadIdx.x, D = a.D;
    const int64_t nrows = static_cast<int64_t>(a.B) * a.H * a.L, r0 = static_cast<int64_t>(blockIdx.x) * kGC;
    const int nv = static_cast<int>(min(static_cast<int64_t>(kGC), nrows - r0));
    auto offs = [&](int t, int64_t sb, int64_t sh, int64_t sl) {
        const int64_t r = r0 + t, h = r % a.H, bl = r / a.H, l = bl % a.L, b = bl / a.L;
        return b * sb + h * sh + l * sl;
    };
    for (int t = 0; t < nv; ++t)
        rows[t][lane] = lane < D ? ld_any(a.x, offs(t, a.x_sb, a.x_sh, a.x_sl) + lane, a.dt) : 0.f;
    __syncthreads();
    if (lane < nv) generic_ln_row(rows[lane], D, a.weight, a.bias, a.dt_norm, a.ln_eps, a.scale, a.dt);
    __syncthreads();
    for (int t = 0; t < nv; ++t)
        if (lane < D) store_elem(a.out, offs(t, a.o_sb, a.o_sh, a.o_sl) + lane, a.dt, rows[t][lane]);
}

hipError_t launch_generic_head_layernorm(const HeadNormArgs &a, hipStream_t stream) {
    const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.L;
    hipLaunchKernelGGL(generic_head_layernorm_kernel, dim3(static_cast<uint32_t>((rows + kGC - 1) / kGC)),
                       dim3(kGD), 0, stream, a);
    return hipGetLastError();
}

}  // namespace prime
