/*
 * prime_oracle.c -- CPU oracle for the PRIME moment-attention hot paths.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels are
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every routine restates, in float64 and plain loops, one algorithm of the
 * reference PyTorch package (src/prime_moment_attention/ in the reference tree);
 * each function names the file:line range it follows.  Tensors are dense
 * row-major arrays:
 *     q, k, v, y      [BH][L][D]        (BH = batch*heads flattened)
 *     S0, K1, K2      [BH][D]
 *     S1, S2          [BH][D][D]        index [key i][value j]
 *     K0              [BH]
 *     lam             [BH]              per-(b,h) decay (the reference has one
 *                                       scalar per module; heads are independent,
 *                                       so a per-head value is the scalar
 *                                       formula applied head by head)
 *
 * Pinning (which independent check holds each routine down) is documented in
 * tests/test_oracle.py next to the checks themselves.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define IDX2(a, b, nb) ((size_t)(a) * (size_t)(nb) + (size_t)(b))

/* ------------------------------------------------------------------------- */
/* Recurrent decode step, applied token by token.                             */
/* attention.py:119-143 (update S*,K* with decay, then read out with the new  */
/* state; den clamped with max(den, eps)).                                    */
/* ------------------------------------------------------------------------- */
void oracle_recurrent(int BH, int L, int D, const double *q, const double *k,
                      const double *v, const double *lam, double eps,
                      double *S0, double *S1, double *S2, double *K0,
                      double *K1, double *K2, double *y)
{
    for (int bh = 0; bh < BH; ++bh) {
        double *s0 = S0 + (size_t)bh * D, *s1 = S1 + (size_t)bh * D * D;
        double *s2 = S2 + (size_t)bh * D * D, *k0 = K0 + bh;
        double *k1 = K1 + (size_t)bh * D, *k2 = K2 + (size_t)bh * D;
        const double l = lam[bh];
        for (int t = 0; t < L; ++t) {
            const double *qt = q + ((size_t)bh * L + t) * D;
            const double *kt = k + ((size_t)bh * L + t) * D;
            const double *vt = v + ((size_t)bh * L + t) * D;
            double *yt = y + ((size_t)bh * L + t) * D;
            /* attention.py:126-132 */
            for (int j = 0; j < D; ++j) s0[j] = l * s0[j] + vt[j];
            for (int i = 0; i < D; ++i)
                for (int j = 0; j < D; ++j) {
                    s1[IDX2(i, j, D)] = l * s1[IDX2(i, j, D)] + kt[i] * vt[j];
                    s2[IDX2(i, j, D)] = l * s2[IDX2(i, j, D)] + kt[i] * kt[i] * vt[j];
                }
            *k0 = l * (*k0) + 1.0;
            for (int i = 0; i < D; ++i) {
                k1[i] = l * k1[i] + kt[i];
                k2[i] = l * k2[i] + kt[i] * kt[i];
            }
            /* attention.py:135-143 */
            double den = *k0;
            for (int i = 0; i < D; ++i) den += qt[i] * k1[i] + 0.5 * qt[i] * qt[i] * k2[i];
            if (den < eps) den = eps;
            for (int j = 0; j < D; ++j) {
                double num = s0[j];
                for (int i = 0; i < D; ++i)
                    num += qt[i] * s1[IDX2(i, j, D)] + 0.5 * qt[i] * qt[i] * s2[IDX2(i, j, D)];
                yt[j] = num / den;
            }
        }
    }
}

/* score weight 1 + q.k + 0.5 (q*q).(k*k)  (attention.py:172-174, chunked_ssd.py:90-92) */
static double taylor_score(int D, const double *qi, const double *kj)
{
    double d1 = 0.0, d2 = 0.0;
    for (int f = 0; f < D; ++f) {
        d1 += qi[f] * kj[f];
        d2 += qi[f] * qi[f] * kj[f] * kj[f];
    }
    return 1.0 + d1 + 0.5 * d2;
}

/* readout of a state (num and den) for one query, without decay factor */
static void state_readout(int D, const double *qt, const double *s0, const double *s1,
                          const double *s2, double k0, const double *k1,
                          const double *k2, double *num, double *den)
{
    double d = k0;
    for (int i = 0; i < D; ++i) d += qt[i] * k1[i] + 0.5 * qt[i] * qt[i] * k2[i];
    *den = d;
    for (int j = 0; j < D; ++j) {
        double n = s0[j];
        for (int i = 0; i < D; ++i)
            n += qt[i] * s1[IDX2(i, j, D)] + 0.5 * qt[i] * qt[i] * s2[IDX2(i, j, D)];
        num[j] = n;
    }
}

/* ------------------------------------------------------------------------- */
/* Chunked SSD core.  chunked_ssd.py:48-184.                                  */
/* Zero-pad L to a multiple of C (:65-77); per chunk: intra Taylor block with */
/* lambda^(i-j) mask (:79-94), carry readout lambda^(i+1)*(state readout)     */
/* (:139-153), y = num / max(den, eps) (:155-157); chunk deltas with weights  */
/* lambda^(C-1-i), zero on padding (:96-111); state carried chunk to chunk,   */
/* S^(c) = lambda^C S^(c-1) + dS^(c-1) (the closed form of :113-137); terminal */
/* state with the lambda^(-pad) correction (:162-182).                         */
/* has_state == 0 starts from zeros (state arrays are outputs only).          */
/* ------------------------------------------------------------------------- */
void oracle_chunked(int BH, int L, int D, int C, const double *q, const double *k,
                    const double *v, const double *lam, double eps, int has_state,
                    double *S0, double *S1, double *S2, double *K0, double *K1,
                    double *K2, double *y)
{
    const int pad = (C - (L % C)) % C;
    const int Lp = L + pad, NC = Lp / C;
    double *num = (double *)malloc(sizeof(double) * D);
    double *cn = (double *)malloc(sizeof(double) * D);
    double *dS1 = (double *)malloc(sizeof(double) * D * D);
    double *dS2 = (double *)malloc(sizeof(double) * D * D);
    double *dS0 = (double *)malloc(sizeof(double) * D);
    double *dK1 = (double *)malloc(sizeof(double) * D);
    double *dK2 = (double *)malloc(sizeof(double) * D);
    double *zero = (double *)calloc(D, sizeof(double));
    for (int bh = 0; bh < BH; ++bh) {
        double *s0 = S0 + (size_t)bh * D, *s1 = S1 + (size_t)bh * D * D;
        double *s2 = S2 + (size_t)bh * D * D, *k0 = K0 + bh;
        double *k1 = K1 + (size_t)bh * D, *k2 = K2 + (size_t)bh * D;
        if (!has_state) {
            memset(s0, 0, sizeof(double) * D);
            memset(s1, 0, sizeof(double) * D * D);
            memset(s2, 0, sizeof(double) * D * D);
            *k0 = 0.0;
            memset(k1, 0, sizeof(double) * D);
            memset(k2, 0, sizeof(double) * D);
        }
        const double l = lam[bh];
        const double lC = pow(l, C);
        const double *qb = q + (size_t)bh * L * D;
        const double *kb = k + (size_t)bh * L * D;
        const double *vb = v + (size_t)bh * L * D;
        double *yb = y + (size_t)bh * L * D;
        for (int c = 0; c < NC; ++c) {
            /* readout: intra block + carry of the state entering chunk c */
            for (int i = 0; i < C; ++i) {
                const int t = c * C + i;
                if (t >= L) break; /* padded rows are sliced off (:159-160) */
                const double *qi = qb + (size_t)t * D;
                double den = 0.0;
                for (int f = 0; f < D; ++f) num[f] = 0.0;
                for (int j = 0; j <= i; ++j) {
                    const int tj = c * C + j;
                    const double *kj = (tj < L) ? kb + (size_t)tj * D : zero;
                    const double *vj = (tj < L) ? vb + (size_t)tj * D : zero;
                    const double a = pow(l, i - j) * taylor_score(D, qi, kj);
                    den += a;
                    for (int f = 0; f < D; ++f) num[f] += a * vj[f];
                }
                double cn_den;
                state_readout(D, qi, s0, s1, s2, *k0, k1, k2, cn, &cn_den);
                const double din = pow(l, i + 1);
                den += din * cn_den;
                if (den < eps) den = eps;
                for (int f = 0; f < D; ++f) yb[(size_t)t * D + f] = (num[f] + din * cn[f]) / den;
            }
            /* chunk deltas (weights lambda^(C-1-i), zero on pad) and carry */
            memset(dS0, 0, sizeof(double) * D);
            memset(dS1, 0, sizeof(double) * D * D);
            memset(dS2, 0, sizeof(double) * D * D);
            memset(dK1, 0, sizeof(double) * D);
            memset(dK2, 0, sizeof(double) * D);
            double dK0 = 0.0;
            for (int j = 0; j < C; ++j) {
                const int tj = c * C + j;
                if (tj >= L) continue;
                const double w = pow(l, C - 1 - j);
                const double *kj = kb + (size_t)tj * D, *vj = vb + (size_t)tj * D;
                dK0 += w;
                for (int f = 0; f < D; ++f) {
                    dS0[f] += w * vj[f];
                    dK1[f] += w * kj[f];
                    dK2[f] += w * kj[f] * kj[f];
                }
                for (int a = 0; a < D; ++a)
                    for (int b = 0; b < D; ++b) {
                        dS1[IDX2(a, b, D)] += w * kj[a] * vj[b];
                        dS2[IDX2(a, b, D)] += w * kj[a] * kj[a] * vj[b];
                    }
            }
            for (int f = 0; f < D; ++f) {
                s0[f] = lC * s0[f] + dS0[f];
                k1[f] = lC * k1[f] + dK1[f];
                k2[f] = lC * k2[f] + dK2[f];
            }
            for (int a = 0; a < D * D; ++a) {
                s1[a] = lC * s1[a] + dS1[a];
                s2[a] = lC * s2[a] + dS2[a];
            }
            *k0 = lC * (*k0) + dK0;
        }
        if (pad > 0) { /* chunked_ssd.py:171-178 */
            const double corr = pow(l, -pad);
            for (int f = 0; f < D; ++f) { s0[f] *= corr; k1[f] *= corr; k2[f] *= corr; }
            for (int a = 0; a < D * D; ++a) { s1[a] *= corr; s2[a] *= corr; }
            *k0 *= corr;
        }
    }
    free(num); free(cn); free(dS1); free(dS2); free(dS0); free(dK1); free(dK2); free(zero);
}

/* ------------------------------------------------------------------------- */
/* Dense prefill, attention.py:160-202 (the module's 1 < L <= chunk_threshold */
/* branch).  Note the reference clamps the intra denominator first and, when  */
/* an incoming state exists, clamps again after adding the carry (:177,185).  */
/* Terminal state (:190-202) is always produced here.                         */
/* ------------------------------------------------------------------------- */
void oracle_dense(int BH, int L, int D, const double *q, const double *k,
                  const double *v, const double *lam, double eps, int has_state,
                  double *S0, double *S1, double *S2, double *K0, double *K1,
                  double *K2, double *y)
{
    double *num = (double *)malloc(sizeof(double) * D);
    double *cn = (double *)malloc(sizeof(double) * D);
    for (int bh = 0; bh < BH; ++bh) {
        double *s0 = S0 + (size_t)bh * D, *s1 = S1 + (size_t)bh * D * D;
        double *s2 = S2 + (size_t)bh * D * D, *k0 = K0 + bh;
        double *k1 = K1 + (size_t)bh * D, *k2 = K2 + (size_t)bh * D;
        const double l = lam[bh];
        const double *qb = q + (size_t)bh * L * D;
        const double *kb = k + (size_t)bh * L * D;
        const double *vb = v + (size_t)bh * L * D;
        double *yb = y + (size_t)bh * L * D;
        for (int i = 0; i < L; ++i) {
            const double *qi = qb + (size_t)i * D;
            double den = 0.0;
            for (int f = 0; f < D; ++f) num[f] = 0.0;
            for (int j = 0; j <= i; ++j) {
                const double a = pow(l, i - j) * taylor_score(D, qi, kb + (size_t)j * D);
                den += a;
                for (int f = 0; f < D; ++f) num[f] += a * vb[(size_t)j * D + f];
            }
            if (den < eps) den = eps; /* :177 */
            if (has_state) {          /* :180-185 */
                double cd;
                state_readout(D, qi, s0, s1, s2, *k0, k1, k2, cn, &cd);
                const double din = pow(l, i + 1);
                for (int f = 0; f < D; ++f) num[f] += din * cn[f];
                den += din * cd;
                if (den < eps) den = eps;
            }
            for (int f = 0; f < D; ++f) yb[(size_t)i * D + f] = num[f] / den;
        }
        /* terminal state :190-202 */
        const double lL = pow(l, L);
        if (!has_state) {
            memset(s0, 0, sizeof(double) * D);
            memset(s1, 0, sizeof(double) * D * D);
            memset(s2, 0, sizeof(double) * D * D);
            *k0 = 0.0;
            memset(k1, 0, sizeof(double) * D);
            memset(k2, 0, sizeof(double) * D);
        }
        for (int f = 0; f < D; ++f) { s0[f] *= lL; k1[f] *= lL; k2[f] *= lL; }
        for (int a = 0; a < D * D; ++a) { s1[a] *= lL; s2[a] *= lL; }
        *k0 *= lL;
        for (int j = 0; j < L; ++j) {
            const double w = pow(l, L - 1 - j);
            const double *kj = kb + (size_t)j * D, *vj = vb + (size_t)j * D;
            *k0 += w;
            for (int f = 0; f < D; ++f) {
                s0[f] += w * vj[f];
                k1[f] += w * kj[f];
                k2[f] += w * kj[f] * kj[f];
            }
            for (int a = 0; a < D; ++a)
                for (int b = 0; b < D; ++b) {
                    s1[IDX2(a, b, D)] += w * kj[a] * vj[b];
                    s2[IDX2(a, b, D)] += w * kj[a] * kj[a] * vj[b];
                }
        }
    }
    free(num);
    free(cn);
}

/* ------------------------------------------------------------------------- */
/* Delta-PRIME feature maps, chunked_delta_prime.py:73-87:                    */
/*   phi = [k/max(|k|,e), (1/sqrt2) k^2/max(|k^2|,e)],  psi = [q, (1/sqrt2) q^2] */
/* q is the already-scaled query (:120).  psi, phi are [BH][L][2D].            */
/* ------------------------------------------------------------------------- */
void oracle_delta_features(int BH, int L, int D, const double *q, const double *k,
                           double eps, double *psi, double *phi)
{
    const double r2 = 1.0 / sqrt(2.0);
    for (size_t t = 0; t < (size_t)BH * L; ++t) {
        const double *qt = q + t * D, *kt = k + t * D;
        double *ps = psi + t * 2 * D, *ph = phi + t * 2 * D;
        double n1 = 0.0, n2 = 0.0;
        for (int f = 0; f < D; ++f) {
            n1 += kt[f] * kt[f];
            n2 += kt[f] * kt[f] * kt[f] * kt[f];
        }
        n1 = sqrt(n1);
        n2 = sqrt(n2);
        if (n1 < eps) n1 = eps;
        if (n2 < eps) n2 = eps;
        for (int f = 0; f < D; ++f) {
            ph[f] = kt[f] / n1;
            ph[D + f] = r2 * (kt[f] * kt[f]) / n2;
            ps[f] = qt[f];
            ps[D + f] = r2 * qt[f] * qt[f];
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Chunked gated delta-PRIME prefill, chunked_delta_prime.py:177-283.         */
/*   psi, phi [BH][L][P] (P = 2D), v [BH][L][D], beta, alpha [BH][L],         */
/*   S [BH][D][P] in/out (has_state == 0 starts from zeros).                  */
/* Per chunk: cum = cumsum(log clamp(alpha,1e-5,1)) (:199-200),               */
/* Lambda_ij = exp(cum_i - cum_j) for i >= j (:203-206), T = I + strict-tril( */
/* Lambda*G*beta_j) (:209-218), u = v - (phi*e^cum) S^T (:238-242), solve     */
/* T E = u by forward substitution (:245), y = tril(psi phi^T * Lambda)(beta  */
/* E) + (psi*e^cum) S^T (:248-255), S <- e^cum_end S + (beta E)^T (phi *      */
/* e^(cum_end-cum)) (:259-264), then the Lyapunov clamp S <- S min(1, B/(|S|_F */
/* + 1e-6)) when bound > 0 (:266-270).  Padded steps use alpha = decay_pad    */
/* (:183) and zero psi/phi/v/beta.                                            */
/* ------------------------------------------------------------------------- */
void oracle_delta_chunked(int BH, int L, int D, int C, const double *psi,
                          const double *phi, const double *v, const double *beta,
                          const double *alpha, double decay_pad, double bound,
                          int has_state, double *S, double *y)
{
    const int P = 2 * D;
    const int pad = (C - (L % C)) % C;
    const int NC = (L + pad) / C;
    double *cum = (double *)malloc(sizeof(double) * C);
    double *u = (double *)malloc(sizeof(double) * C * D);
    double *E = (double *)malloc(sizeof(double) * C * D);
    double *Sn = (double *)malloc(sizeof(double) * D * P);
    double *zp = (double *)calloc(P, sizeof(double));
    double *zd = (double *)calloc(D, sizeof(double));
    for (int bh = 0; bh < BH; ++bh) {
        double *Sb = S + (size_t)bh * D * P;
        if (!has_state) memset(Sb, 0, sizeof(double) * D * P);
        for (int c = 0; c < NC; ++c) {
            const double *ps[256], *ph[256], *vv[256];
            double bt[256], al[256];
            for (int i = 0; i < C; ++i) {
                const int t = c * C + i;
                const size_t o = (size_t)bh * L + t;
                if (t < L) {
                    ps[i] = psi + o * P; ph[i] = phi + o * P; vv[i] = v + o * D;
                    bt[i] = beta[o]; al[i] = alpha[o];
                } else {
                    ps[i] = zp; ph[i] = zp; vv[i] = zd; bt[i] = 0.0; al[i] = decay_pad;
                }
                double a = al[i];
                if (a < 1e-5) a = 1e-5;
                if (a > 1.0) a = 1.0;
                cum[i] = log(a) + (i ? cum[i - 1] : 0.0);
            }
            /* u = v - (phi * e^cum) S^T */
            for (int i = 0; i < C; ++i) {
                const double ec = exp(cum[i]);
                for (int d = 0; d < D; ++d) {
                    double acc = 0.0;
                    for (int e = 0; e < P; ++e) acc += ph[i][e] * ec * Sb[IDX2(d, e, P)];
                    u[IDX2(i, d, D)] = vv[i][d] - acc;
                }
            }
            /* forward substitution: E_i = u_i - sum_{j<i} T_ij E_j */
            for (int i = 0; i < C; ++i) {
                for (int d = 0; d < D; ++d) E[IDX2(i, d, D)] = u[IDX2(i, d, D)];
                for (int j = 0; j < i; ++j) {
                    double g = 0.0;
                    for (int e = 0; e < P; ++e) g += ph[i][e] * ph[j][e];
                    const double tij = exp(cum[i] - cum[j]) * g * bt[j];
                    for (int d = 0; d < D; ++d) E[IDX2(i, d, D)] -= tij * E[IDX2(j, d, D)];
                }
            }
            /* outputs */
            for (int i = 0; i < C; ++i) {
                const int t = c * C + i;
                if (t >= L) break;
                const double ec = exp(cum[i]);
                double *yt = y + ((size_t)bh * L + t) * D;
                for (int d = 0; d < D; ++d) {
                    double acc = 0.0;
                    for (int e = 0; e < P; ++e) acc += ps[i][e] * ec * Sb[IDX2(d, e, P)];
                    yt[d] = acc;
                }
                for (int j = 0; j <= i; ++j) {
                    double g = 0.0;
                    for (int e = 0; e < P; ++e) g += ps[i][e] * ph[j][e];
                    const double a = g * exp(cum[i] - cum[j]) * bt[j];
                    for (int d = 0; d < D; ++d) yt[d] += a * E[IDX2(j, d, D)];
                }
            }
            /* state update */
            const double cend = cum[C - 1];
            const double cdec = exp(cend);
            for (int d = 0; d < D; ++d)
                for (int e = 0; e < P; ++e) {
                    double acc = cdec * Sb[IDX2(d, e, P)];
                    for (int j = 0; j < C; ++j)
                        acc += bt[j] * E[IDX2(j, d, D)] * ph[j][e] * exp(cend - cum[j]);
                    Sn[IDX2(d, e, P)] = acc;
                }
            if (bound > 0.0) {
                double nrm = 0.0;
                for (int a = 0; a < D * P; ++a) nrm += Sn[a] * Sn[a];
                nrm = sqrt(nrm);
                double sc = bound / (nrm + 1e-6);
                if (sc > 1.0) sc = 1.0;
                for (int a = 0; a < D * P; ++a) Sn[a] *= sc;
            }
            memcpy(Sb, Sn, sizeof(double) * D * P);
        }
    }
    free(cum); free(u); free(E); free(Sn); free(zp); free(zd);
}

/* ------------------------------------------------------------------------- */
/* Per-token gated delta rule with decay before prediction (the closed form   */
/* the chunked routine above equals when bound == 0, for every C):            */
/*   S_t = a_t S_{t-1} + b_t (v_t - a_t S_{t-1} phi_t) phi_t^T,  y_t = S_t psi_t */
/* with a_t = clamp(alpha_t, 1e-5, 1).  Independent of chunking; used only to */
/* pin oracle_delta_chunked.                                                   */
/* ------------------------------------------------------------------------- */
void oracle_delta_tokenwise(int BH, int L, int D, const double *psi,
                            const double *phi, const double *v, const double *beta,
                            const double *alpha, int has_state, double *S, double *y)
{
    const int P = 2 * D;
    double *pred = (double *)malloc(sizeof(double) * D);
    for (int bh = 0; bh < BH; ++bh) {
        double *Sb = S + (size_t)bh * D * P;
        if (!has_state) memset(Sb, 0, sizeof(double) * D * P);
        for (int t = 0; t < L; ++t) {
            const size_t o = (size_t)bh * L + t;
            const double *ph = phi + o * P, *ps = psi + o * P, *vt = v + o * D;
            double a = alpha[o];
            if (a < 1e-5) a = 1e-5;
            if (a > 1.0) a = 1.0;
            for (int d = 0; d < D; ++d) {
                double acc = 0.0;
                for (int e = 0; e < P; ++e) acc += Sb[IDX2(d, e, P)] * ph[e];
                pred[d] = a * acc;
            }
            for (int d = 0; d < D; ++d) {
                const double err = beta[o] * (vt[d] - pred[d]);
                for (int e = 0; e < P; ++e) Sb[IDX2(d, e, P)] = a * Sb[IDX2(d, e, P)] + err * ph[e];
            }
            double *yt = y + o * D;
            for (int d = 0; d < D; ++d) {
                double acc = 0.0;
                for (int e = 0; e < P; ++e) acc += Sb[IDX2(d, e, P)] * ps[e];
                yt[d] = acc;
            }
        }
    }
    free(pred);
}

/* ------------------------------------------------------------------------- */
/* Delta-PRIME single-token step, the L == 1 branch of                        */
/* ChunkedGatedDeltaPrimeAttention.forward (chunked_delta_prime.py:140-176):  */
/* prediction with the state as it is (:155-157, no decay first), update      */
/* S = alpha S + (beta err) phi^T (:159-161, alpha not clamped), Lyapunov     */
/* clamp (:163-167), readout y = S psi (:170).  One token per (b, h).          */
/* ------------------------------------------------------------------------- */
void oracle_delta_step(int BH, int D, const double *psi, const double *phi,
                       const double *v, const double *beta, const double *alpha,
                       double bound, double *S, double *y)
{
    const int P = 2 * D;
    for (int bh = 0; bh < BH; ++bh) {
        double *Sb = S + (size_t)bh * D * P;
        const double *ph = phi + (size_t)bh * P, *ps = psi + (size_t)bh * P;
        const double *vt = v + (size_t)bh * D;
        double nrm = 0.0;
        for (int d = 0; d < D; ++d) {
            double vh = 0.0;
            for (int e = 0; e < P; ++e) vh += Sb[IDX2(d, e, P)] * ph[e];
            const double err = beta[bh] * (vt[d] - vh);
            for (int e = 0; e < P; ++e) {
                const double x = alpha[bh] * Sb[IDX2(d, e, P)] + err * ph[e];
                Sb[IDX2(d, e, P)] = x;
                nrm += x * x;
            }
        }
        double sc = 1.0;
        if (bound > 0.0) {
            sc = bound / (sqrt(nrm) + 1e-6);
            if (sc > 1.0) sc = 1.0;
        }
        for (int a = 0; a < D * P; ++a) Sb[a] *= sc;
        for (int d = 0; d < D; ++d) {
            double acc = 0.0;
            for (int e = 0; e < P; ++e) acc += Sb[IDX2(d, e, P)] * ps[e];
            y[(size_t)bh * D + d] = acc;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Selective PRIME, step branch applied token by token (selective.py:384-409):*/
/* per-token decay lam[bh][t], key weights beta (first order) and beta^2 / 2  */
/* (second order) folded into the state, whose S2 / K2 therefore carry the    */
/* 1/2; the readout weighs the second-order term by 1.                        */
/* ------------------------------------------------------------------------- */
void oracle_selective_recurrent(int BH, int L, int D, const double *q, const double *k,
                                const double *v, const double *lam, const double *beta, double eps,
                                double *S0, double *S1, double *S2, double *K0,
                                double *K1, double *K2, double *y)
{
    for (int bh = 0; bh < BH; ++bh) {
        double *s0 = S0 + (size_t)bh * D, *s1 = S1 + (size_t)bh * D * D;
        double *s2 = S2 + (size_t)bh * D * D, *k0 = K0 + bh;
        double *k1 = K1 + (size_t)bh * D, *k2 = K2 + (size_t)bh * D;
        const double b1 = beta[bh], b2 = 0.5 * beta[bh] * beta[bh];
        for (int t = 0; t < L; ++t) {
            const double l = lam[(size_t)bh * L + t];
            const double *qt = q + ((size_t)bh * L + t) * D;
            const double *kt = k + ((size_t)bh * L + t) * D;
            const double *vt = v + ((size_t)bh * L + t) * D;
            double *yt = y + ((size_t)bh * L + t) * D;
            /* selective.py:394-400 */
            for (int j = 0; j < D; ++j) s0[j] = l * s0[j] + vt[j];
            for (int i = 0; i < D; ++i)
                for (int j = 0; j < D; ++j) {
                    s1[IDX2(i, j, D)] = l * s1[IDX2(i, j, D)] + b1 * kt[i] * vt[j];
                    s2[IDX2(i, j, D)] = l * s2[IDX2(i, j, D)] + b2 * kt[i] * kt[i] * vt[j];
                }
            *k0 = l * (*k0) + 1.0;
            for (int i = 0; i < D; ++i) {
                k1[i] = l * k1[i] + b1 * kt[i];
                k2[i] = l * k2[i] + b2 * kt[i] * kt[i];
            }
            /* selective.py:402-408 */
            double den = *k0;
            for (int i = 0; i < D; ++i) den += qt[i] * k1[i] + qt[i] * qt[i] * k2[i];
            if (den < eps) den = eps;
            for (int j = 0; j < D; ++j) {
                double num = s0[j];
                for (int i = 0; i < D; ++i)
                    num += qt[i] * s1[IDX2(i, j, D)] + qt[i] * qt[i] * s2[IDX2(i, j, D)];
                yt[j] = num / den;
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Selective PRIME, parallel branch (selective.py:414-440): C = cumsum(Delta),*/
/* weight(i <- j) = (1 + b q_i.k_j + b^2/2 (q_i*q_i).(k_j*k_j))               */
/*                  * exp(-max(C_i - C_j, 0) / tau) [i >= j],                  */
/* y_i = sum_j weight v_j / max(sum_j weight, eps); the returned state from    */
/* decay_to_end = exp(-(C_L-1 - C_j) / tau).  No incoming state (the branch    */
/* ignores it).                                                               */
/* ------------------------------------------------------------------------- */
void oracle_selective_parallel(int BH, int L, int D, const double *q, const double *k,
                               const double *v, const double *delta, const double *tau,
                               const double *beta, double eps,
                               double *S0, double *S1, double *S2, double *K0,
                               double *K1, double *K2, double *y)
{
    double *C = (double *)malloc(sizeof(double) * (size_t)L);
    double *w = (double *)malloc(sizeof(double) * (size_t)L);
    for (int bh = 0; bh < BH; ++bh) {
        const double b1 = beta[bh], b2 = 0.5 * beta[bh] * beta[bh], ta = tau[bh];
        double acc = 0.0;
        for (int t = 0; t < L; ++t) { acc += delta[(size_t)bh * L + t]; C[t] = acc; }
        for (int i = 0; i < L; ++i) {
            const double *qi = q + ((size_t)bh * L + i) * D;
            double den = 0.0;
            for (int j = 0; j <= i; ++j) {
                const double *kj = k + ((size_t)bh * L + j) * D;
                double s1 = 0.0, s2 = 0.0;
                for (int d = 0; d < D; ++d) { s1 += qi[d] * kj[d]; s2 += qi[d] * qi[d] * kj[d] * kj[d]; }
                const double dd = C[i] - C[j] > 0.0 ? C[i] - C[j] : 0.0;
                w[j] = (1.0 + b1 * s1 + b2 * s2) * exp(-dd / ta);
                den += w[j];
            }
            if (den < eps) den = eps;
            double *yi = y + ((size_t)bh * L + i) * D;
            for (int d = 0; d < D; ++d) {
                double num = 0.0;
                for (int j = 0; j <= i; ++j) num += w[j] * v[((size_t)bh * L + j) * D + d];
                yi[d] = num / den;
            }
        }
        /* selective.py:428-438: the state after the last token */
        double *s0 = S0 + (size_t)bh * D, *s1 = S1 + (size_t)bh * D * D;
        double *s2 = S2 + (size_t)bh * D * D, *k1 = K1 + (size_t)bh * D, *k2 = K2 + (size_t)bh * D;
        memset(s0, 0, sizeof(double) * D); memset(s1, 0, sizeof(double) * D * D);
        memset(s2, 0, sizeof(double) * D * D); memset(k1, 0, sizeof(double) * D);
        memset(k2, 0, sizeof(double) * D);
        K0[bh] = 0.0;
        for (int j = 0; j < L; ++j) {
            const double dd = C[L - 1] - C[j] > 0.0 ? C[L - 1] - C[j] : 0.0;
            const double e = exp(-dd / ta);
            const double *kj = k + ((size_t)bh * L + j) * D, *vj = v + ((size_t)bh * L + j) * D;
            K0[bh] += e;
            for (int a = 0; a < D; ++a) {
                s0[a] += e * vj[a];
                k1[a] += b1 * e * kj[a];
                k2[a] += b2 * e * kj[a] * kj[a];
                for (int c = 0; c < D; ++c) {
                    s1[IDX2(a, c, D)] += b1 * e * kj[a] * vj[c];
                    s2[IDX2(a, c, D)] += b2 * e * kj[a] * kj[a] * vj[c];
                }
            }
        }
    }
    free(C);
    free(w);
}

/* ------------------------------------------------------------------------- */
/* Reverse mode (vector-Jacobian product) of the recurrence.                  */
/* The reference trains through its prefill with torch autograd               */
/* (tests/test_attention.py:50-62, attention.py:77-210); this is the same     */
/* derivative written by hand on the token recurrence of attention.py:119-143,*/
/* in the reference's state coordinates:                                      */
/*   after token t: num_j = s0_j + sum_i q_i s1_ij + 1/2 q_i^2 s2_ij,         */
/*   den = max(k0 + q.k1 + 1/2 q^2.k2, eps), y = num / den;                   */
/*   torch's clamp passes the gradient where den_raw >= eps.                  */
/* Inputs: dy [BH,L,D], dstate_out (adjoint of the final state, NULL = 0).    */
/* Outputs: dq, dk, dv [BH,L,D] and dstate_in (adjoint of state_in).          */
/* The forward states of one sequence are kept in a buffer of L states.       */
/* ------------------------------------------------------------------------- */
void oracle_recurrent_vjp(int BH, int L, int D, const double *q, const double *k,
                          const double *v, const double *lam, double eps,
                          const double *S0i, const double *S1i, const double *S2i,
                          const double *K0i, const double *K1i, const double *K2i,
                          const double *dy, const double *dS0o, const double *dS1o,
                          const double *dS2o, const double *dK0o, const double *dK1o,
                          const double *dK2o, double *dq, double *dk, double *dv,
                          double *dS0, double *dS1, double *dS2, double *dK0, double *dK1,
                          double *dK2)
{
    const size_t DD = (size_t)D * D, NS = 2 * DD + 3 * (size_t)D + 1;
    double *hist = (double *)malloc(sizeof(double) * NS * (size_t)(L > 0 ? L : 1));
    double *cur = (double *)malloc(sizeof(double) * NS);
    double *dnum = (double *)malloc(sizeof(double) * D);
    for (int bh = 0; bh < BH; ++bh) {
        /* state layout in a buffer: s0 | s1 | s2 | k0 | k1 | k2 */
        double *s0 = cur, *s1 = cur + D, *s2 = s1 + DD, *k0 = s2 + DD, *k1 = k0 + 1, *k2 = k1 + D;
        if (S0i) {
            memcpy(s0, S0i + (size_t)bh * D, sizeof(double) * D);
            memcpy(s1, S1i + (size_t)bh * DD, sizeof(double) * DD);
            memcpy(s2, S2i + (size_t)bh * DD, sizeof(double) * DD);
            *k0 = K0i[bh];
            memcpy(k1, K1i + (size_t)bh * D, sizeof(double) * D);
            memcpy(k2, K2i + (size_t)bh * D, sizeof(double) * D);
        } else {
            memset(cur, 0, sizeof(double) * NS);
        }
        const double l = lam[bh];
        for (int t = 0; t < L; ++t) {  /* forward: the state after each token */
            const double *kt = k + ((size_t)bh * L + t) * D, *vt = v + ((size_t)bh * L + t) * D;
            for (int j = 0; j < D; ++j) s0[j] = l * s0[j] + vt[j];
            for (int i = 0; i < D; ++i)
                for (int j = 0; j < D; ++j) {
                    s1[IDX2(i, j, D)] = l * s1[IDX2(i, j, D)] + kt[i] * vt[j];
                    s2[IDX2(i, j, D)] = l * s2[IDX2(i, j, D)] + kt[i] * kt[i] * vt[j];
                }
            *k0 = l * (*k0) + 1.0;
            for (int i = 0; i < D; ++i) {
                k1[i] = l * k1[i] + kt[i];
                k2[i] = l * k2[i] + kt[i] * kt[i];
            }
            memcpy(hist + (size_t)t * NS, cur, sizeof(double) * NS);
        }
        /* adjoint of the state after the current token, same layout */
        double *a0 = dS0 + (size_t)bh * D, *a1 = dS1 + (size_t)bh * DD, *a2 = dS2 + (size_t)bh * DD;
        double *ak0 = dK0 + bh, *ak1 = dK1 + (size_t)bh * D, *ak2 = dK2 + (size_t)bh * D;
        if (dS0o) {
            memcpy(a0, dS0o + (size_t)bh * D, sizeof(double) * D);
            memcpy(a1, dS1o + (size_t)bh * DD, sizeof(double) * DD);
            memcpy(a2, dS2o + (size_t)bh * DD, sizeof(double) * DD);
            *ak0 = dK0o[bh];
            memcpy(ak1, dK1o + (size_t)bh * D, sizeof(double) * D);
            memcpy(ak2, dK2o + (size_t)bh * D, sizeof(double) * D);
        } else {
            memset(a0, 0, sizeof(double) * D); memset(a1, 0, sizeof(double) * DD);
            memset(a2, 0, sizeof(double) * DD); *ak0 = 0.0;
            memset(ak1, 0, sizeof(double) * D); memset(ak2, 0, sizeof(double) * D);
        }
        for (int t = L - 1; t >= 0; --t) {
            const double *h = hist + (size_t)t * NS;
            const double *h0 = h, *h1 = h + D, *h2 = h1 + DD, *hk0 = h2 + DD, *hk1 = hk0 + 1, *hk2 = hk1 + D;
            const double *qt = q + ((size_t)bh * L + t) * D, *kt = k + ((size_t)bh * L + t) * D;
            const double *vt = v + ((size_t)bh * L + t) * D, *gy = dy + ((size_t)bh * L + t) * D;
            double *gq = dq + ((size_t)bh * L + t) * D, *gk = dk + ((size_t)bh * L + t) * D;
            double *gv = dv + ((size_t)bh * L + t) * D;
            /* readout of token t */
            double raw = *hk0;
            for (int i = 0; i < D; ++i) raw += qt[i] * hk1[i] + 0.5 * qt[i] * qt[i] * hk2[i];
            const double den = raw < eps ? eps : raw;
            double dot = 0.0;
            for (int j = 0; j < D; ++j) {
                double num = h0[j];
                for (int i = 0; i < D; ++i) num += qt[i] * h1[IDX2(i, j, D)] + 0.5 * qt[i] * qt[i] * h2[IDX2(i, j, D)];
                dot += gy[j] * num / den;
                dnum[j] = gy[j] / den;
            }
            const double dden = raw >= eps ? -dot / den : 0.0;
            for (int i = 0; i < D; ++i) {
                double g = dden * (hk1[i] + qt[i] * hk2[i]);
                for (int j = 0; j < D; ++j) g += dnum[j] * (h1[IDX2(i, j, D)] + qt[i] * h2[IDX2(i, j, D)]);
                gq[i] = g;
            }
            for (int j = 0; j < D; ++j) a0[j] += dnum[j];
            for (int i = 0; i < D; ++i)
                for (int j = 0; j < D; ++j) {
                    a1[IDX2(i, j, D)] += qt[i] * dnum[j];
                    a2[IDX2(i, j, D)] += 0.5 * qt[i] * qt[i] * dnum[j];
                }
            *ak0 += dden;
            for (int i = 0; i < D; ++i) {
                ak1[i] += qt[i] * dden;
                ak2[i] += 0.5 * qt[i] * qt[i] * dden;
            }
            /* update of token t: state = l * state_before + f(k_t, v_t) */
            for (int j = 0; j < D; ++j) {
                double g = a0[j];
                for (int i = 0; i < D; ++i) g += a1[IDX2(i, j, D)] * kt[i] + a2[IDX2(i, j, D)] * kt[i] * kt[i];
                gv[j] = g;
            }
            for (int i = 0; i < D; ++i) {
                double g1 = 0.0, g2 = 0.0;
                for (int j = 0; j < D; ++j) {
                    g1 += a1[IDX2(i, j, D)] * vt[j];
                    g2 += a2[IDX2(i, j, D)] * vt[j];
                }
                gk[i] = g1 + 2.0 * kt[i] * g2 + ak1[i] + 2.0 * kt[i] * ak2[i];
            }
            for (int j = 0; j < D; ++j) a0[j] *= l;
            for (size_t x = 0; x < DD; ++x) {
                a1[x] *= l;
                a2[x] *= l;
            }
            *ak0 *= l;
            for (int i = 0; i < D; ++i) {
                ak1[i] *= l;
                ak2[i] *= l;
            }
        }
    }
    free(hist);
    free(cur);
    free(dnum);
}

/* ------------------------------------------------------------------------- */
/* Reverse mode of the dense prefill branch (attention.py:160-202) with its   */
/* double clamp.  Per token t the call's own tokens give (readout of the      */
/* call's state C_t, run from zero) num_c, den_c = sum_{j<=t} l^(t-j)         */
/* (1 + q.k_j + 1/2 q^2.k_j^2); an incoming state S adds l^(t+1) times its    */
/* readout (num_s, den_s):                                                    */
/*   D1 = max(den_c, eps) (:177),  D = max(D1 + l^(t+1) den_s, eps) (:185),   */
/*   y = (num_c + l^(t+1) num_s) / D   (without a state: D = D1).             */
/* torch's clamps pass the gradient where their argument >= eps: the outer    */
/* one gates dD, the inner one additionally gates what reaches den_c.  The    */
/* terminal state (:189-202) is l^L S + C_(L-1), as for the recurrence.       */
/* Same arguments and outputs as oracle_recurrent_vjp.                        */
/* ------------------------------------------------------------------------- */
void oracle_dense_vjp(int BH, int L, int D, const double *q, const double *k,
                      const double *v, const double *lam, double eps,
                      const double *S0i, const double *S1i, const double *S2i,
                      const double *K0i, const double *K1i, const double *K2i,
                      const double *dy, const double *dS0o, const double *dS1o,
                      const double *dS2o, const double *dK0o, const double *dK1o,
                      const double *dK2o, double *dq, double *dk, double *dv,
                      double *dS0, double *dS1, double *dS2, double *dK0, double *dK1,
                      double *dK2)
{
    const size_t DD = (size_t)D * D, NS = 2 * DD + 3 * (size_t)D + 1;
    double *hist = (double *)malloc(sizeof(double) * NS * (size_t)(L > 0 ? L : 1));
    double *cs = (double *)calloc(NS, sizeof(double));  /* the call's state */
    double *ac = (double *)malloc(sizeof(double) * NS);  /* its adjoint */
    double *nc = (double *)malloc(sizeof(double) * D), *ns = (double *)malloc(sizeof(double) * D);
    double *gn = (double *)malloc(sizeof(double) * D);
    for (int bh = 0; bh < BH; ++bh) {
        const double l = lam[bh];
        const int has = S0i != NULL;
        const double *i0 = has ? S0i + (size_t)bh * D : NULL, *i1 = has ? S1i + (size_t)bh * DD : NULL;
        const double *i2 = has ? S2i + (size_t)bh * DD : NULL, *ik1 = has ? K1i + (size_t)bh * D : NULL;
        const double *ik2 = has ? K2i + (size_t)bh * D : NULL;
        const double ik0 = has ? K0i[bh] : 0.0;
        /* forward: the call's state after each token (layout s0 | s1 | s2 | k0 | k1 | k2) */
        memset(cs, 0, sizeof(double) * NS);
        double *c0 = cs, *c1 = cs + D, *c2 = c1 + DD, *ck0 = c2 + DD, *ck1 = ck0 + 1, *ck2 = ck1 + D;
        for (int t = 0; t < L; ++t) {
            const double *kt = k + ((size_t)bh * L + t) * D, *vt = v + ((size_t)bh * L + t) * D;
            for (int j = 0; j < D; ++j) c0[j] = l * c0[j] + vt[j];
            for (int i = 0; i < D; ++i)
                for (int j = 0; j < D; ++j) {
                    c1[IDX2(i, j, D)] = l * c1[IDX2(i, j, D)] + kt[i] * vt[j];
                    c2[IDX2(i, j, D)] = l * c2[IDX2(i, j, D)] + kt[i] * kt[i] * vt[j];
                }
            *ck0 = l * (*ck0) + 1.0;
            for (int i = 0; i < D; ++i) {
                ck1[i] = l * ck1[i] + kt[i];
                ck2[i] = l * ck2[i] + kt[i] * kt[i];
            }
            memcpy(hist + (size_t)t * NS, cs, sizeof(double) * NS);
        }
        /* adjoints: ac of the call's state after the current token (from dstate_out),
           the incoming state's in the outputs (its readout terms, then l^L dstate_out) */
        double *a0 = ac, *a1 = ac + D, *a2 = a1 + DD, *ak0 = a2 + DD, *ak1 = ak0 + 1, *ak2 = ak1 + D;
        double *b0 = dS0 + (size_t)bh * D, *b1 = dS1 + (size_t)bh * DD, *b2 = dS2 + (size_t)bh * DD;
        double *bk0 = dK0 + bh, *bk1 = dK1 + (size_t)bh * D, *bk2 = dK2 + (size_t)bh * D;
        memset(ac, 0, sizeof(double) * NS);
        memset(b0, 0, sizeof(double) * D); memset(b1, 0, sizeof(double) * DD);
        memset(b2, 0, sizeof(double) * DD); *bk0 = 0.0;
        memset(bk1, 0, sizeof(double) * D); memset(bk2, 0, sizeof(double) * D);
        if (dS0o) {
            memcpy(a0, dS0o + (size_t)bh * D, sizeof(double) * D);
            memcpy(a1, dS1o + (size_t)bh * DD, sizeof(double) * DD);
            memcpy(a2, dS2o + (size_t)bh * DD, sizeof(double) * DD);
            *ak0 = dK0o[bh];
            memcpy(ak1, dK1o + (size_t)bh * D, sizeof(double) * D);
            memcpy(ak2, dK2o + (size_t)bh * D, sizeof(double) * D);
        }
        for (int t = L - 1; t >= 0; --t) {
            const double *h = hist + (size_t)t * NS;
            const double *h0 = h, *h1 = h + D, *h2 = h1 + DD, *hk0 = h2 + DD, *hk1 = hk0 + 1, *hk2 = hk1 + D;
            const double *qt = q + ((size_t)bh * L + t) * D, *kt = k + ((size_t)bh * L + t) * D;
            const double *vt = v + ((size_t)bh * L + t) * D, *gy = dy + ((size_t)bh * L + t) * D;
            double *gq = dq + ((size_t)bh * L + t) * D, *gk = dk + ((size_t)bh * L + t) * D;
            double *gv = dv + ((size_t)bh * L + t) * D;
            const double w = has ? pow(l, t + 1) : 0.0;
            double den_c, den_s = 0.0;
            state_readout(D, qt, h0, h1, h2, *hk0, hk1, hk2, nc, &den_c);
            if (has) state_readout(D, qt, i0, i1, i2, ik0, ik1, ik2, ns, &den_s);
            const double d1 = den_c < eps ? eps : den_c;
            const double dsum = has ? d1 + w * den_s : den_c;
            const double Dt = dsum < eps ? eps : dsum;
            double dot = 0.0;
            for (int j = 0; j < D; ++j) {
                const double num = nc[j] + (has ? w * ns[j] : 0.0);
                dot += gy[j] * num / Dt;
                gn[j] = gy[j] / Dt;
            }
            const double gD = dsum >= eps ? -dot / Dt : 0.0;  /* outer clamp */
            const double gc = den_c >= eps ? gD : 0.0;        /* inner clamp: the call's share */
            for (int i = 0; i < D; ++i) {
                double g = gc * (hk1[i] + qt[i] * hk2[i]);
                for (int j = 0; j < D; ++j) g += gn[j] * (h1[IDX2(i, j, D)] + qt[i] * h2[IDX2(i, j, D)]);
                if (has) {
                    double gs = gD * (ik1[i] + qt[i] * ik2[i]);
                    for (int j = 0; j < D; ++j) gs += gn[j] * (i1[IDX2(i, j, D)] + qt[i] * i2[IDX2(i, j, D)]);
                    g += w * gs;
                }
                gq[i] = g;
            }
            if (has) {
                for (int j = 0; j < D; ++j) b0[j] += w * gn[j];
                for (int i = 0; i < D; ++i)
                    for (int j = 0; j < D; ++j) {
                        b1[IDX2(i, j, D)] += w * qt[i] * gn[j];
                        b2[IDX2(i, j, D)] += w * 0.5 * qt[i] * qt[i] * gn[j];
                    }
                *bk0 += w * gD;
                for (int i = 0; i < D; ++i) {
                    bk1[i] += w * qt[i] * gD;
                    bk2[i] += w * 0.5 * qt[i] * qt[i] * gD;
                }
            }
            for (int j = 0; j < D; ++j) a0[j] += gn[j];
            for (int i = 0; i < D; ++i)
                for (int j = 0; j < D; ++j) {
                    a1[IDX2(i, j, D)] += qt[i] * gn[j];
                    a2[IDX2(i, j, D)] += 0.5 * qt[i] * qt[i] * gn[j];
                }
            *ak0 += gc;
            for (int i = 0; i < D; ++i) {
                ak1[i] += qt[i] * gc;
                ak2[i] += 0.5 * qt[i] * qt[i] * gc;
            }
            /* token t's update of the call's state: C_t = l C_(t-1) + f(k_t, v_t) */
            for (int j = 0; j < D; ++j) {
                double g = a0[j];
                for (int i = 0; i < D; ++i) g += a1[IDX2(i, j, D)] * kt[i] + a2[IDX2(i, j, D)] * kt[i] * kt[i];
                gv[j] = g;
            }
            for (int i = 0; i < D; ++i) {
                double g1 = 0.0, g2 = 0.0;
                for (int j = 0; j < D; ++j) {
                    g1 += a1[IDX2(i, j, D)] * vt[j];
                    g2 += a2[IDX2(i, j, D)] * vt[j];
                }
                gk[i] = g1 + 2.0 * kt[i] * g2 + ak1[i] + 2.0 * kt[i] * ak2[i];
            }
            for (size_t x = 0; x < NS; ++x) ac[x] *= l;
        }
        if (has && dS0o) {  /* the terminal state carries l^L S */
            const double lL = pow(l, L);
            for (int j = 0; j < D; ++j) b0[j] += lL * dS0o[(size_t)bh * D + j];
            for (size_t x = 0; x < DD; ++x) {
                b1[x] += lL * dS1o[(size_t)bh * DD + x];
                b2[x] += lL * dS2o[(size_t)bh * DD + x];
            }
            *bk0 += lL * dK0o[bh];
            for (int i = 0; i < D; ++i) {
                bk1[i] += lL * dK1o[(size_t)bh * D + i];
                bk2[i] += lL * dK2o[(size_t)bh * D + i];
            }
        }
    }
    free(hist);
    free(cs);
    free(ac);
    free(nc);
    free(ns);
    free(gn);
}
