/*
 * cpu_baseline.c -- float32 CPU restatement of the reference C99 engine's
 * additive PRIME step, used ONLY as the CPU timing baseline (bench.py's
 * cpu_baseline leg) and as a test checker.  Never linked into the product.
 *
 * Loop structure follows c/prime_moment.c:276-312 (additive branch of
 * prime_step_delta: decay-then-add update of S0/K1/K2 and the D x D moments,
 * then readout and clamp) and c/prime_moment.c:332-352 (prime_prefill: the
 * step applied token by token).  Two deliberate differences from the C99 file,
 * so that the numbers it produces are PyTorch semantics (attention.py:126-143):
 *   - S1/S2 are indexed [key i][value j] and the readout contracts q over the
 *     key index (the C99 file stores [value][key] but reads out over the value
 *     index, c/prime_moment.c:283-300);
 *   - eps is a parameter (the C99 default is 1e-4, the module default 1.0);
 *   - q is taken already scaled by 1/sqrt(D) and no LayerNorm is applied, as
 *     at the chunked core boundary (chunked_ssd.py:58-61).
 * OpenMP parallelises over independent (sequence, head) tiles.
 *
 * Layouts: q, k, v, y [N][D] with N = nseq*heads tiles; state per tile:
 *   s0 [N][D], s1 [N][D][D], s2 [N][D][D], k0 [N], k1 [N][D], k2 [N][D].
 */
#include <stddef.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static void step_tile(int D, float lam, float eps, const float *q, const float *k,
                      const float *v, float *s0, float *s1, float *s2, float *k0,
                      float *k1, float *k2, float *y)
{
    *k0 = lam * (*k0) + 1.0f;
    for (int i = 0; i < D; ++i) {
        const float ki = k[i], ki2 = k[i] * k[i];
        k1[i] = lam * k1[i] + ki;
        k2[i] = lam * k2[i] + ki2;
        float *r1 = s1 + (size_t)i * D, *r2 = s2 + (size_t)i * D;
        for (int j = 0; j < D; ++j) {
            r1[j] = lam * r1[j] + ki * v[j];
            r2[j] = lam * r2[j] + ki2 * v[j];
        }
    }
    for (int j = 0; j < D; ++j) {
        s0[j] = lam * s0[j] + v[j];
        y[j] = s0[j];
    }
    float den = *k0;
    for (int i = 0; i < D; ++i) {
        const float qi = q[i], qh = 0.5f * q[i] * q[i];
        den += qi * k1[i] + qh * k2[i];
        const float *r1 = s1 + (size_t)i * D, *r2 = s2 + (size_t)i * D;
        for (int j = 0; j < D; ++j) y[j] += qi * r1[j] + qh * r2[j];
    }
    if (den < eps) den = eps;
    const float inv = 1.0f / den;
    for (int j = 0; j < D; ++j) y[j] *= inv;
}

/* One decode step for N independent tiles; lam indexed by tile % heads. */
void baseline_decode_step(int N, int heads, int D, const float *q, const float *k,
                          const float *v, const float *lam, float eps, float *s0,
                          float *s1, float *s2, float *k0, float *k1, float *k2,
                          float *y, int nthreads)
{
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int n = 0; n < N; ++n) {
        const size_t o = (size_t)n * D, o2 = (size_t)n * D * D;
        step_tile(D, lam[n % heads], eps, q + o, k + o, v + o, s0 + o, s1 + o2, s2 + o2,
                  k0 + n, k1 + o, k2 + o, y + o);
    }
}

/* Sequential prefill (prime_prefill shape): q,k,v,y [N][L][D]. */
void baseline_prefill(int N, int heads, int L, int D, const float *q, const float *k,
                      const float *v, const float *lam, float eps, float *s0,
                      float *s1, float *s2, float *k0, float *k1, float *k2, float *y,
                      int nthreads)
{
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int n = 0; n < N; ++n) {
        const size_t o = (size_t)n * D, o2 = (size_t)n * D * D;
        for (int t = 0; t < L; ++t) {
            const size_t ot = ((size_t)n * L + t) * D;
            step_tile(D, lam[n % heads], eps, q + ot, k + ot, v + ot, s0 + o, s1 + o2,
                      s2 + o2, k0 + n, k1 + o, k2 + o, y + ot);
        }
    }
}
