/*
 * prime_mi355x.h -- C ABI of the MI355X (gfx950) PRIME moment-attention library.
 *
 * All tensors are DEVICE pointers on the current HIP device; every call is
 * asynchronous on the given stream (a hipStream_t passed as void*; NULL is the
 * default stream) and performs no host synchronisation and no allocation.
 * Every entry point returns 0 on success or a negative PRIME_ERR_* code; the
 * message for the last failure on the calling thread is prime_last_error().
 *
 * Shapes follow the reference PyTorch package (src/prime_moment_attention):
 *   q, k, v, y   [B, H, L, D]   any element strides for B, H, L; D contiguous
 *   state        6 separate fp32 buffers, contiguous, in the reference order
 *                (attention.py:108-117, cache.py:15-56):
 *                  S0 [B,H,D]  S1 [B,H,D,D]  S2 [B,H,D,D]  (S* indexed [key][value])
 *                  K0 [B,H,1]  K1 [B,H,D]    K2 [B,H,D]
 *   decay        fp32 [H] device array (the reference's scalar `decay`, widened
 *                to one value per head; pass H copies of the scalar for the
 *                reference behaviour)
 * q is taken PRE-SCALED by 1/sqrt(D), as at the reference's core boundary
 * (chunked_ssd.py:58-61, attention.py:101).
 *
 * Head dim: D = 64 runs the MFMA chunk kernels; the base and selective forms
 * (prefill, decode step, backward, QK-norm) also take 1 <= D <= 63 (the
 * reference's own tests use 32 and 16), run token by token in one wavefront
 * per (sequence, head) with no row-alignment requirement and no workspace
 * beyond the backward's per-token records.  The delta rule takes D <= 64
 * with any chunk (documented at prime_delta_prefill).  prime_accumulate and
 * the split decode readout/update take D = 64 only.
 */
#ifndef PRIME_MI355X_H
#define PRIME_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PRIME_ABI_VERSION 1

/* element types */
#define PRIME_F32  0
#define PRIME_BF16 1
#define PRIME_F16  2

/* error codes */
#define PRIME_OK                   0
#define PRIME_ERR_INVALID_ARG     -1  /* null pointer, bad size, inconsistent shape */
#define PRIME_ERR_UNSUPPORTED_DIM -2  /* head dim not taken by this entry point */
#define PRIME_ERR_UNSUPPORTED_DTYPE -3
#define PRIME_ERR_MISALIGNED      -4  /* pointer/stride breaks 16-byte row alignment */
#define PRIME_ERR_ALIAS           -5  /* output overlaps an input it may not alias */
#define PRIME_ERR_HIP             -6  /* HIP launch / runtime error */

/* flags for prime_chunked_prefill */
#define PRIME_FLAG_DENSE_CLAMP 1u /* reproduce the dense branch's double clamp:
                                     den = max(max(den_call, eps) + carry_init, eps)
                                     (attention.py:177,185) instead of the
                                     recurrence's max(den, eps) */

/* flag for prime_delta_prefill_workspace_size: size the workspace for F32
   q/k/v (the fp32 path's per-chunk records are twice the bf16 path's) */
#define PRIME_FLAG_F32_INPUTS 2u

/* tensor layouts (prime_tensor_t.layout) */
#define PRIME_LAYOUT_STRIDED 0 /* the strided view below */
#define PRIME_LAYOUT_FRAG    1 /* y of the decode steps only: the [B, H*D] output
                                  in the fragment layout of prime_linear_frag
                                  (bf16; B padded to a multiple of 16 rows) */

/* A strided [B, H, L, D] view (decode calls ignore stride_l). */
typedef struct prime_tensor {
    void   *data;
    int32_t dtype;      /* PRIME_F32 / PRIME_BF16 / PRIME_F16 */
    int32_t layout;     /* PRIME_LAYOUT_STRIDED (0) unless stated */
    int64_t stride_b;   /* strides in ELEMENTS */
    int64_t stride_h;
    int64_t stride_l;
} prime_tensor_t;

/* The 6-tuple moment state; each pointer is a contiguous fp32 buffer. */
typedef struct prime_state {
    float *s0, *s1, *s2, *k0, *k1, *k2;
} prime_state_t;

/* ABI version (PRIME_ABI_VERSION) and thread-local last error message. */
int prime_abi_version(void);
const char *prime_last_error(void);

/*
 * One recurrent decode step for B x H independent (sequence, head) tiles.
 * Replaces the L == 1 branch of PrimeMomentAttention.forward
 * (attention.py:119-143): decay-update S0..K2 with the new token, then read out
 * y = (S0 + S1^T q + 1/2 S2^T q^2) / max(K0 + q.K1 + 1/2 q^2.K2, eps) with the
 * updated state.
 *   q, k, v : [B, H(q) / H_kv(k,v), D]; k/v head = h / (H / H_kv) (GQA,
 *             attention.py:92-94)
 *   state_in: NULL for a zero state (attention.py:111-117)
 *   state_out may equal state_in (in place); otherwise they must not overlap.
 *   y       : [B, H, D], F32 or BF16 or F16
 */
int prime_decode_step(const prime_tensor_t *q, const prime_tensor_t *k,
                      const prime_tensor_t *v, int B, int H, int H_kv, int D,
                      const float *decay, float eps, const prime_state_t *state_in,
                      const prime_state_t *state_out, const prime_tensor_t *y,
                      void *stream);

/*
 * The module's QK prologue, applied inside the decode step
 * (attention.py:96-101): q <- LayerNorm(q) * q_scale, k <- LayerNorm(k), each
 * over the head dim with the affine weight and bias (dtype `dtype`, [D] each)
 * and `eps`; the LayerNorm output is rounded to q's / k's dtype first, as the
 * module's LayerNorm returns it.  q_weight NULL: no LayerNorm, only q_scale.
 */
typedef struct prime_qk_norm {
    const void *q_weight, *q_bias, *k_weight, *k_bias;
    int32_t dtype;   /* of the four vectors */
    float eps;       /* LayerNorm eps (torch default 1e-5) */
    float q_scale;   /* 1/sqrt(D) for the module; 1 when q is pre-scaled */
} prime_qk_norm_t;

/*
 * prime_decode_step on the raw projections: q, k are the q_proj / k_proj
 * outputs, normalised and scaled in the kernel by `norm` (see above).  Replaces
 * attention.py:96-143 for L == 1.
 */
int prime_decode_step_qknorm(const prime_tensor_t *q, const prime_tensor_t *k,
                             const prime_tensor_t *v, int B, int H, int H_kv, int D,
                             const float *decay, float eps, const prime_qk_norm_t *norm,
                             const prime_state_t *state_in, const prime_state_t *state_out,
                             const prime_tensor_t *y, void *stream);

/*
 * Residual add + RMSNorm of the PRIME decoder blocks (model.py:47-56, 107-118):
 * x <- x + delta (when delta is not NULL; the sum rounded to `dtype`, as the
 * block's residual add stores it), then out <- x * rsqrt(mean(x^2) + eps) *
 * weight.  x, delta, out: [rows, hidden] contiguous, weight [hidden]; one dtype
 * (F32 / BF16 / F16); hidden a multiple of 4 and at most 4096; every pointer
 * aligned to 4 elements.  out may be x.
 */
int prime_add_rmsnorm(void *x, const void *delta, const void *weight, void *out, int rows,
                      int hidden, int dtype, float eps, void *stream);

/*
 * Exact GELU, y = x * 0.5 * (1 + erf(x / sqrt(2))) computed in fp32 and rounded
 * once to `dtype` (F32 / BF16 / F16): the MLP activation of the GELU decoder
 * blocks (nn.GELU(), primelm_50m.py:64; torch.nn.functional.gelu's default
 * form, the same bits for bf16).  x, y: n contiguous elements, 16-byte
 * aligned; y may be x (in place), otherwise they must not overlap.
 */
int prime_gelu(const void *x, void *y, int64_t n, int dtype, void *stream);

/*
 * Chunked prefill of L tokens for B x H sequences.  Replaces
 * chunked_prime_ssd_core (chunked_ssd.py:48-184) and, with
 * PRIME_FLAG_DENSE_CLAMP, the dense branch of PrimeMomentAttention.forward
 * (attention.py:160-202).  The result does not depend on `chunk` (the reference
 * algorithm is exact for any chunk size); the kernel tiles 64 tokens.
 *   state_in : NULL for zeros; state_out: NULL when no final state is wanted;
 *              state_out may equal state_in.
 *   y        : [B, H, L, D]
 *   workspace: optional device scratch of workspace_bytes (16-byte aligned).
 *              With at least prime_chunked_prefill_workspace_size() bytes the
 *              sequences are split into segments that run in parallel (a
 *              carried-state scan between them) when there are fewer of them
 *              than CUs, or, with more, some run as two halves, the second
 *              starting from the first's end state handed over through the
 *              workspace (bit-identical); with less (or NULL) each sequence
 *              runs as one segment.  Results agree either way.  Calls that
 *              overlap in time must not share a workspace.
 */
int prime_chunked_prefill(const prime_tensor_t *q, const prime_tensor_t *k,
                          const prime_tensor_t *v, int B, int H, int H_kv, int L, int D,
                          int chunk, const float *decay, float eps, unsigned flags,
                          const prime_state_t *state_in, const prime_tensor_t *y,
                          const prime_state_t *state_out, void *workspace,
                          size_t workspace_bytes, void *stream);

/*
 * prime_chunked_prefill on the raw projections: q, k are the q_proj / k_proj
 * outputs, normalised and scaled as the kernels load them by `norm` (see
 * prime_qk_norm_t), bit-identical to prime_head_layernorm on q (with q_scale)
 * and k (scale 1) followed by prime_chunked_prefill.  Replaces
 * attention.py:96-101 together with the prefill branches (:145-202).
 * BF16 q/k/v only; workspace and the other arguments as above.
 */
int prime_chunked_prefill_qknorm(const prime_tensor_t *q, const prime_tensor_t *k,
                                 const prime_tensor_t *v, int B, int H, int H_kv, int L, int D,
                                 int chunk, const float *decay, float eps, unsigned flags,
                                 const prime_qk_norm_t *norm, const prime_state_t *state_in,
                                 const prime_tensor_t *y, const prime_state_t *state_out,
                                 void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes prime_chunked_prefill uses for this shape (0 = none needed). */
size_t prime_chunked_prefill_workspace_size(int B, int H, int L, unsigned flags);

/*
 * Chunked gated delta-rule PRIME prefill.  Replaces the L > 1 branch of
 * ChunkedGatedDeltaPrimeAttention.forward (chunked_delta_prime.py:177-283):
 * per 64-token chunk, u = v - (phi e^cum) S^T, the unit-triangular solve
 * T E = u, y = tril(Psi Phi^T * Lambda) (beta E) + (psi e^cum) S^T,
 * S <- e^cum_end S + (beta E)^T (phi e^(cum_end - cum)), then the Lyapunov
 * clamp S <- S min(1, bound / (|S|_F + 1e-6)).
 *   q, k, v   : [B, H(q) / H_kv, L, D] after the module's projections, QK-norm
 *               and q * 1/sqrt(D) (:107-126); the kernels form psi = [q, q*q/sqrt2]
 *               and phi = [k/max(|k|,feat_eps), (k*k)/max(|k*k|,feat_eps)/sqrt2]
 *               (:73-87).  BF16 or F32 (all three alike).  BF16 inputs run
 *               on bf16 MFMA operands (fp32 accumulation, fp32 state); F32
 *               inputs take an fp32 path (fp32 MFMA operands and records), as
 *               the reference computes in fp32 (:123-127).
 *   beta      : fp32 [B, H, L] contiguous, 0.5 mean sigmoid(write) (:134)
 *   alpha     : fp32 [B, H, L] contiguous, decay (1 - 0.5 mean sigmoid(erase)) (:137)
 *   decay_pad : alpha of the zero tokens padding the last chunk (:189, the
 *               module's decay; the final state keeps that padding's decay)
 *   bound     : Lyapunov bound; <= 0 disables the clamp (:266-270)
 *   chunk     : tokens per clamp (the reference's chunk_size; the result
 *               depends on it).  D = 64 with chunk 64 runs the MFMA kernels
 *               below; any other D in 1 .. 64 or chunk >= 1 runs the token
 *               recurrence the chunk form unrolls (one wavefront per
 *               (sequence, head), the clamp after every `chunk` tokens and
 *               after the padded last chunk; q/k/v of any supported dtype, no
 *               alignment or workspace requirement: workspace may be NULL)
 *   state_in  : fp32 [B, H, D, 2D] or NULL (zero); state_out likewise or NULL;
 *               they may be the same buffer
 *   y         : [B, H, L, D], F32 / BF16 / F16
 *   workspace : at least prime_delta_prefill_workspace_size(B, H, L, f) bytes
 *               (16-byte aligned; f = PRIME_FLAG_F32_INPUTS for F32 inputs,
 *               else 0).  A smaller workspace (at least
 *               prime_delta_prefill_workspace_size(B, H, 64, f)) makes the call
 *               process the sequence in more, shorter windows; results agree.
 * When the workspace holds fewer chunks than the sequence, the per-chunk
 * solve of later windows runs on a side stream while the current window is
 * scanned on `stream` (two windows ahead when the workspace holds three
 * windows of 64 chunks, as the recommended size does; one window ahead with
 * less).  The library keeps one side stream and its events per
 * (device, caller stream), created on the first such call outside graph
 * capture and held for the life of the process; a call holds them for its
 * whole enqueue sequence, so calls on different streams or threads are
 * independent.  Under capture, or past 64 caller streams, the windows run on
 * `stream` alone (same results).
 */
int prime_delta_prefill(const prime_tensor_t *q, const prime_tensor_t *k,
                        const prime_tensor_t *v, const float *beta, const float *alpha,
                        int B, int H, int H_kv, int L, int D, int chunk, float decay_pad,
                        float feat_eps, float bound, const float *state_in,
                        const prime_tensor_t *y, float *state_out, void *workspace,
                        size_t workspace_bytes, void *stream);

/* Workspace bytes of prime_delta_prefill for this shape (flags: 0 for BF16
   inputs, PRIME_FLAG_F32_INPUTS for F32 inputs). */
size_t prime_delta_prefill_workspace_size(int B, int H, int L, unsigned flags);

/*
 * Backward of prime_delta_prefill: gradients of the chunked delta-rule
 * prefill (the autograd graph of chunked_delta_prime.py:177-283 -- features
 * :73-87, the per-chunk triangular solve, the per-chunk Lyapunov clamp) with
 * respect to q, k, v, beta, alpha and the incoming state, given dy (the
 * gradient of y) and dstate_out (of the final state; NULL = zero).
 *   q, k, v, beta, alpha, decay_pad, feat_eps, bound, state_in: as the forward
 *   dy           : [B, H, L, D], BF16 or F32, strided
 *   dq, dk, dv   : fp32 contiguous [B, H, L, D] -- dk and dv per QUERY head
 *                  (the caller sums the H / H_kv heads of a group)
 *   dbeta, dalpha: fp32 [B, H, L]; dalpha is 0 where alpha is outside the
 *                  forward's clamp [1e-5, 1]
 *   dstate_in    : fp32 [B, H, D, 2D] or NULL
 *   workspace    : prime_delta_prefill_backward_workspace_size(B, H, L, D, chunk)
 *                  bytes (the state entering every chunk, recomputed in fp32;
 *                  outside D = 64 with chunk 64 also one chunk's token states
 *                  per (sequence, head), recomputed chunk by chunk for the
 *                  reverse pass)
 * fp32 arithmetic throughout.
 */
size_t prime_delta_prefill_backward_workspace_size(int B, int H, int L, int D, int chunk);
int prime_delta_prefill_backward(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                                 const float *beta, const float *alpha, int B, int H, int H_kv, int L, int D,
                                 int chunk, float decay_pad, float feat_eps, float bound, const float *state_in,
                                 const prime_tensor_t *dy, const float *dstate_out, float *dq, float *dk, float *dv,
                                 float *dbeta, float *dalpha, float *dstate_in, void *workspace,
                                 size_t workspace_bytes, void *stream);

/*
 * One delta-rule PRIME decode step.  Replaces the L == 1 branch of
 * ChunkedGatedDeltaPrimeAttention.forward (chunked_delta_prime.py:140-176),
 * which predicts with the undecayed state: v_hat = S phi, S <- alpha S +
 * beta (v - v_hat) phi^T, Lyapunov clamp, y = S psi.
 *   q, k, v : [B, H(q) / H_kv, D] (stride_l ignored; D = 64, or 1 .. 63 in
 *             one wavefront per (sequence, head)); beta, alpha: fp32 [B, H]
 *   state_in: fp32 [B, H, D, 2D] or NULL; state_out may equal state_in
 *   y       : [B, H, D]
 */
int prime_delta_decode_step(const prime_tensor_t *q, const prime_tensor_t *k,
                            const prime_tensor_t *v, const float *beta, const float *alpha,
                            int B, int H, int H_kv, int D, float feat_eps, float bound,
                            const float *state_in, float *state_out, const prime_tensor_t *y,
                            void *stream);

/*
 * Backward of prime_delta_decode_step: the gradients torch autograd takes
 * through the L == 1 branch (chunked_delta_prime.py:140-176 -- features
 * :73-87, the prediction with the undecayed state, the update with alpha
 * unclamped, the Lyapunov clamp before the readout) with respect to q, k, v,
 * beta, alpha and the incoming state, given dy and dstate_out (the gradient
 * of the new state; NULL = zero).
 *   q, k, v, beta, alpha, feat_eps, bound, state_in: as the forward (D <= 64)
 *   dy           : [B, H, D], any float dtype, strided (stride_l ignored)
 *   dq, dk, dv   : fp32 contiguous [B, H, D] -- dk and dv per QUERY head
 *   dbeta, dalpha: fp32 [B, H]
 *   dstate_in    : fp32 [B, H, D, 2D] or NULL
 * One wavefront per (sequence, head), fp32 arithmetic, no workspace.
 */
int prime_delta_decode_step_backward(const prime_tensor_t *q, const prime_tensor_t *k,
                                     const prime_tensor_t *v, const float *beta, const float *alpha,
                                     int B, int H, int H_kv, int D, float feat_eps, float bound,
                                     const float *state_in, const prime_tensor_t *dy,
                                     const float *dstate_out, float *dq, float *dk, float *dv,
                                     float *dbeta, float *dalpha, float *dstate_in, void *stream);

/*
 * The module's per-head QK-norm on projected rows (attention.py:96-101):
 * out = LayerNorm(x) over D (biased variance, affine weight/bias [D] of
 * param_dtype, epsilon ln_eps) rounded to x's dtype, then multiplied by
 * `scale` and rounded again (pass 1/sqrt(D) for q, 1 for k).  weight = bias =
 * NULL applies the scale only (a module without QK-norm).  x, out: strided
 * [B, H, L, D] views of one dtype, D = 64 (or 1 .. 63); out may be x (the same view) but may
 * not partly overlap it.  The chunked prefill's producer for q and k.
 */
int prime_head_layernorm(const prime_tensor_t *x, const prime_tensor_t *out, int B, int H, int L, int D,
                         const void *weight, const void *bias, int param_dtype, float ln_eps, float scale,
                         void *stream);

/*
 * Linear layer of the PRIME blocks, y = epilogue(x w^T) (F.linear without
 * bias; model.py:59-68, 101-118, 160): x [M, K], w [N, K], y [M, N], all
 * BF16, row strides ldx, ldw, ldy in elements; fp32 accumulation, one
 * rounding to bf16.  Epilogues: PRIME_EPILOGUE_NONE, or PRIME_EPILOGUE_GELU =
 * the exact GELU 0.5 t (1 + erf(t / sqrt 2)) of F.gelu.  Few rows (decode
 * batches) run a skinny kernel; M >= 2048 with N a multiple of 256 a
 * 256 x 256-tile kernel.  K a multiple of 64; N a multiple of 4; x, w rows
 * 16-byte aligned, y rows 8-byte aligned; y may not overlap x or w.
 */
#define PRIME_EPILOGUE_NONE 0
#define PRIME_EPILOGUE_GELU 1
#define PRIME_EPILOGUE_RESIDUAL 2 /* prime_linear_residual only */
int prime_linear(const void *x, const void *w, void *y, int M, int N, int K, int64_t ldx, int64_t ldw,
                 int64_t ldy, int dtype, int epilogue, void *stream);

/*
 * y = r + x . w^T: a projection and the residual add after it in one pass (the
 * blocks' x + o_proj(...) and x + down_proj(...), model.py:107-118).  The
 * product is rounded to bf16 first, then added to r and rounded again, as the
 * separate GEMM and add store it.  r [M, N] with row stride ldr may be y (in
 * place: the residual stream updated where it lies), otherwise disjoint from
 * it; the other arguments as prime_linear.  BF16 only.
 */
int prime_linear_residual(const void *x, const void *w, const void *r, void *y, int M, int N, int K,
                          int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldy, int dtype, void *stream);

/*
 * A decode-step projection with the passes around it folded in (model.py:
 * 47-56, 59-68, 107-118 at one token per sequence): y = epilogue(s_m x w^T),
 * where s_m = rsqrt(mean_k x[m,k]^2 + rms_eps) when rms_eps > 0 (the RMSNorm
 * before the projection; pass w with the norm's weight already multiplied
 * into its columns, w' = w diag(g)) and 1 otherwise; the product (times s_m)
 * is rounded to bf16, then the epilogue: PRIME_EPILOGUE_NONE, _GELU (exact)
 * or _RESIDUAL (y = r + product; r may be y, with the same row stride).
 * BF16; M up to 1024 rows (decode batches); N a multiple of 32, K of 128;
 * x, w rows 16-byte aligned, y and r rows 8-byte aligned.  With the RMS
 * prologue K is the normalised width (the hidden size).  The norm's output
 * is not rounded on its own, unlike RMSNorm followed by F.linear; the
 * difference is within a bf16 rounding of each product.
 */
int prime_linear_fused(const void *x, const void *w, const void *r, void *y, int M, int N, int K, int64_t ldx,
                       int64_t ldw, int64_t ldr, int64_t ldy, int dtype, int epilogue, float rms_eps,
                       void *stream);

/*
 * Selective PRIME (PrimeSelectiveMomentAttention, selective.py:264-444): the
 * same moment recurrence with a decay per token and per head,
 *   l_t = exp(-Delta_t / tau_h)  (Delta_t = softplus(W_delta x_t + b), clamped),
 * and the key scaled by an inverse temperature beta_h:
 *   S0 = l S0 + v;  S1 = l S1 + beta k v^T;  S2 = l S2 + 1/2 beta^2 (k*k) v^T
 *   K0 = l K0 + 1;  K1 = l K1 + beta k;      K2 = l K2 + 1/2 beta^2 k*k
 *   y  = (S0 + S1^T q + S2^T (q*q)) / max(K0 + q.K1 + (q*q).K2, eps)
 * Note the state convention: S2 and K2 include the 1/2 (selective.py:395-400),
 * unlike the base form's.  q arrives pre-scaled by 1/sqrt(D) as for the base
 * form (selective.py:362).
 *
 * prime_selective_prefill: L tokens of q/k/v [B, H(kv), L, 64] (strided as
 * prime_chunked_prefill), BF16 (bf16 MFMA operands, fp32 accumulation and
 * state) or F32 (an fp32 kernel: fp32 MFMA operands throughout, one workgroup
 * per sequence; the reference computes in fp32, selective.py:363-365);
 * prime_selective_prefill_qknorm takes BF16 only.  log_decay fp32 [B, H, L] contiguous = log l_t
 * (natural log, <= 0), k_scale fp32 [H] = beta_h; state_in may be NULL (zero);
 * same y, state_out, workspace rules as prime_chunked_prefill (whose
 * workspace size applies).  Replaces the parallel branch (selective.py:
 * 414-440), which builds the full [L, L] decay matrix; the reference branch
 * ignores an incoming state, a caller reproducing it passes NULL.
 *
 * prime_selective_decode_step: one token; the decays come from `gate`
 * (below), k_scale [H]; norm (may be NULL) as for prime_decode_step_qknorm
 * (the module's QK LayerNorm and q scale applied to raw projections).
 * Replaces selective.py:384-409.
 */
/*
 * prime_selective_log_decay: the per-token log decays prime_selective_prefill
 * takes, from the step-size pre-activations s = delta_proj(x): Delta =
 * clamp(softplus(s), step_min, step_max), each stage rounded to step_dtype
 * as the module's tensors are (selective.py:368), and
 * log_decay[b, h, t] = -Delta / tau[h] (the exponent of selective.py:414-416's
 * decay matrix per token), fp32 [B, H, L] contiguous.  s element (b, t, h)
 * at step + b * step_sb + t * step_sl + h (elements of step_dtype); tau fp32
 * [H]; log_decay must not overlap step or tau.
 */
int prime_selective_log_decay(const void *step, int step_dtype, int64_t step_sb, int64_t step_sl, const float *tau,
                              float step_min, float step_max, int B, int H, int L, float *log_decay, void *stream);

typedef struct prime_selective_gate {
    /* either l_t per (sequence, head), fp32 [B, H] contiguous ... */
    const float *decay;
    /* ... or (decay == NULL) the step-size pre-activations delta_proj(x):
       element (b, h) at step + b * step_sb + h, of step_dtype; the kernel
       forms Delta = clamp(softplus(.), step_min, step_max) rounded to
       step_dtype as the module's tensors are (selective.py:368), and
       l = exp(-Delta / tau[h]) (selective.py:386) */
    const void *step;
    int32_t step_dtype;
    int32_t reserved;
    int64_t step_sb;
    const float *tau;  /* [H] */
    float step_min, step_max;
} prime_selective_gate_t;
int prime_selective_prefill(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v, int B,
                            int H, int H_kv, int L, int D, const float *log_decay, const float *k_scale, float eps,
                            const prime_state_t *state_in, const prime_tensor_t *y, const prime_state_t *state_out,
                            void *workspace, size_t workspace_bytes, void *stream);
/* prime_selective_prefill with the module's QK LayerNorm and scale applied
 * on load by `norm` (selective.py:358-362), as prime_chunked_prefill_qknorm. */
int prime_selective_prefill_qknorm(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                                   int B, int H, int H_kv, int L, int D, const float *log_decay,
                                   const float *k_scale, float eps, const prime_qk_norm_t *norm,
                                   const prime_state_t *state_in, const prime_tensor_t *y,
                                   const prime_state_t *state_out, void *workspace, size_t workspace_bytes,
                                   void *stream);
int prime_selective_decode_step(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v, int B,
                                int H, int H_kv, int D, const prime_selective_gate_t *gate, const float *k_scale,
                                float eps, const prime_qk_norm_t *norm, const prime_state_t *state_in,
                                const prime_state_t *state_out, const prime_tensor_t *y, void *stream);

/*
 * Fragment layout and the decode step's projections.  No counterpart in the
 * reference: they are the MI355X form of the one-token step of
 * PrimeForCausalLM (model.py:101-118 per block, model.py:160 for the lm_head,
 * model.py:230-231 for the greedy token), where each projection sees only a
 * few hundred rows.
 *
 * Fragment layout of a bf16 matrix X[R, K] (K a multiple of 32; R padded to
 * prime_frag_rows(R) = R rounded up to a multiple of 32, padding rows zero or
 * ignored): 16 x 32 blocks in row-block-major order, each block the 64 lane
 * slots of 8 elements of one MFMA operand,
 *   X(r, k) at ((r/16) (K/32) + k/32) * 512 + (r%16 + 16 ((k%32)/8)) * 8 + k%8.
 *
 * prime_pack_frag: out (fragment layout, prime_frag_rows(M) x K) <- M rows of
 * the row-major bf16 matrix src (row stride ld, src_rows rows): row r is src
 * row rows[r] (an embedding gather; ids outside [0, src_rows) give a zero
 * row) or row r when rows is NULL.  Weights are packed once; the step packs
 * its token embeddings per call.
 *
 * prime_linear_frag: y = epilogue(s . (x w^T) + bias) for x (fragment layout,
 * prime_frag_rows(M) x K) and w (fragment layout, N x K), bf16, fp32
 * accumulation, K = 256 x {1, 2, 3, 4, 6, 12}, N a multiple of 16.
 *   flags PRIME_LINEAR_RMS: s = rsqrt(mean_k x^2 + rms_eps) per row (the
 *     RMSNorm before the projection, its weight multiplied into w's columns);
 *     otherwise s = 1.  bias: fp32 [N] or NULL.  The product is rounded to
 *     bf16 once, then
 *   epilogue PRIME_EPILOGUE_GELU: exact-erf GELU, rounded again;
 *   epilogue PRIME_EPILOGUE_RESIDUAL: y = r + product, rounded (r in y's
 *     layout; r == y updates in place).
 *   flags PRIME_LINEAR_OUT_FRAG: y (and r) in the fragment layout
 *     (prime_frag_rows(M) x N, N a multiple of 32); otherwise y row-major
 *     [M, ldy], 8-byte aligned rows.
 *   tokens (row-major output only): the greedy token of every row, argmax of
 *     the rounded products (first index of the largest, NaN largest), into
 *     int64 [M]; y may then be NULL (no logits written).  Needs a workspace
 *     of prime_linear_frag_workspace_size(M, N, K) bytes.
 * y must not overlap x or w.
 */
#define PRIME_LINEAR_RMS      1u
#define PRIME_LINEAR_OUT_FRAG 2u
int prime_frag_rows(int M);
int prime_pack_frag(const void *src, int64_t ld, int64_t src_rows, const int64_t *rows, int M, int K, void *out,
                    void *stream);
size_t prime_linear_frag_workspace_size(int M, int N, int K);
int prime_linear_frag(const void *x, const void *w, const void *r, void *y, int M, int N, int K, int64_t ldy,
                      int epilogue, unsigned flags, float rms_eps, const float *bias, int64_t *tokens,
                      void *workspace, size_t workspace_bytes, void *stream);

/*
 * Greedy token choice of the generate loop (model.py:230-231, argmax over the
 * vocabulary at temperature 0): out[i] = the first index j of the largest
 * logits[i, j], NaN counting as the largest value (torch.argmax's answer).
 * logits: n rows of `vocab` elements (F32 / BF16 / F16), row i starting
 * stride_n elements after row i-1 (stride_n >= vocab); out: int64 [n].
 */
int prime_argmax(const void *logits, int dtype, int n, int vocab, int64_t stride_n, int64_t *out,
                 void *stream);

/*
 * Hybrid window-PRIME pieces (hybrid.py:98-170 calls them through the JIT
 * extension of prime_cpp_kernel.cpp).  The reference's prime_prefill_cpp
 * (prime_cpp_kernel.cpp:6-46) is prime_chunked_prefill with eps = 1e-3 and a
 * zero initial state.
 *
 * prime_accumulate replaces prime_accumulate_evicted_cpp
 * (prime_cpp_kernel.cpp:48-83): the moment state of L tokens of k/v
 * ([B, H_kv, L, D], BF16 or F32, 16-byte rows), no queries and no readout.
 * state_in = NULL starts from zeros (the reference always does); otherwise
 * the tokens are appended to state_in, and state_out may equal state_in.
 * workspace (16-byte aligned) must hold at least B*H*kSlot bytes with
 * kSlot = 33,792 (one per sequence); prime_accumulate_workspace_size() bytes
 * let the sequences split into segments that run in parallel.
 */
int prime_accumulate(const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv, int L, int D,
                     const float *decay, const prime_state_t *state_in, const prime_state_t *state_out,
                     void *workspace, size_t workspace_bytes, void *stream);
size_t prime_accumulate_workspace_size(int B, int H, int L);

/*
 * prime_accumulate without a workspace argument: it allocates nothing.  No
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The segment slots live in a fixed device array of
 * PRIME_NOALLOC_SCRATCH_BYTES inside the library (one per device, held until
 * the process ends); the call needs one 33,792-byte slot per (sequence, head)
 * and fails with PRIME_ERR_INVALID_ARG when B * H exceeds 992.  Within that
 * array the segment plan is the one prime_accumulate picks for a workspace of
 * the same size.  All calls on one device share the array: calls that overlap
 * in time on one device (different streams or threads) race and must be
 * ordered by the caller.  Other arguments and results as prime_accumulate.
 */
#define PRIME_NOALLOC_SCRATCH_BYTES (32u << 20)
int prime_accumulate_noalloc(const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv, int L,
                             int D, const float *decay, const prime_state_t *state_in,
                             const prime_state_t *state_out, void *stream);

/*
 * Backward of prime_chunked_prefill: the reverse-mode derivative the reference
 * obtains from torch autograd when it trains through its prefill
 * (tests/test_attention.py:50-62 through attention.py:77-210 and
 * chunked_ssd.py:48-184).  For output adjoints dy [B, H, L, D] (and
 * dstate_out, the adjoint of the final state; NULL = 0) it writes
 *   dq, dk, dv   [B, H, L, D] (one dtype and one set of strides for the three)
 *   dstate_in    the adjoint of state_in (NULL: not written)
 * with the clamp's gradient passing where den >= eps, as torch's clamp.
 * q (pre-scaled), k, v, decay, eps and state_in are the forward's arguments.
 * k/v must have one head per query head (H_kv == H: the reference module
 * expands grouped k/v before the recurrence, attention.py:92-94).  With
 * PRIME_FLAG_DENSE_CLAMP and an incoming state the derivative is that of the
 * dense branch's double clamp (attention.py:177-185): the inner clamp gates
 * the call's own tokens, the outer one the incoming state's term (without a
 * state the two clamps are the same).  BF16 inputs run on bf16 MFMA operands (fp32
 * accumulation); F32 inputs run fp32 passes (fp32 MFMA operands throughout,
 * one workgroup per sequence, as the reference differentiates in fp32).
 * workspace (16-byte aligned): at least B*H*L*8 bytes (per-token
 * denominators; rounded up to 256), plus B*H*528 bytes for
 * PRIME_FLAG_DENSE_CLAMP with a state; with prime_chunked_prefill_backward_workspace_size()
 * bytes, few long sequences are split into segments that run in parallel
 * (segment-entry states by the forward's state-only pass, dual states by a
 * reverse scan).  Results agree either way.
 */
int prime_chunked_prefill_backward(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                                   int B, int H, int H_kv, int L, int D, const float *decay, float eps,
                                   unsigned flags, const prime_state_t *state_in, const prime_tensor_t *dy,
                                   const prime_state_t *dstate_out, const prime_tensor_t *dq,
                                   const prime_tensor_t *dk, const prime_tensor_t *dv,
                                   const prime_state_t *dstate_in, void *workspace, size_t workspace_bytes,
                                   void *stream);
size_t prime_chunked_prefill_backward_workspace_size(int B, int H, int L);

/*
 * prime_selective_prefill_backward: the adjoint of prime_selective_prefill
 * (torch autograd through selective.py:414-440, and through the step branch
 * :384-409 for a call with an incoming state), F32 q/k/v (convert bf16 inputs
 * first; the passes are the fp32 backward's, one workgroup per sequence).
 * Inputs as for prime_selective_prefill: log_decay fp32 [B,H,L] (log lambda_t,
 * contiguous), k_scale fp32 [H] (beta; the key enters as beta k), state_in in
 * the selective convention (S2, K2 carry the 1/2), or NULL; dy; dstate_out
 * (the final state's adjoint, selective convention) or NULL.  Outputs: dq, dk,
 * dv (one dtype and stride set), dstate_in (or NULL), d_log_decay fp32
 * [B,H,L] (the adjoint of log_decay: every later token's decay factor
 * e^(c_i - c_j) contains log lambda_t, so d_log_decay[t] sums, over the
 * tokens i >= t, phi_q'(i).dphi_q'(i) - phi_k'(i).dphi_k'(i) with the
 * features [1, q, q*q] and [1, beta k, beta^2 k*k/2], plus
 * <dstate_out, state_out>), d_k_scale fp32 [B,H] (the adjoint of k_scale per
 * sequence: sum over the batch for the [H] parameter).  H_kv == H.
 * workspace (16-byte aligned): prime_selective_prefill_backward_workspace_size.
 */
int prime_selective_prefill_backward(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                                     int B, int H, int H_kv, int L, int D, const float *log_decay,
                                     const float *k_scale, float eps, const prime_state_t *state_in,
                                     const prime_tensor_t *dy, const prime_state_t *dstate_out,
                                     const prime_tensor_t *dq, const prime_tensor_t *dk, const prime_tensor_t *dv,
                                     const prime_state_t *dstate_in, float *d_log_decay, float *d_k_scale,
                                     void *workspace, size_t workspace_bytes, void *stream);
size_t prime_selective_prefill_backward_workspace_size(int B, int H, int L);

/*
 * prime_decode_readout replaces prime_query_step_cpp (prime_cpp_kernel.cpp:85-100):
 * y = (S0 + S1^T q + 1/2 S2^T q^2) / max(K0 + q.K1 + 1/2 q^2.K2, eps) against
 * `state` as it is (the reference's eps is 1e-3); the state is not written.
 * q, y: [B, H, D] views (stride_l unused).
 */
int prime_decode_readout(const prime_tensor_t *q, int B, int H, int D, float eps, const prime_state_t *state,
                         const prime_tensor_t *y, void *stream);

/*
 * prime_decode_update replaces prime_step_evict_update_cpp
 * (prime_cpp_kernel.cpp:102-117): one token of k/v ([B, H_kv, D]) appended
 * to the state, no readout.  The reference updates in place: pass
 * state_out == state_in.  state_in = NULL starts from zeros.
 */
int prime_decode_update(const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv, int D,
                        const float *decay, const prime_state_t *state_in, const prime_state_t *state_out,
                        void *stream);

/*
 * Launch timer.  No counterpart in the reference: it serves benchmark harnesses
 * that need the device time of ONE kernel of a multi-kernel call.
 * prime_timer_enable(mask) (process-wide; bit (1 << PRIME_KERNEL_*) selects a
 * kernel, 0 disables) times every launch of the selected kernels with a pair
 * of HIP events that the dispatch itself stamps at its start and end
 * (hipExtLaunchKernel; no extra packets on the stream).  prime_timer_read waits for the recorded
 * events and returns the summed device time and launch count of one kernel
 * since the last reset.  Event objects are created while enabled (never on the
 * default, disabled path) and kept for reuse.
 */
#define PRIME_KERNEL_PREFILL_CHUNKS   0 /* fused chunk loop: y and final state */
#define PRIME_KERNEL_PREFILL_SEGMENTS 1 /* per-segment state contributions */
#define PRIME_KERNEL_SEGMENT_SCAN     2 /* exclusive scan over segments */
#define PRIME_KERNEL_DECODE           3 /* fused decode step */
#define PRIME_KERNEL_DELTA_PREP       4 /* delta rule: per-chunk solve and transfer matrices */
#define PRIME_KERNEL_DELTA_SCAN       5 /* delta rule: sequential scan over chunks */
#define PRIME_KERNEL_DELTA_STEP       6 /* delta rule: decode step */
#define PRIME_KERNEL_BWD_DQ           7 /* prefill backward: dq pass (chunks in order) */
#define PRIME_KERNEL_BWD_DKV          8 /* prefill backward: dk, dv pass (chunks in reverse) */
#define PRIME_KERNEL_BWD_DUAL         9 /* prefill backward: per-segment dual contributions */
#define PRIME_KERNEL_BWD_DUAL_SCAN   10 /* prefill backward: reverse scan over segments */
#define PRIME_KERNEL_COUNT           11

int prime_timer_enable(unsigned mask);
int prime_timer_reset(void);
int prime_timer_read(int kernel, double *total_ms, int64_t *launches);

/*
 * HBM bandwidth probe.  No counterpart in the reference: benchmark harnesses
 * use it for the achievable-bandwidth figure that kernel rooflines are read
 * against.  copy != 0: dst = src over `bytes` (read + write); copy == 0: a
 * read-only pass over src, one 16-byte word per workgroup written to dst
 * (dst must hold `blocks` x 16 bytes).  Nontemporal 16-byte loads and stores,
 * `blocks` workgroups of 256 threads in a grid-stride loop.  bytes a multiple
 * of 16, both pointers 16-byte aligned.
 */
int prime_hbm_stream(const void *src, void *dst, size_t bytes, int copy, int blocks, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PRIME_MI355X_H */
