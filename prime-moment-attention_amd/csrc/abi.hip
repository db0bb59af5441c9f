// C-ABI entry points: argument validation, error reporting and dispatch.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <mutex>
#include <random>

#include "prime_kernels.h"

namespace {

thread_local char g_err[512] = "";

// hand-off value of a paired prefill: the flag words live in a caller's
// workspace that nobody clears, so the value must not be one that leftover
// data holds by accident (small integers, token ids, float patterns, an epoch
// of another process).  High 32 bits: a per-process random nonce with bit 63
// set (never 0, the value a consumed flag is reset to); low 32 bits: a call
// counter, so that calls of one process never share a value within 2^32 calls.
unsigned long long epoch_nonce() {
    std::random_device rd;
    unsigned long long n = (static_cast<unsigned long long>(rd()) << 32) ^ rd();
    n ^= static_cast<unsigned long long>(std::chrono::steady_clock::now().time_since_epoch().count()) * 0x9E3779B97F4A7C15ull;
    n ^= reinterpret_cast<uintptr_t>(&n) * 0xC2B2AE3D27D4EB4Full;
    return (n | 0x8000000000000000ull) & 0xFFFFFFFF00000000ull;
}
const unsigned long long g_epoch_nonce = epoch_nonce();
std::atomic<unsigned int> g_epoch{0};
unsigned long long next_epoch() { return g_epoch_nonce | static_cast<unsigned long long>(++g_epoch); }

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int elem_size(int dt) { return dt == PRIME_F32 ? 4 : 2; }
bool valid_dtype(int dt) { return dt == PRIME_F32 || dt == PRIME_BF16 || dt == PRIME_F16; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// every row start of a strided view is 16-byte aligned
bool rows_aligned(const prime_tensor_t *t, bool use_l) {
    const int64_t es = elem_size(t->dtype);
    if (!aligned16(t->data)) return false;
    if ((t->stride_b * es) % 16 || (t->stride_h * es) % 16) return false;
    if (use_l && (t->stride_l * es) % 16) return false;
    return true;
}

bool overlap(const void *a, size_t na, const void *b, size_t nb) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + nb && y < x + na;
}

// state_out must be exactly state_in (in place) or disjoint from it.
int check_state_alias(const prime_state_t *in, const prime_state_t *out, size_t BH, int D,
                      bool *inplace) {
    *inplace = false;
    if (!in || !out) return PRIME_OK;
    const float *pi[6] = {in->s0, in->s1, in->s2, in->k0, in->k1, in->k2};
    const float *po[6] = {out->s0, out->s1, out->s2, out->k0, out->k1, out->k2};
    const size_t n[6] = {BH * D, BH * D * D, BH * D * D, BH, BH * D, BH * D};
    bool all_same = true, any_same = false;
    for (int i = 0; i < 6; ++i) {
        all_same &= pi[i] == po[i];
        any_same |= pi[i] == po[i];
    }
    if (all_same) {
        *inplace = true;
        return PRIME_OK;
    }
    for (int i = 0; i < 6; ++i)
        for (int j = 0; j < 6; ++j)
            if (overlap(pi[i], n[i] * 4, po[j], n[j] * 4))
                return fail(PRIME_ERR_ALIAS, "state_out buffer %d overlaps state_in buffer %d "
                            "(only a fully in-place state is allowed)", j, i);
    (void)any_same;
    return PRIME_OK;
}

int check_state(const prime_state_t *s, const char *name) {
    if (!s) return PRIME_OK;
    const float *p[6] = {s->s0, s->s1, s->s2, s->k0, s->k1, s->k2};
    for (int i = 0; i < 6; ++i) {
        if (!p[i]) return fail(PRIME_ERR_INVALID_ARG, "%s: buffer %d is null", name, i);
        if ((reinterpret_cast<uintptr_t>(p[i]) & 3u) != 0)
            return fail(PRIME_ERR_MISALIGNED, "%s: buffer %d is not 4-byte aligned", name, i);
    }
    if (!aligned16(s->s1) || !aligned16(s->s2))
        return fail(PRIME_ERR_MISALIGNED, "%s: S1/S2 must be 16-byte aligned", name);
    return PRIME_OK;
}

int check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) return fail(PRIME_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return PRIME_OK;
}

// Head dims below 64 (generic_d.hip): argument descriptor shared by the
// prefill, the decode step and the backward.
int generic_args(prime::GenericArgs &a, const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                 int B, int H, int H_kv, int L, int D, const float *decay, float eps, unsigned flags,
                 const prime_state_t *state_in, const prime_state_t *state_out) {
    if (D < 1 || D > prime::kGenericMaxD)
        return fail(PRIME_ERR_UNSUPPORTED_DIM, "head dim %d unsupported (64, or 1 .. %d)", D, prime::kGenericMaxD);
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv || L <= 0)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d L=%d", B, H, H_kv, L);
    if (flags & ~PRIME_FLAG_DENSE_CLAMP) return fail(PRIME_ERR_INVALID_ARG, "unknown flags 0x%x", flags);
    if (!valid_dtype(q->dtype) || !valid_dtype(k->dtype) || !valid_dtype(v->dtype))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported q/k/v dtype");
    int rc;
    if ((rc = check_state(state_in, "state_in")) || (rc = check_state(state_out, "state_out"))) return rc;
    bool inplace;
    if ((rc = check_state_alias(state_in, state_out, static_cast<size_t>(B) * H, D, &inplace))) return rc;
    a.q = q->data; a.k = k->data; a.v = v->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.q_sl = q->stride_l;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_sl = k->stride_l;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_sl = v->stride_l;
    a.dt_q = q->dtype; a.dt_k = k->dtype; a.dt_v = v->dtype;
    a.B = B; a.H = H; a.group = H / H_kv; a.L = L; a.D = D;
    a.decay = decay; a.eps = eps;
    a.dense_clamp = (flags & PRIME_FLAG_DENSE_CLAMP) ? 1 : 0;
    if (state_in) {
        a.s0i = state_in->s0; a.s1i = state_in->s1; a.s2i = state_in->s2;
        a.k0i = state_in->k0; a.k1i = state_in->k1; a.k2i = state_in->k2;
    }
    if (state_out) {
        a.s0o = state_out->s0; a.s1o = state_out->s1; a.s2o = state_out->s2;
        a.k0o = state_out->k0; a.k1o = state_out->k1; a.k2o = state_out->k2;
    }
    return PRIME_OK;
}

int generic_norm(prime::GenericArgs &a, const prime_qk_norm_t *norm) {
    if (!norm) return PRIME_OK;
    if ((norm->q_weight == nullptr) != (norm->q_bias == nullptr) ||
        (norm->k_weight == nullptr) != (norm->k_bias == nullptr))
        return fail(PRIME_ERR_INVALID_ARG, "QK-norm: LayerNorm weight without bias or bias without weight");
    if ((norm->q_weight || norm->k_weight) && !valid_dtype(norm->dtype))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported norm dtype");
    a.qk_norm = 1;
    a.qn_w = norm->q_weight; a.qn_b = norm->q_bias; a.kn_w = norm->k_weight; a.kn_b = norm->k_bias;
    a.dt_norm = norm->dtype; a.ln_eps = norm->eps; a.q_scale = norm->q_scale;
    return PRIME_OK;
}

}  // namespace

extern "C" {

int prime_abi_version(void) { return PRIME_ABI_VERSION; }

const char *prime_last_error(void) { return g_err; }

}  // extern "C"

namespace {

int decode_impl(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv,
                int D, const float *decay, float eps, const prime_qk_norm_t *norm, const prime_state_t *state_in,
                const prime_state_t *state_out, const prime_tensor_t *y, void *stream,
                const prime_selective_gate_t *gate = nullptr, const float *k_scale = nullptr) {
    g_err[0] = 0;
    const bool selective = gate != nullptr;
    if (!q || !k || !v || !y || !q->data || !k->data || !v->data || !y->data || !(decay || selective) || !state_out ||
        (selective && !k_scale))
        return fail(PRIME_ERR_INVALID_ARG, "prime_decode_step: null argument");
    if (D != prime::kD) {
        // head dims below 64: the generic recurrence over one token
        if (!valid_dtype(y->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported y dtype");
        if (selective && !gate->decay && (!gate->step || !gate->tau || !valid_dtype(gate->step_dtype)))
            return fail(PRIME_ERR_INVALID_ARG, "selective gate: give decay_bh, or step (a supported dtype) and tau");
        if (y->layout != PRIME_LAYOUT_STRIDED)
            return fail(PRIME_ERR_INVALID_ARG, "head dim %d: y must be a strided view", D);
        prime::GenericArgs g{};
        int rc;
        if ((rc = generic_args(g, q, k, v, B, H, H_kv, 1, D, decay, eps, 0u, state_in, state_out)) ||
            (rc = generic_norm(g, norm)))
            return rc;
        g.y = y->data; g.dt_y = y->dtype; g.y_sb = y->stride_b; g.y_sh = y->stride_h; g.y_sl = 0;
        if (selective) {
            g.selective = 1;
            g.k_scale = k_scale;
            g.decay_bh = gate->decay;
            g.step = gate->step; g.step_sb = gate->step_sb; g.dt_step = gate->step_dtype;
            g.tau = gate->tau; g.step_min = gate->step_min; g.step_max = gate->step_max;
        }
        return check_hip(prime::launch_generic_prefill(g, static_cast<hipStream_t>(stream)), "decode launch");
    }
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d", B, H, H_kv);
    if (!valid_dtype(q->dtype) || !valid_dtype(k->dtype) || !valid_dtype(v->dtype) || !valid_dtype(y->dtype))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dtype");
    int rc;
    if ((rc = check_state(state_in, "state_in")) || (rc = check_state(state_out, "state_out"))) return rc;
    bool inplace;
    if ((rc = check_state_alias(state_in, state_out, static_cast<size_t>(B) * H, D, &inplace))) return rc;

    prime::DecodeArgs a{};
    if (norm) {
        a.qn_w = norm->q_weight; a.qn_b = norm->q_bias; a.kn_w = norm->k_weight; a.kn_b = norm->k_bias;
        a.dt_norm = norm->dtype; a.ln_eps = norm->eps;
    }
    a.q = q->data; a.k = k->data; a.v = v->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h;
    a.dt_q = q->dtype; a.dt_k = k->dtype; a.dt_v = v->dtype;
    a.B = B; a.H = H; a.group = H / H_kv;
    a.decay = decay; a.eps = eps;
    if (state_in) {
        a.s0i = state_in->s0; a.s1i = state_in->s1; a.s2i = state_in->s2;
        a.k0i = state_in->k0; a.k1i = state_in->k1; a.k2i = state_in->k2;
    }
    a.s0o = state_out->s0; a.s1o = state_out->s1; a.s2o = state_out->s2;
    a.k0o = state_out->k0; a.k1o = state_out->k1; a.k2o = state_out->k2;
    a.y = y->data; a.dt_y = y->dtype; a.y_sb = y->stride_b; a.y_sh = y->stride_h;
    if (y->layout == PRIME_LAYOUT_FRAG) {
        if (y->dtype != PRIME_BF16 || (H * D) % 32 || !aligned16(y->data))
            return fail(PRIME_ERR_INVALID_ARG, "fragment-layout y: bf16, H*D a multiple of 32, 16-byte aligned");
        a.y_frag = 1;
        a.y_ks = H * D / 32;
    } else if (y->layout != PRIME_LAYOUT_STRIDED) {
        return fail(PRIME_ERR_INVALID_ARG, "unknown y layout %d", y->layout);
    }
    a.q_scale = norm ? norm->q_scale : 1.0f;
    a.k_scale = k_scale; a.selective = selective ? 1 : 0;
    if (gate) {
        a.decay_bh = gate->decay;
        if (!gate->decay) {
            if (!gate->step || !gate->tau) return fail(PRIME_ERR_INVALID_ARG, "selective gate: null step or tau");
            if (!valid_dtype(gate->step_dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported step dtype");
            if (!(gate->step_min > 0.f) || !(gate->step_max >= gate->step_min))
                return fail(PRIME_ERR_INVALID_ARG, "selective gate: bad step bounds");
            a.step = gate->step; a.step_sb = gate->step_sb; a.dt_step = gate->step_dtype; a.tau = gate->tau;
            a.step_min = gate->step_min; a.step_max = gate->step_max;
        }
    }
    return check_hip(prime::launch_decode_step(a, static_cast<hipStream_t>(stream)), "decode launch");
}

}  // namespace

extern "C" {

int prime_decode_step(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                      int B, int H, int H_kv, int D, const float *decay, float eps,
                      const prime_state_t *state_in, const prime_state_t *state_out,
                      const prime_tensor_t *y, void *stream) {
    return decode_impl(q, k, v, B, H, H_kv, D, decay, eps, nullptr, state_in, state_out, y, stream);
}

int prime_decode_step_qknorm(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                             int B, int H, int H_kv, int D, const float *decay, float eps,
                             const prime_qk_norm_t *norm, const prime_state_t *state_in,
                             const prime_state_t *state_out, const prime_tensor_t *y, void *stream) {
    g_err[0] = 0;
    if (!norm) return fail(PRIME_ERR_INVALID_ARG, "prime_decode_step_qknorm: null norm");
    if (norm->q_weight && (!norm->q_bias || !norm->k_weight || !norm->k_bias))
        return fail(PRIME_ERR_INVALID_ARG, "prime_decode_step_qknorm: LayerNorm weight without bias");
    if (!valid_dtype(norm->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported norm dtype");
    return decode_impl(q, k, v, B, H, H_kv, D, decay, eps, norm, state_in, state_out, y, stream);
}

int prime_add_rmsnorm(void *x, const void *delta, const void *weight, void *out, int rows, int hidden,
                      int dtype, float eps, void *stream) {
    g_err[0] = 0;
    if (!x || !weight || !out) return fail(PRIME_ERR_INVALID_ARG, "prime_add_rmsnorm: null argument");
    if (rows <= 0 || hidden <= 0 || hidden % 4)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes rows=%d hidden=%d (hidden must be a multiple of 4)", rows,
                    hidden);
    if (hidden > 4 * 64 * prime::kNormMaxGroups)
        return fail(PRIME_ERR_INVALID_ARG, "hidden=%d above the supported %d", hidden, 4 * 64 * prime::kNormMaxGroups);
    if (!valid_dtype(dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dtype");
    const uintptr_t al = 4 * elem_size(dtype) - 1;  // one 4-element group per load
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(delta) | reinterpret_cast<uintptr_t>(weight) |
         reinterpret_cast<uintptr_t>(out)) & al)
        return fail(PRIME_ERR_MISALIGNED, "x/delta/weight/out must be aligned to 4 elements");
    const size_t n = static_cast<size_t>(rows) * hidden * elem_size(dtype);
    if (delta && overlap(delta, n, x, n)) return fail(PRIME_ERR_ALIAS, "delta overlaps x");
    if (out != x && overlap(out, n, x, n)) return fail(PRIME_ERR_ALIAS, "out overlaps x without being x");
    prime::RmsNormArgs a{};
    a.x = x; a.delta = delta; a.weight = weight; a.out = out;
    a.rows = rows; a.hidden = hidden; a.dt = dtype; a.eps = eps;
    return check_hip(prime::launch_add_rmsnorm(a, static_cast<hipStream_t>(stream)), "add_rmsnorm launch");
}

int prime_gelu(const void *x, void *y, int64_t n, int dtype, void *stream) {
    g_err[0] = 0;
    if (!x || !y) return fail(PRIME_ERR_INVALID_ARG, "prime_gelu: null argument");
    if (n < 0) return fail(PRIME_ERR_INVALID_ARG, "bad size n=%lld", static_cast<long long>(n));
    if (!valid_dtype(dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dtype");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15)
        return fail(PRIME_ERR_MISALIGNED, "x and y must be 16-byte aligned");
    const size_t bytes = static_cast<size_t>(n) * elem_size(dtype);
    if (y != x && overlap(x, bytes, y, bytes)) return fail(PRIME_ERR_ALIAS, "y overlaps x without being x");
    if (n == 0) return PRIME_OK;
    return check_hip(prime::launch_gelu(x, y, n, dtype, static_cast<hipStream_t>(stream)), "gelu launch");
}

int prime_selective_log_decay(const void *step, int step_dtype, int64_t step_sb, int64_t step_sl, const float *tau,
                              float step_min, float step_max, int B, int H, int L, float *log_decay, void *stream) {
    g_err[0] = 0;
    if (!step || !tau || !log_decay) return fail(PRIME_ERR_INVALID_ARG, "prime_selective_log_decay: null argument");
    if (B <= 0 || H <= 0 || L <= 0 || step_sb < 0 || step_sl < 0)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d L=%d step_sb=%lld step_sl=%lld", B, H, L,
                    static_cast<long long>(step_sb), static_cast<long long>(step_sl));
    if (!valid_dtype(step_dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported step dtype");
    if (!(step_min > 0.f) || !(step_max >= step_min))
        return fail(PRIME_ERR_INVALID_ARG, "step bounds must satisfy 0 < step_min <= step_max");
    const int64_t es = elem_size(step_dtype);
    if (reinterpret_cast<uintptr_t>(step) % es || (reinterpret_cast<uintptr_t>(tau) & 3) ||
        (reinterpret_cast<uintptr_t>(log_decay) & 3))
        return fail(PRIME_ERR_MISALIGNED, "step, tau or log_decay misaligned");
    const size_t nout = static_cast<size_t>(B) * H * L * sizeof(float);
    const size_t nstep = static_cast<size_t>((B - 1) * step_sb + (L - 1) * step_sl + H) * es;
    if (overlap(log_decay, nout, step, nstep) || overlap(log_decay, nout, tau, static_cast<size_t>(H) * sizeof(float)))
        return fail(PRIME_ERR_ALIAS, "log_decay overlaps step or tau");
    return check_hip(prime::launch_selective_log_decay(step, step_dtype, step_sb, step_sl, tau, step_min, step_max, B,
                                                       H, L, log_decay, static_cast<hipStream_t>(stream)),
                     "selective log decay launch");
}

int prime_head_layernorm(const prime_tensor_t *x, const prime_tensor_t *out, int B, int H, int L, int D,
                         const void *weight, const void *bias, int param_dtype, float ln_eps, float scale,
                         void *stream) {
    g_err[0] = 0;
    if (!x || !out || !x->data || !out->data) return fail(PRIME_ERR_INVALID_ARG, "prime_head_layernorm: null argument");
    if (D != prime::kD && (D < 1 || D > prime::kGenericMaxD))
        return fail(PRIME_ERR_UNSUPPORTED_DIM, "head dim %d unsupported (64, or 1 .. %d)", D, prime::kGenericMaxD);
    if (B <= 0 || H <= 0 || L <= 0) return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d L=%d", B, H, L);
    if (static_cast<int64_t>(B) * H * L >= (int64_t(1) << 31))
        return fail(PRIME_ERR_INVALID_ARG, "B*H*L = %lld rows exceeds 2^31 - 1",
                    static_cast<long long>(static_cast<int64_t>(B) * H * L));
    if (!valid_dtype(x->dtype) || out->dtype != x->dtype)
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "x and out must share one supported dtype");
    if ((weight == nullptr) != (bias == nullptr))
        return fail(PRIME_ERR_INVALID_ARG, "LayerNorm weight and bias must both be given or both be null");
    if (weight && !valid_dtype(param_dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported parameter dtype");
    if (D == prime::kD && (!rows_aligned(x, true) || !rows_aligned(out, true)))
        return fail(PRIME_ERR_MISALIGNED, "x/out rows must start on 16-byte boundaries");
    const int64_t es = elem_size(x->dtype);
    auto span = [&](const prime_tensor_t *t) {
        return static_cast<size_t>(((B - 1) * t->stride_b + (H - 1) * t->stride_h + (L - 1) * t->stride_l + D) * es);
    };
    const bool same = out->data == x->data && out->stride_b == x->stride_b && out->stride_h == x->stride_h &&
                      out->stride_l == x->stride_l;
    if (!same && overlap(out->data, span(out), x->data, span(x)))
        return fail(PRIME_ERR_ALIAS, "out overlaps x without being the same view");
    prime::HeadNormArgs a{};
    a.x = x->data; a.out = out->data; a.weight = weight; a.bias = bias;
    a.x_sb = x->stride_b; a.x_sh = x->stride_h; a.x_sl = x->stride_l;
    a.o_sb = out->stride_b; a.o_sh = out->stride_h; a.o_sl = out->stride_l;
    a.B = B; a.H = H; a.L = L; a.dt = x->dtype; a.dt_norm = param_dtype;
    a.ln_eps = ln_eps; a.scale = scale; a.D = D;
    if (D != prime::kD)
        return check_hip(prime::launch_generic_head_layernorm(a, static_cast<hipStream_t>(stream)),
                         "head_layernorm launch");
    return check_hip(prime::launch_head_layernorm(a, static_cast<hipStream_t>(stream)), "head_layernorm launch");
}

namespace {

int linear_checks(const char *who, const void *x, const void *w, const void *y, int M, int N, int K, int64_t ldx,
                  int64_t ldw, int64_t ldy, int dtype) {
    if (!x || !w || !y) return fail(PRIME_ERR_INVALID_ARG, "%s: null argument", who);
    if (M <= 0 || N <= 0 || K <= 0 || K % 64 || N % 4)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes M=%d N=%d K=%d (K a multiple of 64, N of 4)", M, N, K);
    if (ldx < K || ldw < K || ldy < N) return fail(PRIME_ERR_INVALID_ARG, "row strides below the row lengths");
    if (dtype != PRIME_BF16) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "%s: BF16 only", who);
    if (!aligned16(x) || !aligned16(w) || (ldx % 8) || (ldw % 8))
        return fail(PRIME_ERR_MISALIGNED, "x and w rows must start on 16-byte boundaries");
    if ((reinterpret_cast<uintptr_t>(y) & 7) || (ldy % 4))
        return fail(PRIME_ERR_MISALIGNED, "y rows must start on 8-byte boundaries");
    const size_t nx = static_cast<size_t>((M - 1) * ldx + K) * 2, nw = static_cast<size_t>((N - 1) * ldw + K) * 2,
                 ny = static_cast<size_t>((M - 1) * ldy + N) * 2;
    if (overlap(y, ny, x, nx) || overlap(y, ny, w, nw)) return fail(PRIME_ERR_ALIAS, "y overlaps x or w");
    return PRIME_OK;
}

}  // namespace

int prime_linear(const void *x, const void *w, void *y, int M, int N, int K, int64_t ldx, int64_t ldw,
                 int64_t ldy, int dtype, int epilogue, void *stream) {
    g_err[0] = 0;
    if (epilogue != PRIME_EPILOGUE_NONE && epilogue != PRIME_EPILOGUE_GELU)
        return fail(PRIME_ERR_INVALID_ARG, "unknown epilogue %d", epilogue);
    int rc;
    if ((rc = linear_checks("prime_linear", x, w, y, M, N, K, ldx, ldw, ldy, dtype))) return rc;
    prime::LinearArgs a{};
    a.x = x; a.w = w; a.y = y; a.ldx = ldx; a.ldw = ldw; a.ldy = ldy;
    a.M = M; a.N = N; a.K = K; a.epilogue = epilogue;
    return check_hip(prime::launch_linear(a, static_cast<hipStream_t>(stream)), "linear launch");
}

int prime_linear_residual(const void *x, const void *w, const void *r, void *y, int M, int N, int K,
                          int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldy, int dtype, void *stream) {
    g_err[0] = 0;
    int rc;
    if ((rc = linear_checks("prime_linear_residual", x, w, y, M, N, K, ldx, ldw, ldy, dtype))) return rc;
    if (!r) return fail(PRIME_ERR_INVALID_ARG, "prime_linear_residual: null r");
    if (ldr < N) return fail(PRIME_ERR_INVALID_ARG, "r row stride below the row length");
    if ((reinterpret_cast<uintptr_t>(r) & 7) || (ldr % 4))
        return fail(PRIME_ERR_MISALIGNED, "r rows must start on 8-byte boundaries");
    const size_t nr = static_cast<size_t>((M - 1) * ldr + N) * 2, ny = static_cast<size_t>((M - 1) * ldy + N) * 2;
    if (!(r == y && ldr == ldy) && overlap(r, nr, y, ny))
        return fail(PRIME_ERR_ALIAS, "r overlaps y (only r == y with the same row stride is allowed)");
    prime::LinearArgs a{};
    a.x = x; a.w = w; a.y = y; a.r = r; a.ldx = ldx; a.ldw = ldw; a.ldy = ldy; a.ldr = ldr;
    a.M = M; a.N = N; a.K = K; a.epilogue = PRIME_EPILOGUE_RESIDUAL;
    return check_hip(prime::launch_linear(a, static_cast<hipStream_t>(stream)), "linear launch");
}

int prime_linear_fused(const void *x, const void *w, const void *r, void *y, int M, int N, int K, int64_t ldx,
                       int64_t ldw, int64_t ldr, int64_t ldy, int dtype, int epilogue, float rms_eps,
                       void *stream) {
    g_err[0] = 0;
    int rc;
    if ((rc = linear_checks("prime_linear_fused", x, w, y, M, N, K, ldx, ldw, ldy, dtype))) return rc;
    if (epilogue != PRIME_EPILOGUE_NONE && epilogue != PRIME_EPILOGUE_GELU && epilogue != PRIME_EPILOGUE_RESIDUAL)
        return fail(PRIME_ERR_INVALID_ARG, "unknown epilogue %d", epilogue);
    if (M > 1024 || N % 32 || K % 128)
        return fail(PRIME_ERR_INVALID_ARG, "prime_linear_fused: M <= 1024, N a multiple of 32, K of 128 (M=%d N=%d K=%d)",
                    M, N, K);
    if (!(rms_eps >= 0.f)) return fail(PRIME_ERR_INVALID_ARG, "prime_linear_fused: rms_eps must be >= 0");
    if (epilogue == PRIME_EPILOGUE_RESIDUAL) {
        if (!r) return fail(PRIME_ERR_INVALID_ARG, "prime_linear_fused: null r");
        if (ldr < N) return fail(PRIME_ERR_INVALID_ARG, "r row stride below the row length");
        if ((reinterpret_cast<uintptr_t>(r) & 7) || (ldr % 4))
            return fail(PRIME_ERR_MISALIGNED, "r rows must start on 8-byte boundaries");
        const size_t nr = static_cast<size_t>((M - 1) * ldr + N) * 2, ny = static_cast<size_t>((M - 1) * ldy + N) * 2;
        if (!(r == y && ldr == ldy) && overlap(r, nr, y, ny))
            return fail(PRIME_ERR_ALIAS, "r overlaps y (only r == y with the same row stride is allowed)");
        const size_t nx = static_cast<size_t>((M - 1) * ldx + K) * 2;
        if (overlap(r, nr, x, nx) && r != y) return fail(PRIME_ERR_ALIAS, "r overlaps x");
    }
    prime::LinearArgs a{};
    a.x = x; a.w = w; a.y = y; a.r = r; a.ldx = ldx; a.ldw = ldw; a.ldy = ldy; a.ldr = ldr;
    a.M = M; a.N = N; a.K = K; a.epilogue = epilogue;
    a.rms = rms_eps > 0.f ? 1 : 0; a.rms_eps = rms_eps;
    return check_hip(prime::launch_linear_rows(a, static_cast<hipStream_t>(stream)), "linear launch");
}

int prime_pack_frag(const void *src, int64_t ld, int64_t src_rows, const int64_t *rows, int M, int K, void *out,
                    void *stream) {
    g_err[0] = 0;
    if (!src || !out) return fail(PRIME_ERR_INVALID_ARG, "prime_pack_frag: null argument");
    if (M <= 0 || K <= 0 || K % 32 || ld < K || src_rows <= 0 || (!rows && src_rows < M))
        return fail(PRIME_ERR_INVALID_ARG, "prime_pack_frag: bad sizes M=%d K=%d ld=%lld src_rows=%lld", M, K,
                    static_cast<long long>(ld), static_cast<long long>(src_rows));
    if (!aligned16(src) || (ld * 2) % 16 || !aligned16(out))
        return fail(PRIME_ERR_MISALIGNED, "prime_pack_frag: src rows and out must be 16-byte aligned");
    if (rows && (reinterpret_cast<uintptr_t>(rows) & 7)) return fail(PRIME_ERR_MISALIGNED, "rows must be 8-byte aligned");
    const int Mp = prime_frag_rows(M);
    const size_t nout = static_cast<size_t>(Mp) * K * 2;
    if (overlap(out, nout, src, static_cast<size_t>((src_rows - 1) * ld + K) * 2))
        return fail(PRIME_ERR_ALIAS, "prime_pack_frag: out overlaps src");
    return check_hip(prime::launch_pack_frag(static_cast<const uint16_t *>(src), ld, rows, M, Mp, K, src_rows,
                                             static_cast<uint16_t *>(out), static_cast<hipStream_t>(stream)),
                     "pack launch");
}

int prime_frag_rows(int M) { return M <= 0 ? 0 : (M + 31) / 32 * 32; }

size_t prime_linear_frag_workspace_size(int M, int N, int K) {
    if (M <= 0 || N <= 0 || N % 16 || K <= 0 || K % 32) return 0;
    prime::FragArgs a{};
    a.M = M; a.Mp = prime_frag_rows(M); a.N = N; a.K = K;
    prime::frag_plan(a);
    return static_cast<size_t>(a.Mp) * a.gn * sizeof(uint64_t);
}

int prime_linear_frag(const void *x, const void *w, const void *r, void *y, int M, int N, int K, int64_t ldy,
                      int epilogue, unsigned flags, float rms_eps, const float *bias, int64_t *tokens,
                      void *workspace, size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    if (!x || !w || (!y && !tokens)) return fail(PRIME_ERR_INVALID_ARG, "prime_linear_frag: null argument");
    if (flags & ~(PRIME_LINEAR_RMS | PRIME_LINEAR_OUT_FRAG))
        return fail(PRIME_ERR_INVALID_ARG, "prime_linear_frag: unknown flags 0x%x", flags);
    const bool out_frag = (flags & PRIME_LINEAR_OUT_FRAG) != 0;
    if (M <= 0 || N <= 0 || N % 16 || (out_frag && N % 32))
        return fail(PRIME_ERR_INVALID_ARG, "prime_linear_frag: M > 0, N a multiple of 16 (32 for a fragment-layout "
                    "output) (M=%d N=%d)", M, N);
    if (!prime::frag_k_supported(K))
        return fail(PRIME_ERR_INVALID_ARG, "prime_linear_frag: K must be 256 x {1, 2, 3, 4, 6, 12} (K=%d)", K);
    if (epilogue != PRIME_EPILOGUE_NONE && epilogue != PRIME_EPILOGUE_GELU && epilogue != PRIME_EPILOGUE_RESIDUAL)
        return fail(PRIME_ERR_INVALID_ARG, "unknown epilogue %d", epilogue);
    if (epilogue == PRIME_EPILOGUE_RESIDUAL && !r) return fail(PRIME_ERR_INVALID_ARG, "prime_linear_frag: null r");
    if ((flags & PRIME_LINEAR_RMS) && !(rms_eps >= 0.f))
        return fail(PRIME_ERR_INVALID_ARG, "prime_linear_frag: rms_eps must be >= 0");
    if (!aligned16(x) || !aligned16(w)) return fail(PRIME_ERR_MISALIGNED, "x and w must be 16-byte aligned");
    const int Mp = prime_frag_rows(M);
    size_t ny = 0;
    if (y || r) {
        if (out_frag) {
            if ((y && !aligned16(y)) || (r && !aligned16(r)))
                return fail(PRIME_ERR_MISALIGNED, "fragment-layout y and r must be 16-byte aligned");
            ny = static_cast<size_t>(Mp) * N * 2;
        } else {
            if (ldy < N) return fail(PRIME_ERR_INVALID_ARG, "y row stride below the row length");
            if (((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(r)) & 7) || ldy % 4)
                return fail(PRIME_ERR_MISALIGNED, "row-major y and r rows must start on 8-byte boundaries");
            ny = static_cast<size_t>((M - 1) * ldy + N) * 2;
        }
    }
    const size_t nx = static_cast<size_t>(Mp) * K * 2, nw = static_cast<size_t>(N) * K * 2;
    if (y && (overlap(y, ny, x, nx) || overlap(y, ny, w, nw)))
        return fail(PRIME_ERR_ALIAS, "prime_linear_frag: y overlaps x or w");
    if (r && r != y && y && overlap(r, ny, y, ny))
        return fail(PRIME_ERR_ALIAS, "r overlaps y (only r == y is allowed)");
    prime::FragArgs a{};
    a.x = static_cast<const uint16_t *>(x); a.w = static_cast<const uint16_t *>(w);
    a.r = static_cast<const uint16_t *>(r); a.y = static_cast<uint16_t *>(y); a.bias = bias;
    a.M = M; a.Mp = Mp; a.N = N; a.K = K; a.KS = K / 32; a.ldy = ldy;
    a.epilogue = epilogue; a.rms = (flags & PRIME_LINEAR_RMS) ? 1 : 0; a.out_frag = out_frag ? 1 : 0;
    a.rms_eps = rms_eps;
    prime::frag_plan(a);
    if (tokens) {
        if (out_frag) return fail(PRIME_ERR_INVALID_ARG, "prime_linear_frag: argmax with a row-major output only");
        if (reinterpret_cast<uintptr_t>(tokens) & 7) return fail(PRIME_ERR_MISALIGNED, "tokens must be 8-byte aligned");
        const size_t need = static_cast<size_t>(Mp) * a.gn * sizeof(uint64_t);
        if (!workspace || workspace_bytes < need)
            return fail(PRIME_ERR_INVALID_ARG, "prime_linear_frag: argmax needs a workspace of %zu bytes", need);
        if (reinterpret_cast<uintptr_t>(workspace) & 7) return fail(PRIME_ERR_MISALIGNED, "workspace misaligned");
        a.keys = static_cast<uint64_t *>(workspace);
        a.tokens = tokens;
    }
    return check_hip(prime::launch_linear_frag(a, static_cast<hipStream_t>(stream)), "linear_frag launch");
}

int prime_argmax(const void *logits, int dtype, int n, int vocab, int64_t stride_n, int64_t *out, void *stream) {
    g_err[0] = 0;
    if (!logits || !out) return fail(PRIME_ERR_INVALID_ARG, "prime_argmax: null argument");
    if (n <= 0 || vocab <= 0 || stride_n < vocab)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes n=%d vocab=%d stride_n=%lld", n, vocab,
                    static_cast<long long>(stride_n));
    if (!valid_dtype(dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dtype");
    if (reinterpret_cast<uintptr_t>(out) & 7) return fail(PRIME_ERR_MISALIGNED, "out must be 8-byte aligned");
    const int64_t es = elem_size(dtype);
    if (reinterpret_cast<uintptr_t>(logits) % es) return fail(PRIME_ERR_MISALIGNED, "logits misaligned");
    prime::ArgmaxArgs a{};
    a.logits = logits; a.out = out; a.stride_n = stride_n;
    a.n = n; a.vocab = vocab; a.dt = dtype;
    a.vector = aligned16(logits) && (stride_n * es) % 16 == 0;
    return check_hip(prime::launch_argmax_rows(a, static_cast<hipStream_t>(stream)), "argmax launch");
}

static int prefill_impl(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v, int B, int H,
                        int H_kv, int L, int D, int chunk, const float *decay, float eps, unsigned flags,
                        const prime_state_t *state_in, const prime_tensor_t *y, const prime_state_t *state_out,
                        void *workspace, size_t workspace_bytes, void *stream, const float *log_decay,
                        const float *k_scale, const prime_qk_norm_t *norm = nullptr) {
    g_err[0] = 0;
    const bool selective = log_decay != nullptr;
    if (!q || !k || !v || !y || !q->data || !k->data || !v->data || !y->data || !(decay || selective) ||
        (selective && !k_scale))
        return fail(PRIME_ERR_INVALID_ARG, "prefill: null argument");
    if (D != prime::kD) {
        // head dims below 64: one wavefront per (sequence, head), chunk size irrelevant
        if (chunk <= 0) return fail(PRIME_ERR_INVALID_ARG, "bad chunk %d", chunk);
        if (selective && flags) return fail(PRIME_ERR_INVALID_ARG, "the selective form takes no flags");
        if (!valid_dtype(y->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported y dtype");
        prime::GenericArgs g{};
        int rc;
        if ((rc = generic_args(g, q, k, v, B, H, H_kv, L, D, decay, eps, flags, state_in, state_out)) ||
            (rc = generic_norm(g, norm)))
            return rc;
        g.y = y->data; g.dt_y = y->dtype; g.y_sb = y->stride_b; g.y_sh = y->stride_h; g.y_sl = y->stride_l;
        if (selective) {
            g.selective = 1;
            g.log_decay = log_decay;
            g.k_scale = k_scale;
        }
        return check_hip(prime::launch_generic_prefill(g, static_cast<hipStream_t>(stream)), "prefill launch");
    }
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv || L <= 0 || chunk <= 0)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d L=%d chunk=%d", B, H, H_kv, L, chunk);
    if (flags & ~PRIME_FLAG_DENSE_CLAMP) return fail(PRIME_ERR_INVALID_ARG, "unknown flags 0x%x", flags);
    if (q->dtype != k->dtype || q->dtype != v->dtype || (q->dtype != PRIME_BF16 && q->dtype != PRIME_F32))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "q/k/v must share dtype BF16 or F32");
    if (!valid_dtype(y->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported y dtype");
    if (!rows_aligned(q, true) || !rows_aligned(k, true) || !rows_aligned(v, true) || !rows_aligned(y, true))
        return fail(PRIME_ERR_MISALIGNED, "q/k/v/y rows must start on 16-byte boundaries");
    int rc;
    if ((rc = check_state(state_in, "state_in")) || (rc = check_state(state_out, "state_out"))) return rc;
    bool inplace;
    if ((rc = check_state_alias(state_in, state_out, static_cast<size_t>(B) * H, D, &inplace))) return rc;

    prime::PrefillArgs a{};
    a.q = q->data; a.k = k->data; a.v = v->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.q_sl = q->stride_l;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_sl = k->stride_l;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_sl = v->stride_l;
    a.dt_in = q->dtype;
    a.B = B; a.H = H; a.group = H / H_kv; a.L = L;
    a.decay = decay; a.eps = eps;
    a.dense_clamp = (flags & PRIME_FLAG_DENSE_CLAMP) ? 1 : 0;
    if (selective && a.dense_clamp) return fail(PRIME_ERR_INVALID_ARG, "the selective form has no dense clamp");
    a.log_decay = log_decay; a.k_scale = k_scale;
    if (norm) {
        if (q->dtype != PRIME_BF16)
            return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "the QK-norm prefill takes BF16 q/k/v");
        if ((norm->q_weight == nullptr) != (norm->q_bias == nullptr) ||
            (norm->k_weight == nullptr) != (norm->k_bias == nullptr))
            return fail(PRIME_ERR_INVALID_ARG, "QK-norm: LayerNorm weight without bias or bias without weight");
        if ((norm->q_weight || norm->k_weight) && !valid_dtype(norm->dtype))
            return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported norm dtype");
        a.qk_norm = 1;
        a.qn_w = norm->q_weight; a.qn_b = norm->q_bias; a.kn_w = norm->k_weight; a.kn_b = norm->k_bias;
        a.dt_norm = norm->dtype; a.ln_eps = norm->eps; a.q_scale = norm->q_scale;
    }
    if (state_in) {
        a.s0i = state_in->s0; a.s1i = state_in->s1; a.s2i = state_in->s2;
        a.k0i = state_in->k0; a.k1i = state_in->k1; a.k2i = state_in->k2;
    }
    if (state_out) {
        a.s0o = state_out->s0; a.s1o = state_out->s1; a.s2o = state_out->s2;
        a.k0o = state_out->k0; a.k1o = state_out->k1; a.k2o = state_out->k2;
    }
    a.y = y->data; a.dt_y = y->dtype;
    a.y_sb = y->stride_b; a.y_sh = y->stride_h; a.y_sl = y->stride_l;
    if (workspace && !aligned16(workspace))
        return fail(PRIME_ERR_MISALIGNED, "workspace must be 16-byte aligned");
    const int S = B * H;
    prime::plan_segments(S, L, a.dense_clamp != 0, workspace ? workspace_bytes : 0, &a.G, &a.cps);
    a.ws = a.G > 1 ? static_cast<float *>(workspace) : nullptr;
    if (a.G == 1 && workspace && q->dtype == PRIME_BF16 && !a.dense_clamp) {
        // more sequences than CUs: the paired split, when the workspace holds it
        int K, pcs;
        prime::plan_pairs(S, L, &K, &pcs);
        if (K > 0 && workspace_bytes >= prime::pair_ws_bytes(K)) {
            a.npair = K;
            a.pcs = pcs;
            a.ws = static_cast<float *>(workspace);
            a.pflag = reinterpret_cast<unsigned long long *>(a.ws + static_cast<size_t>(K) * prime::kWsStride);
            a.epoch = next_epoch();
        }
    }
    (void)inplace;  // in place is safe: each workgroup reads its own state before writing it
    return check_hip(prime::launch_prefill(a, static_cast<hipStream_t>(stream)), "prefill launch");
}

int prime_chunked_prefill(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                          int B, int H, int H_kv, int L, int D, int chunk, const float *decay,
                          float eps, unsigned flags, const prime_state_t *state_in,
                          const prime_tensor_t *y, const prime_state_t *state_out, void *workspace,
                          size_t workspace_bytes, void *stream) {
    if (!decay) {
        g_err[0] = 0;
        return fail(PRIME_ERR_INVALID_ARG, "prime_chunked_prefill: null decay");
    }
    return prefill_impl(q, k, v, B, H, H_kv, L, D, chunk, decay, eps, flags, state_in, y, state_out, workspace,
                        workspace_bytes, stream, nullptr, nullptr);
}

int prime_chunked_prefill_qknorm(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v, int B,
                                 int H, int H_kv, int L, int D, int chunk, const float *decay, float eps,
                                 unsigned flags, const prime_qk_norm_t *norm, const prime_state_t *state_in,
                                 const prime_tensor_t *y, const prime_state_t *state_out, void *workspace,
                                 size_t workspace_bytes, void *stream) {
    if (!decay || !norm) {
        g_err[0] = 0;
        return fail(PRIME_ERR_INVALID_ARG, "prime_chunked_prefill_qknorm: null decay or norm");
    }
    return prefill_impl(q, k, v, B, H, H_kv, L, D, chunk, decay, eps, flags, state_in, y, state_out, workspace,
                        workspace_bytes, stream, nullptr, nullptr, norm);
}

}  // extern "C"

namespace {

// Validation shared by prime_accumulate and prime_accumulate_noalloc; the
// workspace is checked separately (the no-allocation variant brings its own).
int accumulate_checks(const char *who, const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv,
                      int L, int D, const float *decay, const prime_state_t *state_in,
                      const prime_state_t *state_out) {
    if (!k || !v || !k->data || !v->data || !decay || !state_out)
        return fail(PRIME_ERR_INVALID_ARG, "%s: null argument", who);
    if (D != prime::kD) return fail(PRIME_ERR_UNSUPPORTED_DIM, "head dim %d unsupported (only 64)", D);
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv || L <= 0)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d L=%d", B, H, H_kv, L);
    if (k->dtype != v->dtype || (k->dtype != PRIME_BF16 && k->dtype != PRIME_F32))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "k/v must share dtype BF16 or F32");
    if (!rows_aligned(k, true) || !rows_aligned(v, true))
        return fail(PRIME_ERR_MISALIGNED, "k/v rows must start on 16-byte boundaries");
    int rc;
    if ((rc = check_state(state_in, "state_in")) || (rc = check_state(state_out, "state_out"))) return rc;
    bool inplace;
    return check_state_alias(state_in, state_out, static_cast<size_t>(B) * H, D, &inplace);
}

// Launch of a validated accumulate call on a workspace of at least one slot
// per sequence (the segment plan uses as much of workspace_bytes as it pays to).
int accumulate_launch(const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv, int L,
                      const float *decay, const prime_state_t *state_in, const prime_state_t *state_out,
                      void *workspace, size_t workspace_bytes, void *stream) {
    const int S = B * H;
    prime::PrefillArgs a{};
    // q is not read by the state-only kernels; it points at v for safety
    a.q = v->data; a.k = k->data; a.v = v->data;
    a.q_sb = v->stride_b; a.q_sh = v->stride_h; a.q_sl = v->stride_l;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_sl = k->stride_l;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_sl = v->stride_l;
    a.dt_in = k->dtype;
    a.B = B; a.H = H; a.group = H / H_kv; a.L = L;
    a.decay = decay; a.eps = 1.0f;
    if (state_in) {
        a.s0i = state_in->s0; a.s1i = state_in->s1; a.s2i = state_in->s2;
        a.k0i = state_in->k0; a.k1i = state_in->k1; a.k2i = state_in->k2;
    }
    a.s0o = state_out->s0; a.s1o = state_out->s1; a.s2o = state_out->s2;
    a.k0o = state_out->k0; a.k1o = state_out->k1; a.k2o = state_out->k2;
    // G = 1 (one slot per sequence, cps = all chunks) when the workspace holds no more
    prime::plan_segments(S, L, false, workspace_bytes, &a.G, &a.cps);
    a.ws = static_cast<float *>(workspace);
    a.accumulate = 1;
    // in place is safe: the scan reads state_in and the slots before it writes
    // state_out, element by element
    return check_hip(prime::launch_prefill(a, static_cast<hipStream_t>(stream)), "accumulate launch");
}

}  // namespace

// Scratch of prime_accumulate_noalloc: the segment slots live in this fixed
// device array instead of a caller workspace.  Every slot a call reads is
// written earlier in the same call (the state-only pass writes all 8,385
// state floats of each of its slots before the scan reads them), so nothing
// needs clearing between calls.  One copy per device, held until the process
// ends; calls that overlap on one device share it and race.
static __device__ __align__(256) float scratch[PRIME_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

// The array's device address, looked up once per device with that device
// current (the host-side name `scratch` is only a stand-in for the symbol).
std::mutex g_scratch_mu;
void *g_scratch_ptr[64] = {};

int scratch_address(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(PRIME_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= 64) return fail(PRIME_ERR_HIP, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return fail(PRIME_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return PRIME_OK;
}

}  // namespace

extern "C" {

int prime_accumulate(const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv, int L, int D,
                     const float *decay, const prime_state_t *state_in, const prime_state_t *state_out,
                     void *workspace, size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    int rc;
    if ((rc = accumulate_checks("prime_accumulate", k, v, B, H, H_kv, L, D, decay, state_in, state_out)))
        return rc;
    if (!workspace) return fail(PRIME_ERR_INVALID_ARG, "prime_accumulate: null workspace");
    if (!aligned16(workspace)) return fail(PRIME_ERR_MISALIGNED, "workspace must be 16-byte aligned");
    const size_t slot = static_cast<size_t>(B) * H * prime::kWsStride * sizeof(float);
    if (workspace_bytes < slot)
        return fail(PRIME_ERR_INVALID_ARG, "workspace of %zu bytes is below the minimum %zu", workspace_bytes, slot);
    return accumulate_launch(k, v, B, H, H_kv, L, decay, state_in, state_out, workspace, workspace_bytes, stream);
}

int prime_accumulate_noalloc(const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv, int L,
                             int D, const float *decay, const prime_state_t *state_in,
                             const prime_state_t *state_out, void *stream) {
    g_err[0] = 0;
    int rc;
    if ((rc = accumulate_checks("prime_accumulate_noalloc", k, v, B, H, H_kv, L, D, decay, state_in, state_out)))
        return rc;
    const size_t slot = static_cast<size_t>(B) * H * prime::kWsStride * sizeof(float);
    if (slot > PRIME_NOALLOC_SCRATCH_BYTES)
        return fail(PRIME_ERR_INVALID_ARG,
                    "prime_accumulate_noalloc: B*H = %d sequences need %zu bytes of scratch, above its fixed %zu "
                    "(at most %zu sequences); use prime_accumulate with a workspace",
                    B * H, slot, static_cast<size_t>(PRIME_NOALLOC_SCRATCH_BYTES),
                    static_cast<size_t>(PRIME_NOALLOC_SCRATCH_BYTES) / (prime::kWsStride * sizeof(float)));
    void *ws = nullptr;
    if ((rc = scratch_address(&ws))) return rc;
    return accumulate_launch(k, v, B, H, H_kv, L, decay, state_in, state_out, ws, PRIME_NOALLOC_SCRATCH_BYTES,
                             stream);
}

namespace {
// per-token denominators, rounded up to a slot boundary
size_t bwd_token_bytes(int B, int H, int L) {
    return (static_cast<size_t>(B) * H * L * 2 * sizeof(float) + 255) & ~static_cast<size_t>(255);
}
// the dense double clamp with an incoming state: kBwdCorr floats per sequence
size_t bwd_corr_bytes(int B, int H) { return static_cast<size_t>(B) * H * prime::kBwdCorr * sizeof(float); }
}  // namespace

namespace {
// segment slots of the backward's plan for bf16 (per_cu 2) or fp32 (1) inputs
size_t bwd_slot_bytes(int B, int H, int L, int per_cu, int *G, int *cps) {
    prime::plan_backward_segments(B * H, L, G, cps, per_cu);
    return *G > 1 ? static_cast<size_t>(B) * H * *G * prime::kWsStride * sizeof(float) : 0;
}
}  // namespace

size_t prime_chunked_prefill_backward_workspace_size(int B, int H, int L) {
    if (B <= 0 || H <= 0 || L <= 0) return 0;
    int G, cps;
    // enough for either plan (the inputs' dtype is not an argument)
    const size_t slots = std::max(bwd_slot_bytes(B, H, L, 2, &G, &cps), bwd_slot_bytes(B, H, L, 1, &G, &cps));
    return bwd_token_bytes(B, H, L) + std::max(slots, bwd_corr_bytes(B, H));
}

int prime_chunked_prefill_backward(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                                   int B, int H, int H_kv, int L, int D, const float *decay, float eps,
                                   unsigned flags, const prime_state_t *state_in, const prime_tensor_t *dy,
                                   const prime_state_t *dstate_out, const prime_tensor_t *dq,
                                   const prime_tensor_t *dk, const prime_tensor_t *dv,
                                   const prime_state_t *dstate_in, void *workspace, size_t workspace_bytes,
                                   void *stream) {
    g_err[0] = 0;
    if (!q || !k || !v || !dy || !dq || !dk || !dv || !q->data || !k->data || !v->data || !dy->data || !dq->data ||
        !dk->data || !dv->data || !decay || !workspace)
        return fail(PRIME_ERR_INVALID_ARG, "prime_chunked_prefill_backward: null argument");
    if (D != prime::kD) {
        // head dims below 64: the generic reverse pass (workspace: the per-token
        // denominators, as the 64 path's minimum)
        if (H_kv != H)
            return fail(PRIME_ERR_INVALID_ARG, "backward takes k/v with one head per query head (H_kv=%d, H=%d)",
                        H_kv, H);
        if (!valid_dtype(dy->dtype) || !valid_dtype(dq->dtype))
            return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dy / gradient dtype");
        if (dk->dtype != dq->dtype || dv->dtype != dq->dtype || dk->stride_b != dq->stride_b ||
            dv->stride_b != dq->stride_b || dk->stride_h != dq->stride_h || dv->stride_h != dq->stride_h ||
            dk->stride_l != dq->stride_l || dv->stride_l != dq->stride_l)
            return fail(PRIME_ERR_INVALID_ARG, "dq, dk and dv must share dtype and strides");
        if (B > 0 && H > 0 && L > 0 && (workspace_bytes < bwd_token_bytes(B, H, L) || !aligned16(workspace)))
            return fail(PRIME_ERR_INVALID_ARG, "workspace of %zu bytes (16-byte aligned) is below the %zu needed",
                        workspace_bytes, bwd_token_bytes(B, H, L));
        prime::GenericArgs g{};
        int rc;
        if ((rc = generic_args(g, q, k, v, B, H, H_kv, L, D, decay, eps, flags, state_in, nullptr)) ||
            (rc = check_state(dstate_out, "dstate_out")) || (rc = check_state(dstate_in, "dstate_in")))
            return rc;
        g.dy = dy->data; g.dt_dy = dy->dtype; g.dy_sb = dy->stride_b; g.dy_sh = dy->stride_h; g.dy_sl = dy->stride_l;
        if (dstate_out) {
            g.ds0 = dstate_out->s0; g.ds1 = dstate_out->s1; g.ds2 = dstate_out->s2;
            g.dk0 = dstate_out->k0; g.dk1 = dstate_out->k1; g.dk2 = dstate_out->k2;
        }
        g.dq = dq->data; g.dk = dk->data; g.dv = dv->data; g.dt_g = dq->dtype;
        g.g_sb = dq->stride_b; g.g_sh = dq->stride_h; g.g_sl = dq->stride_l;
        if (dstate_in) {
            g.dsi0 = dstate_in->s0; g.dsi1 = dstate_in->s1; g.dsi2 = dstate_in->s2;
            g.dki0 = dstate_in->k0; g.dki1 = dstate_in->k1; g.dki2 = dstate_in->k2;
        }
        g.ws = static_cast<float *>(workspace);
        return check_hip(prime::launch_generic_backward(g, static_cast<hipStream_t>(stream)), "backward launch");
    }
    if (B <= 0 || H <= 0 || L <= 0) return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d L=%d", B, H, L);
    if (H_kv != H)
        return fail(PRIME_ERR_INVALID_ARG, "backward takes k/v with one head per query head (H_kv=%d, H=%d): "
                    "expand grouped k/v first, as the reference module does", H_kv, H);
    if (flags & ~PRIME_FLAG_DENSE_CLAMP) return fail(PRIME_ERR_INVALID_ARG, "unknown flags 0x%x", flags);
    const bool dense_in = (flags & PRIME_FLAG_DENSE_CLAMP) && state_in;
    if (q->dtype != k->dtype || q->dtype != v->dtype || (q->dtype != PRIME_BF16 && q->dtype != PRIME_F32))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "q/k/v must share dtype BF16 or F32");
    if (!valid_dtype(dy->dtype) || !valid_dtype(dq->dtype))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dy / gradient dtype");
    if (dk->dtype != dq->dtype || dv->dtype != dq->dtype || dk->stride_b != dq->stride_b ||
        dv->stride_b != dq->stride_b || dk->stride_h != dq->stride_h || dv->stride_h != dq->stride_h ||
        dk->stride_l != dq->stride_l || dv->stride_l != dq->stride_l)
        return fail(PRIME_ERR_INVALID_ARG, "dq, dk and dv must share dtype and strides");
    if (!rows_aligned(q, true) || !rows_aligned(k, true) || !rows_aligned(v, true) || !rows_aligned(dy, true))
        return fail(PRIME_ERR_MISALIGNED, "q/k/v/dy rows must start on 16-byte boundaries");
    const size_t need = bwd_token_bytes(B, H, L);
    const size_t need_all = need + (dense_in ? bwd_corr_bytes(B, H) : 0);
    if (workspace_bytes < need_all || !aligned16(workspace))
        return fail(PRIME_ERR_INVALID_ARG, "workspace of %zu bytes (16-byte aligned) is below the %zu needed",
                    workspace_bytes, need_all);
    int rc;
    if ((rc = check_state(state_in, "state_in")) || (rc = check_state(dstate_out, "dstate_out")) ||
        (rc = check_state(dstate_in, "dstate_in")))
        return rc;
    prime::BwdArgs a{};
    a.q = q->data; a.k = k->data; a.v = v->data; a.dy = dy->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.q_sl = q->stride_l;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_sl = k->stride_l;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_sl = v->stride_l;
    a.dy_sb = dy->stride_b; a.dy_sh = dy->stride_h; a.dy_sl = dy->stride_l;
    a.dt_in = q->dtype; a.dt_dy = dy->dtype;
    a.B = B; a.H = H; a.L = L; a.decay = decay; a.eps = eps;
    if (state_in) {
        a.s0i = state_in->s0; a.s1i = state_in->s1; a.s2i = state_in->s2;
        a.k0i = state_in->k0; a.k1i = state_in->k1; a.k2i = state_in->k2;
    }
    if (dstate_out) {
        a.ds0o = dstate_out->s0; a.ds1o = dstate_out->s1; a.ds2o = dstate_out->s2;
        a.dk0o = dstate_out->k0; a.dk1o = dstate_out->k1; a.dk2o = dstate_out->k2;
    }
    a.dq = dq->data; a.dk = dk->data; a.dv = dv->data; a.dt_g = dq->dtype;
    a.g_sb = dq->stride_b; a.g_sh = dq->stride_h; a.g_sl = dq->stride_l;
    if (dstate_in) {
        a.ds0i = dstate_in->s0; a.ds1i = dstate_in->s1; a.ds2i = dstate_in->s2;
        a.dk0i = dstate_in->k0; a.dk1i = dstate_in->k1; a.dk2i = dstate_in->k2;
    }
    a.inv_den = static_cast<float *>(workspace);
    a.g_den = a.inv_den + static_cast<size_t>(B) * H * L;
    // (fp32 inputs: the fp32 passes run one workgroup per CU)
    const size_t slots = bwd_slot_bytes(B, H, L, q->dtype == PRIME_F32 ? 1 : 2, &a.G, &a.cps);
    if (dense_in || (a.G > 1 && workspace_bytes < need + slots)) {
        // (the dense double clamp carries the call's K apart from the incoming
        // one from token 0)
        a.G = 1;  // one segment per sequence in the workspace given
        a.cps = (L + 63) / 64;
    }
    a.ws = a.G > 1 ? reinterpret_cast<float *>(static_cast<char *>(workspace) + need) : nullptr;
    if (dense_in) {
        a.dense_in = 1;
        a.kcorr = reinterpret_cast<float *>(static_cast<char *>(workspace) + need);
    }
    return check_hip(prime::launch_prefill_backward(a, static_cast<hipStream_t>(stream)), "backward launch");
}

size_t prime_selective_prefill_backward_workspace_size(int B, int H, int L) {
    if (B <= 0 || H <= 0 || L <= 0) return 0;
    // the per-token denominators (8 bytes), the query-side decay terms (4), one float per sequence
    return bwd_token_bytes(B, H, L) + static_cast<size_t>(B) * H * L * sizeof(float) +
           static_cast<size_t>(B) * H * sizeof(float);
}

int prime_selective_prefill_backward(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                                     int B, int H, int H_kv, int L, int D, const float *log_decay,
                                     const float *k_scale, float eps, const prime_state_t *state_in,
                                     const prime_tensor_t *dy, const prime_state_t *dstate_out,
                                     const prime_tensor_t *dq, const prime_tensor_t *dk, const prime_tensor_t *dv,
                                     const prime_state_t *dstate_in, float *d_log_decay, float *d_k_scale,
                                     void *workspace, size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    if (!q || !k || !v || !dy || !dq || !dk || !dv || !q->data || !k->data || !v->data || !dy->data || !dq->data ||
        !dk->data || !dv->data || !log_decay || !k_scale || !d_log_decay || !d_k_scale || !workspace)
        return fail(PRIME_ERR_INVALID_ARG, "prime_selective_prefill_backward: null argument");
    if (D != prime::kD) {
        // head dims below 64: the generic reverse pass in its selective form
        if (H_kv != H)
            return fail(PRIME_ERR_INVALID_ARG, "backward takes k/v with one head per query head (H_kv=%d, H=%d)",
                        H_kv, H);
        if (!valid_dtype(dy->dtype) || !valid_dtype(dq->dtype))
            return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dy / gradient dtype");
        if (dk->dtype != dq->dtype || dv->dtype != dq->dtype || dk->stride_b != dq->stride_b ||
            dv->stride_b != dq->stride_b || dk->stride_h != dq->stride_h || dv->stride_h != dq->stride_h ||
            dk->stride_l != dq->stride_l || dv->stride_l != dq->stride_l)
            return fail(PRIME_ERR_INVALID_ARG, "dq, dk and dv must share dtype and strides");
        if (B > 0 && H > 0 && L > 0 &&
            (workspace_bytes < prime_selective_prefill_backward_workspace_size(B, H, L) || !aligned16(workspace)))
            return fail(PRIME_ERR_INVALID_ARG, "workspace of %zu bytes (16-byte aligned) is below the %zu needed",
                        workspace_bytes, prime_selective_prefill_backward_workspace_size(B, H, L));
        prime::GenericArgs g{};
        int rc;
        if ((rc = generic_args(g, q, k, v, B, H, H_kv, L, D, nullptr, eps, 0u, state_in, nullptr)) ||
            (rc = check_state(dstate_out, "dstate_out")) || (rc = check_state(dstate_in, "dstate_in")))
            return rc;
        g.selective = 1;
        g.log_decay = log_decay;
        g.k_scale = k_scale;
        g.dy = dy->data; g.dt_dy = dy->dtype; g.dy_sb = dy->stride_b; g.dy_sh = dy->stride_h; g.dy_sl = dy->stride_l;
        if (dstate_out) {
            g.ds0 = dstate_out->s0; g.ds1 = dstate_out->s1; g.ds2 = dstate_out->s2;
            g.dk0 = dstate_out->k0; g.dk1 = dstate_out->k1; g.dk2 = dstate_out->k2;
        }
        g.dq = dq->data; g.dk = dk->data; g.dv = dv->data; g.dt_g = dq->dtype;
        g.g_sb = dq->stride_b; g.g_sh = dq->stride_h; g.g_sl = dq->stride_l;
        if (dstate_in) {
            g.dsi0 = dstate_in->s0; g.dsi1 = dstate_in->s1; g.dsi2 = dstate_in->s2;
            g.dki0 = dstate_in->k0; g.dki1 = dstate_in->k1; g.dki2 = dstate_in->k2;
        }
        g.ws = static_cast<float *>(workspace);
        g.pq = reinterpret_cast<float *>(static_cast<char *>(workspace) + bwd_token_bytes(B, H, L));
        g.dlogd = d_log_decay;
        g.dkscale = d_k_scale;
        return check_hip(prime::launch_generic_backward(g, static_cast<hipStream_t>(stream)), "backward launch");
    }
    if (B <= 0 || H <= 0 || L <= 0) return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d L=%d", B, H, L);
    if (H_kv != H)
        return fail(PRIME_ERR_INVALID_ARG, "backward takes k/v with one head per query head (H_kv=%d, H=%d): "
                    "expand grouped k/v first, as the reference module does", H_kv, H);
    if (q->dtype != PRIME_F32 || k->dtype != PRIME_F32 || v->dtype != PRIME_F32)
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "selective backward: F32 q/k/v (the reference differentiates "
                    "the selective branch in fp32; convert bf16 inputs first)");
    if (!valid_dtype(dy->dtype) || !valid_dtype(dq->dtype))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dy / gradient dtype");
    if (dk->dtype != dq->dtype || dv->dtype != dq->dtype || dk->stride_b != dq->stride_b ||
        dv->stride_b != dq->stride_b || dk->stride_h != dq->stride_h || dv->stride_h != dq->stride_h ||
        dk->stride_l != dq->stride_l || dv->stride_l != dq->stride_l)
        return fail(PRIME_ERR_INVALID_ARG, "dq, dk and dv must share dtype and strides");
    if (!rows_aligned(q, true) || !rows_aligned(k, true) || !rows_aligned(v, true) || !rows_aligned(dy, true))
        return fail(PRIME_ERR_MISALIGNED, "q/k/v/dy rows must start on 16-byte boundaries");
    const size_t need = prime_selective_prefill_backward_workspace_size(B, H, L);
    if (workspace_bytes < need || !aligned16(workspace))
        return fail(PRIME_ERR_INVALID_ARG, "workspace of %zu bytes (16-byte aligned) is below the %zu needed",
                    workspace_bytes, need);
    int rc;
    if ((rc = check_state(state_in, "state_in")) || (rc = check_state(dstate_out, "dstate_out")) ||
        (rc = check_state(dstate_in, "dstate_in")))
        return rc;
    prime::BwdArgs a{};
    a.q = q->data; a.k = k->data; a.v = v->data; a.dy = dy->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.q_sl = q->stride_l;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_sl = k->stride_l;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_sl = v->stride_l;
    a.dy_sb = dy->stride_b; a.dy_sh = dy->stride_h; a.dy_sl = dy->stride_l;
    a.dt_in = q->dtype; a.dt_dy = dy->dtype;
    a.B = B; a.H = H; a.L = L; a.decay = k_scale; a.eps = eps;  // (decay: not read in the selective form)
    if (state_in) {
        a.s0i = state_in->s0; a.s1i = state_in->s1; a.s2i = state_in->s2;
        a.k0i = state_in->k0; a.k1i = state_in->k1; a.k2i = state_in->k2;
    }
    if (dstate_out) {
        a.ds0o = dstate_out->s0; a.ds1o = dstate_out->s1; a.ds2o = dstate_out->s2;
        a.dk0o = dstate_out->k0; a.dk1o = dstate_out->k1; a.dk2o = dstate_out->k2;
    }
    a.dq = dq->data; a.dk = dk->data; a.dv = dv->data; a.dt_g = dq->dtype;
    a.g_sb = dq->stride_b; a.g_sh = dq->stride_h; a.g_sl = dq->stride_l;
    if (dstate_in) {
        a.ds0i = dstate_in->s0; a.ds1i = dstate_in->s1; a.ds2i = dstate_in->s2;
        a.dk0i = dstate_in->k0; a.dk1i = dstate_in->k1; a.dk2i = dstate_in->k2;
    }
    const size_t ntok = static_cast<size_t>(B) * H * L;
    a.inv_den = static_cast<float *>(workspace);
    a.g_den = a.inv_den + ntok;
    a.pq = reinterpret_cast<float *>(static_cast<char *>(workspace) + bwd_token_bytes(B, H, L));
    a.fin = a.pq + ntok;
    a.G = 1;
    a.cps = (L + 63) / 64;
    a.logd = log_decay; a.kscale = k_scale; a.dlogd = d_log_decay; a.dkscale = d_k_scale;
    return check_hip(prime::launch_prefill_backward_f32(a, static_cast<hipStream_t>(stream)), "backward launch");
}

int prime_decode_readout(const prime_tensor_t *q, int B, int H, int D, float eps, const prime_state_t *state,
                         const prime_tensor_t *y, void *stream) {
    g_err[0] = 0;
    if (!q || !q->data || !y || !y->data || !state)
        return fail(PRIME_ERR_INVALID_ARG, "prime_decode_readout: null argument");
    if (D != prime::kD) return fail(PRIME_ERR_UNSUPPORTED_DIM, "head dim %d unsupported (only 64)", D);
    if (B <= 0 || H <= 0) return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d", B, H);
    if (!valid_dtype(q->dtype) || !valid_dtype(y->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dtype");
    int rc;
    if ((rc = check_state(state, "state"))) return rc;
    prime::DecodeArgs a{};
    a.q = q->data; a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.dt_q = q->dtype;
    a.k = q->data; a.v = q->data; a.dt_k = a.dt_v = q->dtype;  // not read
    a.B = B; a.H = H; a.group = 1; a.eps = eps; a.q_scale = 1.0f;
    a.s0i = state->s0; a.s1i = state->s1; a.s2i = state->s2; a.k0i = state->k0; a.k1i = state->k1; a.k2i = state->k2;
    a.s0o = state->s0; a.s1o = state->s1; a.s2o = state->s2; a.k0o = state->k0; a.k1o = state->k1; a.k2o = state->k2;
    a.y = y->data; a.dt_y = y->dtype; a.y_sb = y->stride_b; a.y_sh = y->stride_h;
    a.no_update = 1;
    return check_hip(prime::launch_decode_step(a, static_cast<hipStream_t>(stream)), "readout launch");
}

int prime_decode_update(const prime_tensor_t *k, const prime_tensor_t *v, int B, int H, int H_kv, int D,
                        const float *decay, const prime_state_t *state_in, const prime_state_t *state_out,
                        void *stream) {
    g_err[0] = 0;
    if (!k || !v || !k->data || !v->data || !decay || !state_out)
        return fail(PRIME_ERR_INVALID_ARG, "prime_decode_update: null argument");
    if (D != prime::kD) return fail(PRIME_ERR_UNSUPPORTED_DIM, "head dim %d unsupported (only 64)", D);
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d", B, H, H_kv);
    if (!valid_dtype(k->dtype) || !valid_dtype(v->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dtype");
    int rc;
    if ((rc = check_state(state_in, "state_in")) || (rc = check_state(state_out, "state_out"))) return rc;
    bool inplace;
    if ((rc = check_state_alias(state_in, state_out, static_cast<size_t>(B) * H, D, &inplace))) return rc;
    prime::DecodeArgs a{};
    a.k = k->data; a.v = v->data; a.q = k->data;  // q not read
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.v_sb = v->stride_b; a.v_sh = v->stride_h;
    a.dt_k = k->dtype; a.dt_v = v->dtype; a.dt_q = k->dtype;
    a.B = B; a.H = H; a.group = H / H_kv; a.decay = decay; a.eps = 1.0f; a.q_scale = 1.0f;
    if (state_in) {
        a.s0i = state_in->s0; a.s1i = state_in->s1; a.s2i = state_in->s2;
        a.k0i = state_in->k0; a.k1i = state_in->k1; a.k2i = state_in->k2;
    }
    a.s0o = state_out->s0; a.s1o = state_out->s1; a.s2o = state_out->s2;
    a.k0o = state_out->k0; a.k1o = state_out->k1; a.k2o = state_out->k2;
    a.y = state_out->s0; a.dt_y = PRIME_F32;  // not written
    a.no_readout = 1;
    return check_hip(prime::launch_decode_step(a, static_cast<hipStream_t>(stream)), "update launch");
}

int prime_selective_prefill(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v, int B,
                            int H, int H_kv, int L, int D, const float *log_decay, const float *k_scale, float eps,
                            const prime_state_t *state_in, const prime_tensor_t *y, const prime_state_t *state_out,
                            void *workspace, size_t workspace_bytes, void *stream) {
    if (!log_decay || !k_scale) {
        g_err[0] = 0;
        return fail(PRIME_ERR_INVALID_ARG, "prime_selective_prefill: null log_decay or k_scale");
    }
    return prefill_impl(q, k, v, B, H, H_kv, L, D, 64, nullptr, eps, 0, state_in, y, state_out, workspace,
                        workspace_bytes, stream, log_decay, k_scale);
}

int prime_selective_prefill_qknorm(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v, int B,
                                   int H, int H_kv, int L, int D, const float *log_decay, const float *k_scale,
                                   float eps, const prime_qk_norm_t *norm, const prime_state_t *state_in,
                                   const prime_tensor_t *y, const prime_state_t *state_out, void *workspace,
                                   size_t workspace_bytes, void *stream) {
    if (!log_decay || !k_scale || !norm) {
        g_err[0] = 0;
        return fail(PRIME_ERR_INVALID_ARG, "prime_selective_prefill_qknorm: null log_decay, k_scale or norm");
    }
    return prefill_impl(q, k, v, B, H, H_kv, L, D, 64, nullptr, eps, 0, state_in, y, state_out, workspace,
                        workspace_bytes, stream, log_decay, k_scale, norm);
}

int prime_selective_decode_step(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v, int B,
                                int H, int H_kv, int D, const prime_selective_gate_t *gate, const float *k_scale,
                                float eps, const prime_qk_norm_t *norm, const prime_state_t *state_in,
                                const prime_state_t *state_out, const prime_tensor_t *y, void *stream) {
    if (!gate || !k_scale) {
        g_err[0] = 0;
        return fail(PRIME_ERR_INVALID_ARG, "prime_selective_decode_step: null gate or k_scale");
    }
    if (norm && norm->q_weight && (!norm->q_bias || !norm->k_weight || !norm->k_bias)) {
        g_err[0] = 0;
        return fail(PRIME_ERR_INVALID_ARG, "prime_selective_decode_step: LayerNorm weight without bias");
    }
    if (norm && !valid_dtype(norm->dtype)) {
        g_err[0] = 0;
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported norm dtype");
    }
    return decode_impl(q, k, v, B, H, H_kv, D, nullptr, eps, norm, state_in, state_out, y, stream, gate, k_scale);
}

}  // extern "C"

namespace {

// The delta rule's shapes outside the MFMA kernels (D = 64 with chunk 64):
// head dims 1 .. 64 with any chunk, token by token (delta_gen.hip).
bool delta_generic(int D, int chunk) { return D != prime::kD || chunk != prime::kDeltaChunk; }

int delta_gen_args(prime::DeltaGenArgs &a, const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                   const float *beta, const float *alpha, int B, int H, int H_kv, int L, int D, int chunk,
                   float decay_pad, float feat_eps, float bound, const float *state_in, const float *state_out) {
    if (D < 1 || D > prime::kDeltaGenMaxD)
        return fail(PRIME_ERR_UNSUPPORTED_DIM, "head dim %d unsupported (1 .. %d)", D, prime::kDeltaGenMaxD);
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv || L <= 0 || chunk <= 0)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d L=%d chunk=%d", B, H, H_kv, L, chunk);
    if (!valid_dtype(q->dtype) || !valid_dtype(k->dtype) || !valid_dtype(v->dtype))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported q/k/v dtype");
    const size_t sbytes = static_cast<size_t>(B) * H * D * 2 * D * sizeof(float);
    if (state_in && state_out && state_in != state_out && overlap(state_in, sbytes, state_out, sbytes))
        return fail(PRIME_ERR_ALIAS, "state_out overlaps state_in (only a fully in-place state is allowed)");
    a.q = q->data; a.k = k->data; a.v = v->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.q_sl = q->stride_l;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_sl = k->stride_l;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_sl = v->stride_l;
    a.dt_q = q->dtype; a.dt_k = k->dtype; a.dt_v = v->dtype;
    a.B = B; a.H = H; a.group = H / H_kv; a.L = L; a.D = D; a.chunk = chunk;
    a.beta = beta; a.alpha = alpha;
    a.decay_pad = decay_pad; a.feat_eps = feat_eps; a.bound = bound;
    a.state_in = state_in;
    return PRIME_OK;
}

}  // namespace

extern "C" {

size_t prime_delta_prefill_workspace_size(int B, int H, int L, unsigned flags) {
    if (B <= 0 || H <= 0 || L <= 0) return 0;
    const int NC = (L + prime::kDeltaChunk - 1) / prime::kDeltaChunk;
    const int win = NC < prime::kDeltaDefaultWindow ? NC : prime::kDeltaDefaultWindow;
    const size_t S = static_cast<size_t>(B) * H;
    const size_t rec = prime::delta_rec_bytes((flags & PRIME_FLAG_F32_INPUTS) ? PRIME_F32 : PRIME_BF16);
    return S * prime::kDeltaStateBytes + S * static_cast<size_t>(win) * rec;
}

int prime_delta_prefill(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                        const float *beta, const float *alpha, int B, int H, int H_kv, int L, int D,
                        int chunk, float decay_pad, float feat_eps, float bound, const float *state_in,
                        const prime_tensor_t *y, float *state_out, void *workspace, size_t workspace_bytes,
                        void *stream) {
    g_err[0] = 0;
    if (!q || !k || !v || !y || !q->data || !k->data || !v->data || !y->data || !beta || !alpha)
        return fail(PRIME_ERR_INVALID_ARG, "prime_delta_prefill: null argument");
    if (delta_generic(D, chunk)) {
        prime::DeltaGenArgs g{};
        int rc;
        if ((rc = delta_gen_args(g, q, k, v, beta, alpha, B, H, H_kv, L, D, chunk, decay_pad, feat_eps, bound,
                                 state_in, state_out)))
            return rc;
        if (!valid_dtype(y->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported y dtype");
        g.state_out = state_out;
        g.y = y->data; g.dt_y = y->dtype; g.y_sb = y->stride_b; g.y_sh = y->stride_h; g.y_sl = y->stride_l;
        return check_hip(prime::launch_delta_gen_forward(g, static_cast<hipStream_t>(stream)), "delta prefill launch");
    }
    if (!workspace) return fail(PRIME_ERR_INVALID_ARG, "prime_delta_prefill: null workspace");
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv || L <= 0)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d L=%d", B, H, H_kv, L);
    if (q->dtype != k->dtype || q->dtype != v->dtype || (q->dtype != PRIME_BF16 && q->dtype != PRIME_F32))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "q/k/v must share dtype BF16 or F32");
    if (!valid_dtype(y->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported y dtype");
    if (!rows_aligned(q, true) || !rows_aligned(k, true) || !rows_aligned(v, true) || !rows_aligned(y, true))
        return fail(PRIME_ERR_MISALIGNED, "q/k/v/y rows must start on 16-byte boundaries");
    if (!aligned16(workspace)) return fail(PRIME_ERR_MISALIGNED, "workspace must be 16-byte aligned");
    if ((state_in && !aligned16(state_in)) || (state_out && !aligned16(state_out)))
        return fail(PRIME_ERR_MISALIGNED, "state buffers must be 16-byte aligned");
    const size_t S = static_cast<size_t>(B) * H;
    const size_t sbytes = S * prime::kDeltaStateBytes;
    if (state_in && state_out && state_in != state_out && overlap(state_in, sbytes, state_out, sbytes))
        return fail(PRIME_ERR_ALIAS, "state_out overlaps state_in (only a fully in-place state is allowed)");
    const size_t rec = prime::delta_rec_bytes(q->dtype);
    if (workspace_bytes < sbytes + S * rec)
        return fail(PRIME_ERR_INVALID_ARG, "workspace of %zu bytes is below the minimum %zu for %s inputs%s",
                    workspace_bytes, sbytes + S * rec, q->dtype == PRIME_F32 ? "F32" : "BF16",
                    q->dtype == PRIME_F32 ? " (size it with PRIME_FLAG_F32_INPUTS)" : "");
    const int NC = (L + prime::kDeltaChunk - 1) / prime::kDeltaChunk;
    const size_t cap_sz = (workspace_bytes - sbytes) / (S * rec);
    const int cap = static_cast<int>(cap_sz < static_cast<size_t>(NC) ? cap_sz : static_cast<size_t>(NC) + 1);

    prime::DeltaArgs a{};
    a.q = q->data; a.k = k->data; a.v = v->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.q_sl = q->stride_l;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_sl = k->stride_l;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_sl = v->stride_l;
    a.dt_in = q->dtype;
    a.B = B; a.H = H; a.group = H / H_kv; a.L = L;
    a.beta = beta; a.alpha = alpha;
    a.decay_pad = decay_pad; a.feat_eps = feat_eps; a.bound = bound;
    a.state_in = state_in; a.state_out = state_out;
    a.y = y->data; a.dt_y = y->dtype;
    a.y_sb = y->stride_b; a.y_sh = y->stride_h; a.y_sl = y->stride_l;
    a.ws_state = static_cast<float *>(workspace);
    a.ws_rec = static_cast<uint8_t *>(workspace) + sbytes;
    return check_hip(prime::launch_delta_prefill(a, NC, cap, static_cast<hipStream_t>(stream)),
                     "delta prefill launch");
}

size_t prime_delta_prefill_backward_workspace_size(int B, int H, int L, int D, int chunk) {
    if (B <= 0 || H <= 0 || L <= 0 || D < 1 || D > prime::kDeltaGenMaxD || chunk <= 0) return 0;
    if (delta_generic(D, chunk)) return prime::delta_gen_backward_ws_bytes(B, H, L, D, chunk);
    const size_t NC = (static_cast<size_t>(L) + prime::kDeltaChunk - 1) / prime::kDeltaChunk;
    return static_cast<size_t>(B) * H * NC * prime::kDeltaStateBytes;
}

int prime_delta_prefill_backward(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                                 const float *beta, const float *alpha, int B, int H, int H_kv, int L, int D,
                                 int chunk, float decay_pad, float feat_eps, float bound, const float *state_in,
                                 const prime_tensor_t *dy, const float *dstate_out, float *dq, float *dk, float *dv,
                                 float *dbeta, float *dalpha, float *dstate_in, void *workspace,
                                 size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    if (!q || !k || !v || !dy || !q->data || !k->data || !v->data || !dy->data || !beta || !alpha || !dq || !dk ||
        !dv || !dbeta || !dalpha || !workspace)
        return fail(PRIME_ERR_INVALID_ARG, "prime_delta_prefill_backward: null argument");
    if (delta_generic(D, chunk)) {
        prime::DeltaGenArgs g{};
        int rc;
        if ((rc = delta_gen_args(g, q, k, v, beta, alpha, B, H, H_kv, L, D, chunk, decay_pad, feat_eps, bound,
                                 state_in, nullptr)))
            return rc;
        if (!valid_dtype(dy->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dy dtype");
        const size_t need = prime_delta_prefill_backward_workspace_size(B, H, L, D, chunk);
        if (workspace_bytes < need || !aligned16(workspace))
            return fail(PRIME_ERR_INVALID_ARG, "workspace of %zu bytes (16-byte aligned) is below the %zu needed",
                        workspace_bytes, need);
        g.dy = dy->data; g.dt_dy = dy->dtype; g.dy_sb = dy->stride_b; g.dy_sh = dy->stride_h; g.dy_sl = dy->stride_l;
        g.dstate_out = dstate_out;
        g.dq = dq; g.dk = dk; g.dv = dv; g.dbeta = dbeta; g.dalpha = dalpha; g.dstate_in = dstate_in;
        g.ws = static_cast<float *>(workspace);
        return check_hip(prime::launch_delta_gen_backward(g, static_cast<hipStream_t>(stream)),
                         "delta backward launch");
    }
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv || L <= 0)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d L=%d", B, H, H_kv, L);
    if (q->dtype != k->dtype || q->dtype != v->dtype || (q->dtype != PRIME_BF16 && q->dtype != PRIME_F32))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "q/k/v must share dtype BF16 or F32");
    if (dy->dtype != PRIME_BF16 && dy->dtype != PRIME_F32)
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "dy must be BF16 or F32");
    if (!rows_aligned(q, true) || !rows_aligned(k, true) || !rows_aligned(v, true) || !rows_aligned(dy, true))
        return fail(PRIME_ERR_MISALIGNED, "q/k/v/dy rows must start on 16-byte boundaries");
    if (!aligned16(workspace)) return fail(PRIME_ERR_MISALIGNED, "workspace must be 16-byte aligned");
    if (workspace_bytes < prime_delta_prefill_backward_workspace_size(B, H, L, D, chunk))
        return fail(PRIME_ERR_INVALID_ARG, "workspace of %zu bytes is below the %zu this shape needs", workspace_bytes,
                    prime_delta_prefill_backward_workspace_size(B, H, L, D, chunk));
    prime::DeltaBwdArgs a{};
    a.q = q->data; a.k = k->data; a.v = v->data; a.dy = dy->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h; a.q_sl = q->stride_l;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h; a.k_sl = k->stride_l;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h; a.v_sl = v->stride_l;
    a.dy_sb = dy->stride_b; a.dy_sh = dy->stride_h; a.dy_sl = dy->stride_l;
    a.dt_in = q->dtype; a.dt_dy = dy->dtype;
    a.B = B; a.H = H; a.group = H / H_kv; a.L = L;
    a.beta = beta; a.alpha = alpha;
    a.decay_pad = decay_pad; a.feat_eps = feat_eps; a.bound = bound;
    a.state_in = state_in; a.dstate_out = dstate_out;
    a.dq = dq; a.dk = dk; a.dv = dv; a.dbeta = dbeta; a.dalpha = dalpha; a.dstate_in = dstate_in;
    a.ws = static_cast<float *>(workspace);
    return check_hip(prime::launch_delta_backward(a, static_cast<hipStream_t>(stream)), "delta backward launch");
}

int prime_delta_decode_step_backward(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                                     const float *beta, const float *alpha, int B, int H, int H_kv, int D,
                                     float feat_eps, float bound, const float *state_in, const prime_tensor_t *dy,
                                     const float *dstate_out, float *dq, float *dk, float *dv, float *dbeta,
                                     float *dalpha, float *dstate_in, void *stream) {
    g_err[0] = 0;
    if (!q || !k || !v || !dy || !q->data || !k->data || !v->data || !dy->data || !beta || !alpha || !dq || !dk ||
        !dv || !dbeta || !dalpha)
        return fail(PRIME_ERR_INVALID_ARG, "prime_delta_decode_step_backward: null argument");
    prime::DeltaGenArgs g{};
    int rc;
    if ((rc = delta_gen_args(g, q, k, v, beta, alpha, B, H, H_kv, 1, D, 1, 1.0f, feat_eps, bound, state_in,
                             nullptr)))
        return rc;
    if (!valid_dtype(dy->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dy dtype");
    const size_t sbytes = static_cast<size_t>(B) * H * D * 2 * D * sizeof(float);
    if (dstate_in && ((state_in && overlap(dstate_in, sbytes, state_in, sbytes)) ||
                      (dstate_out && overlap(dstate_in, sbytes, dstate_out, sbytes))))
        return fail(PRIME_ERR_ALIAS, "dstate_in overlaps state_in or dstate_out");
    g.step = 1;
    g.q_sl = g.k_sl = g.v_sl = 0;
    g.dy = dy->data; g.dt_dy = dy->dtype; g.dy_sb = dy->stride_b; g.dy_sh = dy->stride_h; g.dy_sl = 0;
    g.dstate_out = dstate_out;
    g.dq = dq; g.dk = dk; g.dv = dv; g.dbeta = dbeta; g.dalpha = dalpha; g.dstate_in = dstate_in;
    return check_hip(prime::launch_delta_gen_step_backward(g, static_cast<hipStream_t>(stream)),
                     "delta step backward launch");
}

int prime_delta_decode_step(const prime_tensor_t *q, const prime_tensor_t *k, const prime_tensor_t *v,
                            const float *beta, const float *alpha, int B, int H, int H_kv, int D,
                            float feat_eps, float bound, const float *state_in, float *state_out,
                            const prime_tensor_t *y, void *stream) {
    g_err[0] = 0;
    if (!q || !k || !v || !y || !q->data || !k->data || !v->data || !y->data || !beta || !alpha || !state_out)
        return fail(PRIME_ERR_INVALID_ARG, "prime_delta_decode_step: null argument");
    if (D != prime::kD) {
        // head dims below 64: the token-sequential kernel in the step's form
        prime::DeltaGenArgs g{};
        int rc;
        if ((rc = delta_gen_args(g, q, k, v, beta, alpha, B, H, H_kv, 1, D, 1, 1.0f, feat_eps, bound, state_in,
                                 state_out)))
            return rc;
        if (!valid_dtype(y->dtype)) return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported y dtype");
        g.step = 1;
        g.q_sl = g.k_sl = g.v_sl = 0;
        g.state_out = state_out;
        g.y = y->data; g.dt_y = y->dtype; g.y_sb = y->stride_b; g.y_sh = y->stride_h; g.y_sl = 0;
        return check_hip(prime::launch_delta_gen_forward(g, static_cast<hipStream_t>(stream)), "delta step launch");
    }
    if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv)
        return fail(PRIME_ERR_INVALID_ARG, "bad sizes B=%d H=%d H_kv=%d", B, H, H_kv);
    if (!valid_dtype(q->dtype) || !valid_dtype(k->dtype) || !valid_dtype(v->dtype) || !valid_dtype(y->dtype))
        return fail(PRIME_ERR_UNSUPPORTED_DTYPE, "unsupported dtype");
    if ((state_in && !aligned16(state_in)) || !aligned16(state_out))
        return fail(PRIME_ERR_MISALIGNED, "state buffers must be 16-byte aligned");
    const size_t sbytes = static_cast<size_t>(B) * H * prime::kDeltaStateBytes;
    if (state_in && state_in != state_out && overlap(state_in, sbytes, state_out, sbytes))
        return fail(PRIME_ERR_ALIAS, "state_out overlaps state_in (only a fully in-place state is allowed)");
    prime::DeltaStepArgs a{};
    a.q = q->data; a.k = k->data; a.v = v->data;
    a.q_sb = q->stride_b; a.q_sh = q->stride_h;
    a.k_sb = k->stride_b; a.k_sh = k->stride_h;
    a.v_sb = v->stride_b; a.v_sh = v->stride_h;
    a.dt_q = q->dtype; a.dt_k = k->dtype; a.dt_v = v->dtype;
    a.B = B; a.H = H; a.group = H / H_kv;
    a.beta = beta; a.alpha = alpha;
    a.feat_eps = feat_eps; a.bound = bound;
    a.state_in = state_in; a.state_out = state_out;
    a.y = y->data; a.dt_y = y->dtype; a.y_sb = y->stride_b; a.y_sh = y->stride_h;
    return check_hip(prime::launch_delta_step(a, static_cast<hipStream_t>(stream)), "delta step launch");
}

size_t prime_accumulate_workspace_size(int B, int H, int L) {
    if (B <= 0 || H <= 0 || L <= 0) return 0;
    int G, cps;
    prime::plan_segments(B * H, L, false, static_cast<size_t>(-1), &G, &cps);
    return static_cast<size_t>(B) * H * (G > 1 ? G : 1) * prime::kWsStride * sizeof(float);
}

size_t prime_chunked_prefill_workspace_size(int B, int H, int L, unsigned flags) {
    if (B <= 0 || H <= 0 || L <= 0) return 0;
    int G, cps;
    prime::plan_segments(B * H, L, (flags & PRIME_FLAG_DENSE_CLAMP) != 0, static_cast<size_t>(-1), &G, &cps);
    if (G > 1) return static_cast<size_t>(B) * H * G * prime::kWsStride * sizeof(float);
    if (flags & PRIME_FLAG_DENSE_CLAMP) return 0;
    int K, pcs;
    prime::plan_pairs(B * H, L, &K, &pcs);
    return K > 0 ? prime::pair_ws_bytes(K) : 0;
}

}  // extern "C"
