// Kernel argument blocks and launchers shared by the kernels and the C-ABI layer.
#pragma once

#include <hip/hip_ext.h>

#include "prime_common.h"

namespace prime {

struct DecodeArgs {
    const void *q, *k, *v;
    int64_t q_sb, q_sh, k_sb, k_sh, v_sb, v_sh;
    int dt_q, dt_k, dt_v;
    int B, H, group;
    const float *decay;
    float eps;
    const float *s0i, *s1i, *s2i, *k0i, *k1i, *k2i;  // all null => zero state
    float *s0o, *s1o, *s2o, *k0o, *k1o, *k2o;
    void *y;
    int dt_y;
    int64_t y_sb, y_sh;
    int y_frag, y_ks;  // y in the fragment layout [B padded / 16][H D / 32][512] (bf16)
    // optional prologue: q <- LN(q) * q_scale, k <- LN(k) (LN over the head dim,
    // affine; qn_w == nullptr: no LN), LN output rounded to dt_q / dt_k
    const void *qn_w, *qn_b, *kn_w, *kn_b;
    int dt_norm;
    float ln_eps, q_scale;
    // selective form: decay per (sequence, head) [B, H] instead of per head,
    // k scaled by k_scale[h] (beta), S2 / K2 carrying the 1/2 (selective != 0)
    const float *decay_bh;
    const float *k_scale;
    int selective;
    // selective, decay_bh == null: l = exp(-clamp(softplus(step)) / tau)
    const void *step;
    int64_t step_sb;
    int dt_step;
    const float *tau;
    float step_min, step_max;
    // hybrid-window pieces: no_update = read out the incoming state only
    // (k, v unused, no state written); no_readout = update only (q, y unused)
    int no_update, no_readout;
};

// Residual add + RMSNorm rows (norm.hip).
struct RmsNormArgs {
    void *x;              // [rows, hidden], updated in place when delta is given
    const void *delta;    // [rows, hidden] or null
    const void *weight;   // [hidden]
    void *out;            // [rows, hidden]
    int rows, hidden, dt;
    float eps;
};
struct ArgmaxArgs {
    const void *logits;   // n rows of `vocab` logits, row i at logits + i * stride_n elements
    int64_t *out;         // [n]
    int64_t stride_n;
    int n, vocab, dt;
    int vector;           // rows 16-byte aligned: 16-byte loads, element-wise tail
};
hipError_t launch_argmax_rows(const ArgmaxArgs &a, hipStream_t stream);

// Per-head LayerNorm (+ scale) of projected q or k rows (norm.hip).
struct HeadNormArgs {
    const void *x;        // [B, H, L, D] view, element strides below
    void *out;            // same shape, own strides; may be x itself
    const void *weight, *bias;  // [D] each, or null (no LayerNorm: scale only)
    int64_t x_sb, x_sh, x_sl, o_sb, o_sh, o_sl;
    int B, H, L, dt, dt_norm;
    float ln_eps, scale;
    int D;                // 64 (norm.hip), or below 64 (generic_d.hip)
};
hipError_t launch_head_layernorm(const HeadNormArgs &a, hipStream_t stream);
hipError_t launch_generic_head_layernorm(const HeadNormArgs &a, hipStream_t stream);

// Skinny bf16 linear layer y = epilogue(x w^T) (gemm.hip).
struct LinearArgs {
    const void *x, *w;
    void *y;
    int64_t ldx, ldw, ldy;  // row strides in elements
    int M, N, K, epilogue;
    const void *r;          // PRIME_EPILOGUE_RESIDUAL: y = r + x w^T (r may be y)
    int64_t ldr;
    int rms;                // rows scaled by rsqrt(mean_k x^2 + rms_eps) before the epilogue
    float rms_eps;
};
hipError_t launch_linear(const LinearArgs &a, hipStream_t stream);
// few-row kernel with the RMS prologue (gemm_rows.hip): N % 32 == 0, K % 128 == 0
bool linear_rows_fits(const LinearArgs &a);
hipError_t launch_linear_rows(const LinearArgs &a, hipStream_t stream);
// 256 x 256-tile kernel for many rows (gemm_tile.hip): M >= 256, N % 256 == 0, K % 64 == 0
bool linear_tile_fits(const LinearArgs &a);
hipError_t launch_linear_tile(const LinearArgs &a, hipStream_t stream);

// Fragment-layout projections (gemm_frag.hip): x [Mp/16][K/32][512] and
// w [N/16][K/32][512] bf16 blocks; y row-major [M, ldy] or fragment layout
// [Mp/16][N/32][512]; r in y's layout.
struct FragArgs {
    const uint16_t *x, *w, *r;
    uint16_t *y;               // may be null when tokens is set
    const float *bias;         // fp32 [N] or null
    uint64_t *keys;            // argmax tile keys [Mp][gn] or null
    int64_t *tokens;           // argmax per row [M] or null (then keys is null)
    int M, Mp, N, K, KS;       // KS = K / 32
    int64_t ldy;
    int epilogue, rms, out_frag;
    float rms_eps;
    int mt, nt, gm, gn;        // tile (16-row blocks) and grid (row tiles, column tiles)
    int persistent;            // lm_head kernel: mt = m-blocks per row half, nt = row halves,
                               // gn = column-tile ranges per row tile
};
void frag_tile(int Mp, int N, int K, int *MT, int *NT);
void frag_plan(FragArgs &a);  // fills persistent, mt, nt, gm, gn from M, Mp, N, K
bool frag_k_supported(int K);
hipError_t launch_linear_frag(const FragArgs &a, hipStream_t stream);
hipError_t launch_pack_frag(const uint16_t *src, int64_t ld, const int64_t *idx, int M, int Mp, int K,
                            int64_t nrows_src, uint16_t *out, hipStream_t stream);

constexpr int kNormMaxGroups = 16;  // 4-element groups per lane: hidden <= 4 * 64 * 16 = 4096
hipError_t launch_add_rmsnorm(const RmsNormArgs &a, hipStream_t stream);
hipError_t launch_gelu(const void *x, void *y, int64_t n, int dt, hipStream_t stream);
hipError_t launch_selective_log_decay(const void *step, int dt, int64_t sb, int64_t sl, const float *tau, float dmin,
                                      float dmax, int B, int H, int L, float *out, hipStream_t stream);

struct PrefillArgs {
    const void *q, *k, *v;
    int64_t q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl;
    int dt_in;  // PRIME_BF16 or PRIME_F32 (all three inputs)
    int B, H, group, L;
    const float *decay;
    float eps;
    int dense_clamp;
    const float *s0i, *s1i, *s2i, *k0i, *k1i, *k2i;  // null => zero state
    float *s0o, *s1o, *s2o, *k0o, *k1o, *k2o;        // null => no final state
    void *y;
    int dt_y;
    int64_t y_sb, y_sh, y_sl;
    // segment-parallel scan (G > 1): each sequence is cut into G segments of
    // `cps` chunks; ws holds one packed fp32 state slot per (sequence, segment)
    int G, cps;
    int nseg_launch;  // segments covered by the current launch (G or G - 1)
    float *ws;
    // selective form (null for the base form): per-token natural-log decays
    // [B, H, L] replace `decay`; k is scaled by k_scale[h] (beta) and the
    // S2 / K2 state components carry the 1/2 of the module's convention
    const float *log_decay;
    const float *k_scale;
    // accumulate only (no q, no y): every segment's contribution from zero,
    // then an inclusive scan that writes the final state
    int accumulate;
    // segment-entry states only (G > 1): the state-only pass and the
    // exclusive scan, leaving the state entering segment s in slot s
    int states_only;
    // QK LayerNorm on load (bf16 inputs): each q and k row is normalised with
    // the per-column weight and bias (the module's nn.LayerNorm, eps ln_eps) and
    // rounded to bf16, and q is then scaled by q_scale and rounded again;
    // qn_w null: q is only scaled; kn_w null: k is used as it is
    int qk_norm;
    const void *qn_w, *qn_b, *kn_w, *kn_b;
    int dt_norm;
    float ln_eps, q_scale;
    // paired split (bf16 fused kernel, G == 1, more sequences than CUs): the
    // first npair sequences run as two workgroups, chunks [0, pcs) and
    // [pcs, NC).  Grid order: the npair first parts, the other sequences
    // whole, then the npair second parts.  A first part writes its end state
    // to ws slot `seq` and then pflag[seq] = epoch (release); the second part
    // waits for that value (acquire, bounded), resets the flag to 0 and
    // starts from the slot.
    int npair, pcs;
    unsigned long long *pflag;
    unsigned long long epoch;
};

// packed fp32 state slot in the workspace: S1 | S2 | S0 | K1 | K2 | K0
constexpr int kWsS1 = 0, kWsS2 = 4096, kWsS0 = 8192, kWsK1 = 8256, kWsK2 = 8320, kWsK0 = 8384;
constexpr int kWsStride = 8448;  // floats per slot (33,792 bytes)
constexpr int kWsElems = 8385;   // state floats per slot
constexpr int kWsDecay = 8385;   // selective: the segment's log2 decay (not part of the scanned state)

// Backward of the chunked prefill (prefill_bwd.hip): the adjoints of q, k,
// v and of the incoming state for output adjoints dy (and of the final state).
struct BwdArgs {
    // segments per sequence (G > 1: slot s of `ws` holds the state entering
    // segment s for the dq pass, then the dual state at its end for the dk/dv pass)
    int G, cps;
    float *ws;
    const void *q, *k, *v, *dy;
    int64_t q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, dy_sb, dy_sh, dy_sl;
    int dt_in, dt_dy;  // q/k/v: PRIME_BF16 or PRIME_F32; dy: any
    int B, H, L;
    const float *decay;
    float eps;
    const float *s0i, *s1i, *s2i, *k0i, *k1i, *k2i;         // incoming state (null => zero)
    const float *ds0o, *ds1o, *ds2o, *dk0o, *dk1o, *dk2o;   // adjoint of the final state (null => 0)
    void *dq, *dk, *dv;
    int dt_g;
    int64_t g_sb, g_sh, g_sl;                               // strides of dq, dk, dv
    float *ds0i, *ds1i, *ds2i, *dk0i, *dk1i, *dk2i;         // adjoint of the incoming state (null => none)
    float *inv_den, *g_den;                                 // [B*H, L] fp32, written by the dq pass
    // the dense branch's double clamp with an incoming state (G == 1): the dq
    // pass carries the call's own K moments apart from the incoming ones and
    // writes, per sequence, kBwdCorr floats to kcorr (the incoming K adjoint's
    // share that the inner clamp withholds from the call's tokens: features
    // [K1; K2/2], then K0), which the dk/dv pass adds to that adjoint
    int dense_in;
    float *kcorr;
    // selective form (fp32 passes only): per-token natural-log decays logd
    // [B*H, L] and the key scale kscale [H] (k enters as kscale[h] k); the
    // states in the selective convention (S2, K2 carry the 1/2).  Outputs:
    // dlogd [B*H, L] (the log decays' adjoint) and dkscale [B*H] (the key
    // scale's adjoint per sequence).  Scratch: pq [B*H, L], fin [B*H].
    const float *logd, *kscale;
    float *dlogd, *dkscale, *pq, *fin;
};
constexpr int kBwdCorr = 132;  // floats per sequence in BwdArgs::kcorr (128 features, K0, padding)

hipError_t launch_prefill_backward(const BwdArgs &a, hipStream_t stream);
// fp32 inputs: the fp32 dq and dk/dv passes, one workgroup per sequence (prefill_bwd_f32.hip)
hipError_t launch_prefill_backward_f32(const BwdArgs &a, hipStream_t stream);
// segments per sequence for the backward: enough (sequence, segment) units to
// fill per_cu workgroups per CU (2 for the bf16 passes, 1 for the fp32 ones),
// at least 8 chunks per segment
void plan_backward_segments(int S, int L, int *G, int *cps, int per_cu = 2);
// the reverse scan over segments of the backward's dual states (prefill_bwd.hip)
hipError_t launch_bwd_dual_scan(const BwdArgs &a, hipStream_t stream);
int device_cus();  // compute units of the current device (cached)

hipError_t launch_decode_step(const DecodeArgs &a, hipStream_t stream);
hipError_t launch_prefill(PrefillArgs a, hipStream_t stream);
// the scan over a prefill's segments: slot s <- the state entering segment s
// (prefill.hip)
hipError_t launch_segment_scan(const PrefillArgs &a, hipStream_t stream);
// selective form with fp32 inputs: one fp32 kernel over each sequence's chunks (selective_f32.hip)
hipError_t launch_selective_f32(const PrefillArgs &a, hipStream_t stream);
// segments per sequence for the launch plan, given the workspace the caller has
void plan_segments(int S, int L, bool dense_clamp, size_t ws_bytes, int *G, int *cps);
// paired split for the bf16 fused kernel when S exceeds the CU count (K = 0:
// none pays); its workspace: K slots, then K 8-byte flags
void plan_pairs(int S, int L, int *K, int *pcs);
inline size_t pair_ws_bytes(int K) {
    return static_cast<size_t>(K) * (kWsStride * sizeof(float) + sizeof(unsigned long long));
}
// spin bound of a second part's wait (iterations of a ~0.2 us sleep plus a load)
constexpr int kPairSpin = 1 << 22;

// Chunked gated delta-rule prefill (delta.hip).
struct DeltaArgs {
    const void *q, *k, *v;
    int64_t q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl;
    int dt_in;  // PRIME_BF16 or PRIME_F32 (all three inputs)
    int B, H, group, L;
    const float *beta, *alpha;  // [B, H, L]
    float decay_pad, feat_eps, bound;
    const float *state_in;      // [B, H, D, 2D] or null
    float *state_out;           // [B, H, D, 2D] or null
    void *y;
    int dt_y;
    int64_t y_sb, y_sh, y_sl;
    float *ws_state;            // [B*H][D*2D]: state between windows
    uint8_t *ws_rec;            // [B*H][window][record]
    int c0, nw;                 // window: chunks c0 .. c0 + nw - 1
    int first, last;            // window is the first / last of the call
};

// Head dims below 64 (generic_d.hip): one wavefront per (sequence, head).
struct GenericArgs {
    const void *q, *k, *v;
    int64_t q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl;
    int dt_q, dt_k, dt_v;
    int B, H, group, L, D;
    const float *decay;
    float eps;
    int dense_clamp;
    const float *s0i, *s1i, *s2i, *k0i, *k1i, *k2i;  // incoming state or null
    float *s0o, *s1o, *s2o, *k0o, *k1o, *k2o;        // final state or null
    void *y;
    int dt_y;
    int64_t y_sb, y_sh, y_sl;
    int qk_norm;  // forward only: LayerNorm weights (may be null) and q scale
    const void *qn_w, *qn_b, *kn_w, *kn_b;
    int dt_norm;
    float ln_eps, q_scale;
    // backward
    const void *dy;
    int dt_dy;
    int64_t dy_sb, dy_sh, dy_sl;
    const float *ds0, *ds1, *ds2, *dk0, *dk1, *dk2;  // adjoint of the final state or null
    void *dq, *dk, *dv;
    int dt_g;
    int64_t g_sb, g_sh, g_sl;
    float *dsi0, *dsi1, *dsi2, *dki0, *dki1, *dki2;  // adjoint of the incoming state or null
    float *ws;                                        // [B*H][L][2]
    // selective form: a decay per token, k weighted by k_scale[h] (beta), S2
    // and K2 carrying the 1/2; decays from log_decay [B*H][L] (natural log), or
    // for one token (the decode step) from decay_bh [B*H] or the step-size
    // pre-activations (l = exp(-clamp(softplus(step)) / tau), each stage
    // rounded to dt_step)
    int selective;
    const float *log_decay, *k_scale, *decay_bh, *tau;
    const void *step;
    int64_t step_sb;
    int dt_step;
    float step_min, step_max;
    float *dlogd;    // backward: [B*H][L], the log decays' adjoint
    float *dkscale;  // backward: [B*H], beta's adjoint per sequence
    float *pq;       // backward scratch: [B*H][L]
};
constexpr int kGenericMaxD = 63;
hipError_t launch_generic_prefill(const GenericArgs &a, hipStream_t stream);
hipError_t launch_generic_backward(const GenericArgs &a, hipStream_t stream);

// Backward of the delta-rule prefill (delta_bwd.hip): q, k, v, dy strided
// [B, H(kv), L, D]; gradients fp32 contiguous, dk / dv per query head
// ([B, H, L, D]); ws = [B*H][chunks][D*2D] fp32 (the state entering each chunk).
struct DeltaBwdArgs {
    const void *q, *k, *v, *dy;
    int64_t q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, dy_sb, dy_sh, dy_sl;
    int dt_in, dt_dy;
    int B, H, group, L;
    const float *beta, *alpha;  // [B, H, L]
    float decay_pad, feat_eps, bound;
    const float *state_in;      // [B, H, D, 2D] or null
    const float *dstate_out;    // [B, H, D, 2D] or null
    float *dq, *dk, *dv;        // [B, H, L, D]
    float *dbeta, *dalpha;      // [B, H, L]
    float *dstate_in;           // [B, H, D, 2D] or null
    float *ws;
};
hipError_t launch_delta_backward(const DeltaBwdArgs &a, hipStream_t stream);

// The delta rule at head dims up to 64 and any chunk size (delta_gen.hip):
// one wavefront per (sequence, head), the recurrence token by token.
struct DeltaGenArgs {
    const void *q, *k, *v, *dy;
    int64_t q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, dy_sb, dy_sh, dy_sl;
    int dt_q, dt_k, dt_v, dt_dy;
    int B, H, group, L, D, chunk;
    int step;                   // 1: the decode step's form (L == 1)
    const float *beta, *alpha;  // [B, H, L]
    float decay_pad, feat_eps, bound;
    const float *state_in;      // [B, H, D, 2D] or null
    float *state_out;           // [B, H, D, 2D] or null
    void *y;
    int dt_y;
    int64_t y_sb, y_sh, y_sl;
    const float *dstate_out;    // backward: [B, H, D, 2D] or null
    float *dq, *dk, *dv;        // [B, H, L, D] fp32 contiguous
    float *dbeta, *dalpha;      // [B, H, L]
    float *dstate_in;           // [B, H, D, 2D] or null
    float *ws;                  // backward workspace (delta_gen_backward_ws_bytes)
};
constexpr int kDeltaGenMaxD = 64;
hipError_t launch_delta_gen_forward(const DeltaGenArgs &a, hipStream_t stream);
hipError_t launch_delta_gen_backward(const DeltaGenArgs &a, hipStream_t stream);
hipError_t launch_delta_gen_step_backward(const DeltaGenArgs &a, hipStream_t stream);
size_t delta_gen_backward_ws_bytes(int B, int H, int L, int D, int chunk);

// One delta-rule decode step (delta.hip).
struct DeltaStepArgs {
    const void *q, *k, *v;
    int64_t q_sb, q_sh, k_sb, k_sh, v_sb, v_sh;
    int dt_q, dt_k, dt_v;
    int B, H, group;
    const float *beta, *alpha;  // [B, H]
    float feat_eps, bound;
    const float *state_in;      // [B, H, D, 2D] or null
    float *state_out;
    void *y;
    int dt_y;
    int64_t y_sb, y_sh;
};

constexpr int kDeltaChunk = 64;
constexpr size_t kDeltaStateBytes = static_cast<size_t>(kD) * 2 * kD * sizeof(float);  // one (b,h) state
constexpr size_t kDeltaRecBytes = 73984;         // per-chunk transfer record, bf16 inputs (multiple of 256)
constexpr size_t kDeltaRecBytesF32 = 147712;     // per-chunk transfer record, fp32 inputs (fp32 operands)
constexpr int kDeltaDefaultWindow = 192;         // record chunks of the recommended workspace (3 windows of 64)

// Record bytes per chunk for inputs of dtype `dt_in`.
inline size_t delta_rec_bytes(int dt_in) { return dt_in == PRIME_F32 ? kDeltaRecBytesF32 : kDeltaRecBytes; }

// Launch the delta prefill over every window (prep + scan per window); cap =
// chunks of record space per (sequence, head) in the workspace.
hipError_t launch_delta_prefill(DeltaArgs a, int NC, int cap, hipStream_t stream);
hipError_t launch_delta_step(const DeltaStepArgs &a, hipStream_t stream);
// fp32-input prep and scan kernels of one window (delta_f32.hip)
void launch_delta_prep_f32(const DeltaArgs &a, hipStream_t s);
void launch_delta_scan_f32(const DeltaArgs &a, hipStream_t s);

// Launch timer (the C-ABI prime_timer_* calls).  timer_events(kernel) hands
// out the event pair for one launch of `kernel` while that kernel is being
// timed (both null otherwise); the launch passes them to hipExtLaunchKernelGGL,
// which stamps them with the dispatch's own start and end times (no marker
// packets between kernels).  timer_drop() withdraws a pair whose launch failed.
struct TimerEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
TimerEvents timer_events(int kernel);
void timer_drop(const TimerEvents &t);

// bf16-input prefill kernels (prefill_bf16.hip): the state-only segment pass
// (256 threads) or the fused chunk loop (512 threads) over `grid` workgroups.
void launch_prefill_bf16(const PrefillArgs &a, bool state_only, int grid, hipStream_t stream, TimerEvents t);

}  // namespace prime
