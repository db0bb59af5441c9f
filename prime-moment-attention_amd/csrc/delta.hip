// Chunked gated delta-rule PRIME (ChunkedGatedDeltaPrimeAttention,
// chunked_delta_prime.py:25-283) on gfx950.
//
// Per (sequence, head) the state S is [D = 64 values][P = 128 features]; a
// 64-token chunk with features psi_i, phi_i, values v_i, write rates beta_i
// and cumulative log-decays cum_i does (chunked_delta_prime.py:199-270)
//   E   = T^-1 (V - diag(e^cum) Phi S^T),   T = I + N,
//         N_ij = [i>j] e^(cum_i - cum_j) (phi_i . phi_j) beta_j
//   y   = A E + diag(e^cum) Psi S^T,  A_ij = [i>=j] e^(cum_i - cum_j) (psi_i . phi_j) beta_j
//   S'  = e^cum_63 S + E^T diag(omega) Phi,  omega_j = beta_j e^(cum_63 - cum_j)
//   S'' = S' min(1, bound / (|S'|_F + 1e-6))
// Everything but S depends on the chunk alone, so the work splits into
//   delta_prep_kernel (all chunks in parallel): the solve X = T^-1 [V | diag(e^cum) Phi]
//     = [U | W], then the chunk's transfer record
//       Y0 = A U,  Z = diag(e^cum) Psi - A W,  R0 = U^T diag(omega) Phi,
//       M = W^T diag(omega) Phi,  e^cum_63
//     so that  y = Y0 + Z S^T  and  S' = e^cum_63 S - S M + R0;
//   delta_scan_kernel (one workgroup per (sequence, head), chunks in order):
//     y^T = Y0^T + S Z^T and S'^T = e^cum_63 S^T - M^T S^T + R0^T on bf16 MFMA,
//     the state S^T held in fp32 accumulators, then the clamp (one barrier).
// The scan's MFMA operands of S are its accumulators repacked: lane l holds
// S^T[16eb + 4g + r][d = 16dw + l%16] (g = l/16), and the 8 k-slots of an
// operand take rows 4g..4g+3 of two adjacent 16-row tiles, a fixed permutation
// of the contraction index that the prep kernel applies to the other operand.
// Records are written in exactly the lane order the scan reads them.
//
// The sequence is processed in windows of chunks (prep then scan per window),
// so the workspace is bounded by the window, not by L.

#include <mutex>

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kP = 2 * kD;        // features
constexpr int kP136 = kP + 8;     // 128-wide rows, 16-byte row reads
constexpr int kP72 = kD + 8;      // 64-wide rows, 16 / 8-byte row reads
constexpr int kRecMT = 0;         // -M^T A operands   [8 eb'][4 ks][64 lanes] x 16 B
constexpr int kRecZB = 32768;     // Z^T B operands    [4 tb][4 ks][64 lanes] x 16 B
constexpr int kRecR0 = 49152;     // R0^T acc tiles    [8 eb][4 dw][64 lanes] x 8 B (bf16x4)
constexpr int kRecY0 = 65536;     // Y0^T acc tiles    [4 tb][4 dw][64 lanes] x 8 B
constexpr int kRecSC = 73728;     // e^cum_63 (fp32)

static_assert(kRecSC + 16 <= static_cast<int>(kDeltaRecBytes), "record layout");

typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

// 16 consecutive inputs of one row (bf16 or fp32; 32- or 64-byte aligned), zero when !valid
__device__ __forceinline__ void load16(const void *p, int64_t off, int dt, bool valid, float (&o)[16]) {
    if (!valid) {
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] = 0.f;
        return;
    }
    if (dt == PRIME_BF16) {
        const u32x4 *s = reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p) + off);
        const u32x4 a = s[0], b = s[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(a[i] << 16);
            o[2 * i + 1] = __uint_as_float(a[i] & 0xFFFF0000u);
            o[8 + 2 * i] = __uint_as_float(b[i] << 16);
            o[8 + 2 * i + 1] = __uint_as_float(b[i] & 0xFFFF0000u);
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

__device__ __forceinline__ uint2 pack4(f32x4 x) { return uint2{pack2(x[0], x[1]), pack2(x[2], x[3])}; }

__device__ __forceinline__ f32x4 unpack4(uint2 u) {
    return f32x4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u), __uint_as_float(u.y << 16),
                 __uint_as_float(u.y & 0xFFFF0000u)};
}

__device__ __forceinline__ bf16x8 pack8x(f32x4 a, f32x4 b) {
    return as_bf16x8(u32x4{pack2(a[0], a[1]), pack2(a[2], a[3]), pack2(b[0], b[1]), pack2(b[2], b[3])});
}

// operand of 8 tokens (k-slots 0..3: rows r0..r0+3, 4..7: rows r0+16..r0+19) of
// one column, read transposed from a row-major bf16 tile
__device__ __forceinline__ bf16x8 tr8(const uint16_t *p0, int pitch) {
    const uint2 a = lds_tr(p0), b = lds_tr(p0 + 16 * pitch);
    return as_bf16x8(u32x4{a.x, a.y, b.x, b.y});
}

// 4 + 4 bf16 of one row at columns c and c + 16 (the same k-slot permutation)
__device__ __forceinline__ bf16x8 row8p(const uint16_t *row, int c) {
    const uint2 a = *reinterpret_cast<const uint2 *>(row + c), b = *reinterpret_cast<const uint2 *>(row + c + 16);
    return as_bf16x8(u32x4{a.x, a.y, b.x, b.y});
}

}  // namespace

// ---------------------------------------------------------------------------
// Per-chunk transfer records.  One workgroup (256 threads) per (seq, chunk).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 1) void delta_prep_kernel(const DeltaArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sPhi[kC][kP136];  // phi rows (bf16)
    __shared__ __attribute__((aligned(16))) uint16_t sPsi[kC][kP136];  // psi rows
    __shared__ __attribute__((aligned(16))) uint16_t sV[kC][kP72];     // v rows
    __shared__ __attribute__((aligned(16))) float sN[kC][kC + 4];      // N (strictly lower), fp32
    __shared__ __attribute__((aligned(16))) uint16_t sA[kC][kP72];     // A (lower), bf16
    // the solve's results, transposed (one row per column of X = [U | W]):
    __shared__ __attribute__((aligned(16))) uint16_t sUt[kD][kP72];    // U^T, U = T^-1 V
    __shared__ __attribute__((aligned(16))) uint16_t sUwt[kD][kP72];   // (diag(omega) U)^T
    __shared__ __attribute__((aligned(16))) uint16_t sWt[kP][kP72];    // W^T, W = T^-1 diag(e^cum) Phi
    __shared__ __attribute__((aligned(16))) uint16_t sWwt[kP][kP72];   // (diag(omega) W)^T
    __shared__ __attribute__((aligned(16))) float sCum[kC], sBeta[kC], sEc[kC], sOm[kC];  // cum, beta, e^cum, omega

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int tr_r = c16 >> 2, tr_c = 4 * (c16 & 3);
    const int Sq = a.B * a.H;
    const int unit = blockIdx.x;
    if (unit >= Sq * a.nw) return;
    const int seq = unit / a.nw, cw = unit - seq * a.nw;
    const int c = a.c0 + cw;
    const int b = seq / a.H, h = seq - b * a.H, hk = h / a.group;

    // ---- features (chunked_delta_prime.py:73-87): thread = (token tid/4, 16 dims)
    {
        const int i = tid >> 2, d0 = 16 * (tid & 3);
        const int t = c * kC + i;
        const bool valid = t < a.L;
        const int tc = valid ? t : a.L - 1;
        const int64_t qo = b * a.q_sb + h * a.q_sh + tc * a.q_sl + d0;
        const int64_t ko = b * a.k_sb + hk * a.k_sh + tc * a.k_sl + d0;
        const int64_t vo = b * a.v_sb + hk * a.v_sh + tc * a.v_sl + d0;
        float qv[16], kv[16], vv[16];
        load16(a.q, qo, a.dt_in, valid, qv);
        load16(a.k, ko, a.dt_in, valid, kv);
        load16(a.v, vo, a.dt_in, valid, vv);
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float k2 = kv[e] * kv[e];
            s1 += k2;
            s2 += k2 * k2;
        }
        s1 += xor_lane<1>(s1);
        s1 += xor_lane<2>(s1);
        s2 += xor_lane<1>(s2);
        s2 += xor_lane<2>(s2);
        const float r1 = 1.0f / fmaxf(sqrtf(s1), a.feat_eps);
        const float r2 = 0.70710678118654752f / fmaxf(sqrtf(s2), a.feat_eps);
        float ph[16], ph2[16], ps2[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            ph[e] = kv[e] * r1;
            ph2[e] = kv[e] * kv[e] * r2;
            ps2[e] = 0.70710678118654752f * qv[e] * qv[e];
        }
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int o = 8 * hf;
            *reinterpret_cast<u32x4 *>(&sPhi[i][d0 + o]) = u32x4{pack2(ph[o], ph[o + 1]), pack2(ph[o + 2], ph[o + 3]),
                                                                  pack2(ph[o + 4], ph[o + 5]), pack2(ph[o + 6], ph[o + 7])};
            *reinterpret_cast<u32x4 *>(&sPhi[i][kD + d0 + o]) =
                u32x4{pack2(ph2[o], ph2[o + 1]), pack2(ph2[o + 2], ph2[o + 3]), pack2(ph2[o + 4], ph2[o + 5]),
                      pack2(ph2[o + 6], ph2[o + 7])};
            *reinterpret_cast<u32x4 *>(&sPsi[i][d0 + o]) = u32x4{pack2(qv[o], qv[o + 1]), pack2(qv[o + 2], qv[o + 3]),
                                                                  pack2(qv[o + 4], qv[o + 5]), pack2(qv[o + 6], qv[o + 7])};
            *reinterpret_cast<u32x4 *>(&sPsi[i][kD + d0 + o]) =
                u32x4{pack2(ps2[o], ps2[o + 1]), pack2(ps2[o + 2], ps2[o + 3]), pack2(ps2[o + 4], ps2[o + 5]),
                      pack2(ps2[o + 6], ps2[o + 7])};
            *reinterpret_cast<u32x4 *>(&sV[i][d0 + o]) = u32x4{pack2(vv[o], vv[o + 1]), pack2(vv[o + 2], vv[o + 3]),
                                                                pack2(vv[o + 4], vv[o + 5]), pack2(vv[o + 6], vv[o + 7])};
        }
    }
    // ---- cumulative log-decay (:199-201), padding tokens: beta 0, alpha decay_pad (:186-189)
    if (wave == 0) {
        const int t = c * kC + lane;
        const bool valid = t < a.L;
        const int64_t o = static_cast<int64_t>(seq) * a.L + t;
        const float bt = valid ? a.beta[o] : 0.f;
        const float al = valid ? a.alpha[o] : a.decay_pad;
        float cum = logf(fminf(fmaxf(al, 1e-5f), 1.0f));
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) {
            const float x = __shfl_up(cum, s, kWave);
            if (lane >= s) cum += x;
        }
        const float cend = __shfl(cum, 63, kWave);
        sCum[lane] = cum;
        sBeta[lane] = bt;
        sEc[lane] = expf(cum);
        sOm[lane] = bt * expf(cend - cum);
    }
    __syncthreads();

    // ---- N and A (:203-218, :248-250): row block of wave w, column blocks jb <= w
    {
        const int w = wave;
        bf16x8 fa[4], fs[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            fa[ks] = as_bf16x8(lds128(&sPhi[16 * w + c16][32 * ks + 8 * g]));
            fs[ks] = as_bf16x8(lds128(&sPsi[16 * w + c16][32 * ks + 8 * g]));
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            f32x4 gr = {0.f, 0.f, 0.f, 0.f}, ga = {0.f, 0.f, 0.f, 0.f};
            if (jb <= w) {
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const bf16x8 fb = as_bf16x8(lds128(&sPhi[16 * jb + c16][32 * ks + 8 * g]));
                    gr = mfma(fa[ks], fb, gr);
                    ga = mfma(fs[ks], fb, ga);
                }
            }
            const int j = 16 * jb + c16;
            const float cj = sCum[j], bj = sBeta[j];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * w + 4 * g + r;
                const float lam = i >= j ? expf(sCum[i] - cj) * bj : 0.f;
                sN[i][j] = i > j ? lam * gr[r] : 0.f;
                sA[i][j] = f32_to_bf16_bits(lam * ga[r]);
            }
        }
    }
    __syncthreads();

    // ---- solve T X = [V | diag(e^cum) Phi] (:242-245): thread = one of 192 columns,
    // forward substitution in fp32 registers, each row's sum in four partial
    // sums (four short dependent chains instead of one long one).  Row i of N
    // is read as broadcast 16-byte LDS reads; its offset and the row's result
    // pass through empty asm statements so that the compiler neither hoists
    // all 504 reads to the top nor sinks the rows' arithmetic to their last
    // use (either spills).  The column is then stored transposed, 16 bytes at
    // a time.
    if (tid < kD + kP) {
        const int col = tid;
        const float *nbase = &sN[0][0];
        float x[kC];
#pragma unroll
        for (int i = 0; i < kC; ++i)
            x[i] = col < kD ? bf16_bits_to_f32(sV[i][col]) : sEc[i] * bf16_bits_to_f32(sPhi[i][col - kD]);
#pragma unroll
        for (int i = 1; i < kC; ++i) {
            int ro = i * (kC + 4);
            asm volatile("" : "+v"(ro));
            float acc[4] = {x[i], 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < i; j += 4) {
                const f32x4 n4 = *reinterpret_cast<const f32x4 *>(nbase + ro + j);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (j + e < i) acc[e] -= n4[e] * x[j + e];
            }
            float r = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            asm volatile("" : "+v"(r));  // x[i] is final here (no sinking into later rows)
            x[i] = r;
        }
        uint16_t *dx = col < kD ? &sUt[col][0] : &sWt[col - kD][0];
        uint16_t *dw = col < kD ? &sUwt[col][0] : &sWwt[col - kD][0];
#pragma unroll
        for (int i0 = 0; i0 < kC; i0 += 8) {
            const f32x4 o0 = *reinterpret_cast<const f32x4 *>(&sOm[i0]);
            const f32x4 o1 = *reinterpret_cast<const f32x4 *>(&sOm[i0 + 4]);
            *reinterpret_cast<u32x4 *>(dx + i0) = u32x4{pack2(x[i0], x[i0 + 1]), pack2(x[i0 + 2], x[i0 + 3]),
                                                        pack2(x[i0 + 4], x[i0 + 5]), pack2(x[i0 + 6], x[i0 + 7])};
            *reinterpret_cast<u32x4 *>(dw + i0) =
                u32x4{pack2(o0[0] * x[i0], o0[1] * x[i0 + 1]), pack2(o0[2] * x[i0 + 2], o0[3] * x[i0 + 3]),
                      pack2(o1[0] * x[i0 + 4], o1[1] * x[i0 + 5]), pack2(o1[2] * x[i0 + 6], o1[3] * x[i0 + 7])};
        }
    }
    __syncthreads();

    // ---- transfer record, in the scan's lane order
    uint8_t *rec = a.ws_rec + (static_cast<size_t>(seq) * a.nw + cw) * kDeltaRecBytes;
    const int w = wave;
    // Y0^T tile (d-block w, token block tb) = U^T A^T
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            if (kt == 1 && tb < 2) continue;  // A is lower triangular
            const bf16x8 ua = row8p(&sUt[16 * w + c16][0], 32 * kt + 4 * g);
            const bf16x8 ab = row8p(&sA[16 * tb + c16][0], 32 * kt + 4 * g);
            acc = mfma(ua, ab, acc);
        }
        *reinterpret_cast<uint2 *>(rec + kRecY0 + ((tb * 4 + w) * 64 + lane) * 8) = pack4(acc);
    }
    // Z^T tiles (feature blocks 2w, 2w+1; token block tb) = diag(e^cum) Psi^T - W^T A^T
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        f32x4 zt[2];
        const int i = 16 * tb + c16;
        const float ec = sEc[i];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int eb = 2 * w + hf;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                if (kt == 1 && tb < 2) continue;
                const bf16x8 wa = row8p(&sWt[16 * eb + c16][0], 32 * kt + 4 * g);
                const bf16x8 ab = row8p(&sA[i][0], 32 * kt + 4 * g);
                acc = mfma(wa, ab, acc);
            }
            const f32x4 ps = unpack4(*reinterpret_cast<const uint2 *>(&sPsi[i][16 * eb + 4 * g]));
#pragma unroll
            for (int r = 0; r < 4; ++r) zt[hf][r] = ec * ps[r] - acc[r];
        }
        *reinterpret_cast<bf16x8 *>(rec + kRecZB + ((tb * 4 + w) * 64 + lane) * 16) = pack8x(zt[0], zt[1]);
    }
    // R0^T tiles (feature blocks 2w, 2w+1; every d-block) = Phi^T diag(omega) U
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int eb = 2 * w + hf;
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const bf16x8 pa = tr8(&sPhi[32 * kt + 4 * g + tr_r][16 * eb + tr_c], kP136);
                const bf16x8 ub = row8p(&sUwt[16 * dw + c16][0], 32 * kt + 4 * g);
                acc = mfma(pa, ub, acc);
            }
            *reinterpret_cast<uint2 *>(rec + kRecR0 + ((eb * 4 + dw) * 64 + lane) * 8) = pack4(acc);
        }
    }
    // -M^T as the scan's A operands: M tiles (rows e in blocks 2w, 2w+1; columns e')
    // = (diag(omega) W)^T Phi, packed two row blocks per k-step
#pragma unroll
    for (int ebp = 0; ebp < 8; ++ebp) {
        f32x4 m[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int eb = 2 * w + hf;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const bf16x8 wa = row8p(&sWwt[16 * eb + c16][0], 32 * kt + 4 * g);
                const bf16x8 pb = tr8(&sPhi[32 * kt + 4 * g + tr_r][16 * ebp + tr_c], kP136);
                acc = mfma(wa, pb, acc);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) m[hf][r] = -acc[r];
        }
        *reinterpret_cast<bf16x8 *>(rec + kRecMT + ((ebp * 4 + w) * 64 + lane) * 16) = pack8x(m[0], m[1]);
    }
    if (tid == 0) *reinterpret_cast<float *>(rec + kRecSC) = sEc[kC - 1];
}

// ---------------------------------------------------------------------------
// Sequential scan over a window's chunks.  One workgroup of 8 waves per
// (sequence, head) in two roles, one wave of each per SIMD:
//   state waves 0..3 carry the recurrence: wave s owns the state rows of
//     feature blocks 2s and 2s+1 (S^T tiles for every value block dv: 32
//     MFMAs per chunk) and publishes them as bf16 MFMA operand packs;
//   y waves 4..7 compute the output off that chain: wave 4+t the y tiles of
//     token block t for all four value blocks (16 MFMAs per chunk) from the
//     same packs, and write the previous chunk's y out.
// Only the state update carries into the next chunk, so the y work overlaps
// the state waves' chain instead of lengthening it.  Each wave loads only its
// role's share of each chunk's record, into registers, one chunk ahead,
// through a buffer descriptor (a fixed per-lane offset and scalar offsets: no
// per-load address arithmetic).  Pack (dv, ks) = rows 4g..4g+3 of feature
// blocks 2ks and 2ks+1 at value column 16dv + l%16, written whole by state
// wave ks.  The Lyapunov scale of chunk c is applied inside chunk c+1 (the
// packs hold the unscaled state), so one barrier per chunk suffices:
//   y_c      = Y0 + sc_c (S~_c Z^T)
//   S~_{c+1} = sc_c (e^cum_63 S~_c - M^T S~_c) + R0,  sc_{c+1} from |S~_{c+1}|_F.
// ---------------------------------------------------------------------------
namespace {

constexpr int kScanWaves = 8;
constexpr int kStateWaves = 4;             // waves 0..3: the state; 4..7: y
constexpr int kYThreads = (kScanWaves - kStateWaves) * kWave;
constexpr int kBufWord3 = 0x00020000;  // raw buffer descriptor, word 3 (gfx9 family)

// a state wave's share of a chunk record, in registers
struct RecS {
    bf16x8 mt[2][4];  // -M^T A operands: feature blocks 2s + fi, k-step ks
    uint2 r0[2][4];   // R0^T tiles: feature blocks 2s + fi, value block dv
    float e63;
};

// a y wave's share: the Z^T B operands and the Y0^T tiles of its token block
// (a token block per y wave: each wave loads a quarter of Z, where a value
// block per wave had every y wave load all of it -- 48 KB of the CU's 120 KB
// of record loads per chunk were such duplicates, and the loads' issue
// through the CU's memory pipeline was the longest phase of the y waves'
// chunk, which is the chain's critical path)
struct RecY {
    bf16x8 zb[4];  // k-step ks
    uint2 y0[4];   // value block dv
};

__device__ __forceinline__ bf16x8 bload16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return as_bf16x8(__builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0)));
}

__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// `ro`: byte offset of the chunk's record inside the window (uniform)
__device__ __forceinline__ void load_recs(RecS &R, __amdgpu_buffer_rsrc_t rs, int ro, int sw, int lane) {
    const int v16 = lane * 16, v8 = lane * 8;
#pragma unroll
    for (int fi = 0; fi < 2; ++fi)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) R.mt[fi][ks] = bload16(rs, v16, ro + kRecMT + ((2 * sw + fi) * 4 + ks) * 1024);
#pragma unroll
    for (int fi = 0; fi < 2; ++fi)
#pragma unroll
        for (int dv = 0; dv < 4; ++dv) R.r0[fi][dv] = bload8(rs, v8, ro + kRecR0 + ((2 * sw + fi) * 4 + dv) * 512);
    R.e63 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, 0, ro + kRecSC, 0));
}

__device__ __forceinline__ void load_recy(RecY &R, __amdgpu_buffer_rsrc_t rs, int ro, int tb, int lane) {
    const int v16 = lane * 16, v8 = lane * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) R.zb[ks] = bload16(rs, v16, ro + kRecZB + (tb * 4 + ks) * 1024);
#pragma unroll
    for (int dv = 0; dv < 4; ++dv) R.y0[dv] = bload8(rs, v8, ro + kRecY0 + (tb * 4 + dv) * 512);
}

template <int DTY>
__device__ __forceinline__ void store_y4(uint8_t *p, f32x4 v) {
    if constexpr (DTY == PRIME_BF16) {
        *reinterpret_cast<uint2 *>(p) = pack4(v);
    } else if constexpr (DTY == PRIME_F32) {
        *reinterpret_cast<f32x4 *>(p) = v;
    } else {
        uint16_t *h = reinterpret_cast<uint16_t *>(p);
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = f32_to_h16_bits(v[r]);
    }
}

// y of one chunk is staged in LDS, [64 tokens][64 values] of the output dtype
// with rows padded by 16 bytes (16-byte aligned rows whose starts move four
// banks per row, so the tile writes of 16 rows meet no bank twice), and
// written to global memory in the next chunk as whole 16-byte row segments.
// Direct stores of the accumulator tiles (8 bytes per lane over 16 rows)
// were the scan's largest cost.
template <int DTY>
struct YStage {
    static constexpr int es = DTY == PRIME_F32 ? 4 : 2;
    static constexpr int pitch = kD * es + 16;  // bytes per token row
    static constexpr int bytes = kC * pitch;    // one chunk
};

// Write a staged chunk of y (LDS) to global memory: thread t of `nt` takes
// 16-byte segments t, t + nt, ... of the chunk's rows.  GUARD skips tokens at
// or past L; only the call's last chunk can hold such tokens, and only the
// write after the loop can reach it, so the writes inside the loop carry no
// condition (a conditional store would leave the compiler to count
// outstanding memory operations for both paths, and its conservative count
// would then wait for the store at the next record wait).
template <int DTY, bool GUARD, int NT = kYThreads>
__device__ __forceinline__ void y_write(const DeltaArgs &a, int c, const uint8_t *ystage, uint8_t *ychunk,
                                        int64_t yrow_bytes, int t) {
    using YS = YStage<DTY>;
    constexpr int segs = kD * YS::es / 16;  // 16-byte segments per row
    static_assert((kC * segs) % NT == 0, "whole segments per thread");
    // a fixed trip count, so that the compiler counts this thread's stores exactly
#pragma unroll
    for (int j = 0; j < kC * segs / NT; ++j) {
        const int i = t + j * NT;
        const int row = i / segs, sg = i - row * segs;
        if (!GUARD || c * kC + row < a.L)
            *reinterpret_cast<u32x4 *>(ychunk + row * yrow_bytes + 16 * sg) =
                *reinterpret_cast<const u32x4 *>(ystage + row * YS::pitch + 16 * sg);
    }
}

// the pending Lyapunov scale of the state entering the next chunk (every wave)
__device__ __forceinline__ float clamp_scale(const DeltaArgs &a, const float *red) {
    if (!(a.bound > 0.f)) return 1.0f;
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kStateWaves; ++i) t += red[i];
    return fminf(1.0f, a.bound / (sqrtf(t) + 1e-6f));
}

// One chunk of a state wave.  `cur` holds this chunk's record share; `nxt2`
// receives the share of the chunk after the next one: the state waves keep
// three register sets in rotation, so each share is loaded two chunk periods
// before its use (with one, the chain waited on the memory latency of every
// chunk's share: 4.38 ms against 3.50 ms at config 5 with no loads at all).
__device__ __forceinline__ void state_chunk(const DeltaArgs &a, int cw, int sw, int lane, __amdgpu_buffer_rsrc_t rs,
                                            f32x4 (&st)[2][4], float &sc, const RecS &cur, RecS &nxt2,
                                            bf16x8 (*sPk)[4][4][64], float (*sRed)[kStateWaves]) {
    const int buf = cw & 1;
    // share of chunk cw + 2 (clamped to the window: the duplicate is unused),
    // one load instruction after every two MFMAs below: issued as one group,
    // the 17 loads stalled the wave ~900 cycles before its first MFMA
    const int ro2 = min(cw + 2, a.nw - 1) * static_cast<int>(kDeltaRecBytes);
    nxt2.e63 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, 0, ro2 + kRecSC, 0));
    bf16x8 pk[4][4];
#pragma unroll
    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) pk[dv][ks] = sPk[buf][dv][ks][lane];
    // ---- S~'^T = sc (e^cum_63 S~^T - M^T S~^T) + R0^T on feature blocks 2sw, 2sw + 1:
    // the eight accumulator chains (value block x feature block) interleaved
    // k-step by k-step, so that no MFMA waits for the one before it (two
    // chains at a time left the matrix unit idle between dependent issues)
    float ss = 0.f;
    f32x4 x[4][2];
#pragma unroll
    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
        for (int fi = 0; fi < 2; ++fi)
#pragma unroll
            for (int r = 0; r < 4; ++r) x[dv][fi][r] = cur.e63 * st[fi][dv][r];
    const int v16 = lane * 16, v8 = lane * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int dv = 0; dv < 4; ++dv)
#pragma unroll
            for (int fi = 0; fi < 2; ++fi) {
                x[dv][fi] = mfma(cur.mt[fi][ks], pk[dv][ks], x[dv][fi]);
                __builtin_amdgcn_sched_barrier(0);
                const int q = (ks * 4 + dv) * 2 + fi;  // 0..31
                if (q & 1) {
                    const int l = q >> 1;  // 0..15: the -M^T operands, then the R0^T tiles
                    if (l < 8)
                        nxt2.mt[l >> 2][l & 3] = bload16(rs, v16, ro2 + kRecMT + ((2 * sw + (l >> 2)) * 4 + (l & 3)) * 1024);
                    else
                        nxt2.r0[(l - 8) >> 2][(l - 8) & 3] =
                            bload8(rs, v8, ro2 + kRecR0 + ((2 * sw + ((l - 8) >> 2)) * 4 + ((l - 8) & 3)) * 512);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
    // the pending Lyapunov scale of the state entering this chunk (its norm was
    // reduced in the previous chunk): read here, under the MFMAs, not before them
    sc = cw == 0 ? 1.0f : clamp_scale(a, sRed[buf ^ 1]);
#pragma unroll
    for (int dv = 0; dv < 4; ++dv) {
#pragma unroll
        for (int fi = 0; fi < 2; ++fi) {
            const f32x4 r0 = unpack4(cur.r0[fi][dv]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                x[dv][fi][r] = sc * x[dv][fi][r] + r0[r];
                ss += x[dv][fi][r] * x[dv][fi][r];
            }
            st[fi][dv] = x[dv][fi];
        }
        // pack (dv, sw) of the next chunk: rows 4g..4g+3 of both feature blocks
        const uint2 lo = pack4(x[dv][0]), hi = pack4(x[dv][1]);
        sPk[buf ^ 1][dv][sw][lane] = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
    }
    ss = wave_sum(ss);
    if (lane == 0) sRed[buf][sw] = ss;  // Lyapunov clamp (:266-270): applied in the next chunk
    __syncthreads();
}

// One chunk of a y wave: y^T tiles of token block tb (all value blocks) = Y0^T +
// sc S~ Z^T into the chunk's LDS stage, after writing the previous chunk's
// staged y (WRITE_PREV) to global memory.
template <int DTY, bool WRITE_PREV>
__device__ __forceinline__ void y_chunk(const DeltaArgs &a, int cw, int tb, int lane, int g, int c16,
                                        __amdgpu_buffer_rsrc_t rs, float &sc, const RecY &cur, RecY &nxt,
                                        bf16x8 (*sPk)[4][4][64], float (*sRed)[kStateWaves], uint8_t *sY,
                                        uint8_t *ychunk, int64_t yrow_bytes, int ty) {
    using YS = YStage<DTY>;
    const int buf = cw & 1;
    load_recy(nxt, rs, min(cw + 1, a.nw - 1) * static_cast<int>(kDeltaRecBytes), tb, lane);
    bf16x8 pk[4][4];
#pragma unroll
    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) pk[dv][ks] = sPk[buf][dv][ks][lane];
    uint8_t *ys = sY + buf * YS::bytes;
    f32x4 p[4];  // the four value blocks' chains, interleaved k-step by k-step
#pragma unroll
    for (int dv = 0; dv < 4; ++dv) p[dv] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int dv = 0; dv < 4; ++dv) p[dv] = mfma(pk[dv][ks], cur.zb[ks], p[dv]);
    sc = cw == 0 ? 1.0f : clamp_scale(a, sRed[buf ^ 1]);  // the scale of the state entering this chunk
#pragma unroll
    for (int dv = 0; dv < 4; ++dv) {
        const f32x4 y0 = unpack4(cur.y0[dv]);
        f32x4 yv;
#pragma unroll
        for (int r = 0; r < 4; ++r) yv[r] = y0[r] + sc * p[dv][r];
        store_y4<DTY>(ys + (16 * tb + c16) * YS::pitch + (16 * dv + 4 * g) * YS::es, yv);
    }
    // the previous chunk's y, staged before the last barrier: stored after this
    // chunk's use of `cur`, so that the wait for `cur` (loaded one chunk ago)
    // covers only stores issued a chunk ago, never the loads of `nxt` just issued
    if constexpr (WRITE_PREV)
        y_write<DTY, false>(a, a.c0 + cw - 1, sY + (buf ^ 1) * YS::bytes, ychunk - kC * yrow_bytes, yrow_bytes, ty);
    __syncthreads();
}

}  // namespace

template <int DTY>
__global__ __launch_bounds__(kScanWaves * kWave, 1) void delta_scan_kernel(const DeltaArgs a) {
    __shared__ __attribute__((aligned(16))) bf16x8 sPk[2][4][4][64];  // [buf][dv][ks][lane]
    __shared__ __attribute__((aligned(16))) uint8_t sY[2 * YStage<DTY>::bytes];  // y of two chunks
    __shared__ float sRed[2][kStateWaves];

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int seq = blockIdx.x;
    if (seq >= a.B * a.H) return;
    const int b = seq / a.H, h = seq - b * a.H;
    const size_t sofs = static_cast<size_t>(seq) * kD * kP;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        a.ws_rec + static_cast<size_t>(seq) * a.nw * kDeltaRecBytes, 0,
        static_cast<int>(static_cast<size_t>(a.nw) * kDeltaRecBytes), kBufWord3);
    float sc = 1.0f;  // pending Lyapunov scale of the state in the packs

    // the y rows of the window's first chunk, advanced by one chunk per step
    constexpr int es = YStage<DTY>::es;
    const int64_t yrow_bytes = a.y_sl * es;
    uint8_t *ychunk = static_cast<uint8_t *>(a.y) +
                      (b * a.y_sb + h * a.y_sh + static_cast<int64_t>(a.c0) * kC * a.y_sl) * es;
    const int64_t ystep = kC * yrow_bytes;

    if (w < kStateWaves) {
        const int sw = w;
        // ---- state entering the window: st[fi][dv][r] = S[d = 16dv + c16][e = 16(2sw + fi) + 4g + r]
        const float *src = a.first ? a.state_in : a.ws_state;
        f32x4 st[2][4];
#pragma unroll
        for (int fi = 0; fi < 2; ++fi)
#pragma unroll
            for (int dv = 0; dv < 4; ++dv)
                st[fi][dv] = src ? *reinterpret_cast<const f32x4 *>(src + sofs + (16 * dv + c16) * kP +
                                                                    16 * (2 * sw + fi) + 4 * g)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dv = 0; dv < 4; ++dv) {
            const uint2 lo = pack4(st[0][dv]), hi = pack4(st[1][dv]);
            sPk[0][dv][sw][lane] = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
        }
        RecS ra, rb, rc;
        load_recs(ra, rs, 0, sw, lane);
        load_recs(rb, rs, min(1, a.nw - 1) * static_cast<int>(kDeltaRecBytes), sw, lane);
        __syncthreads();
        int cw = 0;
        for (; cw + 2 < a.nw; cw += 3) {
            state_chunk(a, cw, sw, lane, rs, st, sc, ra, rc, sPk, sRed);
            state_chunk(a, cw + 1, sw, lane, rs, st, sc, rb, ra, sPk, sRed);
            state_chunk(a, cw + 2, sw, lane, rs, st, sc, rc, rb, sPk, sRed);
        }
        if (cw < a.nw) state_chunk(a, cw, sw, lane, rs, st, sc, ra, rc, sPk, sRed);
        if (cw + 1 < a.nw) state_chunk(a, cw + 1, sw, lane, rs, st, sc, rb, ra, sPk, sRed);
        // ---- state leaving the window (the pending scale applied)
        sc = clamp_scale(a, sRed[(a.nw - 1) & 1]);
        float *dst = a.last ? a.state_out : a.ws_state;
        if (dst) {
#pragma unroll
            for (int fi = 0; fi < 2; ++fi)
#pragma unroll
                for (int dv = 0; dv < 4; ++dv) {
                    f32x4 x = st[fi][dv];
#pragma unroll
                    for (int r = 0; r < 4; ++r) x[r] *= sc;
                    *reinterpret_cast<f32x4 *>(dst + sofs + (16 * dv + c16) * kP + 16 * (2 * sw + fi) + 4 * g) = x;
                }
        }
    } else {
        const int v = w - kStateWaves, ty = tid - kStateWaves * kWave;  // v: this wave's token block
        RecY ra, rb;
        load_recy(ra, rs, 0, v, lane);
        __syncthreads();
        // chunk 0 (no earlier y to write), then pairs of chunks writing the y of
        // the chunk before each
        y_chunk<DTY, false>(a, 0, v, lane, g, c16, rs, sc, ra, rb, sPk, sRed, sY, ychunk, yrow_bytes, ty);
        ychunk += ystep;
        int cw = 1;
        for (; cw + 1 < a.nw; cw += 2) {
            y_chunk<DTY, true>(a, cw, v, lane, g, c16, rs, sc, rb, ra, sPk, sRed, sY, ychunk, yrow_bytes, ty);
            y_chunk<DTY, true>(a, cw + 1, v, lane, g, c16, rs, sc, ra, rb, sPk, sRed, sY, ychunk + ystep,
                               yrow_bytes, ty);
            ychunk += 2 * ystep;
        }
        if (cw < a.nw) {
            y_chunk<DTY, true>(a, cw, v, lane, g, c16, rs, sc, rb, ra, sPk, sRed, sY, ychunk, yrow_bytes, ty);
            ychunk += ystep;
        }
        // the last chunk's y (staged before the last barrier)
        y_write<DTY, true>(a, a.c0 + a.nw - 1, sY + ((a.nw - 1) & 1) * YStage<DTY>::bytes, ychunk - ystep,
                           yrow_bytes, ty);
    }
}

// ---------------------------------------------------------------------------
// Decode step (chunked_delta_prime.py:140-176).  One wave per (b, h); lane d
// holds state row S[d][0..127].
// ---------------------------------------------------------------------------
constexpr int kStepWaves = 4;

__global__ __launch_bounds__(kStepWaves * 64) void delta_step_kernel(const DeltaStepArgs a) {
    __shared__ __attribute__((aligned(16))) float sPhi[kStepWaves][kP];
    __shared__ __attribute__((aligned(16))) float sPsi[kStepWaves][kP];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * kStepWaves + wave;
    const bool active = t < a.B * a.H;
    const int tt = active ? t : 0;
    const int b = tt / a.H, h = tt - b * a.H, hk = h / a.group;
    const float qv = load_elem(a.q, b * a.q_sb + h * a.q_sh + lane, a.dt_q);
    const float kv = load_elem(a.k, b * a.k_sb + hk * a.k_sh + lane, a.dt_k);
    const float vv = load_elem(a.v, b * a.v_sb + hk * a.v_sh + lane, a.dt_v);
    const float k2 = kv * kv;
    const float s1 = wave_sum(k2), s2 = wave_sum(k2 * k2);
    sPhi[wave][lane] = kv / fmaxf(sqrtf(s1), a.feat_eps);
    sPhi[wave][kD + lane] = 0.70710678118654752f * k2 / fmaxf(sqrtf(s2), a.feat_eps);
    sPsi[wave][lane] = qv;
    sPsi[wave][kD + lane] = 0.70710678118654752f * qv * qv;
    __syncthreads();
    const size_t so = static_cast<size_t>(tt) * kD * kP + static_cast<size_t>(lane) * kP;
    f32x4 s[kP / 4];
#pragma unroll
    for (int i = 0; i < kP / 4; ++i)
        s[i] = a.state_in ? *reinterpret_cast<const f32x4 *>(a.state_in + so + 4 * i) : f32x4{0.f, 0.f, 0.f, 0.f};
    float vhat = 0.f;
#pragma unroll
    for (int i = 0; i < kP / 4; ++i) {
        const f32x4 p = *reinterpret_cast<const f32x4 *>(&sPhi[wave][4 * i]);
#pragma unroll
        for (int r = 0; r < 4; ++r) vhat += s[i][r] * p[r];
    }
    const float bt = a.beta[tt], al = a.alpha[tt];
    const float err = bt * (vv - vhat);
    float ss = 0.f, yv = 0.f;
#pragma unroll
    for (int i = 0; i < kP / 4; ++i) {
        const f32x4 p = *reinterpret_cast<const f32x4 *>(&sPhi[wave][4 * i]);
        const f32x4 q = *reinterpret_cast<const f32x4 *>(&sPsi[wave][4 * i]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[i][r] = al * s[i][r] + err * p[r];
            ss += s[i][r] * s[i][r];
            yv += s[i][r] * q[r];
        }
    }
    ss = wave_sum(ss);
    const float sc = a.bound > 0.f ? fminf(1.0f, a.bound / (sqrtf(ss) + 1e-6f)) : 1.0f;
    if (active) {
#pragma unroll
        for (int i = 0; i < kP / 4; ++i) {
            f32x4 x = s[i];
#pragma unroll
            for (int r = 0; r < 4; ++r) x[r] *= sc;
            *reinterpret_cast<f32x4 *>(a.state_out + so + 4 * i) = x;
        }
        store_elem(a.y, b * a.y_sb + h * a.y_sh + lane, a.dt_y, sc * yv);
    }
}

namespace {

// Side stream and events for overlapping the prep of window w+1 with the scan
// of window w (the scan occupies one CU per (sequence, head); the prep fills
// the rest).  One set per (device, caller stream), created on first use
// outside any graph capture, default priority, kept for the life of the
// process.  A call holds its set's lock for its whole enqueue sequence, so
// that calls on different streams never share events and calls from several
// host threads on one stream do not interleave their records and waits.
// The record space is used as up to kRecParts parts of one window each: with
// three, the prep of window w+2 waits only for the scan of window w-1, so it
// runs a whole window ahead of the scan that reads it and the scan stream
// never stalls on a cross-stream event (with two, every window paid the event
// latency twice: prep waiting for the scan two windows back, then the scan
// for that prep).
constexpr int kRecParts = 3;

struct SideStream {
    int dev = -1;
    hipStream_t caller = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t start = nullptr, prep[kRecParts] = {nullptr, nullptr, nullptr}, scan[kRecParts] = {nullptr, nullptr, nullptr};
    std::mutex mu;
};

constexpr int kMaxSideStreams = 64;
std::mutex g_side_mu;
SideStream g_side[kMaxSideStreams];
int g_side_n = 0;

// The set of (current device, caller); null when it does not exist and may
// not be created now (capture in progress, or the table is full): the caller
// then runs the windows on its own stream alone.
SideStream *side_stream(hipStream_t caller, bool may_create) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(g_side_mu);
    for (int i = 0; i < g_side_n; ++i)
        if (g_side[i].dev == dev && g_side[i].caller == caller) return &g_side[i];
    if (!may_create || g_side_n >= kMaxSideStreams) return nullptr;
    SideStream &x = g_side[g_side_n];
    const unsigned f = hipEventDisableTiming;
    if (hipStreamCreateWithFlags(&x.s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&x.start, f) != hipSuccess) return nullptr;
    for (int i = 0; i < kRecParts; ++i)
        if (hipEventCreateWithFlags(&x.prep[i], f) != hipSuccess || hipEventCreateWithFlags(&x.scan[i], f) != hipSuccess)
            return nullptr;
    x.dev = dev;
    x.caller = caller;
    ++g_side_n;  // published last: a half-built set is never found
    return &x;
}

void launch_prep(const DeltaArgs &a, hipStream_t s) {
    if (a.dt_in == PRIME_F32) return launch_delta_prep_f32(a, s);
    const TimerEvents t = timer_events(PRIME_KERNEL_DELTA_PREP);
    hipExtLaunchKernelGGL(delta_prep_kernel, dim3(a.B * a.H * a.nw), dim3(256), 0, s, t.start, t.stop, 0, a);
    if (hipPeekAtLastError() != hipSuccess) timer_drop(t);
}

void launch_scan(const DeltaArgs &a, hipStream_t s) {
    if (a.dt_in == PRIME_F32) return launch_delta_scan_f32(a, s);
    const TimerEvents t = timer_events(PRIME_KERNEL_DELTA_SCAN);
    const dim3 grid(a.B * a.H), block(kScanWaves * kWave);
    if (a.dt_y == PRIME_BF16)
        hipExtLaunchKernelGGL(delta_scan_kernel<PRIME_BF16>, grid, block, 0, s, t.start, t.stop, 0, a);
    else if (a.dt_y == PRIME_F32)
        hipExtLaunchKernelGGL(delta_scan_kernel<PRIME_F32>, grid, block, 0, s, t.start, t.stop, 0, a);
    else
        hipExtLaunchKernelGGL(delta_scan_kernel<PRIME_F16>, grid, block, 0, s, t.start, t.stop, 0, a);
    if (hipPeekAtLastError() != hipSuccess) timer_drop(t);
}

DeltaArgs window_args(DeltaArgs a, int c0, int window, int NC, uint8_t *rec) {
    a.c0 = c0;
    a.nw = NC - c0 < window ? NC - c0 : window;
    a.first = c0 == 0;
    a.last = c0 + a.nw >= NC;
    a.ws_rec = rec;
    return a;
}

}  // namespace

// `cap` = chunks of record space per (sequence, head) in the workspace.  One
// window when the sequence fits; otherwise two record halves alternate: the
// prep of window w+1 (side stream) writes one half while the scan of window w
// (caller's stream) reads the other.
hipError_t launch_delta_prefill(DeltaArgs a, int NC, int cap, hipStream_t stream) {
    uint8_t *rec0 = a.ws_rec;
    SideStream *ss = nullptr;
    if (NC > cap && cap >= 2) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess) cs = hipStreamCaptureStatusActive;
        ss = side_stream(stream, cs == hipStreamCaptureStatusNone);
    }
    if (ss == nullptr) {
        // one window at a time on the caller's stream
        const int window = NC <= cap ? NC : cap;
        for (int c0 = 0; c0 < NC; c0 += window) {
            const DeltaArgs w = window_args(a, c0, window, NC, rec0);
            launch_prep(w, stream);
            launch_scan(w, stream);
        }
        return hipGetLastError();
    }
    std::lock_guard<std::mutex> lk(ss->mu);
    // parts of the record space: three when it holds three windows of 64
    // chunks or more (the recommended workspace does), else two halves
    const int nparts = cap >= kRecParts * 64 ? kRecParts : 2;
    const int part = cap / nparts;
    const size_t part_bytes = static_cast<size_t>(a.B) * a.H * part * delta_rec_bytes(a.dt_in);
    const int nwin = (NC + part - 1) / part;
    hipError_t e;
    if ((e = hipEventRecord(ss->start, stream)) != hipSuccess) return e;
    if ((e = hipStreamWaitEvent(ss->s, ss->start, 0)) != hipSuccess) return e;
    // preps of the first nparts - 1 windows: their parts are free
    for (int w = 0; w + 1 < nparts && w < nwin; ++w) {
        launch_prep(window_args(a, w * part, part, NC, rec0 + w * part_bytes), ss->s);
        if ((e = hipEventRecord(ss->prep[w], ss->s)) != hipSuccess) return e;
    }
    for (int w = 0; w < nwin; ++w) {
        const int pb = w % nparts;
        if ((e = hipStreamWaitEvent(stream, ss->prep[pb], 0)) != hipSuccess) return e;
        launch_scan(window_args(a, w * part, part, NC, rec0 + pb * part_bytes), stream);
        if ((e = hipEventRecord(ss->scan[pb], stream)) != hipSuccess) return e;
        const int wn = w + nparts - 1;  // the next window to prepare
        if (wn < nwin) {
            const int nb = wn % nparts;
            // its part was last read by the scan of window wn - nparts = w - 1
            if (w >= 1 && (e = hipStreamWaitEvent(ss->s, ss->scan[nb], 0)) != hipSuccess) return e;
            launch_prep(window_args(a, wn * part, part, NC, rec0 + nb * part_bytes), ss->s);
            if ((e = hipEventRecord(ss->prep[nb], ss->s)) != hipSuccess) return e;
        }
    }
    return hipGetLastError();
}

hipError_t launch_delta_step(const DeltaStepArgs &a, hipStream_t stream) {
    const int n = a.B * a.H;
    const TimerEvents t = timer_events(PRIME_KERNEL_DELTA_STEP);
    hipExtLaunchKernelGGL(delta_step_kernel, dim3((n + kStepWaves - 1) / kStepWaves), dim3(kStepWaves * 64), 0, stream,
                          t.start, t.stop, 0, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) timer_drop(t);
    return e;
}

}  // namespace prime
