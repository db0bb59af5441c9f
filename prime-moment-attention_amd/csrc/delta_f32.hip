// Chunked gated delta-rule PRIME for fp32 inputs, in fp32 throughout
// (ChunkedGatedDeltaPrimeAttention computes the prefill in fp32,
// chunked_delta_prime.py:123-127 and :177-283).
//
// Same split as the bf16 path: a prep kernel over all chunks of a window
// solves T X = [V | diag(e^cum) Phi] = [U | W] and writes the chunk's transfer
// record (Y0 = A U, Z = diag(e^cum) Psi - A W, R0 = U^T diag(omega) Phi,
// M = W^T diag(omega) Phi, e^cum_63), and a scan kernel per (sequence, head)
// applies, chunk by chunk,
//   y = Y0 + Z S^T,   S' = e^cum_63 S - S M + R0,   then the Lyapunov clamp.
// Here every product is an fp32 MFMA (v_mfma_f32_16x16x4_f32: lane l holds
// A[l%16][k = l/16] and B[k = l/16][l%16]; the accumulator holds
// D[4(l/16) + r][l%16]) and the records hold fp32, so the result carries fp32
// rounding only (the bf16 path rounds its operands to bf16: about 5e-3
// relative for fp32 inputs).
//
// k-step mappings.  Contractions over the 128 features take, in k-step s
// (0..31), features {s, 32 + s, 64 + s, 96 + s} (k-slot g = l/16 holds
// feature 32g + s), so that a lane's 32 operands of one row are contiguous;
// contractions over the 64 tokens of a chunk take tokens 4s + g (s = 0..15).
// The scan's record operands are stored in the order the scan reads them:
//   MT [8 fb][64 lanes][32 s]   -M^T[16 fb + l%16][32 (l/16) + s]   (A operand)
//   ZB [4 tb][64 lanes][32 s]   Z^T[32 (l/16) + s][16 tb + l%16]     (B operand)
//   R0 [8 fb][4 dv][64 lanes]   R0^T accumulator tiles (4 floats per lane)
//   Y0 [4 dv][4 tb][64 lanes]   Y0^T accumulator tiles

#include "prefill_common.h"

namespace prime {
namespace {

constexpr int kP = 2 * kD;         // features
constexpr int kFMT = 0;
constexpr int kFZB = 65536;
constexpr int kFR0 = 98304;
constexpr int kFY0 = 131072;
constexpr int kFSC = 147456;       // e^cum_63
static_assert(kFSC + 16 <= static_cast<int>(kDeltaRecBytesF32), "record layout");

constexpr int kPF = kP + 4;        // phi / psi rows: 16-byte reads of 16 rows fall on distinct bank quads
constexpr int kPN = kC + 4;        // N, A rows
constexpr int kPX = 3 * kD + 16;   // X rows: scalar reads of 4 rows x 16 columns meet no bank twice

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }
__device__ __forceinline__ f32x4 ld4(const uint8_t *p) { return *reinterpret_cast<const f32x4 *>(p); }
__device__ __forceinline__ void st4(float *p, f32x4 v) { *reinterpret_cast<f32x4 *>(p) = v; }
__device__ __forceinline__ void st4(uint8_t *p, f32x4 v) { *reinterpret_cast<f32x4 *>(p) = v; }

}  // namespace

// ---------------------------------------------------------------------------
// Per-chunk transfer records, fp32.  One workgroup (256 threads) per (seq, chunk).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 1) void delta_prep_f32_kernel(const DeltaArgs a) {
    __shared__ __attribute__((aligned(16))) float sPhi[kC][kPF];
    __shared__ __attribute__((aligned(16))) float sPsi[kC][kPF];
    __shared__ __attribute__((aligned(16))) float sN[kC][kPN];   // N (strictly lower)
    __shared__ __attribute__((aligned(16))) float sA[kC][kPN];   // A (lower tiles only)
    __shared__ __attribute__((aligned(16))) float sX[kC][kPX];   // X = [U | W], one row per token
    __shared__ __attribute__((aligned(16))) float sCum[kC], sBeta[kC], sEc[kC], sOm[kC];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int unit = blockIdx.x;
    if (unit >= a.B * a.H * a.nw) return;
    const int seq = unit / a.nw, cw = unit - seq * a.nw;
    const int c = a.c0 + cw;
    const int b = seq / a.H, h = seq - b * a.H, hk = h / a.group;
    const float *qf = static_cast<const float *>(a.q);
    const float *kf = static_cast<const float *>(a.k);
    const float *vf = static_cast<const float *>(a.v);

    // ---- features (chunked_delta_prime.py:73-87): thread = (token tid/4, 16 dims)
    {
        const int i = tid >> 2, d0 = 16 * (tid & 3);
        const int t = c * kC + i;
        const bool valid = t < a.L;
        const int64_t tc = valid ? t : a.L - 1;
        const float *qp = qf + b * a.q_sb + h * a.q_sh + tc * a.q_sl + d0;
        const float *kp = kf + b * a.k_sb + hk * a.k_sh + tc * a.k_sl + d0;
        f32x4 qv[4], kv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            qv[j] = valid ? ld4(qp + 4 * j) : f32x4{0.f, 0.f, 0.f, 0.f};
            kv[j] = valid ? ld4(kp + 4 * j) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float k2 = kv[j][r] * kv[j][r];
                s1 += k2;
                s2 += k2 * k2;
            }
        s1 += xor_lane<1>(s1);
        s1 += xor_lane<2>(s1);
        s2 += xor_lane<1>(s2);
        s2 += xor_lane<2>(s2);
        const float r1 = 1.0f / fmaxf(sqrtf(s1), a.feat_eps);
        const float r2 = 0.70710678118654752f / fmaxf(sqrtf(s2), a.feat_eps);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4 p1, p2, q2;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p1[r] = kv[j][r] * r1;
                p2[r] = kv[j][r] * kv[j][r] * r2;
                q2[r] = 0.70710678118654752f * qv[j][r] * qv[j][r];
            }
            st4(&sPhi[i][d0 + 4 * j], p1);
            st4(&sPhi[i][kD + d0 + 4 * j], p2);
            st4(&sPsi[i][d0 + 4 * j], qv[j]);
            st4(&sPsi[i][kD + d0 + 4 * j], q2);
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

    // ---- N and A (:203-218, :248-250) on the 10 lower 16x16 tiles; wave w takes tiles w, w+4, w+8
    for (int ti = wave; ti < 10; ti += 4) {
        const int ib = ti < 1 ? 0 : ti < 3 ? 1 : ti < 6 ? 2 : 3;
        const int jb = ti - ib * (ib + 1) / 2;
        const float *pa = &sPhi[16 * ib + c16][32 * g];
        const float *sa = &sPsi[16 * ib + c16][32 * g];
        const float *pb = &sPhi[16 * jb + c16][32 * g];
        f32x4 gr = {0.f, 0.f, 0.f, 0.f}, ga = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q4 = 0; q4 < 8; ++q4) {
            const f32x4 x = ld4(pa + 4 * q4), y = ld4(sa + 4 * q4), z = ld4(pb + 4 * q4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                gr = mfma4(x[r], z[r], gr);
                ga = mfma4(y[r], z[r], ga);
            }
        }
        const int j = 16 * jb + c16;
        const float cj = sCum[j], bj = sBeta[j];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * ib + 4 * g + r;
            const float lam = i >= j ? expf(sCum[i] - cj) * bj : 0.f;
            sN[i][j] = i > j ? lam * gr[r] : 0.f;
            sA[i][j] = lam * ga[r];
        }
    }
    __syncthreads();

    // ---- solve T X = [V | diag(e^cum) Phi] (:242-245): thread = one of 192 columns,
    // forward substitution in registers, each row's sum in four partial sums.
    // The empty asm statements keep the compiler from hoisting all row reads
    // to the top or sinking a row's arithmetic to its last use (either spills).
    if (tid < kD + kP) {
        const int col = tid;
        const float *nbase = &sN[0][0];
        float x[kC];
        if (col < kD) {
            const float *vp = vf + b * a.v_sb + hk * a.v_sh + col;
#pragma unroll
            for (int i = 0; i < kC; ++i) {
                const int t = c * kC + i;
                x[i] = t < a.L ? vp[static_cast<int64_t>(t) * a.v_sl] : 0.f;
            }
        } else {
#pragma unroll
            for (int i = 0; i < kC; ++i) x[i] = sEc[i] * sPhi[i][col - kD];
        }
#pragma unroll
        for (int i = 1; i < kC; ++i) {
            int ro = i * kPN;
            asm volatile("" : "+v"(ro));
            float acc[4] = {x[i], 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < i; j += 4) {
                const f32x4 n4 = ld4(nbase + ro + j);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (j + e < i) acc[e] -= n4[e] * x[j + e];
            }
            float r = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            asm volatile("" : "+v"(r));
            x[i] = r;
        }
#pragma unroll
        for (int i = 0; i < kC; ++i) sX[i][col] = x[i];
    }
    __syncthreads();

    // ---- transfer record, in the scan's operand order
    uint8_t *rec = a.ws_rec + (static_cast<size_t>(seq) * a.nw + cw) * kDeltaRecBytesF32;
    const int w = wave;
    // Y0^T tiles (value block w, token block tb) = U^T A^T (A is zero above token 16 tb + 15)
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4 * (tb + 1); ++s) {
            const int j = 4 * s + g;
            acc = mfma4(sX[j][16 * w + c16], sA[16 * tb + c16][j], acc);
        }
        st4(rec + kFY0 + ((w * 4 + tb) * 64 + lane) * 16, acc);
    }
    // Z^T tiles (feature blocks 2w, 2w+1; token block tb) = diag(e^cum) Psi^T - W^T A^T
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int eb = 2 * w + hf;
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4 * (tb + 1); ++s) {
                const int j = 4 * s + g;
                acc = mfma4(sX[j][kD + 16 * eb + c16], sA[16 * tb + c16][j], acc);
            }
            const int tok = 16 * tb + c16;
            const float ec = sEc[tok];
            const f32x4 ps = ld4(&sPsi[tok][16 * eb + 4 * g]);
            f32x4 z;
#pragma unroll
            for (int r = 0; r < 4; ++r) z[r] = ec * ps[r] - acc[r];
            // feature 16 eb + 4g + r = 32 (eb/2) + (16 (eb&1) + 4g + r)
            st4(rec + kFZB + ((tb * 64 + 16 * (eb >> 1) + c16) * 32 + 16 * (eb & 1) + 4 * g) * 4, z);
        }
    }
    // R0^T tiles (feature blocks 2w, 2w+1; value block dv) = Phi^T diag(omega) U
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int eb = 2 * w + hf;
#pragma unroll
        for (int dv = 0; dv < 4; ++dv) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int j = 4 * s + g;
                acc = mfma4(sOm[j] * sPhi[j][16 * eb + c16], sX[j][16 * dv + c16], acc);
            }
            st4(rec + kFR0 + ((eb * 4 + dv) * 64 + lane) * 16, acc);
        }
    }
    // M tiles (rows f' in block ebp, columns f in blocks 2w, 2w+1) = W^T diag(omega) Phi,
    // stored negated as the scan's A operands of -M^T (row f, k-slot feature f')
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int eb = 2 * w + hf;
#pragma unroll 2
        for (int ebp = 0; ebp < 8; ++ebp) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int j = 4 * s + g;
                acc = mfma4(sX[j][kD + 16 * ebp + c16], sOm[j] * sPhi[j][16 * eb + c16], acc);
            }
            f32x4 m;
#pragma unroll
            for (int r = 0; r < 4; ++r) m[r] = -acc[r];
            st4(rec + kFMT + ((eb * 64 + 16 * (ebp >> 1) + c16) * 32 + 16 * (ebp & 1) + 4 * g) * 4, m);
        }
    }
    if (tid == 0) *reinterpret_cast<float *>(rec + kFSC) = sEc[kC - 1];
}

// ---------------------------------------------------------------------------
// Sequential scan over a window's chunks, fp32.  One workgroup of 8 waves per
// (sequence, head).  Wave w owns the state rows of feature block w (S^T tiles
// for the four value blocks, 128 MFMAs per chunk) and the y tiles of token
// block w/2, value blocks 2(w&1) and 2(w&1)+1 (64 MFMAs).  The state is
// exchanged through LDS in the operand order sS[dv][16 g + c][s] =
// S^T[32 g + s][16 dv + c]: one row of 32 contiguous floats per lane serves
// as the B operand of the state update and as the A operand of y.  Records
// are read one chunk ahead.  As in the bf16 scan, the Lyapunov scale of chunk
// c is applied inside chunk c+1 (one barrier per chunk):
//   y_c      = Y0 + sc_c (S~_c Z^T)
//   S~_{c+1} = sc_c (e^cum_63 S~_c - M^T S~_c) + R0,  sc_{c+1} from |S~_{c+1}|_F.
// ---------------------------------------------------------------------------
namespace {

constexpr int kScanWavesF = 8;
constexpr int kPS = 32 + 4;        // sS rows: 16-byte reads of 16 rows fall on distinct bank quads

// the part of a record read one chunk ahead (the Z^T operands, needed only
// by the last two value blocks, are read at the start of their chunk)
struct RecF {
    f32x4 mt[8];   // -M^T operands, k-steps 4q..4q+3
    f32x4 r0[4];   // R0^T tiles of feature block w
    f32x4 y0[2];   // Y0^T tiles of value blocks 2(w&1) + j, token block w/2
    float e63;
};

__device__ __forceinline__ void load_recf(RecF &R, const uint8_t *rc, int w, int lane) {
    const int tb = w >> 1, dvy = 2 * (w & 1);
#pragma unroll
    for (int q = 0; q < 8; ++q) R.mt[q] = ld4(rc + kFMT + ((w * 64 + lane) * 32 + 4 * q) * 4);
#pragma unroll
    for (int dv = 0; dv < 4; ++dv) R.r0[dv] = ld4(rc + kFR0 + ((w * 4 + dv) * 64 + lane) * 16);
#pragma unroll
    for (int j = 0; j < 2; ++j) R.y0[j] = ld4(rc + kFY0 + (((dvy + j) * 4 + tb) * 64 + lane) * 16);
    R.e63 = *reinterpret_cast<const float *>(rc + kFSC);
}

template <int DTY>
__device__ __forceinline__ void store_y4f(void *y, int64_t idx, f32x4 v) {
    if constexpr (DTY == PRIME_F32) {
        *reinterpret_cast<f32x4 *>(static_cast<float *>(y) + idx) = v;
    } else if constexpr (DTY == PRIME_BF16) {
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + idx) = uint2{pack2(v[0], v[1]), pack2(v[2], v[3])};
    } else {
        uint16_t *p = static_cast<uint16_t *>(y) + idx;
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = f32_to_h16_bits(v[r]);
    }
}

// state update of value block DV, and with Y the y tile of that value block
template <int DTY, int DV, bool Y>
__device__ __forceinline__ void scan_block(const DeltaArgs &a, const RecF &R, const f32x4 (&zb)[8], f32x4 (&st)[4],
                                           float sc, float &ss,
                                           const float (*sSb)[64][kPS], int lane, int g, int64_t ytok, bool yvalid,
                                           int64_t ybase) {
    f32x4 so[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) so[q] = ld4(&sSb[DV][lane][4 * q]);
    f32x4 x, p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = R.e63 * st[DV][r];
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            x = mfma4(R.mt[q][r], so[q][r], x);
            if constexpr (Y) p = mfma4(so[q][r], zb[q][r], p);
        }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        x[r] = sc * x[r] + R.r0[DV][r];
        ss += x[r] * x[r];
    }
    st[DV] = x;
    if constexpr (Y) {
        f32x4 yv;
#pragma unroll
        for (int r = 0; r < 4; ++r) yv[r] = R.y0[DV & 1][r] + sc * p[r];
        if (yvalid) store_y4f<DTY>(a.y, ybase + ytok * a.y_sl + 16 * DV + 4 * g, yv);
    }
}

// one chunk: the value blocks without y tiles first, so that the loads of
// the record's y operands have the longest time to arrive
template <int DTY>
__device__ __forceinline__ void scan_chunk_f32(const DeltaArgs &a, int w, const RecF &R, const f32x4 (&zb)[8],
                                               f32x4 (&st)[4], float sc,
                                               float &ss, const float (*sSb)[64][kPS], int lane, int g,
                                               int64_t ytok, bool yvalid, int64_t ybase) {
    if (w & 1) {
        scan_block<DTY, 0, false>(a, R, zb, st, sc, ss, sSb, lane, g, ytok, yvalid, ybase);
        scan_block<DTY, 1, false>(a, R, zb, st, sc, ss, sSb, lane, g, ytok, yvalid, ybase);
        scan_block<DTY, 2, true>(a, R, zb, st, sc, ss, sSb, lane, g, ytok, yvalid, ybase);
        scan_block<DTY, 3, true>(a, R, zb, st, sc, ss, sSb, lane, g, ytok, yvalid, ybase);
    } else {
        scan_block<DTY, 2, false>(a, R, zb, st, sc, ss, sSb, lane, g, ytok, yvalid, ybase);
        scan_block<DTY, 3, false>(a, R, zb, st, sc, ss, sSb, lane, g, ytok, yvalid, ybase);
        scan_block<DTY, 0, true>(a, R, zb, st, sc, ss, sSb, lane, g, ytok, yvalid, ybase);
        scan_block<DTY, 1, true>(a, R, zb, st, sc, ss, sSb, lane, g, ytok, yvalid, ybase);
    }
}

// One chunk of the window: `cur` holds its record share, `nxt` receives the next chunk's.
template <int DTY>
__device__ __forceinline__ void scan_step(const DeltaArgs &a, int cw, int w, int lane, int g, int c16,
                                          const uint8_t *rec0, const RecF &cur, RecF &nxt, f32x4 (&st)[4], float &sc,
                                          float (*sS)[4][64][kPS], float (*sRed)[kScanWavesF], int64_t ybase) {
    const int buf = cw & 1;
    f32x4 zb[8];
    const uint8_t *rz = rec0 + static_cast<size_t>(cw) * kDeltaRecBytesF32 + kFZB + ((w >> 1) * 64 + lane) * 128;
#pragma unroll
    for (int q = 0; q < 8; ++q) zb[q] = ld4(rz + 16 * q);
    load_recf(nxt, rec0 + static_cast<size_t>(min(cw + 1, a.nw - 1)) * kDeltaRecBytesF32, w, lane);
    const int64_t ytok = static_cast<int64_t>(a.c0 + cw) * kC + 16 * (w >> 1) + c16;
    float ss = 0.f;
    scan_chunk_f32<DTY>(a, w, cur, zb, st, sc, ss, sS[buf], lane, g, ytok, ytok < a.L, ybase);
#pragma unroll
    for (int dv = 0; dv < 4; ++dv) st4(&sS[buf ^ 1][dv][16 * (w >> 1) + c16][16 * (w & 1) + 4 * g], st[dv]);
    ss = wave_sum(ss);
    if (lane == 0) sRed[buf][w] = ss;
    __syncthreads();
    // ---- Lyapunov clamp (:266-270), kept as the pending scale of the state
    sc = 1.0f;
    if (a.bound > 0.f) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < kScanWavesF; ++i) t += sRed[buf][i];
        sc = fminf(1.0f, a.bound / (sqrtf(t) + 1e-6f));
    }
}

}  // namespace

template <int DTY>
__global__ __launch_bounds__(kScanWavesF * kWave, 1) void delta_scan_f32_kernel(const DeltaArgs a) {
    __shared__ __attribute__((aligned(16))) float sS[2][4][64][kPS];  // [buf][dv][16 g + c][s]
    __shared__ float sRed[2][kScanWavesF];

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int seq = blockIdx.x;
    if (seq >= a.B * a.H) return;
    const int b = seq / a.H, h = seq - b * a.H;
    const size_t sofs = static_cast<size_t>(seq) * kD * kP;
    const uint8_t *rec0 = a.ws_rec + static_cast<size_t>(seq) * a.nw * kDeltaRecBytesF32;

    // ---- state entering the window: st[dv][r] = S[d = 16dv + c16][e = 16w + 4g + r]
    const float *src = a.first ? a.state_in : a.ws_state;
    f32x4 st[4];
#pragma unroll
    for (int dv = 0; dv < 4; ++dv)
        st[dv] = src ? ld4(src + sofs + (16 * dv + c16) * kP + 16 * w + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
    // feature 16w + 4g + r = 32 (w/2) + (16 (w&1) + 4g + r)
#pragma unroll
    for (int dv = 0; dv < 4; ++dv) st4(&sS[0][dv][16 * (w >> 1) + c16][16 * (w & 1) + 4 * g], st[dv]);
    float sc = 1.0f;
    RecF ra, rb;
    load_recf(ra, rec0, w, lane);
    __syncthreads();

    const int64_t ybase = b * a.y_sb + h * a.y_sh;
    // chunks in pairs, the two record register sets swapping roles (no copies)
    int cw = 0;
    for (; cw + 1 < a.nw; cw += 2) {
        scan_step<DTY>(a, cw, w, lane, g, c16, rec0, ra, rb, st, sc, sS, sRed, ybase);
        scan_step<DTY>(a, cw + 1, w, lane, g, c16, rec0, rb, ra, st, sc, sS, sRed, ybase);
    }
    if (cw < a.nw) scan_step<DTY>(a, cw, w, lane, g, c16, rec0, ra, rb, st, sc, sS, sRed, ybase);

    // ---- state leaving the window (the pending scale applied)
    float *dst = a.last ? a.state_out : a.ws_state;
    if (dst) {
#pragma unroll
        for (int dv = 0; dv < 4; ++dv) {
            f32x4 x = st[dv];
#pragma unroll
            for (int r = 0; r < 4; ++r) x[r] *= sc;
            st4(dst + sofs + (16 * dv + c16) * kP + 16 * w + 4 * g, x);
        }
    }
}

void launch_delta_prep_f32(const DeltaArgs &a, hipStream_t s) {
    const TimerEvents t = timer_events(PRIME_KERNEL_DELTA_PREP);
    hipExtLaunchKernelGGL(delta_prep_f32_kernel, dim3(a.B * a.H * a.nw), dim3(256), 0, s, t.start, t.stop, 0, a);
    if (hipPeekAtLastError() != hipSuccess) timer_drop(t);
}

void launch_delta_scan_f32(const DeltaArgs &a, hipStream_t s) {
    const TimerEvents t = timer_events(PRIME_KERNEL_DELTA_SCAN);
    const dim3 grid(a.B * a.H), block(kScanWavesF * kWave);
    if (a.dt_y == PRIME_BF16)
        hipExtLaunchKernelGGL(delta_scan_f32_kernel<PRIME_BF16>, grid, block, 0, s, t.start, t.stop, 0, a);
    else if (a.dt_y == PRIME_F32)
        hipExtLaunchKernelGGL(delta_scan_f32_kernel<PRIME_F32>, grid, block, 0, s, t.start, t.stop, 0, a);
    else
        hipExtLaunchKernelGGL(delta_scan_f32_kernel<PRIME_F16>, grid, block, 0, s, t.start, t.stop, 0, a);
    if (hipPeekAtLastError() != hipSuccess) timer_drop(t);
}

}  // namespace prime
