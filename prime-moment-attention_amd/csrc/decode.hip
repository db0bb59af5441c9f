// Fused recurrent decode step for PRIME moment attention (gfx950).
//
// Semantics: attention.py:119-143 of the reference -- per (sequence, head) tile
//   S0 = l S0 + v ; S1 = l S1 + k v^T ; S2 = l S2 + (k*k) v^T
//   K0 = l K0 + 1 ; K1 = l K1 + k     ; K2 = l K2 + k*k
//   y  = (S0 + S1^T q + 1/2 S2^T q^2) / max(K0 + q.K1 + 1/2 q^2.K2, eps)
// read out with the UPDATED state.
//
// Design: the step is HBM-bound (67.6 KB of state traffic per tile against
// ~33 kflop).  W wavefronts own one tile (W = 4: each wave 16 key rows, 8 KB
// of S1/S2).  Lane l owns value columns 4*(l&15)..+3 and key rows
// {R0 + 4r + (l>>4)}, r = 0 .. 64/(4W) - 1, R0 = (64/W) * wave, so each
// wave-wide 128-bit load/store instruction touches four consecutive 256-byte
// rows: one contiguous 1 KB segment.  A wave issues its q/k/v loads and then
// every S1/S2 load of its rows before any math, so the QK-norm reductions run
// while the state is in flight; the update and readout are fused per row, and
// the key contraction ends with two cross-lane butterflies and one sum of the
// W waves' partial numerators through LDS.  Quarter tiles keep a wave at about
// 8 KB in flight and few registers (eight waves per SIMD): a launch at
// B = 256 x 12 heads is 12,288 short waves, and the memory system stays busy
// through the last of them (an in-place stream with whole or half tiles per
// wave ran 6-7 % slower on MI355X).  The S1/S2 loads and stores are
// nontemporal: each state byte is touched once per step, and with the
// streaming hint the stores leave the caches as the loads arrive.  The
// denominator is a wavefront reduction.  state_in may alias state_out: every
// element is read and written by the same lane.

#include "prime_kernels.h"

namespace prime {

constexpr int kDecodeWaves = 4;  // waves per tile (each a quarter of the key rows)

// x rounded to dtype dt (to nearest even), returned as fp32
__device__ __forceinline__ float round_to(float x, int dt) {
    if (dt == PRIME_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
    if (dt == PRIME_F16) return h16_bits_to_f32(f32_to_h16_bits(x));
    return x;
}

// Element idx of a q/k/v/step/norm operand as raw bits (2 or 4 bytes), and
// their value: the loads carry no conversion in a dtype branch, so a wave
// issues all of them, and its state loads, before it waits for any.
__device__ __forceinline__ uint32_t load_bits(const void *p, int64_t idx, int dt) {
    if (dt == PRIME_F32) return static_cast<const uint32_t *>(p)[idx];
    return static_cast<const uint16_t *>(p)[idx];
}
__device__ __forceinline__ float bits_value(uint32_t u, int dt) {
    if (dt == PRIME_BF16) return __uint_as_float(u << 16);
    if (dt == PRIME_F16) return h16_bits_to_f32(static_cast<uint16_t>(u));
    return __uint_as_float(u);
}

template <int W, bool HAS_IN>
__global__ __launch_bounds__(W * kWave) void decode_step_kernel(const DecodeArgs a) {
    constexpr int RPW = kD / W;  // key rows per wave
    constexpr int NR = RPW / 4;  // row iterations per lane
    __shared__ float sh[W][4][kD];     // per wave: q, k, v, updated S0
    __shared__ f32x4 sacc[W - 1][16];  // waves 1 .. W-1: readout numerators (row group 0 lanes)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x;  // the grid is exactly B * H tiles
    const int b = t / a.H, h = t - (t / a.H) * a.H, hk = h / a.group;
    const int rg = lane >> 4;  // row group: rows 4r + rg
    const int cg = lane & 15;  // column group: columns 4cg..4cg+3
    const size_t tb = static_cast<size_t>(t) * (kD * kD);
    const size_t tv = static_cast<size_t>(t) * kD;
    const int rb = RPW * wave;  // this wave's first key row

    // loads, all issued before the first wait: the token's q, k, v, the gate
    // and the QK-norm parameters, wave 0's small moments, then the S1/S2 rows
    uint32_t qb = 0, kb = 0, vb = 0, gb = 0, nqw = 0, nqb = 0, nkw = 0, nkb = 0;
    if (!a.no_readout) qb = load_bits(a.q, b * a.q_sb + h * a.q_sh + lane, a.dt_q);
    if (!a.no_update) {
        kb = load_bits(a.k, b * a.k_sb + hk * a.k_sh + lane, a.dt_k);
        vb = load_bits(a.v, b * a.v_sb + hk * a.v_sh + lane, a.dt_v);
    }
    if (!a.decay_bh && a.step) gb = load_bits(a.step, b * a.step_sb + h, a.dt_step);
    if (a.qn_w) {
        nqw = load_bits(a.qn_w, lane, a.dt_norm);
        nqb = load_bits(a.qn_b, lane, a.dt_norm);
        nkw = load_bits(a.kn_w, lane, a.dt_norm);
        nkb = load_bits(a.kn_b, lane, a.dt_norm);
    }
    float s0v = 0.f, k1v = 0.f, k2v = 0.f, k0v = 0.f;
    f32x4 r1[NR], r2[NR];
    if constexpr (HAS_IN) {
        if (wave == 0) {
            s0v = a.s0i[tv + lane];
            k1v = a.k1i[tv + lane];
            k2v = a.k2i[tv + lane];
            k0v = a.k0i[t];
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const size_t o = tb + (rb + 4 * r + rg) * kD + 4 * cg;
            r1[r] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.s1i + o));
            r2[r] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.s2i + o));
        }
    } else {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            r1[r] = f32x4{0.f, 0.f, 0.f, 0.f};
            r2[r] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }

    float qv = bits_value(qb, a.dt_q), kv = bits_value(kb, a.dt_k), vv = bits_value(vb, a.dt_v);
    if (a.qn_w) {
        // the module's QK LayerNorm (attention.py:96-98, biased variance),
        // output rounded to the input dtype as the module's LayerNorm returns it
        const float qm = wave_sum(qv) * (1.0f / kD), km = wave_sum(kv) * (1.0f / kD);
        const float qd = qv - qm, kd = kv - km;
        const float qr = rsqrtf(wave_sum(qd * qd) * (1.0f / kD) + a.ln_eps);
        const float kr = rsqrtf(wave_sum(kd * kd) * (1.0f / kD) + a.ln_eps);
        qv = qd * qr * bits_value(nqw, a.dt_norm) + bits_value(nqb, a.dt_norm);
        kv = kd * kr * bits_value(nkw, a.dt_norm) + bits_value(nkb, a.dt_norm);
        if (a.dt_q == PRIME_BF16) qv = bf16_bits_to_f32(f32_to_bf16_bits(qv));
        if (a.dt_k == PRIME_BF16) kv = bf16_bits_to_f32(f32_to_bf16_bits(kv));
    }
    qv *= a.q_scale;  // 1/sqrt(D) (attention.py:101); exact for powers of two
    if (a.k_scale) kv *= a.k_scale[h];  // selective: beta k (selective.py:394-400)
    // the 1/2 of the second-order term sits on the k side in the selective
    // state convention (S2 = 1/2 beta^2 sum k^2 v), on the q side otherwise
    const float h2k = a.selective ? 0.5f : 1.0f, h2q = a.selective ? 1.0f : 0.5f;

    float lam;
    if (a.decay_bh) {
        lam = a.decay_bh[b * a.H + h];
    } else if (a.step) {
        // selective gate (selective.py:368, 386): Delta = clamp(softplus(s)),
        // each stage rounded to the step dtype as the module's tensors are
        const float s = bits_value(gb, a.dt_step);
        float d = s > 20.f ? s : log1pf(expf(s));
        d = round_to(d, a.dt_step);
        d = round_to(fminf(fmaxf(d, a.step_min), a.step_max), a.dt_step);
        lam = expf(-d / a.tau[h]);
    } else if (!a.no_update) {
        lam = a.decay[h];
    } else {
        lam = 1.0f;  // readout only: the state as it is (k = v = 0 above)
    }

    // small moments (lane l owns element l; used by wave 0 only)
    const float s0n = lam * s0v + vv;
    const float k1n = lam * k1v + kv;
    const float k2n = lam * k2v + h2k * kv * kv;
    const float k0n = lam * k0v + (a.no_update ? 0.0f : 1.0f);
    sh[wave][0][lane] = qv;
    sh[wave][1][lane] = kv;
    sh[wave][2][lane] = vv;
    sh[wave][3][lane] = s0n;
    // each wave reads only its own rows of sh: a wave-local ordering suffices
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const f32x4 v4 = *reinterpret_cast<const f32x4 *>(&sh[wave][2][4 * cg]);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int row = rb + 4 * r + rg;
        const float kr = sh[wave][1][row];
        const float qr = sh[wave][0][row];
        const float kr2 = h2k * kr * kr;
        const float qh = h2q * qr * qr;
        f32x4 n1, n2;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            n1[c] = lam * r1[r][c] + kr * v4[c];
            n2[c] = lam * r2[r][c] + kr2 * v4[c];
            acc[c] += qr * n1[c] + qh * n2[c];
        }
        if (!a.no_update) {
            const size_t o = tb + row * kD + 4 * cg;
            __builtin_nontemporal_store(n1, reinterpret_cast<f32x4 *>(a.s1o + o));
            __builtin_nontemporal_store(n2, reinterpret_cast<f32x4 *>(a.s2o + o));
        }
    }
    // sum the four row groups (lanes cg, cg+16, cg+32, cg+48), then the W waves
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        acc[c] += __shfl_xor(acc[c], 16, kWave);
        acc[c] += __shfl_xor(acc[c], 32, kWave);
    }
    if (wave > 0 && rg == 0) sacc[wave - 1][cg] = acc;
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
        const f32x4 o = sacc[w][cg];
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += o[c];
    }
    const float den = k0n + wave_sum(qv * k1n + h2q * qv * qv * k2n);
    const float inv = 1.0f / fmaxf(den, a.eps);

    if (!a.no_update) {
        a.s0o[tv + lane] = s0n;
        a.k1o[tv + lane] = k1n;
        a.k2o[tv + lane] = k2n;
        if (lane == 0) a.k0o[t] = k0n;
    }
    if (rg == 0 && !a.no_readout) {
        const f32x4 s04 = *reinterpret_cast<const f32x4 *>(&sh[wave][3][4 * cg]);
        // (y in the fragment layout: the four columns of a lane are one lane
        // slot's consecutive elements)
        const int64_t yo = a.y_frag ? frag_index(b, h * kD + 4 * cg, a.y_ks) : b * a.y_sb + h * a.y_sh + 4 * cg;
#pragma unroll
        for (int c = 0; c < 4; ++c) store_elem(a.y, yo + c, a.dt_y, (s04[c] + acc[c]) * inv);
    }
}

hipError_t launch_decode_step(const DecodeArgs &a, hipStream_t stream) {
    const int blocks = a.B * a.H;  // one workgroup per tile, no more (the kernel has no bounds check)
    const TimerEvents t = timer_events(PRIME_KERNEL_DECODE);
    if (a.s1i != nullptr)
        hipExtLaunchKernelGGL((decode_step_kernel<kDecodeWaves, true>), dim3(blocks), dim3(kDecodeWaves * kWave), 0,
                              stream, t.start, t.stop, 0, a);
    else
        hipExtLaunchKernelGGL((decode_step_kernel<kDecodeWaves, false>), dim3(blocks), dim3(kDecodeWaves * kWave), 0,
                              stream, t.start, t.stop, 0, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) timer_drop(t);
    return e;
}

}  // namespace prime
