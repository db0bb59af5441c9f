"""CPU oracle for the PRIME moment-attention hot paths (TEST INFRASTRUCTURE).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module.  It is the checker the HIP library is
compared against, never part of the product path.

Three layers:

* ``liboracle.so`` (``prime_oracle.c``): float64 loop restatements of the
  reference algorithms -- recurrence (attention.py:119-143), chunked SSD core
  (chunked_ssd.py:48-184), dense prefill (attention.py:160-202), delta-PRIME
  features and chunked delta prefill (chunked_delta_prime.py:73-87,177-283).
* independent numpy closed forms (``closed_form_*``) written from the
  mathematics, used by the tests to pin the C restatement;
* ``RefEngine``: a ctypes binding of the reference's own C99 engine
  (c/prime_moment.c) when it has been built into ``oracle/_ref``.

All arrays are float64 numpy arrays in [BH, L, D] / state layouts documented in
``prime_oracle.c``.  State tuples follow the reference order
(S0, S1, S2, K0, K1, K2) with K0 shaped [BH].
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libprime_ref.so")
_lib = None

_dp = ctypes.POINTER(ctypes.c_double)
_fp = ctypes.POINTER(ctypes.c_float)


def build(with_ref: bool = True) -> None:
    """Compile liboracle.so (and _ref when the reference sources exist)."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)
    if with_ref and os.path.isdir("/root/reference/c"):
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build(with_ref=False)
        L = ctypes.CDLL(_LIB_PATH)
        i, d = ctypes.c_int, ctypes.c_double
        L.oracle_recurrent.argtypes = [i, i, i, _dp, _dp, _dp, _dp, d] + [_dp] * 7
        L.oracle_chunked.argtypes = [i, i, i, i, _dp, _dp, _dp, _dp, d, i] + [_dp] * 7
        L.oracle_dense.argtypes = [i, i, i, _dp, _dp, _dp, _dp, d, i] + [_dp] * 7
        L.oracle_delta_features.argtypes = [i, i, i, _dp, _dp, d, _dp, _dp]
        L.oracle_delta_chunked.argtypes = [i, i, i, i, _dp, _dp, _dp, _dp, _dp, d, d, i, _dp, _dp]
        L.oracle_delta_tokenwise.argtypes = [i, i, i, _dp, _dp, _dp, _dp, _dp, i, _dp, _dp]
        L.oracle_delta_step.argtypes = [i, i, _dp, _dp, _dp, _dp, _dp, d, _dp, _dp]
        L.oracle_selective_recurrent.argtypes = [i, i, i, _dp, _dp, _dp, _dp, _dp, d] + [_dp] * 7
        L.oracle_selective_parallel.argtypes = [i, i, i, _dp, _dp, _dp, _dp, _dp, _dp, d] + [_dp] * 7
        L.oracle_recurrent_vjp.argtypes = [i, i, i, _dp, _dp, _dp, _dp, d] + [_dp] * 6 + [_dp] + [_dp] * 6 + [
            _dp] * 3 + [_dp] * 6
        L.oracle_dense_vjp.argtypes = L.oracle_recurrent_vjp.argtypes
        f = ctypes.c_float
        L.baseline_decode_step.argtypes = [i, i, i, _fp, _fp, _fp, _fp, f] + [_fp] * 7 + [i]
        L.baseline_prefill.argtypes = [i, i, i, i, _fp, _fp, _fp, _fp, f] + [_fp] * 7 + [i]
        _lib = L
    return _lib


def _c64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _p(a: np.ndarray):
    return a.ctypes.data_as(_dp)


def zero_state(BH: int, D: int) -> Tuple[np.ndarray, ...]:
    return (np.zeros((BH, D)), np.zeros((BH, D, D)), np.zeros((BH, D, D)),
            np.zeros((BH,)), np.zeros((BH, D)), np.zeros((BH, D)))


def _state_copy(state, BH, D):
    if state is None:
        return zero_state(BH, D), 0
    s = tuple(_c64(x).copy() for x in state)
    s = (s[0].reshape(BH, D), s[1].reshape(BH, D, D), s[2].reshape(BH, D, D),
         s[3].reshape(BH), s[4].reshape(BH, D), s[5].reshape(BH, D))
    return s, 1


def _lam(lam, BH):
    lam = np.asarray(lam, dtype=np.float64).reshape(-1)
    if lam.size == 1:
        lam = np.full(BH, float(lam[0]))
    assert lam.size == BH
    return np.ascontiguousarray(lam)


def recurrent(q, k, v, lam, eps=1.0, state=None):
    """Token-by-token decode steps (attention.py:119-143).  q,k,v [BH,L,D]."""
    q, k, v = _c64(q), _c64(k), _c64(v)
    BH, L, D = q.shape
    s, _ = _state_copy(state, BH, D)
    y = np.zeros_like(q)
    lib().oracle_recurrent(BH, L, D, _p(q), _p(k), _p(v), _p(_lam(lam, BH)), eps,
                           *[_p(x) for x in s], _p(y))
    return y, s


def chunked(q, k, v, lam, eps=1.0, chunk=64, state=None):
    """Chunked SSD core (chunked_ssd.py:48-184).  Returns (y, final_state)."""
    q, k, v = _c64(q), _c64(k), _c64(v)
    BH, L, D = q.shape
    s, has = _state_copy(state, BH, D)
    y = np.zeros_like(q)
    lib().oracle_chunked(BH, L, D, chunk, _p(q), _p(k), _p(v), _p(_lam(lam, BH)), eps, has,
                         *[_p(x) for x in s], _p(y))
    return y, s


def dense(q, k, v, lam, eps=1.0, state=None):
    """Dense prefill (attention.py:160-202), including its double clamp."""
    q, k, v = _c64(q), _c64(k), _c64(v)
    BH, L, D = q.shape
    s, has = _state_copy(state, BH, D)
    y = np.zeros_like(q)
    lib().oracle_dense(BH, L, D, _p(q), _p(k), _p(v), _p(_lam(lam, BH)), eps, has,
                       *[_p(x) for x in s], _p(y))
    return y, s


def selective_recurrent(q, k, v, lam_t, beta, eps=1.0, state=None):
    """Selective PRIME step branch token by token (selective.py:384-409):
    lam_t [BH, L] per-token decays, beta [BH]; state in the selective
    convention (S2, K2 carry the 1/2)."""
    q, k, v = _c64(q), _c64(k), _c64(v)
    BH, L, D = q.shape
    s, _ = _state_copy(state, BH, D)
    y = np.zeros_like(q)
    lib().oracle_selective_recurrent(BH, L, D, _p(q), _p(k), _p(v), _p(_c64(lam_t).reshape(BH, L)),
                                     _p(_lam(beta, BH)), eps, *[_p(x) for x in s], _p(y))
    return y, s


def selective_parallel(q, k, v, delta, tau, beta, eps=1.0):
    """Selective PRIME parallel branch (selective.py:414-440): delta [BH, L]
    (the softplus step sizes), tau and beta [BH]; no incoming state."""
    q, k, v = _c64(q), _c64(k), _c64(v)
    BH, L, D = q.shape
    s = zero_state(BH, D)
    y = np.zeros_like(q)
    lib().oracle_selective_parallel(BH, L, D, _p(q), _p(k), _p(v), _p(_c64(delta).reshape(BH, L)),
                                    _p(_lam(tau, BH)), _p(_lam(beta, BH)), eps, *[_p(x) for x in s], _p(y))
    return y, s


def recurrent_vjp(q, k, v, lam, dy, eps=1.0, state=None, dstate=None):
    """Reverse mode of the recurrence (attention.py:119-143): returns
    (dq, dk, dv, dstate_in) for the output adjoint dy [BH,L,D] and the final
    state's adjoint dstate (None = 0); dstate_in is the adjoint of `state`
    (zero state when None)."""
    q, k, v, dy = _c64(q), _c64(k), _c64(v), _c64(dy)
    BH, L, D = q.shape
    si = None if state is None else _state_copy(state, BH, D)[0]
    so = None if dstate is None else _state_copy(dstate, BH, D)[0]
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    ds = zero_state(BH, D)
    null = [None] * 6
    lib().oracle_recurrent_vjp(BH, L, D, _p(q), _p(k), _p(v), _p(_lam(lam, BH)), eps,
                               *([_p(x) for x in si] if si else null), _p(dy),
                               *([_p(x) for x in so] if so else null), _p(dq), _p(dk), _p(dv),
                               *[_p(x) for x in ds])
    return dq, dk, dv, ds


def dense_vjp(q, k, v, lam, dy, eps=1.0, state=None, dstate=None):
    """Reverse mode of the dense prefill branch with its double clamp
    (attention.py:160-202); same arguments and results as recurrent_vjp."""
    q, k, v, dy = _c64(q), _c64(k), _c64(v), _c64(dy)
    BH, L, D = q.shape
    si = None if state is None else _state_copy(state, BH, D)[0]
    so = None if dstate is None else _state_copy(dstate, BH, D)[0]
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    ds = zero_state(BH, D)
    null = [None] * 6
    lib().oracle_dense_vjp(BH, L, D, _p(q), _p(k), _p(v), _p(_lam(lam, BH)), eps,
                           *([_p(x) for x in si] if si else null), _p(dy),
                           *([_p(x) for x in so] if so else null), _p(dq), _p(dk), _p(dv),
                           *[_p(x) for x in ds])
    return dq, dk, dv, ds


def delta_features(q, k, eps=1e-5):
    """psi, phi feature maps (chunked_delta_prime.py:73-87); q pre-scaled."""
    q, k = _c64(q), _c64(k)
    BH, L, D = q.shape
    psi = np.zeros((BH, L, 2 * D))
    phi = np.zeros((BH, L, 2 * D))
    lib().oracle_delta_features(BH, L, D, _p(q), _p(k), eps, _p(psi), _p(phi))
    return psi, phi


def delta_chunked(psi, phi, v, beta, alpha, decay_pad, bound=25.0, chunk=64, state=None):
    """Chunked delta-PRIME prefill (chunked_delta_prime.py:177-283)."""
    psi, phi, v = _c64(psi), _c64(phi), _c64(v)
    beta, alpha = _c64(beta), _c64(alpha)
    BH, L, D = v.shape
    assert chunk <= 256
    S = np.zeros((BH, D, 2 * D)) if state is None else _c64(state).reshape(BH, D, 2 * D).copy()
    y = np.zeros_like(v)
    lib().oracle_delta_chunked(BH, L, D, chunk, _p(psi), _p(phi), _p(v), _p(beta), _p(alpha),
                               decay_pad, bound, 0 if state is None else 1, _p(S), _p(y))
    return y, S


def delta_tokenwise(psi, phi, v, beta, alpha, state=None):
    """Per-token gated delta rule (decay before prediction), no clamp."""
    psi, phi, v = _c64(psi), _c64(phi), _c64(v)
    beta, alpha = _c64(beta), _c64(alpha)
    BH, L, D = v.shape
    S = np.zeros((BH, D, 2 * D)) if state is None else _c64(state).reshape(BH, D, 2 * D).copy()
    y = np.zeros_like(v)
    lib().oracle_delta_tokenwise(BH, L, D, _p(psi), _p(phi), _p(v), _p(beta), _p(alpha),
                                 0 if state is None else 1, _p(S), _p(y))
    return y, S


def delta_step(psi, phi, v, beta, alpha, bound=25.0, state=None):
    """Delta-PRIME L == 1 step (chunked_delta_prime.py:140-176): psi/phi [BH, 2D],
    v [BH, D], beta/alpha [BH]; returns (y [BH, D], S [BH, D, 2D])."""
    psi, phi, v = _c64(psi), _c64(phi), _c64(v)
    beta, alpha = _c64(beta), _c64(alpha)
    BH, D = v.shape
    S = np.zeros((BH, D, 2 * D)) if state is None else _c64(state).reshape(BH, D, 2 * D).copy()
    y = np.zeros_like(v)
    lib().oracle_delta_step(BH, D, _p(psi), _p(phi), _p(v), _p(beta), _p(alpha), float(bound), _p(S), _p(y))
    return y, S


# --------------------------------------------------------------------------
# Independent closed forms (numpy), written from the mathematics, not from the
# C restatement: y_t = [sum_{j<=t} w_tj v_j + lam^{t+1} N_init(q_t)] /
#                      max(sum_{j<=t} w_tj + lam^{t+1} D_init(q_t), eps),
# w_tj = lam^{t-j} (1 + q_t.k_j + 1/2 (q_t*q_t).(k_j*k_j)).
# Final state: S1 = lam^L S1_init + sum_j lam^{L-1-j} k_j v_j^T, etc.
# --------------------------------------------------------------------------
def closed_form(q, k, v, lam, eps=1.0, state=None):
    q, k, v = _c64(q), _c64(k), _c64(v)
    BH, L, D = q.shape
    lam = _lam(lam, BH)
    y = np.zeros_like(q)
    st = []
    s, _ = _state_copy(state, BH, D)
    for b in range(BH):
        l = lam[b]
        t = np.arange(L)
        diff = t[:, None] - t[None, :]
        mask = np.where(diff >= 0, l ** np.maximum(diff, 0), 0.0)
        W = mask * (1.0 + q[b] @ k[b].T + 0.5 * (q[b] ** 2) @ (k[b] ** 2).T)
        num = W @ v[b]
        den = W.sum(1)
        s0, s1, s2, k0, k1, k2 = (s[0][b], s[1][b], s[2][b], s[3][b], s[4][b], s[5][b])
        din = l ** (t + 1.0)
        num = num + din[:, None] * (s0[None, :] + q[b] @ s1 + 0.5 * (q[b] ** 2) @ s2)
        den = den + din * (k0 + q[b] @ k1 + 0.5 * (q[b] ** 2) @ k2)
        y[b] = num / np.maximum(den, eps)[:, None]
        w = l ** (L - 1.0 - t)
        lL = l ** L
        st.append((lL * s0 + (w[:, None] * v[b]).sum(0),
                   lL * s1 + (k[b] * w[:, None]).T @ v[b],
                   lL * s2 + ((k[b] ** 2) * w[:, None]).T @ v[b],
                   lL * k0 + w.sum(),
                   lL * k1 + (k[b] * w[:, None]).sum(0),
                   lL * k2 + ((k[b] ** 2) * w[:, None]).sum(0)))
    out = tuple(np.stack([x[i] for x in st]) for i in range(6))
    return y, out


def closed_form_delta(psi, phi, v, beta, alpha, state=None):
    """Unrolled gated delta rule as a sequence of rank-1 matrix products:
    S_t = S_{t-1} a_t (I - b_t phi_t phi_t^T) + b_t v_t phi_t^T, y_t = S_t psi_t.
    (Algebraically the same recurrence as oracle_delta_tokenwise, written as a
    product of transition matrices so the two are independent.)"""
    psi, phi, v = _c64(psi), _c64(phi), _c64(v)
    beta, alpha = _c64(beta), _c64(alpha)
    BH, L, D = v.shape
    P = 2 * D
    S = np.zeros((BH, D, P)) if state is None else _c64(state).reshape(BH, D, P).copy()
    y = np.zeros_like(v)
    I = np.eye(P)
    for b in range(BH):
        for t in range(L):
            a = min(max(alpha[b, t], 1e-5), 1.0)
            Tm = a * (I - beta[b, t] * np.outer(phi[b, t], phi[b, t]))
            S[b] = S[b] @ Tm + beta[b, t] * np.outer(v[b, t], phi[b, t])
            y[b, t] = S[b] @ psi[b, t]
    return y, S


# --------------------------------------------------------------------------
# Input recipe shared by tests, smoke and bench (seeded; q,k L2-normalised,
# optionally rounded to bf16; q then scaled by 1/sqrt(D)).
# --------------------------------------------------------------------------
def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bfloat16, returned as float32 values."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).reshape(a.shape)


def make_inputs(shape, seed=0, bf16=True, scale_q=True, normalize=True):
    """q, k, v ~ N(0,1) [.., D] float32; q,k L2-normalised along D; bf16-rounded
    after normalising when bf16; q scaled by 1/sqrt(D) (exact in bf16 for D=64)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(shape, dtype=np.float32)
    k = rng.standard_normal(shape, dtype=np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    if normalize:
        q = q / np.maximum(np.linalg.norm(q, axis=-1, keepdims=True), 1e-12)
        k = k / np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), 1e-12)
    if bf16:
        q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
    if scale_q:
        q = (q * np.float32(1.0 / np.sqrt(shape[-1]))).astype(np.float32)
    return q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)


def rel_err(got, ref) -> float:
    """max|got - ref| / max|ref| (the tolerance measure used throughout)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    if den == 0.0:
        return float(np.max(np.abs(got)))
    return float(np.max(np.abs(got - ref)) / den)


# --------------------------------------------------------------------------
# fp32 CPU baseline (timing) -- cpu_baseline.c
# --------------------------------------------------------------------------
def _pf(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def baseline_decode_step(q, k, v, lam_heads, eps, state, y, heads, nthreads):
    N, D = q.shape
    lib().baseline_decode_step(N, heads, D, _pf(q), _pf(k), _pf(v), _pf(lam_heads), eps,
                               *[_pf(x) for x in state], _pf(y), nthreads)


def baseline_prefill(q, k, v, lam_heads, eps, state, y, heads, nthreads):
    N, L, D = q.shape
    lib().baseline_prefill(N, heads, L, D, _pf(q), _pf(k), _pf(v), _pf(lam_heads), eps,
                           *[_pf(x) for x in state], _pf(y), nthreads)


# --------------------------------------------------------------------------
# The reference C99 engine (c/prime_moment.{h,c}) built into oracle/_ref.
# --------------------------------------------------------------------------
class _Cfg(ctypes.Structure):  # prime_config_t, c/prime_moment.h:29-38
    _fields_ = [("num_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("decay", ctypes.c_float), ("eps", ctypes.c_float),
                ("use_qk_norm", ctypes.c_int), ("use_delta_rule", ctypes.c_int),
                ("lyapunov_bound", ctypes.c_float), ("use_harmonic_rope", ctypes.c_int)]


class _State(ctypes.Structure):  # prime_state_t, c/prime_moment.h:40-59
    _fields_ = [("num_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("state_bytes", ctypes.c_size_t)] + [(n, _fp) for n in
                                                      ("s0", "s1", "s2", "k0", "k1", "k2")]


def ref_available() -> bool:
    return os.path.exists(_REF_PATH)


class RefEngine:
    """Additive-mode reference C99 engine for H heads of one sequence.

    Its S1/S2 are stored [value][key] (c/prime_moment.c:283-289) and its
    readout contracts q over the value index (:292-300); ``state()`` returns
    the arrays as stored, so callers transpose to compare with [key][value].
    """

    def __init__(self, heads: int, D: int, decay: float, eps: float):
        L = ctypes.CDLL(_REF_PATH)
        L.prime_state_create.restype = ctypes.POINTER(_State)
        L.prime_state_create.argtypes = [ctypes.c_int, ctypes.c_int]
        L.prime_state_free.argtypes = [ctypes.POINTER(_State)]
        L.prime_step.argtypes = [ctypes.POINTER(_Cfg), ctypes.POINTER(_State), _fp, _fp, _fp, _fp]
        L.prime_prefill.argtypes = [ctypes.POINTER(_Cfg), ctypes.POINTER(_State), ctypes.c_int,
                                    _fp, _fp, _fp, _fp]
        self._L = L
        self.H, self.D = heads, D
        self.cfg = _Cfg(heads, D, decay, eps, 0, 0, 0.0, 0)
        self.st = L.prime_state_create(heads, D)
        if not self.st:
            raise RuntimeError("prime_state_create failed")

    def __del__(self):
        try:
            self._L.prime_state_free(self.st)
        except Exception:
            pass

    def step(self, q, k, v) -> np.ndarray:
        """q (unscaled: the engine scales by 1/sqrt(D) itself), k, v [H, D] float32."""
        q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
        out = np.zeros((self.H, self.D), dtype=np.float32)
        self._L.prime_step(ctypes.byref(self.cfg), self.st, _pf(q), _pf(k), _pf(v), _pf(out))
        return out

    def prefill(self, q, k, v) -> np.ndarray:
        """q, k, v [L, H, D] float32 (token-major, as prime_prefill walks them)."""
        q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
        out = np.zeros_like(q)
        self._L.prime_prefill(ctypes.byref(self.cfg), self.st, q.shape[0], _pf(q), _pf(k),
                              _pf(v), _pf(out))
        return out

    def state(self):
        H, D = self.H, self.D
        s = self.st.contents

        def arr(p, shape):
            return np.ctypeslib.as_array(p, shape=shape).copy()
        return (arr(s.s0, (H, D)), arr(s.s1, (H, D, D)), arr(s.s2, (H, D, D)),
                arr(s.k0, (H,)), arr(s.k1, (H, D)), arr(s.k2, (H, D)))
