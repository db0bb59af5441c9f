"""Pins for the CPU oracle (oracle/prime_oracle.c) -- CPU only.

Each oracle routine is checked against something it was not written from:
  recurrent      <- numpy closed form (independent); known answers (single
                    token y = v, clamp branch y = v*den/eps, lambda = 1 prefix
                    sums, k = 0 only decays); the reference's own C99 engine
                    built from /root/reference sources (state update and a
                    transposed readout), when oracle/_ref exists.
  chunked        <- recurrent for C in {1, 7, 64}, ragged L (pad path), L < C,
                    incoming state; state-carry invariant prefill(a)+prefill(b)
                    == prefill(a||b); golden fixtures from the reference.
  dense          <- closed form without state; golden fixtures from the
                    reference module for the incoming-state double clamp.
  delta_chunked  <- per-token delta rule and an unrolled transition-matrix
                    product (bound = 0, several C); golden fixtures from the
                    reference for the active Lyapunov clamp.
  selective      <- the parallel branch (selective.py:414-440, a separate
                    O(L^2) routine) against the step branch applied token by
                    token; beta = 1 with a constant step reduces to the base
                    recurrence with S2, K2 halved; one token gives y = v.
  selective_ref  <- (the float64 torch composition the selective backward
                    tests differentiate) the step branch token by token, with
                    and without an incoming state, the eps clamp active.
A planted-mistake check (oracle_plant_check) shows the pins detect a wrong
index/sign in a modified copy of the formula.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _rand(BH, L, D, seed, normalize=True, bf16=False):
    q, k, v = O.make_inputs((BH, L, D), seed=seed, bf16=bf16, normalize=normalize)
    return q.astype(np.float64), k.astype(np.float64), v.astype(np.float64)


def _rand_state(BH, D, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((BH, D)) * scale, rng.standard_normal((BH, D, D)) * 0.1 * scale,
            rng.standard_normal((BH, D, D)) * 0.1 * scale, np.abs(rng.standard_normal(BH)) * 5 + 1,
            rng.standard_normal((BH, D)) * 0.1, np.abs(rng.standard_normal((BH, D))) * 0.1)


def _close(a, b, tol=1e-11):
    assert O.rel_err(a, b) < tol, O.rel_err(a, b)


def _states_close(s, t, tol=1e-11):
    for x, y in zip(s, t):
        _close(np.asarray(x).reshape(-1), np.asarray(y).reshape(-1), tol)


# ---------------------------------------------------------------- recurrent
@pytest.mark.parametrize("with_state", [False, True])
def test_recurrent_matches_closed_form(with_state):
    BH, L, D = 3, 37, 8
    q, k, v = _rand(BH, L, D, 1)
    lam = np.array([0.9, 0.99, 0.95])
    st = _rand_state(BH, D, 2) if with_state else None
    y, s = O.recurrent(q, k, v, lam, eps=1.0, state=st)
    yc, sc = O.closed_form(q, k, v, lam, eps=1.0, state=st)
    _close(y, yc)
    _states_close(s, sc)


def test_recurrent_single_token_known_answers():
    D = 16
    rng = np.random.default_rng(3)
    k = rng.standard_normal((1, 1, D))
    v = rng.standard_normal((1, 1, D))
    # den = 1 + s + s^2/2 with s = q.k ; pick q so that s = +0.5 (den >= 1) and s = -0.3 (den < 1)
    for s_target, clamped in ((0.5, False), (-0.3, True)):
        q = k * (s_target / np.sum(k * k))
        y, _ = O.recurrent(q, k, v, 0.9, eps=1.0)
        q2k2 = np.sum(q ** 2 * k ** 2)
        den = 1 + s_target + 0.5 * q2k2
        if clamped:
            assert den < 1.0
            _close(y, v * den / 1.0)
        else:
            _close(y, v)


def test_recurrent_lambda_one_prefix_sums_and_k_zero_decay():
    BH, L, D = 2, 9, 4
    q, k, v = _rand(BH, L, D, 4)
    _, s = O.recurrent(q, k, v, 1.0)
    _close(s[1], np.einsum("bli,blj->bij", k, v))
    _close(s[2], np.einsum("bli,blj->bij", k * k, v))
    _close(s[3], np.full(BH, float(L)))
    # k = 0 tokens: S1, S2, K1, K2 only decay
    st = _rand_state(BH, D, 5)
    _, s2 = O.recurrent(q, np.zeros_like(k), v, 0.9, state=st)
    _close(s2[1], st[1] * 0.9 ** L)
    _close(s2[4], st[4] * 0.9 ** L)


@pytest.mark.skipif(not O.ref_available(), reason="reference C99 engine not built (oracle/_ref)")
def test_recurrent_against_reference_c_engine():
    """The reference engine (additive mode, no LN, no clamp) must produce the same
    state as the oracle (S1/S2 transposed: it stores [value][key]) and a y equal to
    the oracle state read out with its transposed contraction."""
    H, D, L = 4, 64, 12
    q, k, v = O.make_inputs((L, H, D), seed=6, bf16=True)  # q pre-scaled by 1/8 (exact)
    lam = 0.9995
    eng = O.RefEngine(H, D, lam, 1.0)
    y_ref = eng.prefill(q * 8.0, k, v)  # the engine applies 1/sqrt(D) itself
    lam32 = float(np.float32(lam))
    y, s = O.recurrent(q.transpose(1, 0, 2), k.transpose(1, 0, 2), v.transpose(1, 0, 2),
                       lam32, eps=1.0)
    rs = eng.state()
    tol = 2e-5  # the engine runs in float32
    _close(rs[0], s[0], tol)
    _close(rs[1], s[1].transpose(0, 2, 1), tol)
    _close(rs[2], s[2].transpose(0, 2, 1), tol)
    _close(rs[3], s[3], tol)
    _close(rs[4], s[4], tol)
    _close(rs[5], s[5], tol)
    # last token: transposed readout of the oracle's state
    qt = q[-1].astype(np.float64)
    den = s[3] + np.sum(qt * s[4], -1) + 0.5 * np.sum(qt * qt * s[5], -1)
    num = s[0] + np.einsum("hd,hed->he", qt, s[1]) + 0.5 * np.einsum("hd,hed->he", qt * qt, s[2])
    _close(y_ref[-1], num / np.maximum(den, 1.0)[:, None], tol)


# ---------------------------------------------------------------- chunked
@pytest.mark.parametrize("L,C", [(64, 64), (100, 64), (13, 64), (50, 7), (20, 1), (192, 32)])
@pytest.mark.parametrize("with_state", [False, True])
def test_chunked_equals_recurrence(L, C, with_state):
    BH, D = 2, 8
    q, k, v = _rand(BH, L, D, 7)
    lam = np.array([0.97, 0.9995])
    st = _rand_state(BH, D, 8) if with_state else None
    yr, sr = O.recurrent(q, k, v, lam, eps=1.0, state=st)
    yc, sc = O.chunked(q, k, v, lam, eps=1.0, chunk=C, state=st)
    _close(yc, yr, 1e-10)
    _states_close(sc, sr, 1e-10)


def test_chunked_state_carry_invariant():
    BH, L1, L2, D = 2, 70, 90, 8
    q, k, v = _rand(BH, L1 + L2, D, 9)
    lam = np.array([0.99, 0.999])
    y_all, s_all = O.chunked(q, k, v, lam, chunk=64)
    y1, s1 = O.chunked(q[:, :L1], k[:, :L1], v[:, :L1], lam, chunk=64)
    y2, s2 = O.chunked(q[:, L1:], k[:, L1:], v[:, L1:], lam, chunk=64, state=s1)
    _close(np.concatenate([y1, y2], 1), y_all, 1e-10)
    _states_close(s2, s_all, 1e-10)


@pytest.mark.parametrize("carry", ["dense", "scan"])
def test_config1_cpu_plumbing(carry):
    """BASELINE config 1 on the CPU reference path: fp32, B=1, H=12, L=512,
    D=64, q/k/v ~ N(0,1) with q/k L2-normalised, lambda 0.9995 per head.  The
    recurrent readout O_t (attention.py:119-143) against the chunked form at
    chunk 64 (chunked_ssd.py:48-184): the fp64 restatements agree to
    rounding, and the fp32 PyTorch-CPU restatement (with the reference's
    O(Nc^2) carry, or the O(Nc) scan) within the fp32 tolerance 1e-3."""
    import torch
    from oracle import torch_cpu as T
    B, H, L, D = 1, 12, 512, 64
    q, k, v = O.make_inputs((B, H, L, D), seed=1, bf16=False)
    lam = np.full(H, 0.9995)
    yr, sr = O.recurrent(q.reshape(H, L, D), k.reshape(H, L, D), v.reshape(H, L, D), lam)
    yc, sc = O.chunked(q.reshape(H, L, D), k.reshape(H, L, D), v.reshape(H, L, D), lam, chunk=64)
    _close(yc, yr, 1e-10)
    _states_close(sc, sr, 1e-10)
    y, st = T.chunked_core(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                           torch.tensor(lam, dtype=torch.float32), chunk=64, carry=carry)
    assert y.dtype == torch.float32
    assert O.rel_err(y.double().numpy().reshape(H, L, D), yr) < 1e-3
    for a, b in zip(st, sr):
        assert O.rel_err(a.double().numpy().reshape(-1), np.asarray(b).reshape(-1)) < 1e-3


@pytest.mark.parametrize("carry", ["dense", "scan"])
@pytest.mark.parametrize("L,with_state", [(200, False), (129, True), (64, True)])
def test_torch_cpu_restatement_matches_oracle(carry, L, with_state):
    """The fp32 PyTorch CPU baseline (oracle/torch_cpu.py) agrees with the fp64
    oracle to fp32 accuracy, for both inter-chunk carries, per-head lambda, a
    ragged last chunk and an incoming state; its decode step agrees with the
    recurrence."""
    import torch
    from oracle import torch_cpu as T
    B, H, D = 2, 3, 16
    q, k, v = _rand(B * H, L, D, 31)
    lam = np.array([0.97, 0.995, 0.9999])
    st = _rand_state(B * H, D, 32) if with_state else None
    yo, so = O.chunked(q, k, v, np.tile(lam, B), chunk=64, state=st)
    t = lambda x: torch.tensor(x, dtype=torch.float32).reshape(B, H, *x.shape[1:])
    tst = None
    if st is not None:
        tst = tuple(torch.tensor(x, dtype=torch.float32).reshape(B, H, *x.shape[1:]) for x in st)
    y, s = T.chunked_core(t(q), t(k), t(v), torch.tensor(lam), chunk=64, state=tst, carry=carry)
    _close(y.double().numpy().reshape(B * H, L, D), yo, 1e-5)
    _states_close([x.double().numpy() for x in s], so, 1e-5)
    # one decode step from the final state equals the recurrence on L + 1 tokens
    q1, k1, v1 = _rand(B * H, 1, D, 33)
    yr, _ = O.recurrent(q1, k1, v1, np.tile(lam, B), state=so)
    yd, _ = T.decode_step(t(q1[:, 0]), t(k1[:, 0]), t(v1[:, 0]), torch.tensor(lam), 1.0, s)
    _close(yd.double().numpy().reshape(B * H, D), yr[:, 0], 1e-5)


def test_chunked_eps_clamp_active():
    """Early tokens with den < eps: the chunked form must clamp exactly like the
    recurrence (unnormalised inputs give s = q.k far from 0)."""
    BH, L, D = 4, 40, 8
    q, k, v = _rand(BH, L, D, 10, normalize=False)
    yr, _ = O.recurrent(q, k, v, 0.9, eps=1.0)
    yc, _ = O.chunked(q, k, v, 0.9, eps=1.0, chunk=16)
    # the clamp branch is exercised: token 0 of sequence 3 has den < eps, and its
    # output is v * den / eps rather than v
    den0 = 1 + np.sum(q[:, 0] * k[:, 0], -1) + 0.5 * np.sum(q[:, 0] ** 2 * k[:, 0] ** 2, -1)
    assert den0[3] < 1.0
    _close(yr[3, 0], v[3, 0] * den0[3])
    _close(yc, yr, 1e-10)


# ---------------------------------------------------------------- dense
def test_dense_without_state_matches_closed_form():
    BH, L, D = 2, 33, 8
    q, k, v = _rand(BH, L, D, 11)
    y, s = O.dense(q, k, v, np.array([0.99, 0.95]))
    yc, sc = O.closed_form(q, k, v, np.array([0.99, 0.95]))
    _close(y, yc)
    _states_close(s, sc)


def test_dense_with_state_terminal_state_matches_closed_form():
    BH, L, D = 2, 21, 8
    q, k, v = _rand(BH, L, D, 12)
    st = _rand_state(BH, D, 13)
    _, s = O.dense(q, k, v, 0.98, state=st)
    _, sc = O.closed_form(q, k, v, 0.98, state=st)
    _states_close(s, sc)


# ---------------------------------------------------------------- delta
def _delta_inputs(BH, L, D, seed):
    q, k, v = _rand(BH, L, D, seed)
    psi, phi = O.delta_features(q, k)
    rng = np.random.default_rng(seed + 100)
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((BH, L))))
    alpha = rng.uniform(0.9, 0.999, (BH, L))
    return psi, phi, v, beta, alpha


def test_delta_features_known_answer():
    D = 4
    q = np.array([[[0.5, -0.25, 0.0, 1.0]]])
    k = np.array([[[3.0, 0.0, -4.0, 0.0]]])
    psi, phi = O.delta_features(q, k)
    r2 = 1 / np.sqrt(2)
    _close(phi[0, 0], [0.6, 0.0, -0.8, 0.0, r2 * 9 / np.sqrt(81 + 256), 0, r2 * 16 / np.sqrt(337), 0])
    _close(psi[0, 0], [0.5, -0.25, 0.0, 1.0, r2 * 0.25, r2 * 0.0625, 0.0, r2])
    # zero key: normalisation clamps at eps, features are 0
    _, phi0 = O.delta_features(q, np.zeros((1, 1, D)))
    _close(phi0, np.zeros((1, 1, 2 * D)))


@pytest.mark.parametrize("L,C", [(64, 64), (50, 16), (37, 64), (30, 1)])
def test_delta_chunked_equals_tokenwise_without_clamp(L, C):
    BH, D = 2, 8
    psi, phi, v, beta, alpha = _delta_inputs(BH, L, D, 14)
    yt, St = O.delta_tokenwise(psi, phi, v, beta, alpha)
    yc, Sc = O.delta_chunked(psi, phi, v, beta, alpha, decay_pad=0.99, bound=0.0, chunk=C)
    _close(yc, yt, 1e-9)
    # the reference pads with alpha = decay (chunked_delta_prime.py:183) and never
    # undoes it, so the returned state carries decay^pad from the padded steps
    pad = (C - L % C) % C
    _close(Sc, St * 0.99 ** pad, 1e-9)


def test_delta_tokenwise_matches_transition_products():
    BH, L, D = 2, 23, 4
    psi, phi, v, beta, alpha = _delta_inputs(BH, L, D, 15)
    S0 = np.random.default_rng(16).standard_normal((BH, D, 2 * D))
    yt, St = O.delta_tokenwise(psi, phi, v, beta, alpha, state=S0)
    yp, Sp = O.closed_form_delta(psi, phi, v, beta, alpha, state=S0)
    _close(yt, yp)
    _close(St, Sp)


def test_delta_chunked_clamp_bounds_norm():
    BH, L, D = 1, 256, 8
    psi, phi, v, beta, alpha = _delta_inputs(BH, L, D, 17)
    _, S = O.delta_chunked(psi, phi, v * 50.0, beta, np.ones_like(alpha), 0.99, bound=5.0, chunk=32)
    assert np.linalg.norm(S[0]) <= 5.0 + 1e-9


# ---------------------------------------------------------------- golden fixtures
def _gold(name):
    p = os.path.join(GOLD, name)
    if not os.path.exists(p):
        pytest.skip(f"golden fixture {name} not generated")
    return np.load(p, allow_pickle=False)


def test_golden_dense_with_state_double_clamp():
    g = _gold("ref_dense_state.npz")
    st = tuple(g[f"s{i}"] for i in range(6))
    y, s = O.dense(g["q"], g["k"], g["v"], float(g["decay"]), eps=float(g["eps"]), state=st)
    _close(y, g["y"], 2e-5)
    _states_close(s, tuple(g[f"o{i}"] for i in range(6)), 2e-5)
    # the fixture exercises the double clamp: a single clamp (the recurrence's)
    # gives a visibly different answer on the same inputs
    y1, _ = O.chunked(g["q"], g["k"], g["v"], float(g["decay"]), eps=float(g["eps"]),
                      chunk=64, state=st)
    assert O.rel_err(y1, g["y"]) > 1e-3


def test_golden_chunked_core_rejects_state():
    """Reference behaviour record: its chunked core raises on an incoming state
    (chunked_ssd.py:129-137 broadcasts [B,H,1,D] against [1,1,Nc,1,1]); this
    build carries the state as the recurrence defines it instead."""
    p = os.path.join(GOLD, "ref_chunked_state.txt")
    if not os.path.exists(p):
        pytest.skip("record not generated")
    assert "RuntimeError" in open(p).read()


def test_golden_delta_chunked_with_clamp():
    g = _gold("ref_delta.npz")
    y, S = O.delta_chunked(g["psi"], g["phi"], g["v"], g["beta"], g["alpha"],
                           float(g["decay"]), bound=float(g["bound"]), chunk=int(g["chunk"]))
    _close(y, g["y"], 2e-4)
    _close(S, g["S"], 2e-4)
    # the clamp is active in this fixture: without it the answer differs
    y0, _ = O.delta_chunked(g["psi"], g["phi"], g["v"], g["beta"], g["alpha"],
                            float(g["decay"]), bound=0.0, chunk=int(g["chunk"]))
    assert O.rel_err(y0, g["y"]) > 1e-3
    # and the features restated in the oracle match the reference's own
    psi, phi = O.delta_features(g["q"], g["k"])
    _close(psi, g["psi"], 1e-6)
    _close(phi, g["phi"], 1e-6)


# ---------------------------------------------------------------- planted mistake
def test_oracle_plant_check():
    """A plausible mistake (readout contracting over the value index instead of
    the key index, i.e. S1 transposed) must be caught by the closed-form pin."""
    BH, L, D = 1, 10, 6
    q, k, v = _rand(BH, L, D, 18)
    st = _rand_state(BH, D, 19)
    stT = (st[0], st[1].transpose(0, 2, 1), st[2].transpose(0, 2, 1), st[3], st[4], st[5])
    y_bad, _ = O.recurrent(q, k, v, 0.95, state=stT)
    yc, _ = O.closed_form(q, k, v, 0.95, state=st)
    assert O.rel_err(y_bad, yc) > 1e-4


# ---------------------------------------------------------------- delta step (L == 1 branch)
def test_delta_step_known_answers():
    """chunked_delta_prime.py:140-176: zero state gives S = beta v phi^T and
    y = beta (phi . psi) v; a perfectly predicted value (v = S phi) or phi = 0
    leaves alpha S; with alpha = 1 the step equals the decay-before-predict
    per-token rule; the clamp bounds |S|_F."""
    rng = np.random.default_rng(40)
    BH, D = 3, 8
    q, k = rng.standard_normal((2, BH, 1, D))
    psi, phi = O.delta_features(q, k)
    psi, phi = psi[:, 0], phi[:, 0]
    v = rng.standard_normal((BH, D))
    beta = rng.uniform(0.1, 0.5, BH)
    alpha = rng.uniform(0.9, 0.99, BH)
    y, S = O.delta_step(psi, phi, v, beta, alpha, bound=0.0)
    _close(S, beta[:, None, None] * v[:, :, None] * phi[:, None, :])
    _close(y, (beta * np.einsum("be,be->b", phi, psi))[:, None] * v)
    S0 = rng.standard_normal((BH, D, 2 * D)) * 0.1
    vp = np.einsum("bde,be->bd", S0, phi)
    _, S1 = O.delta_step(psi, phi, vp, beta, alpha, bound=0.0, state=S0)
    _close(S1, alpha[:, None, None] * S0)
    _, S2 = O.delta_step(psi, np.zeros_like(phi), v, beta, alpha, bound=0.0, state=S0)
    _close(S2, alpha[:, None, None] * S0)
    one = np.ones(BH)
    yt, St = O.delta_tokenwise(psi[:, None], phi[:, None], v[:, None], beta[:, None], one[:, None], state=S0)
    ys, Ss = O.delta_step(psi, phi, v, beta, one, bound=0.0, state=S0)
    _close(ys, yt[:, 0])
    _close(Ss, St)
    yb, Sb = O.delta_step(psi, phi, 50 * v, beta, alpha, bound=2.0, state=S0)
    nrm = np.sqrt((Sb ** 2).sum(axis=(1, 2)))
    assert np.all(np.abs(nrm - 2.0) < 1e-5), nrm
    _close(yb, np.einsum("bde,be->bd", Sb, psi))


def _sel_inputs(BH, L, D, seed):
    q, k, v = _rand(BH, L, D, seed)
    rng = np.random.default_rng(seed + 1)
    delta = np.log1p(np.exp(rng.standard_normal((BH, L))))  # softplus
    tau = rng.uniform(4.0, 300.0, BH)
    beta = rng.uniform(0.5, 3.0, BH)
    return q, k, v, delta, tau, beta


@pytest.mark.parametrize("L", [1, 9, 70])
def test_selective_parallel_equals_token_steps(L):
    """The reference's two selective branches agree: the O(L^2) parallel form
    with C = cumsum(Delta) and the per-token step with lam_t = exp(-Delta_t / tau)."""
    BH, D = 3, 8
    q, k, v, delta, tau, beta = _sel_inputs(BH, L, D, 90 + L)
    yp, sp = O.selective_parallel(q, k, v, delta, tau, beta, eps=1e-5)
    lam = np.exp(-delta / tau[:, None])
    yr, sr = O.selective_recurrent(q, k, v, lam, beta, eps=1e-5)
    np.testing.assert_allclose(yp, yr, rtol=1e-10, atol=1e-12)
    for a, b in zip(sp, sr):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


def test_selective_reduces_to_base_recurrence():
    """beta = 1 and one decay per head: the base recurrence, with the selective
    state's S2 and K2 being half the base ones (the 1/2 moves into the state)."""
    BH, L, D = 2, 40, 8
    q, k, v = _rand(BH, L, D, 95)
    lam = np.array([0.97, 0.999])
    yb, sb = O.recurrent(q, k, v, lam, eps=0.5)
    ys, ss = O.selective_recurrent(q, k, v, np.repeat(lam[:, None], L, 1), np.ones(BH), eps=0.5)
    np.testing.assert_allclose(ys, yb, rtol=1e-12, atol=1e-13)
    for i, (a, b) in enumerate(zip(ss, sb)):
        np.testing.assert_allclose(a, b * (0.5 if i in (2, 5) else 1.0), rtol=1e-12, atol=1e-13)


def test_selective_single_token_is_v():
    BH, D = 4, 8
    q, k, v, delta, tau, beta = _sel_inputs(BH, 1, D, 97)
    y, s = O.selective_parallel(q, k, v, delta, tau, beta, eps=1e-5)
    np.testing.assert_allclose(y, v, rtol=1e-12)
    np.testing.assert_allclose(s[4], beta[:, None] * k[:, 0], rtol=1e-12)
    np.testing.assert_allclose(s[5], 0.5 * beta[:, None] ** 2 * k[:, 0] ** 2, rtol=1e-12)


@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("eps", [1.0, 6.0])
def test_selective_torch_composition_matches_token_steps(with_state, eps):
    """tests/selective_ref.py (the parallel form with the incoming state
    decayed by e^(c_i)) against oracle_selective_recurrent; eps = 6 makes the
    denominator clamp active for some tokens."""
    import torch
    from selective_ref import selective_forward
    B, H, L, D = 2, 2, 37, 8
    BH = B * H
    q, k, v, delta, tau, beta = _sel_inputs(BH, L, D, 98)
    lam = np.exp(-delta / tau[:, None])
    st = None
    if with_state:
        rng = np.random.default_rng(99)
        st = (rng.standard_normal((BH, D)), 0.1 * rng.standard_normal((BH, D, D)),
              0.1 * rng.standard_normal((BH, D, D)), 3.0 + rng.random(BH), 0.1 * rng.standard_normal((BH, D)),
              0.1 * np.abs(rng.standard_normal((BH, D))))
    yr, sr = O.selective_recurrent(q, k, v, lam, beta, eps=eps, state=st)
    t = lambda x, *sh: torch.from_numpy(np.ascontiguousarray(x, dtype=np.float64)).reshape(*sh)
    shapes = [(B, H, D), (B, H, D, D), (B, H, D, D), (B, H, 1), (B, H, D), (B, H, D)]
    ts = tuple(t(x, *sh) for x, sh in zip(st, shapes)) if st is not None else None
    y, so = selective_forward(t(q, B, H, L, D), t(k, B, H, L, D), t(v, B, H, L, D), t(np.log(lam), B, H, L),
                              t(beta, B, H), eps, ts)
    if eps > 1.0:  # the clamp changes some outputs
        y_free, _ = selective_forward(t(q, B, H, L, D), t(k, B, H, L, D), t(v, B, H, L, D),
                                      t(np.log(lam), B, H, L), t(beta, B, H), -1e30, ts)
        assert not torch.allclose(y, y_free)
    np.testing.assert_allclose(y.reshape(BH, L, D).numpy(), yr, rtol=1e-9, atol=1e-11)
    for a, b in zip(so, sr):
        np.testing.assert_allclose(a.reshape(-1).numpy(), np.asarray(b).reshape(-1), rtol=1e-9, atol=1e-11)


# ---------------------------------------------------------------- reverse mode
def _vjp_case(BH, L, seed, with_state, normalize=True, eps=1.0, D=64):
    q, k, v = O.make_inputs((BH, L, D), seed=seed, bf16=False, normalize=normalize)
    rng = np.random.default_rng(seed + 1)
    lam = rng.uniform(0.9, 0.999, BH)
    st = _random_state(BH, D, seed + 2) if with_state else None
    dy = rng.standard_normal((BH, L, D))
    ds = tuple(rng.standard_normal(x.shape) for x in O.zero_state(BH, D))
    return q, k, v, lam, st, dy, ds


def _random_state(BH, D, seed):
    q, k, v = O.make_inputs((BH, 16, D), seed=seed, bf16=False)
    return O.recurrent(q, k, v, 0.95)[1]


def _objective(q, k, v, lam, st, dy, ds, eps):
    y, so = O.recurrent(q, k, v, lam, eps=eps, state=st)
    return float((y * dy).sum() + sum((a * b).sum() for a, b in zip(so, ds)))


@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("normalize,eps", [(True, 1.0), (False, 1e-3)])
def test_recurrent_vjp_matches_finite_differences(with_state, normalize, eps):
    """Directional derivatives of <dy, y> + <dstate, state_out> by central
    differences of the forward recurrence, against the hand-written reverse
    mode, along random directions of q, k, v and the incoming state."""
    BH, L = 2, 6
    q, k, v, lam, st, dy, ds = _vjp_case(BH, L, 300, with_state, normalize, eps)
    dq, dk, dv, dst = O.recurrent_vjp(q, k, v, lam, dy, eps=eps, state=st, dstate=ds)
    rng = np.random.default_rng(301)
    h = 1e-6
    for _ in range(4):
        tq, tk, tv = (rng.standard_normal(q.shape) for _ in range(3))
        ts = tuple(rng.standard_normal(x.shape) for x in O.zero_state(BH, 64)) if with_state else None
        move = lambda s: (q + s * tq, k + s * tk, v + s * tv,
                          None if st is None else tuple(a + s * b for a, b in zip(st, ts)))
        fp = _objective(*move(h)[:3], lam, move(h)[3], dy, ds, eps)
        fm = _objective(*move(-h)[:3], lam, move(-h)[3], dy, ds, eps)
        fd = (fp - fm) / (2 * h)
        an = float((dq * tq).sum() + (dk * tk).sum() + (dv * tv).sum())
        if with_state:
            an += float(sum((a * b).sum() for a, b in zip(dst, ts)))
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (fd, an)


def test_recurrent_vjp_clamped_tokens_pass_no_denominator_gradient():
    """A token whose denominator is below eps: its output is num / eps, so dq
    of that token only carries the numerator term (element-wise check by
    central differences on every q element of that token)."""
    BH, L, eps = 1, 4, 1e-3
    q, k, v = O.make_inputs((BH, L, 64), seed=310, bf16=False, normalize=False)
    # token 3 queries against -K1: its denominator is negative (clamped)
    _, so = O.recurrent(q[:, :3], k[:, :3], v[:, :3], 0.99)
    K1, K2 = so[4], so[5]
    kk = k[:, 3]
    K1n = 0.99 * K1 + kk
    K2n = 0.99 * K2 + kk * kk
    a = (K1n * K1n).sum(-1) / (K1n * K1n * K2n).sum(-1)
    q, k, v = (x.astype(np.float64) for x in (q, k, v))  # perturbations below float32 resolution
    q[:, 3] = -a[:, None] * K1n
    y, st = O.recurrent(q, k, v, 0.99, eps=eps)
    assert (st[3] + (q[:, 3] * st[4]).sum(-1) + 0.5 * (q[:, 3] ** 2 * st[5]).sum(-1) < eps).all()
    dy = np.random.default_rng(311).standard_normal(y.shape)
    dq = O.recurrent_vjp(q, k, v, 0.99, dy, eps=eps)[0]
    h = 1e-6
    for i in range(64):
        qp, qm = q.copy(), q.copy()
        qp[0, 3, i] += h
        qm[0, 3, i] -= h
        fd = (((O.recurrent(qp, k, v, 0.99, eps=eps)[0] - O.recurrent(qm, k, v, 0.99, eps=eps)[0]) * dy).sum()
              / (2 * h))
        assert abs(fd - dq[0, 3, i]) <= 1e-6 * max(1.0, abs(fd))


@pytest.mark.parametrize("with_state", [False, True])
def test_recurrent_vjp_matches_torch_autograd_of_dense_branch(with_state):
    """torch's float64 autograd through the dense branch's formula
    (attention.py:160-202; one clamp, as its L == 1 and chunked forms,
    chunked_ssd.py:156) gives the same dq, dk, dv and state adjoints."""
    import torch
    BH, L, D, eps = 3, 9, 64, 1.0
    q, k, v, lam, st, dy, _ = _vjp_case(BH, L, 320, with_state)
    dq, dk, dv, dst = O.recurrent_vjp(q, k, v, lam, dy, eps=eps, state=st)
    T = lambda x: torch.tensor(x, dtype=torch.float64, requires_grad=True)
    tq, tk, tv = T(q), T(k), T(v)
    ts = [T(x) for x in st] if with_state else None
    lam_t = torch.tensor(lam, dtype=torch.float64).view(BH, 1, 1)
    idx = torch.arange(L, dtype=torch.float64)
    diff = idx.view(L, 1) - idx.view(1, L)
    dm = torch.where(diff >= 0, lam_t ** diff.clamp(min=0), torch.zeros(()))
    A = dm * (1.0 + tq @ tk.transpose(1, 2) + 0.5 * (tq * tq) @ (tk * tk).transpose(1, 2))
    num = A @ tv
    den = A.sum(-1, keepdim=True)
    if with_state:
        S0, S1, S2, K0, K1, K2 = ts
        into = lam_t ** (idx + 1).view(1, L, 1)
        num = num + into * (S0.unsqueeze(1) + tq @ S1 + 0.5 * (tq * tq) @ S2)
        den = den + into * (K0.view(BH, 1, 1) + (tq * K1.unsqueeze(1)).sum(-1, keepdim=True)
                            + 0.5 * (tq * tq * K2.unsqueeze(1)).sum(-1, keepdim=True))
    y = num / den.clamp(min=eps)
    (y * torch.tensor(dy)).sum().backward()
    for got, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        assert np.abs(got - ref.numpy()).max() <= 1e-10 * max(1.0, np.abs(ref.numpy()).max())
    if with_state:
        for got, ref in zip(dst, ts):
            r = ref.grad.numpy().reshape(got.shape)
            assert np.abs(got - r).max() <= 1e-10 * max(1.0, np.abs(r).max())


# ---------------------------------------------------------------- reverse mode of the dense branch
def _dense_objective(q, k, v, lam, st, dy, ds, eps):
    y, so = O.dense(q, k, v, lam, eps=eps, state=st)
    return float((y * dy).sum() + sum((a * b).sum() for a, b in zip(so, ds)))


def _dense_gates(q, k, v, lam, st, eps):
    """Per token: the call's own denominator den_c and max(den_c, eps) + the
    incoming state's term (the arguments of the two clamps, attention.py:177, 185)."""
    BH, L, D = q.shape
    lam = np.broadcast_to(np.asarray(lam, np.float64), (BH,))
    dc, d1 = np.zeros((BH, L)), np.zeros((BH, L))
    for t in range(L):
        _, c = O.recurrent(q[:, :t + 1], k[:, :t + 1], v[:, :t + 1], lam, eps=eps)
        qt = q[:, t]
        dc[:, t] = c[3].reshape(BH) + (qt * c[4]).sum(-1) + 0.5 * (qt * qt * c[5]).sum(-1)
        ds = st[3].reshape(BH) + (qt * st[4]).sum(-1) + 0.5 * (qt * qt * st[5]).sum(-1)
        d1[:, t] = np.maximum(dc[:, t], eps) + lam ** (t + 1) * ds
    return dc, d1


@pytest.mark.parametrize("k0", [None, -1.5])
def test_dense_vjp_matches_finite_differences(k0):
    """Directional derivatives of <dy, y> + <dstate, state_out> through the
    dense branch's double clamp with an incoming state (central differences of
    oracle_dense), with the inner clamp active on some tokens and, for a state
    with a negative K0, the outer clamp on others."""
    BH, L, eps = 2, 6, 2.5
    q, k, v, lam, st, dy, ds = _vjp_case(BH, L, 330, True)
    if k0 is not None:
        st = tuple(np.full_like(x, k0) if i == 3 else x for i, x in enumerate(st))
    dc, d1 = _dense_gates(q, k, v, lam, st, eps)
    assert (dc < eps).any() and (dc >= eps).any()
    if k0 is not None:
        assert (d1 < eps).any() and (d1 >= eps).any()
    assert np.abs(dc - eps).min() > 1e-4 and np.abs(d1 - eps).min() > 1e-4  # no kink within the steps
    dq, dk, dv, dst = O.dense_vjp(q, k, v, lam, dy, eps=eps, state=st, dstate=ds)
    rng = np.random.default_rng(331)
    h = 1e-7
    for _ in range(4):
        tq, tk, tv = (rng.standard_normal(q.shape) for _ in range(3))
        ts = tuple(rng.standard_normal(x.shape) for x in O.zero_state(BH, 64))
        move = lambda s: (q + s * tq, k + s * tk, v + s * tv, tuple(a + s * b for a, b in zip(st, ts)))
        fp = _dense_objective(*move(h)[:3], lam, move(h)[3], dy, ds, eps)
        fm = _dense_objective(*move(-h)[:3], lam, move(-h)[3], dy, ds, eps)
        fd = (fp - fm) / (2 * h)
        an = float((dq * tq).sum() + (dk * tk).sum() + (dv * tv).sum() + sum((a * b).sum() for a, b in zip(dst, ts)))
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (fd, an)


def test_dense_vjp_equals_recurrent_vjp_where_the_clamps_coincide():
    """Without a state the dense branch has one clamp; with a state and the
    inner clamp nowhere active the two clamps act as one.  Either way the
    reverse mode is the recurrence's."""
    BH, L = 3, 40
    q, k, v, lam, st, dy, ds = _vjp_case(BH, L, 340, True)
    for eps, state in ((1.0, None), (1e-3, st)):
        a = O.dense_vjp(q, k, v, lam, dy, eps=eps, state=state, dstate=ds)
        b = O.recurrent_vjp(q, k, v, lam, dy, eps=eps, state=state, dstate=ds)
        for x, y in zip(a[:3], b[:3]):
            np.testing.assert_allclose(x, y, rtol=1e-10, atol=1e-12)
        if state is not None:
            for x, y in zip(a[3], b[3]):
                np.testing.assert_allclose(x, y, rtol=1e-10, atol=1e-12)


def test_dense_vjp_matches_torch_autograd_of_the_double_clamp():
    """torch's float64 autograd through the dense branch as the reference
    writes it (attention.py:160-185: den clamped, the carry added, clamped
    again) gives the same dq, dk, dv and incoming-state adjoint."""
    import torch
    BH, L, D, eps = 3, 9, 64, 2.5
    q, k, v, lam, st, dy, _ = _vjp_case(BH, L, 350, True)
    dc, _ = _dense_gates(q, k, v, lam, st, eps)
    assert (dc < eps).any()
    dq, dk, dv, dst = O.dense_vjp(q, k, v, lam, dy, eps=eps, state=st)
    T = lambda x: torch.tensor(x, dtype=torch.float64, requires_grad=True)
    tq, tk, tv = T(q), T(k), T(v)
    ts = [T(x) for x in st]
    lam_t = torch.tensor(lam, dtype=torch.float64).view(BH, 1, 1)
    idx = torch.arange(L, dtype=torch.float64)
    diff = idx.view(L, 1) - idx.view(1, L)
    dm = torch.where(diff >= 0, lam_t ** diff.clamp(min=0), torch.zeros(()))
    A = dm * (1.0 + tq @ tk.transpose(1, 2) + 0.5 * (tq * tq) @ (tk * tk).transpose(1, 2))
    num = A @ tv
    den = A.sum(-1, keepdim=True).clamp(min=eps)
    S0, S1, S2, K0, K1, K2 = ts
    into = lam_t ** (idx + 1).view(1, L, 1)
    num = num + into * (S0.unsqueeze(1) + tq @ S1 + 0.5 * (tq * tq) @ S2)
    den = (den + into * (K0.view(BH, 1, 1) + (tq * K1.unsqueeze(1)).sum(-1, keepdim=True)
                         + 0.5 * (tq * tq * K2.unsqueeze(1)).sum(-1, keepdim=True))).clamp(min=eps)
    ((num / den) * torch.tensor(dy)).sum().backward()
    for got, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        assert np.abs(got - ref.numpy()).max() <= 1e-10 * max(1.0, np.abs(ref.numpy()).max())
    for got, ref in zip(dst, ts):
        r = ref.grad.numpy().reshape(got.shape)
        assert np.abs(got - r).max() <= 1e-10 * max(1.0, np.abs(r).max())


# ---------------------------------------------------------------- delta backward reference
def _delta_case(B, H, L, D, seed, bound):
    import torch
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, H, L, D, generator=g, dtype=torch.float64), dim=-1) / D ** 0.5
    k = torch.randn(B, H, L, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, H, L, D, generator=g, dtype=torch.float64)
    beta = torch.sigmoid(torch.randn(B, H, L, generator=g, dtype=torch.float64)) * 0.5
    alpha = 0.999 * (1 - 0.5 * torch.sigmoid(torch.randn(B, H, L, generator=g, dtype=torch.float64) - 2.5))
    state = torch.randn(B, H, D, 2 * D, generator=g, dtype=torch.float64) * 0.3
    return q, k, v, beta, alpha, state


@pytest.mark.parametrize("L,bound,D,C", [(64 * 3 + 17, 25.0, 64, 64), (64 * 2 + 5, 1.5, 64, 64), (40, 0.8, 64, 64),
                                         (100, 1.0, 32, 32), (23, 0.7, 8, 5), (130, 25.0, 16, 100)])
def test_delta_torch_restatement_matches_oracle(L, bound, D, C):
    """tests/delta_ref.py (differentiable torch ops) computes what the fp64 C
    oracle computes: y and the final state, ragged L, incoming state, the
    clamp active (bounds below 25 engage it) or not, at the head dims and
    chunk sizes the kernels take."""
    import torch
    import delta_ref as R
    B, H = 1, 2
    q, k, v, beta, alpha, state = _delta_case(B, H, L, D, L, bound)
    y, S = R.delta_chunked(q, k, v, beta, alpha, 0.9995, 1e-5, bound, C, state)
    psi, phi = O.delta_features(q.reshape(B * H, L, D).numpy(), k.reshape(B * H, L, D).numpy(), eps=1e-5)
    yo, So = O.delta_chunked(psi, phi, v.reshape(B * H, L, D).numpy(), beta.reshape(B * H, L).numpy(),
                             alpha.reshape(B * H, L).numpy(), 0.9995, bound=bound, chunk=C,
                             state=state.reshape(B * H, D, 2 * D).numpy())
    assert O.rel_err(y.reshape(B * H, L, D).numpy(), yo) < 1e-12
    assert O.rel_err(S.reshape(B * H, D, 2 * D).numpy(), So) < 1e-12
    if bound < 25.0:
        assert float(S.norm(dim=(-2, -1)).max()) <= bound * (1 + 1e-9)


@pytest.mark.parametrize("bound,D", [(25.0, 64), (0.7, 64), (1.0, 16), (25.0, 7)])
def test_delta_step_torch_restatement_matches_oracle(bound, D):
    """tests/delta_ref.py::delta_step computes what oracle_delta_step computes
    (the L == 1 branch, chunked_delta_prime.py:140-176): y and the new state,
    with an incoming state, the clamp engaged (bound below the state's norm)
    or not."""
    import torch
    import delta_ref as R
    B, H = 2, 3
    q, k, v, beta, alpha, state = (t[:, :, 0] if t.dim() == 4 and i < 3 else t[..., 0] if i in (3, 4) else t
                                   for i, t in enumerate(_delta_case(B, H, 1, D, 11 + D, bound)))
    y, S = R.delta_step(q, k, v, beta, alpha, 1e-5, bound, state)
    psi, phi = O.delta_features(q.reshape(B * H, 1, D).numpy(), k.reshape(B * H, 1, D).numpy(), eps=1e-5)
    yo, So = O.delta_step(psi[:, 0], phi[:, 0], v.reshape(B * H, D).numpy(), beta.reshape(-1).numpy(),
                          alpha.reshape(-1).numpy(), bound=bound, state=state.reshape(B * H, D, 2 * D).numpy())
    assert O.rel_err(y.reshape(B * H, D).numpy(), yo) < 1e-12
    assert O.rel_err(S.reshape(B * H, D, 2 * D).numpy(), So) < 1e-12
    if bound < 25.0:
        assert float(S.norm(dim=(-2, -1)).max()) <= bound * (1 + 1e-9)


@pytest.mark.parametrize("bound", [25.0, 0.6])
def test_delta_step_torch_autograd_matches_central_differences(bound):
    """fp64 autograd of the step restatement against central differences of
    the loss along random directions, for every input (q, k, v, beta, alpha,
    the incoming state), with (bound 0.6) the clamp active."""
    import torch
    import delta_ref as R
    B, H, D = 2, 1, 8
    xs = [t[:, :, 0] if i < 3 else t[..., 0] if i in (3, 4) else t
          for i, t in enumerate(_delta_case(B, H, 1, D, 5, bound))]
    g = torch.Generator().manual_seed(19)
    ry = torch.randn(B, H, D, generator=g, dtype=torch.float64)
    rs = torch.randn(B, H, D, 2 * D, generator=g, dtype=torch.float64)

    def loss(*a):
        y, S = R.delta_step(*a[:5], 1e-5, bound, a[5])
        return (y * ry).sum() + (S * rs).sum()

    for t in xs:
        t.requires_grad_(True)
    grads = torch.autograd.grad(loss(*xs), xs)
    with torch.no_grad():
        if bound < 25.0:
            _, S = R.delta_step(*xs[:5], 1e-5, 0.0, xs[5])
            assert float(S.norm(dim=(-2, -1)).min()) > bound  # the clamp is active
        for i, (x, gr) in enumerate(zip(xs, grads)):
            u = torch.randn(x.shape, generator=g, dtype=torch.float64)
            h = 1e-6
            xp = [t.detach().clone() for t in xs]
            xm = [t.detach().clone() for t in xs]
            xp[i] += h * u
            xm[i] -= h * u
            fd = (loss(*xp) - loss(*xm)) / (2 * h)
            an = (gr * u).sum()
            assert abs(float(fd - an)) <= 1e-6 * max(1.0, abs(float(an))), (i, float(fd), float(an))


@pytest.mark.parametrize("bound", [25.0, 0.6])
def test_delta_torch_autograd_matches_central_differences(bound):
    """fp64 autograd of the restatement against central differences of the
    loss along random directions, for every input (q, k, v, beta, alpha, the
    incoming state), with two chunks, a ragged tail and (bound 0.6) the
    per-chunk clamp active: the reference gradients are the function's."""
    import torch
    import delta_ref as R
    B, H, L, D = 1, 1, 64 + 21, 8
    xs = list(_delta_case(B, H, L, D, 3, bound))
    g = torch.Generator().manual_seed(9)
    ry = torch.randn(B, H, L, D, generator=g, dtype=torch.float64)
    rs = torch.randn(B, H, D, 2 * D, generator=g, dtype=torch.float64)

    def loss(*a):
        y, S = R.delta_chunked(*a[:5], 0.9995, 1e-5, bound, 64, a[5])
        return (y * ry).sum() + (S * rs).sum()

    for t in xs:
        t.requires_grad_(True)
    grads = torch.autograd.grad(loss(*xs), xs)
    with torch.no_grad():
        for i, (x, gr) in enumerate(zip(xs, grads)):
            u = torch.randn(x.shape, generator=g, dtype=torch.float64)
            h = 1e-6
            xp = [t.detach().clone() for t in xs]
            xm = [t.detach().clone() for t in xs]
            xp[i] += h * u
            xm[i] -= h * u
            fd = (loss(*xp) - loss(*xm)) / (2 * h)
            an = (gr * u).sum()
            assert abs(float(fd - an)) <= 1e-6 * max(1.0, abs(float(an))), (i, float(fd), float(an))
