"""GPU parity of the hybrid window-PRIME entry points (prime_accumulate,
prime_decode_readout, prime_decode_update) and of the drop-in for the
reference's C++ extension (prime_cpp_kernel.cpp:6-117, called from
hybrid.py:98-170), against the oracle's recurrence (attention.py:119-143
restated in oracle/prime_oracle.c; eps 1e-3 as prime_cpp_kernel.cpp:40, :96).

The readout and the update are checked through the recurrence itself: the
oracle's y_t is the readout of q_t against the state after token t, and that
state is the state after t - 1 updated with token t."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib
from prime_moment_attention.hybrid import get_cpp_kernel

from gpu_util import (TOL_BF16, TOL_F32, assert_close, assert_state_close, random_state,
                      state_to_dev, state_to_np, to_dev, to_np, dev)

pytestmark = pytest.mark.gpu

D = 64
EPS = 1e-3


def _lams(H, seed):
    return np.random.default_rng(seed).uniform(0.99, 0.9999, H).astype(np.float32)


def _expand(x, grp):
    return np.repeat(x, grp, axis=1)


@pytest.mark.parametrize("B,H,L", [(1, 1, 1), (2, 3, 13), (2, 2, 200), (1, 3, 64 * 37 + 5)])
@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_accumulate_matches_recurrence(B, H, L, with_state, dtype):
    BH = B * H
    bf = dtype == torch.bfloat16
    q, k, v = O.make_inputs((B, H, L, D), seed=100 + L, bf16=bf)
    lam = _lams(H, L)
    st0 = random_state(BH, D, 101 + L) if with_state else None
    _, so = O.recurrent(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D),
                        np.tile(lam.astype(np.float64), B), state=st0)
    st = _lib.new_state(B, H, D, dev())
    _lib.accumulate(to_dev(k, dtype), to_dev(v, dtype), to_dev(lam),
                    state_to_dev(st0, B, H, D) if with_state else None, st)
    torch.cuda.synchronize()
    assert_state_close(state_to_np(st, BH, D), so, TOL_BF16 if bf else TOL_F32)


@pytest.mark.parametrize("with_state", [False, True])
def test_accumulate_segmented_equals_one_slot_and_inplace(with_state):
    """The segment-parallel plan (recommended workspace) and one slot per
    sequence (minimum workspace) agree; state_out may be state_in."""
    B, H, L = 2, 3, 64 * 41 + 17
    BH = B * H
    q, k, v = O.make_inputs((B, H, L, D), seed=110, bf16=True)
    lam = to_dev(_lams(H, 110))
    st0 = random_state(BH, D, 111)
    full = _lib.accumulate_workspace_size(B, H, L)
    one = BH * 33792
    assert full > one, "this shape should split into segments"
    outs = []
    for nbytes in (full, one):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev())
        st = state_to_dev(st0, B, H, D) if with_state else _lib.new_state(B, H, D, dev())
        _lib.accumulate(to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16), lam,
                        st if with_state else None, st, workspace=ws)
        torch.cuda.synchronize()
        outs.append(state_to_np(st, BH, D))
    assert_state_close(outs[0], outs[1], 2e-3)
    _, so = O.recurrent(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D),
                        np.tile(_lams(H, 110).astype(np.float64), B), state=st0 if with_state else None)
    assert_state_close(outs[0], so, TOL_BF16)


def test_accumulate_gqa():
    B, H, Hkv, L = 2, 4, 2, 150
    BH = B * H
    _, k, v = O.make_inputs((B, Hkv, L, D), seed=120, bf16=True)
    lam = _lams(H, 120)
    q0 = np.zeros((BH, L, D))
    _, so = O.recurrent(q0, _expand(k, 2).reshape(BH, L, D), _expand(v, 2).reshape(BH, L, D),
                        np.tile(lam.astype(np.float64), B))
    st = _lib.new_state(B, H, D, dev())
    _lib.accumulate(to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16), to_dev(lam), None, st, H=H)
    torch.cuda.synchronize()
    assert_state_close(state_to_np(st, BH, D), so, TOL_BF16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_readout_is_the_recurrence_output(dtype):
    """Readout of q_L against the state after L tokens = the recurrence's y_L;
    the state is left as it was (bit for bit)."""
    B, H, L = 3, 5, 40
    BH = B * H
    bf = dtype == torch.bfloat16
    q, k, v = O.make_inputs((B, H, L, D), seed=130, bf16=bf, normalize=False)
    lam = np.tile(_lams(H, 130).astype(np.float64), B)
    yo, so = O.recurrent(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D), lam, eps=EPS)
    st = state_to_dev(so, B, H, D)
    before = [t.clone() for t in st]
    y = torch.empty(B, H, D, device=dev(), dtype=dtype)
    _lib.decode_readout(to_dev(q[:, :, L - 1], dtype), EPS, st, y)
    torch.cuda.synchronize()
    assert_close(to_np(y), yo.reshape(B, H, L, D)[:, :, L - 1], TOL_BF16 if bf else TOL_F32, "y")
    for a, b in zip(st, before):
        assert torch.equal(a, b)


def test_readout_eps_clamp():
    """A query whose denominator is negative: the clamp decides the output.
    state_3 does not depend on q_3, so q_3 is chosen from it, as
    q = -a K1 with a minimising K0 + q.K1 + 1/2 q^2.K2."""
    B, H, T = 1, 2, 3
    BH = B * H
    q, k, v = O.make_inputs((B, H, T, D), seed=131, bf16=False, normalize=False)
    lam = np.full(BH, 0.99)
    args = (k.reshape(BH, T, D), v.reshape(BH, T, D), lam)
    _, so = O.recurrent(q.reshape(BH, T, D), *args, eps=EPS)
    K0, K1, K2 = so[3], so[4], so[5]
    a = (K1 * K1).sum(-1) / (K1 * K1 * K2).sum(-1)
    q3 = -a[:, None] * K1
    den = K0 + (q3 * K1).sum(-1) + 0.5 * (q3 * q3 * K2).sum(-1)
    assert (den < 0).all(), den
    qall = q.reshape(BH, T, D).astype(np.float64).copy()
    qall[:, T - 1] = q3
    yo, _ = O.recurrent(qall, *args, eps=EPS)
    y = torch.empty(B, H, D, device=dev())
    _lib.decode_readout(to_dev(q3.reshape(B, H, D)), EPS, state_to_dev(so, B, H, D), y)
    torch.cuda.synchronize()
    assert_close(to_np(y), yo[:, T - 1].reshape(B, H, D), TOL_F32, "y")


@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("Hkv", [4, 2])
def test_update_is_one_recurrence_step(inplace, Hkv):
    B, H, L = 2, 4, 20
    BH = B * H
    grp = H // Hkv
    q, k, v = O.make_inputs((B, Hkv, L, D), seed=140, bf16=False)
    ke, ve = _expand(k, grp).reshape(BH, L, D), _expand(v, grp).reshape(BH, L, D)
    lam = _lams(H, 140)
    lamt = np.tile(lam.astype(np.float64), B)
    _, s_prev = O.recurrent(np.zeros((BH, L - 1, D)), ke[:, :L - 1], ve[:, :L - 1], lamt)
    _, s_last = O.recurrent(np.zeros((BH, L, D)), ke, ve, lamt)
    st_in = state_to_dev(s_prev, B, H, D)
    st_out = st_in if inplace else _lib.new_state(B, H, D, dev())
    _lib.decode_update(to_dev(k[:, :, L - 1]), to_dev(v[:, :, L - 1]), to_dev(lam), st_in, st_out, H=H)
    torch.cuda.synchronize()
    assert_state_close(state_to_np(st_out, BH, D), s_last, TOL_F32)


def test_update_from_zero_state():
    B, H = 2, 3
    _, k, v = O.make_inputs((B, H, 1, D), seed=141, bf16=False)
    lam = _lams(H, 141)
    _, so = O.recurrent(np.zeros((B * H, 1, D)), k.reshape(B * H, 1, D), v.reshape(B * H, 1, D),
                        np.tile(lam.astype(np.float64), B))
    st = _lib.new_state(B, H, D, dev())
    _lib.decode_update(to_dev(k[:, :, 0]), to_dev(v[:, :, 0]), to_dev(lam), None, st)
    torch.cuda.synchronize()
    assert_state_close(state_to_np(st, B * H, D), so, TOL_F32)


def test_cpp_kernel_dropin_prefill_then_decode():
    """The reference's hybrid flow (hybrid.py:98-170): prime_prefill_cpp over
    L tokens, then per token prime_step_evict_update_cpp + prime_query_step_cpp;
    equals the recurrence over all tokens at eps 1e-3 (fp32 inputs)."""
    B, H, L, n = 2, 3, 77, 4
    BH = B * H
    decay = 0.9995
    q, k, v = O.make_inputs((B, H, L + n, D), seed=150, bf16=False)
    yo, so = O.recurrent(q.reshape(BH, L + n, D), k.reshape(BH, L + n, D), v.reshape(BH, L + n, D),
                         decay, eps=EPS)
    yo = yo.reshape(B, H, L + n, D)
    m = get_cpp_kernel()
    out, S0, S1, S2, K0, K1, K2 = m.prime_prefill_cpp(to_dev(q[:, :, :L]), to_dev(k[:, :, :L]),
                                                      to_dev(v[:, :, :L]), decay)
    assert tuple(K0.shape) == (B, H, 1) and tuple(S1.shape) == (B, H, D, D)
    ys = []
    for t in range(L, L + n):
        m.prime_step_evict_update_cpp(to_dev(k[:, :, t]), to_dev(v[:, :, t]), S0, S1, S2, K0, K1, K2, decay)
        ys.append(to_np(m.prime_query_step_cpp(to_dev(q[:, :, t]), S0, S1, S2, K0, K1, K2)))
    torch.cuda.synchronize()
    assert_close(to_np(out), yo[:, :, :L], TOL_F32, "prefill y")
    assert_close(np.stack(ys, 2), yo[:, :, L:], TOL_F32, "decode y")
    assert_state_close(state_to_np((S0, S1, S2, K0, K1, K2), BH, D), so, TOL_F32)


def test_cpp_kernel_dropin_accumulate_evicted():
    B, H, L = 1, 2, 300
    decay = 0.9995
    _, k, v = O.make_inputs((B, H, L, D), seed=151, bf16=False)
    _, so = O.recurrent(np.zeros((B * H, L, D)), k.reshape(B * H, L, D), v.reshape(B * H, L, D), decay)
    m = get_cpp_kernel()
    st = m.prime_accumulate_evicted_cpp(to_dev(k), to_dev(v), decay)
    torch.cuda.synchronize()
    assert len(st) == 6 and tuple(st[3].shape) == (B, H, 1)
    assert_state_close(state_to_np(st, B * H, D), so, TOL_F32)
    empty = m.prime_accumulate_evicted_cpp(to_dev(k[:, :, :0]), to_dev(v[:, :, :0]), decay)
    assert all(float(t.abs().max()) == 0.0 for t in empty)


def test_hybrid_entry_points_reject_bad_arguments():
    B, H, L = 1, 2, 70
    k = torch.zeros(B, H, L, D, device=dev(), dtype=torch.bfloat16)
    lam = to_dev(np.full(H, 0.99, np.float32))
    st = _lib.new_state(B, H, D, dev())
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.accumulate(k, k, lam, None, st, workspace=torch.empty(1024, dtype=torch.uint8, device=dev()))
    with pytest.raises(RuntimeError, match="dtype"):
        _lib.accumulate(k, k.float(), lam, None, st)
    with pytest.raises(ValueError, match="shape"):
        _lib.decode_readout(k[:, :, 0], EPS, st, torch.empty(B, H + 1, D, device=dev()))
    part = list(_lib.new_state(B, H, D, dev()))
    part[1] = st[1]
    with pytest.raises(RuntimeError, match="overlaps"):
        _lib.decode_update(k[:, :, 0], k[:, :, 0], lam, st, tuple(part))
