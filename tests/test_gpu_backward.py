"""GPU parity of the chunked-prefill backward (prime_chunked_prefill_backward)
against the oracle's reverse mode of the recurrence (oracle_recurrent_vjp,
the derivative of attention.py:119-143 that torch autograd gives the
reference when it trains through its prefill, tests/test_attention.py:50-62).

The kernel's MFMA operands are bf16 for bf16 and fp32 inputs alike, so every
case is held to the bf16 tolerance, 2e-2 (max|d| / max|ref| per tensor)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib

from gpu_util import (TOL_BF16, assert_close, assert_state_close, random_state, state_to_dev, state_to_np,
                      to_dev, to_np, dev)

pytestmark = pytest.mark.gpu

D = 64


def _run(B, H, L, dtype, with_state, with_dstate, seed, normalize=True, eps=1.0, dense_clamp=False,
         gdtype=torch.float32):
    BH = B * H
    bf = dtype == torch.bfloat16
    q, k, v = O.make_inputs((B, H, L, D), seed=seed, bf16=bf, normalize=normalize)
    rng = np.random.default_rng(seed + 1)
    lam = rng.uniform(0.99, 0.9999, H).astype(np.float32)
    dy = rng.standard_normal((B, H, L, D)).astype(np.float32)
    if bf:
        dy = O.bf16_round(dy)
    st0 = random_state(BH, D, seed + 2) if with_state else None
    ds = tuple(0.1 * rng.standard_normal(x.shape) for x in O.zero_state(BH, D)) if with_dstate else None
    lamt = np.tile(lam.astype(np.float64), B)
    ref = O.recurrent_vjp(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D), lamt,
                          dy.reshape(BH, L, D), eps=eps, state=st0, dstate=ds)
    g = [torch.empty(B, H, L, D, device=dev(), dtype=gdtype) for _ in range(3)]
    dsi = _lib.new_state(B, H, D, dev()) if with_state else None
    _lib.chunked_prefill_backward(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(lam), eps,
                                  state_to_dev(st0, B, H, D) if with_state else None,
                                  to_dev(dy, torch.bfloat16 if bf else torch.float32),
                                  state_to_dev(ds, B, H, D) if with_dstate else None, *g, dsi,
                                  flags=1 if dense_clamp else 0)
    torch.cuda.synchronize()
    return ref, [to_np(t).reshape(BH, L, D) for t in g], (state_to_np(dsi, BH, D) if with_state else None)


def _check(ref, got, dsi, tol=TOL_BF16):
    # dq and dk vanish analytically for one token from a zero state (y = v):
    # their error is then measured against the gradient scale of dv
    floor = 0.1 * np.abs(ref[2]).max()
    for name, r, x in zip(("dq", "dk", "dv"), ref[:3], got):
        assert np.isfinite(x).all(), name
        e = np.abs(x - r).max() / max(np.abs(r).max(), floor)
        assert e < tol, f"{name}: rel err {e:.3e} >= {tol}"
    if dsi is not None:
        assert_state_close(dsi, ref[3], tol, "dstate_in")


@pytest.mark.parametrize("B,H,L", [(1, 1, 1), (1, 2, 13), (2, 3, 64), (2, 2, 200), (1, 2, 1000)])
@pytest.mark.parametrize("with_state", [False, True])
def test_backward_bf16_matches_oracle(B, H, L, with_state):
    ref, got, dsi = _run(B, H, L, torch.bfloat16, with_state, with_state, seed=400 + L)
    _check(ref, got, dsi)


@pytest.mark.parametrize("B,H,L", [(2, 2, 77), (1, 3, 130)])
def test_backward_f32_inputs(B, H, L):
    ref, got, dsi = _run(B, H, L, torch.float32, True, True, seed=410 + L)
    _check(ref, got, dsi)


def test_backward_final_state_adjoint_only():
    """dy = 0 with a final-state adjoint: only the state path carries gradient."""
    B, H, L = 2, 2, 150
    BH = B * H
    q, k, v = O.make_inputs((B, H, L, D), seed=420, bf16=True)
    lam = np.array([0.995, 0.9995], np.float32)
    ds = tuple(np.random.default_rng(421).standard_normal(x.shape) for x in O.zero_state(BH, D))
    ref = O.recurrent_vjp(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D),
                          np.tile(lam.astype(np.float64), B), np.zeros((BH, L, D)), state=None, dstate=ds)
    g = [torch.empty(B, H, L, D, device=dev()) for _ in range(3)]
    _lib.chunked_prefill_backward(to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16),
                                  to_dev(lam), 1.0, None, torch.zeros(B, H, L, D, device=dev(), dtype=torch.bfloat16),
                                  state_to_dev(ds, B, H, D), *g, None)
    torch.cuda.synchronize()
    assert float(g[0].abs().max()) == 0.0  # q does not reach the final state
    assert_close(to_np(g[1]).reshape(BH, L, D), ref[1], TOL_BF16, "dk")
    assert_close(to_np(g[2]).reshape(BH, L, D), ref[2], TOL_BF16, "dv")


@pytest.mark.parametrize("eps", [1.0, 1e-3])
def test_backward_clamp_active(eps):
    """Unnormalised q/k: some denominators fall below eps (clamped tokens pass
    no denominator gradient)."""
    ref, got, dsi = _run(2, 2, 100, torch.float32, False, False, seed=430, normalize=False, eps=eps)
    _check(ref, got, dsi)


def test_backward_dense_flag_without_state_and_bf16_grads():
    ref, got, dsi = _run(1, 3, 300, torch.bfloat16, False, False, seed=440, dense_clamp=True,
                         gdtype=torch.bfloat16)
    _check(ref, got, dsi)


def test_backward_rejects_bad_arguments():
    B, H, L = 1, 2, 70
    x = torch.zeros(B, H, L, D, device=dev(), dtype=torch.bfloat16)
    g = [torch.empty(B, H, L, D, device=dev()) for _ in range(3)]
    lam = to_dev(np.full(H, 0.99, np.float32))
    st = _lib.new_state(B, H, D, dev(), zero=True)
    with pytest.raises(RuntimeError, match="double clamp"):
        _lib.chunked_prefill_backward(x, x, x, lam, 1.0, st, x, None, *g, None, flags=1)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.chunked_prefill_backward(x, x, x, lam, 1.0, None, x, None, *g, None,
                                      workspace=torch.empty(64, dtype=torch.uint8, device=dev()))
    with pytest.raises(RuntimeError, match="share dtype"):
        _lib.chunked_prefill_backward(x, x, x, lam, 1.0, None, x, None, g[0], g[1], g[2].bfloat16(), None)
