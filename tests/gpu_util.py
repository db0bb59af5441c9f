"""Helpers shared by the GPU parity tests (not collected: no test_ prefix)."""
import numpy as np
import torch

from oracle import oracle as O

TOL_BF16 = 2e-2  # bf16 inputs
TOL_F32 = 1e-3   # fp32 inputs


def dev():
    return torch.device("cuda:0")


def to_dev(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev(), dtype)


def to_np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def state_to_dev(st, B, H, D):
    shapes = [(B, H, D), (B, H, D, D), (B, H, D, D), (B, H, 1), (B, H, D), (B, H, D)]
    return tuple(to_dev(np.asarray(s).reshape(sh)) for s, sh in zip(st, shapes))


def state_to_np(st, BH, D):
    shapes = [(BH, D), (BH, D, D), (BH, D, D), (BH,), (BH, D), (BH, D)]
    return tuple(to_np(s).reshape(sh) for s, sh in zip(st, shapes))


def assert_state_close(got, ref, tol, what=""):
    names = ("S0", "S1", "S2", "K0", "K1", "K2")
    for n, g, r in zip(names, got, ref):
        e = O.rel_err(np.asarray(g).reshape(-1), np.asarray(r).reshape(-1))
        assert e < tol, f"{what} state {n}: rel err {e:.3e} >= {tol}"


def assert_close(got, ref, tol, what=""):
    e = O.rel_err(got, ref)
    assert e < tol, f"{what}: rel err {e:.3e} >= {tol}"
    return e


def random_state(BH, D, seed, tokens=32, lam=0.99):
    """A realistic state: the recurrence run over `tokens` random tokens."""
    q, k, v = O.make_inputs((BH, tokens, D), seed=seed, bf16=False)
    _, st = O.recurrent(q, k, v, lam)
    return st
