"""GPU parity of the chunked prefill (prime_chunked_prefill) against the oracle
(chunked_ssd.py:48-184 / attention.py:160-202 restated in oracle/prime_oracle.c)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib
from prime_moment_attention.chunked_ssd import chunked_prime_ssd_core, prime_prefill

from gpu_util import (TOL_BF16, TOL_F32, assert_close, assert_state_close, random_state,
                      state_to_dev, state_to_np, to_dev, to_np, dev)

pytestmark = pytest.mark.gpu

D = 64


def _case(B, H, L, in_dtype, with_state, seed, Hkv=None, normalize=True, eps=1.0,
          dense_clamp=False, inplace=False):
    Hkv = Hkv or H
    BH = B * H
    bf = in_dtype == torch.bfloat16
    q, _, _ = O.make_inputs((B, H, L, D), seed=seed, bf16=bf, normalize=normalize)
    _, k, v = O.make_inputs((B, Hkv, L, D), seed=seed + 1, bf16=bf, normalize=normalize)
    rng = np.random.default_rng(seed)
    lam = rng.uniform(0.99, 0.9999, H).astype(np.float32)
    st0 = random_state(BH, D, seed + 2) if with_state else None
    grp = H // Hkv
    ke, ve = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    args = (q.reshape(BH, L, D), ke.reshape(BH, L, D), ve.reshape(BH, L, D),
            np.tile(lam.astype(np.float64), B))
    if dense_clamp:
        yo, so = O.dense(*args, eps=eps, state=st0)
    else:
        yo, so = O.chunked(*args, eps=eps, chunk=64, state=st0)
    st_in = state_to_dev(st0, B, H, D) if with_state else None
    y, st = prime_prefill(to_dev(q, in_dtype), to_dev(k, in_dtype), to_dev(v, in_dtype),
                          state=st_in, decay=to_dev(lam), eps=eps, return_state=True,
                          dense_clamp=dense_clamp, state_out=st_in if inplace else None)
    torch.cuda.synchronize()
    return yo.reshape(B, H, L, D), so, to_np(y), state_to_np(st, BH, D)


SHAPES = [(1, 1, 64), (2, 3, 200), (1, 2, 13), (2, 2, 1000), (1, 1, 1)]


@pytest.mark.parametrize("B,H,L", SHAPES)
@pytest.mark.parametrize("with_state", [False, True])
def test_prefill_bf16_matches_oracle(B, H, L, with_state):
    yo, so, y, s = _case(B, H, L, torch.bfloat16, with_state, seed=20 + L)
    assert_close(y, yo, TOL_BF16, "y")
    assert_state_close(s, so, TOL_BF16)


@pytest.mark.parametrize("B,H,L", [(2, 3, 200), (1, 2, 77)])
@pytest.mark.parametrize("with_state", [False, True])
def test_prefill_f32_matches_oracle(B, H, L, with_state):
    yo, so, y, s = _case(B, H, L, torch.float32, with_state, seed=30 + L)
    assert_close(y, yo, TOL_F32, "y")
    assert_state_close(s, so, TOL_F32)


def test_prefill_one_slice_per_sequence():
    """More than 160 sequences: one workgroup owns all 64 value columns."""
    yo, so, y, s = _case(1, 170, 70, torch.bfloat16, True, seed=40)
    assert_close(y, yo, TOL_BF16, "y")
    assert_state_close(s, so, TOL_BF16)


def test_prefill_inplace_state_and_gqa():
    yo, so, y, s = _case(2, 4, 150, torch.bfloat16, True, seed=41, Hkv=2, inplace=True)
    assert_close(y, yo, TOL_BF16, "y")
    assert_state_close(s, so, TOL_BF16)


@pytest.mark.parametrize("with_state", [False, True])
def test_prefill_dense_clamp_matches_dense_branch(with_state):
    """Unnormalised q/k: den < eps for early tokens, and the dense branch clamps
    the intra denominator before adding the carry (attention.py:177,185)."""
    yo, so, y, s = _case(2, 2, 100, torch.bfloat16, with_state, seed=42, normalize=False,
                         dense_clamp=True)
    assert_close(y, yo, TOL_BF16, "y")
    assert_state_close(s, so, TOL_BF16)


def test_prefill_eps_clamp_recurrence():
    yo, so, y, s = _case(2, 2, 130, torch.bfloat16, False, seed=43, normalize=False)
    assert_close(y, yo, TOL_BF16, "y")


def test_prefill_state_carry_invariant():
    """prefill(a) then prefill(b, state) == prefill(a || b)."""
    B, H, L1, L2 = 2, 3, 100, 157
    q, k, v = O.make_inputs((B, H, L1 + L2, D), seed=44, bf16=True)
    lam = to_dev(np.array([0.99, 0.995, 0.9999], np.float32))
    t = lambda x: to_dev(x, torch.bfloat16)
    y_all, s_all = chunked_prime_ssd_core(t(q), t(k), t(v), decay=lam, return_state=True)
    y1, s1 = chunked_prime_ssd_core(t(q[:, :, :L1]), t(k[:, :, :L1]), t(v[:, :, :L1]), decay=lam,
                                    return_state=True)
    y2, s2 = chunked_prime_ssd_core(t(q[:, :, L1:]), t(k[:, :, L1:]), t(v[:, :, L1:]), state=s1,
                                    decay=lam, return_state=True)
    torch.cuda.synchronize()
    assert_close(np.concatenate([to_np(y1), to_np(y2)], 2), to_np(y_all), 5e-3, "y")
    assert_state_close(state_to_np(s2, B * H, D), state_to_np(s_all, B * H, D), 5e-3)


def test_prefill_then_decode_equals_longer_prefill():
    B, H, L = 2, 2, 129
    q, k, v = O.make_inputs((B, H, L + 1, D), seed=45, bf16=True)
    lam = to_dev(np.array([0.995, 0.9995], np.float32))
    t = lambda x: to_dev(x, torch.bfloat16)
    y_all, _ = chunked_prime_ssd_core(t(q), t(k), t(v), decay=lam)
    _, st = chunked_prime_ssd_core(t(q[:, :, :L]), t(k[:, :, :L]), t(v[:, :, :L]), decay=lam,
                                   return_state=True)
    yd = torch.empty(B, H, D, device=dev())
    st2 = _lib.new_state(B, H, D, dev())
    _lib.decode_step(t(q[:, :, L]), t(k[:, :, L]), t(v[:, :, L]), lam, 1.0, st, st2, yd)
    torch.cuda.synchronize()
    assert_close(to_np(yd), to_np(y_all[:, :, L]), 5e-3, "y")


def test_prefill_config2_shape_subset():
    """BASELINE config 2 (B=8, H=12, L=8192, bf16, per-head lambda in
    [0.99, 0.9999], zero state); three sequences checked against the oracle,
    all outputs finite."""
    B, H, L = 8, 12, 8192
    q, k, v = O.make_inputs((B, H, L, D), seed=2, bf16=True)
    rng = np.random.default_rng(2)
    lam = rng.uniform(0.99, 0.9999, H).astype(np.float32)
    t = lambda x: to_dev(x, torch.bfloat16)
    y, st = chunked_prime_ssd_core(t(q), t(k), t(v), decay=to_dev(lam), return_state=True)
    torch.cuda.synchronize()
    yn = to_np(y)
    assert np.isfinite(yn).all()
    sn = state_to_np(st, B * H, D)
    for (b, h) in [(0, 0), (3, 7), (7, 11)]:
        yo, so = O.chunked(q[b, h][None], k[b, h][None], v[b, h][None], float(lam[h]), chunk=64)
        assert_close(yn[b, h], yo[0], TOL_BF16, f"y[{b},{h}]")
        assert_state_close(tuple(x[b * H + h][None] for x in sn), so, TOL_BF16)


def test_prefill_rejects_bad_arguments():
    x = torch.zeros(1, 1, 8, D, device=dev(), dtype=torch.bfloat16)
    lam = to_dev(np.ones(1, np.float32))
    with pytest.raises(RuntimeError, match="dtype"):
        _lib.chunked_prefill(x, x.float(), x, lam, 1.0, 64, None, x.float(), None)
    with pytest.raises(RuntimeError, match="16-byte"):
        xs = torch.zeros(1, 1, 9 * D + 1, device=dev(), dtype=torch.bfloat16)[..., 1:].view(1, 1, 9, D)
        _lib.chunked_prefill(xs, xs, xs, lam, 1.0, 64, None,
                             torch.zeros(1, 1, 9, D, device=dev()), None)
    with pytest.raises(ValueError, match="shape"):
        _lib.chunked_prefill(x, x, x, lam, 1.0, 64, None, torch.zeros(1, 1, 7, D, device=dev()), None)


@pytest.mark.parametrize("with_state", [False, True])
def test_prefill_segmented_equals_one_segment(with_state):
    """The segment-parallel plan (workspace) and one segment per sequence (no
    workspace) agree, with an incoming state and a ragged last chunk."""
    B, H, L = 1, 3, 64 * 37 + 5
    BH = B * H
    q, k, v = O.make_inputs((B, H, L, D), seed=46, bf16=True)
    lam = to_dev(np.array([0.99, 0.995, 0.9999], np.float32))
    st0 = state_to_dev(random_state(BH, D, 47), B, H, D) if with_state else None
    assert _lib.workspace_size(B, H, L) > 0
    t = lambda x: to_dev(x, torch.bfloat16)
    outs = []
    for ws in (None, torch.empty(0, dtype=torch.uint8, device=dev())):
        y = torch.empty(B, H, L, D, device=dev())
        st = _lib.new_state(B, H, D, dev())
        _lib.chunked_prefill(t(q), t(k), t(v), lam, 1.0, 64, st0, y, st, 0, workspace=ws)
        torch.cuda.synchronize()
        outs.append((to_np(y), state_to_np(st, BH, D)))
    assert_close(outs[0][0], outs[1][0], 2e-3, "y")
    assert_state_close(outs[0][1], outs[1][1], 2e-3)
    yo, so = O.chunked(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D),
                       np.array([0.99, 0.995, 0.9999]), state=None if st0 is None else
                       state_to_np(st0, BH, D))
    assert_close(outs[0][0], yo.reshape(B, H, L, D), TOL_BF16, "y vs oracle")
    assert_state_close(outs[0][1], so, TOL_BF16)
