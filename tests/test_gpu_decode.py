"""GPU parity of the fused decode step (prime_decode_step) against the oracle
recurrence (attention.py:119-143 restated in oracle/prime_oracle.c)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib

from gpu_util import (TOL_BF16, TOL_F32, assert_close, assert_state_close, random_state,
                      state_to_dev, state_to_np, to_dev, to_np, dev)

pytestmark = pytest.mark.gpu

D = 64


def _run(B, H, Hkv, in_dtype, y_dtype, with_state, seed, inplace=False, lam=None):
    BH = B * H
    rng = np.random.default_rng(seed)
    q, _, _ = O.make_inputs((B, H, D), seed=seed, bf16=in_dtype == torch.bfloat16)
    _, k, v = O.make_inputs((B, Hkv, D), seed=seed + 1, bf16=in_dtype == torch.bfloat16)
    lam = rng.uniform(0.99, 0.9999, H).astype(np.float32) if lam is None else lam
    st0 = random_state(BH, D, seed + 2) if with_state else None
    # oracle: expand GQA heads (head h uses kv head h // (H/Hkv))
    grp = H // Hkv
    ke = np.repeat(k, grp, axis=1)
    ve = np.repeat(v, grp, axis=1)
    yo, so = O.recurrent(q.reshape(BH, 1, D), ke.reshape(BH, 1, D), ve.reshape(BH, 1, D),
                         np.tile(lam.astype(np.float64), B), eps=1.0, state=st0)
    tq, tk, tv = to_dev(q, in_dtype), to_dev(k, in_dtype), to_dev(v, in_dtype)
    decay = to_dev(lam)
    st_in = state_to_dev(st0, B, H, D) if with_state else None
    st_out = st_in if inplace else _lib.new_state(B, H, D, dev())
    y = torch.empty(B, H, D, device=dev(), dtype=y_dtype)
    _lib.decode_step(tq, tk, tv, decay, 1.0, st_in, st_out, y)
    torch.cuda.synchronize()
    return yo.reshape(B, H, D), so, to_np(y), state_to_np(st_out, BH, D)


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_state", [False, True])
def test_decode_matches_oracle(in_dtype, with_state):
    yo, so, y, s = _run(5, 6, 6, in_dtype, torch.float32, with_state, seed=10)
    tol = TOL_F32 if in_dtype == torch.float32 else TOL_BF16
    # the arithmetic is fp32 throughout, so even bf16 inputs match tightly
    assert_close(y, yo, min(tol, 1e-4), "y")
    assert_state_close(s, so, min(tol, 1e-5))


@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float16])
def test_decode_low_precision_output(y_dtype):
    yo, so, y, s = _run(3, 4, 4, torch.bfloat16, y_dtype, True, seed=11)
    assert_close(y, yo, 1e-2, "y")
    assert_state_close(s, so, 1e-5)


def test_decode_inplace_and_gqa():
    yo, so, y, s = _run(4, 8, 2, torch.bfloat16, torch.float32, True, seed=12, inplace=True)
    assert_close(y, yo, 1e-4, "y")
    assert_state_close(s, so, 1e-5)


def test_decode_zero_state_single_token_is_v():
    """Known answer: zero state and den >= eps give y = v exactly (up to fp32)."""
    B, H = 2, 3
    q = np.zeros((B, H, D), np.float32)  # den = 1 exactly
    _, k, v = O.make_inputs((B, H, D), seed=13, bf16=True)
    y = torch.empty(B, H, D, device=dev())
    st = _lib.new_state(B, H, D, dev())
    _lib.decode_step(to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16),
                     to_dev(np.full(H, 0.9, np.float32)), 1.0, None, st, y)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_np(y), v.astype(np.float64))


def test_decode_strided_views():
    """q/k/v as [B, 1, H, D] projections viewed [B, H, D] (the module's layout)."""
    B, H = 3, 5
    BH = B * H
    q, k, v = O.make_inputs((B, 1, H, D), seed=14, bf16=True)
    lam = np.full(H, 0.995, np.float32)
    st0 = random_state(BH, D, 15)

    def strided(x):  # token 1 of a [B, H, 2, D] buffer: strides (2HD, 2D, 1)
        buf = torch.zeros(B, H, 2, D, device=dev(), dtype=torch.bfloat16)
        buf[:, :, 1] = to_dev(x, torch.bfloat16).transpose(1, 2)[:, :, 0]
        return buf[:, :, 1]
    tq, tk, tv = strided(q), strided(k), strided(v)
    assert not tq.is_contiguous()
    st_out = _lib.new_state(B, H, D, dev())
    y = torch.empty(B, H, D, device=dev())
    _lib.decode_step(tq, tk, tv, to_dev(lam), 1.0, state_to_dev(st0, B, H, D), st_out, y)
    torch.cuda.synchronize()
    yo, so = O.recurrent(q.transpose(0, 2, 1, 3).reshape(BH, 1, D), k.transpose(0, 2, 1, 3).reshape(BH, 1, D),
                         v.transpose(0, 2, 1, 3).reshape(BH, 1, D), np.tile(lam.astype(np.float64), B),
                         state=st0)
    assert_close(to_np(y), yo.reshape(B, H, D), 1e-4, "y")
    assert_state_close(state_to_np(st_out, BH, D), so, 1e-5)


def test_decode_many_steps_constant_state_and_parity():
    """20 in-place steps: state bytes constant, result equals the recurrence."""
    B, H, T = 2, 4, 20
    BH = B * H
    q, k, v = O.make_inputs((B, H, T, D), seed=16, bf16=True)
    lam = np.full(H, 0.999, np.float32)
    st = _lib.new_state(B, H, D, dev(), zero=True)
    ptrs = [t.data_ptr() for t in st]
    ys = []
    for t in range(T):
        y = torch.empty(B, H, D, device=dev())
        _lib.decode_step(to_dev(q[:, :, t], torch.bfloat16), to_dev(k[:, :, t], torch.bfloat16),
                         to_dev(v[:, :, t], torch.bfloat16), to_dev(lam), 1.0, st, st, y)
        ys.append(to_np(y))
    assert [t.data_ptr() for t in st] == ptrs
    yo, so = O.recurrent(q.reshape(BH, T, D), k.reshape(BH, T, D), v.reshape(BH, T, D), 0.999)
    yg = np.stack(ys, 2).reshape(BH, T, D)
    assert_close(yg, yo, 1e-4, "y")
    assert_state_close(state_to_np(st, BH, D), so, 1e-5)


def test_decode_rejects_bad_arguments():
    B, H = 1, 2
    x = torch.zeros(B, H, D, device=dev())
    st = _lib.new_state(B, H, D, dev())
    dec = to_dev(np.ones(H, np.float32))
    xw = torch.zeros(B, H, 96, device=dev())
    with pytest.raises(RuntimeError, match="head dim"):  # 64, or 1 .. 63
        _lib.decode_step(xw, xw, xw, dec, 1.0, None, _lib.new_state(B, H, 96, dev()), xw)
    # partially overlapping in/out state
    st_bad = (st[0], st[1], st[2], st[3], st[4], st[4])
    st_in = _lib.new_state(B, H, D, dev())
    st_in = (st_in[0], st_in[1], st_in[2], st_in[3], st_in[4], st[5])
    with pytest.raises(RuntimeError, match="overlaps"):
        _lib.decode_step(x, x, x, dec, 1.0, st_in, st, x)
    del st_bad


@pytest.mark.parametrize("qk_norm", [True, False])
def test_decode_qknorm_prologue_matches_module_ops(qk_norm):
    """prime_decode_step_qknorm on raw projections == LayerNorm + scale in torch
    (attention.py:96-101) followed by prime_decode_step."""
    import torch.nn as nn
    B, H = 3, 4
    torch.manual_seed(5)
    qn, kn = nn.LayerNorm(D).to(dev()).bfloat16(), nn.LayerNorm(D).to(dev()).bfloat16()
    with torch.no_grad():
        for m in (qn, kn):
            m.weight.uniform_(0.5, 1.5)
            m.bias.uniform_(-0.2, 0.2)
    q = torch.randn(B, H, D, device=dev()).bfloat16()
    k = torch.randn(B, H, D, device=dev()).bfloat16()
    v = torch.randn(B, H, D, device=dev()).bfloat16()
    lam = to_dev(np.full(H, 0.99, np.float32))
    st0 = state_to_dev(random_state(B * H, D, 17), B, H, D)
    with torch.no_grad():
        qr, kr = (qn(q), kn(k)) if qk_norm else (q, k)
        qr = qr * 0.125
    y_ref = torch.empty(B, H, D, device=dev())
    s_ref = _lib.new_state(B, H, D, dev())
    _lib.decode_step(qr, kr, v, lam, 1.0, st0, s_ref, y_ref)
    y = torch.empty(B, H, D, device=dev())
    s = _lib.new_state(B, H, D, dev())
    norm = _lib.qk_norm(qn if qk_norm else None, kn if qk_norm else None, 0.125, torch.bfloat16)
    _lib.decode_step_qknorm(q, k, v, lam, 1.0, norm, st0, s, y)
    torch.cuda.synchronize()
    assert_close(to_np(y), to_np(y_ref), 5e-3, "y")
    assert_state_close(state_to_np(s, B * H, D), state_to_np(s_ref, B * H, D), 5e-3)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
def test_add_rmsnorm_matches_torch(dtype, tol):
    """prime_add_rmsnorm: x <- x + delta (rounded to dtype), out = RMSNorm(x) * w
    (model.py:47-56) against the fp32 formula on the rounded sum."""
    rows, hid = 37, 768
    torch.manual_seed(6)
    x = torch.randn(rows, hid, device=dev()).to(dtype)
    d = torch.randn(rows, hid, device=dev()).to(dtype)
    w = (torch.rand(hid, device=dev()) + 0.5).to(dtype)
    xs = (x + d)  # torch's add in dtype: the rounded sum the kernel must store
    ref = xs.float() * torch.rsqrt(xs.float().pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    out = torch.empty_like(x)
    xk = x.clone()
    _lib.add_rmsnorm(xk, d, w, out, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(xk, xs)
    assert_close(to_np(out), to_np(ref), tol, "out")
    out2 = torch.empty_like(x)
    _lib.add_rmsnorm(xs, None, w, out2, 1e-6)  # no delta: x untouched, same normalisation
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
