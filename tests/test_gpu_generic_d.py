"""GPU parity of the head dims below 64 (generic_d.hip: one wavefront per
(sequence, head), the recurrence token by token) against the oracle, whose
restatement takes any D: the chunked prefill (chunked_ssd.py:48-184, with its
own chunk size or none -- the result does not depend on it) and the dense
branch's double clamp (attention.py:160-202), the decode step
(attention.py:119-143), the backward (oracle_recurrent_vjp / oracle_dense_vjp),
the QK LayerNorm applied on load and prime_head_layernorm; then the
reference's own module tests at head_dim 32 (tests/test_attention.py,
tests/test_chunked_ssd_parity.py) and its model test at head_dim 16
(tests/test_model.py), each with a parity check added.

Tolerances as for head dim 64: bf16 inputs 2e-2, fp32 inputs 1e-3
(max|d| / max|ref| per tensor)."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from oracle import torch_cpu as TC
from prime_moment_attention import _lib
from prime_moment_attention.chunked_ssd import prime_prefill

from gpu_util import (TOL_BF16, TOL_F32, assert_close, assert_state_close, random_state, state_to_dev, state_to_np,
                      to_dev, to_np, dev)

pytestmark = pytest.mark.gpu


def _inputs(B, H, Hkv, L, D, dtype, seed, normalize=True):
    """q (scaled by 1/sqrt(D)), k, v as the device will hold them (bf16-rounded
    after the scale when bf16, so both sides see the same values)."""
    bf = dtype == torch.bfloat16
    q, _, _ = O.make_inputs((B, H, L, D), seed=seed, bf16=bf, normalize=normalize)
    _, k, v = O.make_inputs((B, Hkv, L, D), seed=seed + 1, bf16=bf, normalize=normalize)
    if bf:
        q = O.bf16_round(q)
    return q, k, v


def _prefill_case(B, H, L, D, dtype, with_state, seed, Hkv=None, normalize=True, eps=1.0, dense_clamp=False,
                  inplace=False):
    Hkv = Hkv or H
    BH = B * H
    q, k, v = _inputs(B, H, Hkv, L, D, dtype, seed, normalize)
    lam = np.random.default_rng(seed).uniform(0.99, 0.9999, H).astype(np.float32)
    st0 = random_state(BH, D, seed + 2) if with_state else None
    grp = H // Hkv
    ke, ve = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    args = (q.reshape(BH, L, D), ke.reshape(BH, L, D), ve.reshape(BH, L, D), np.tile(lam.astype(np.float64), B))
    if dense_clamp:
        yo, so = O.dense(*args, eps=eps, state=st0)
    else:
        yo, so = O.chunked(*args, eps=eps, chunk=64, state=st0)
    print(f"[generic prefill] B={B} H={H} Hkv={Hkv} L={L} D={D} {dtype} state={with_state} dense={dense_clamp}",
          flush=True)
    st_in = state_to_dev(st0, B, H, D) if with_state else None
    y, st = prime_prefill(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), state=st_in, decay=to_dev(lam),
                          eps=eps, return_state=True, dense_clamp=dense_clamp,
                          state_out=st_in if inplace else None)
    torch.cuda.synchronize()
    return yo.reshape(B, H, L, D), so, to_np(y), state_to_np(st, BH, D)


@pytest.mark.parametrize("D", [32, 16, 48, 7, 63])
@pytest.mark.parametrize("B,H,L", [(2, 3, 200), (1, 2, 13), (1, 1, 1)])
@pytest.mark.parametrize("with_state", [False, True])
def test_generic_prefill_bf16_matches_oracle(D, B, H, L, with_state):
    yo, so, y, s = _prefill_case(B, H, L, D, torch.bfloat16, with_state, seed=D + L)
    assert_close(y, yo, TOL_BF16, "y")
    assert_state_close(s, so, TOL_BF16)


@pytest.mark.parametrize("D", [32, 24])
@pytest.mark.parametrize("with_state", [False, True])
def test_generic_prefill_f32_matches_oracle(D, with_state):
    yo, so, y, s = _prefill_case(2, 2, 300, D, torch.float32, with_state, seed=3 * D)
    assert_close(y, yo, TOL_F32, "y")
    assert_state_close(s, so, TOL_F32)


def test_generic_prefill_inplace_state_and_gqa():
    yo, so, y, s = _prefill_case(2, 4, 150, 32, torch.bfloat16, True, seed=41, Hkv=2, inplace=True)
    assert_close(y, yo, TOL_BF16, "y")
    assert_state_close(s, so, TOL_BF16)


@pytest.mark.parametrize("with_state", [False, True])
def test_generic_prefill_dense_clamp_matches_dense_branch(with_state):
    """Unnormalised q/k: den < eps for early tokens; with a state the dense
    branch clamps the call's denominator before adding the state's readout
    (attention.py:177,185)."""
    yo, so, y, s = _prefill_case(1, 2, 90, 32, torch.float32, with_state, seed=5, normalize=False, eps=4.0,
                                 dense_clamp=True)
    assert_close(y, yo, TOL_F32, "y")
    assert_state_close(s, so, TOL_F32)


def test_generic_prefill_strided_output_and_long_sequence():
    """y written through the o_proj input layout [B, L, H, D] (strides), a
    sequence of many staged chunks."""
    B, H, L, D = 1, 2, 1100, 32
    q, k, v = _inputs(B, H, H, L, D, torch.bfloat16, 77)
    lam = np.full(H, 0.995, np.float32)
    yo, so = O.chunked(q.reshape(B * H, L, D), k.reshape(B * H, L, D), v.reshape(B * H, L, D),
                       np.tile(lam.astype(np.float64), B), eps=1.0, chunk=64)
    y_bl = torch.empty(B, L, H, D, device=dev(), dtype=torch.bfloat16)
    st = _lib.new_state(B, H, D, dev())
    _lib.chunked_prefill(to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16),
                         to_dev(lam), 1.0, 64, None, y_bl.transpose(1, 2), st)
    torch.cuda.synchronize()
    assert_close(to_np(y_bl.transpose(1, 2)), yo.reshape(B, H, L, D), TOL_BF16, "y")
    assert_state_close(state_to_np(st, B * H, D), so, TOL_BF16)


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, TOL_BF16), (torch.float32, TOL_F32)])
@pytest.mark.parametrize("D", [32, 16])
def test_generic_decode_matches_oracle(dtype, tol, D):
    B, H, Hkv = 3, 4, 2
    q, k, v = _inputs(B, H, Hkv, 1, D, dtype, 90 + D)
    lam = np.random.default_rng(D).uniform(0.99, 0.999, H).astype(np.float32)
    st0 = random_state(B * H, D, 11)
    grp = H // Hkv
    ke, ve = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    yo, so = O.recurrent(q.reshape(B * H, 1, D), ke.reshape(B * H, 1, D), ve.reshape(B * H, 1, D),
                         np.tile(lam.astype(np.float64), B), eps=1.0, state=st0)
    st_in = state_to_dev(st0, B, H, D)
    y = torch.empty(B, H, D, device=dev(), dtype=torch.float32)
    so_d = _lib.new_state(B, H, D, dev())
    _lib.decode_step(to_dev(q[:, :, 0], dtype), to_dev(k[:, :, 0], dtype), to_dev(v[:, :, 0], dtype), to_dev(lam),
                     1.0, st_in, so_d, y)
    torch.cuda.synchronize()
    assert_close(to_np(y), yo.reshape(B, H, D), tol, "y")
    assert_state_close(state_to_np(so_d, B * H, D), so, tol)
    # in place (state_out is state_in), from a zero state
    z = _lib.new_state(B, H, D, dev(), zero=True)
    _lib.decode_step(to_dev(q[:, :, 0], dtype), to_dev(k[:, :, 0], dtype), to_dev(v[:, :, 0], dtype), to_dev(lam),
                     1.0, z, z, y)
    torch.cuda.synchronize()
    yo1, _ = O.recurrent(q.reshape(B * H, 1, D), ke.reshape(B * H, 1, D), ve.reshape(B * H, 1, D),
                         np.tile(lam.astype(np.float64), B), eps=1.0)
    assert_close(to_np(y), yo1.reshape(B, H, D), tol, "y from zero")


def _layernorms(D, dtype, seed):
    torch.manual_seed(seed)
    qn, kn = torch.nn.LayerNorm(D).to(dev(), dtype), torch.nn.LayerNorm(D).to(dev(), dtype)
    with torch.no_grad():
        for m in (qn, kn):
            m.weight.uniform_(0.5, 1.5)
            m.bias.uniform_(-0.2, 0.2)
    return qn, kn


@pytest.mark.parametrize("qk_norm", [True, False])
def test_generic_decode_qknorm_prologue_matches_module_ops(qk_norm):
    """prime_decode_step_qknorm on raw projections == LayerNorm + scale in torch
    (attention.py:96-101) followed by prime_decode_step."""
    B, H, D = 3, 4, 32
    qn, kn = _layernorms(D, torch.bfloat16, 5)
    q, k, v = (torch.randn(B, H, D, device=dev()).bfloat16() for _ in range(3))
    lam = to_dev(np.full(H, 0.99, np.float32))
    st0 = state_to_dev(random_state(B * H, D, 17), B, H, D)
    scale = 1.0 / math.sqrt(D)
    with torch.no_grad():
        qr, kr = (qn(q), kn(k)) if qk_norm else (q, k)
        qr = qr * scale
    y_ref, s_ref = torch.empty(B, H, D, device=dev()), _lib.new_state(B, H, D, dev())
    _lib.decode_step(qr, kr, v, lam, 1.0, st0, s_ref, y_ref)
    y, s = torch.empty(B, H, D, device=dev()), _lib.new_state(B, H, D, dev())
    norm = _lib.qk_norm(qn if qk_norm else None, kn if qk_norm else None, scale, torch.bfloat16)
    _lib.decode_step_qknorm(q, k, v, lam, 1.0, norm, st0, s, y)
    torch.cuda.synchronize()
    assert_close(to_np(y), to_np(y_ref), 5e-3, "y")
    assert_state_close(state_to_np(s, B * H, D), state_to_np(s_ref, B * H, D), 5e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_ln", [True, False])
def test_generic_head_layernorm_matches_module_ops(dtype, with_ln):
    """prime_head_layernorm at D = 32 in place on the projection layout ==
    nn.LayerNorm then * scale (attention.py:96-101), fp32 within 1e-5; bf16:
    the LayerNorm output may differ by one bf16 ulp (rsqrt and the order of the
    fp32 sums against torch's), which the scale 1/sqrt(32) -- not a power of two
    -- carries into a second rounding: two ulps of the result."""
    B, L, H, D = 3, 137, 5, 32
    ln, _ = _layernorms(D, dtype, 4)
    raw = (torch.randn(B, L, H * D, device=dev()) * 3 + 0.5).to(dtype)
    x = raw.view(B, L, H, D).transpose(1, 2)
    scale = 1.0 / math.sqrt(D)
    with torch.no_grad():
        ref = (ln(x) if with_ln else x) * scale
    _lib.head_layernorm(x, x, ln if with_ln else None, scale)
    torch.cuda.synchronize()
    d = (x.float() - ref.float()).abs()
    bound = ref.float().abs() * 2 ** -6 + 1e-6 if dtype == torch.bfloat16 else 1e-5 * (1 + ref.float().abs())
    assert bool((d <= bound).all()), float(d.max())


@pytest.mark.parametrize("with_state", [False, True])
def test_generic_prefill_qknorm_on_load_equals_normalising_first(with_state):
    """The prefill's QK LayerNorm on load and prime_head_layernorm share one
    row routine: the outputs are bit-identical."""
    B, H, L, D = 2, 3, 150, 32
    qn, kn = _layernorms(D, torch.bfloat16, 6)
    q = torch.randn(B, L, H, D, device=dev()).bfloat16().transpose(1, 2)
    k = torch.randn(B, L, H, D, device=dev()).bfloat16().transpose(1, 2)
    v = torch.randn(B, H, L, D, device=dev()).bfloat16()
    lam = to_dev(np.full(H, 0.995, np.float32))
    st0 = state_to_dev(random_state(B * H, D, 8), B, H, D) if with_state else None
    scale = 1.0 / math.sqrt(D)
    norm = _lib.qk_norm(qn, kn, scale, torch.bfloat16)
    y1, s1 = torch.empty(B, H, L, D, device=dev()), _lib.new_state(B, H, D, dev())
    _lib.chunked_prefill(q, k, v, lam, 1.0, 64, st0, y1, s1, qk_norm=norm)
    qc, kc = q.clone(), k.clone()
    _lib.head_layernorm(qc, qc, qn, scale)
    _lib.head_layernorm(kc, kc, kn, 1.0)
    y2, s2 = torch.empty(B, H, L, D, device=dev()), _lib.new_state(B, H, D, dev())
    _lib.chunked_prefill(qc, kc, v, lam, 1.0, 64, st0, y2, s2)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    for a, b in zip(s1, s2):
        assert torch.equal(a, b)


def _backward_case(B, H, L, D, dtype, with_state, with_dstate, seed, normalize=True, eps=1.0, dense=False):
    BH = B * H
    bf = dtype == torch.bfloat16
    q, k, v = _inputs(B, H, H, L, D, dtype, seed, normalize)
    rng = np.random.default_rng(seed + 1)
    lam = rng.uniform(0.99, 0.9999, H).astype(np.float32)
    dy = rng.standard_normal((B, H, L, D)).astype(np.float32)
    if bf:
        dy = O.bf16_round(dy)
    st0 = random_state(BH, D, seed + 2) if with_state else None
    ds = tuple(0.1 * rng.standard_normal(x.shape) for x in O.zero_state(BH, D)) if with_dstate else None
    vjp = O.dense_vjp if dense else O.recurrent_vjp
    ref = vjp(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D), np.tile(lam.astype(np.float64), B),
              dy.reshape(BH, L, D), eps=eps, state=st0, dstate=ds)
    print(f"[generic bwd] B={B} H={H} L={L} D={D} {dtype} state={with_state} dstate={with_dstate} dense={dense}",
          flush=True)
    g = [torch.empty(B, H, L, D, device=dev(), dtype=torch.float32) for _ in range(3)]
    dsi = _lib.new_state(B, H, D, dev()) if with_state else None
    _lib.chunked_prefill_backward(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(lam), eps,
                                  state_to_dev(st0, B, H, D) if with_state else None,
                                  to_dev(dy, torch.bfloat16 if bf else torch.float32),
                                  state_to_dev(ds, B, H, D) if with_dstate else None, *g, dsi,
                                  flags=1 if dense else 0)
    torch.cuda.synchronize()
    got = [to_np(t).reshape(BH, L, D) for t in g]
    for name, r, x in zip(("dq", "dk", "dv"), ref[:3], got):
        assert np.isfinite(x).all(), name
        e = np.abs(x - r).max() / max(np.abs(r).max(), 1e-300)
        assert e < TOL_F32, f"{name}: rel err {e:.3e}"
    if with_state:
        assert_state_close(state_to_np(dsi, BH, D), ref[3], TOL_F32, "dstate_in")


@pytest.mark.parametrize("D", [32, 16, 7])
@pytest.mark.parametrize("L", [1, 70, 300])
@pytest.mark.parametrize("with_state,with_dstate", [(False, False), (True, True)])
def test_generic_backward_matches_oracle_vjp(D, L, with_state, with_dstate):
    """fp32 arithmetic on the inputs both sides see: held to 1e-3 also for bf16."""
    _backward_case(2, 2, L, D, torch.float32, with_state, with_dstate, seed=D * 7 + L)


def test_generic_backward_bf16_inputs():
    _backward_case(1, 3, 130, 32, torch.bfloat16, True, False, seed=12)


@pytest.mark.parametrize("with_state", [False, True])
def test_generic_backward_dense_clamp(with_state):
    _backward_case(1, 2, 60, 32, torch.float32, with_state, with_state, seed=13, normalize=False, eps=4.0,
                   dense=True)


def test_generic_entry_points_reject_bad_arguments():
    B, H, L, D = 1, 2, 10, 32
    x = torch.zeros(B, H, L, D, device=dev())
    lam = to_dev(np.full(H, 0.99, np.float32))
    xw = torch.zeros(B, H, L, 80, device=dev())
    with pytest.raises(RuntimeError, match="head dim"):  # 64, or 1 .. 63
        _lib.chunked_prefill(xw, xw, xw, lam, 1.0, 64, None, xw.clone(), _lib.new_state(B, H, 80, dev()))
    g = [torch.empty(B, H, L, D, device=dev()) for _ in range(3)]
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.chunked_prefill_backward(x, x, x, lam, 1.0, None, x, None, *g, None,
                                      workspace=torch.empty(16, dtype=torch.uint8, device=dev()))
    with pytest.raises(RuntimeError, match="flags"):
        _lib.chunked_prefill(x, x, x, lam, 1.0, 64, None, x.clone(), None, flags=4)


# ---- the reference's module tests at head_dim 32 (tests/test_attention.py) ----

def _attn(dtype=torch.float32):
    from prime_moment_attention import PrimeMomentAttention
    torch.manual_seed(42)
    return PrimeMomentAttention(hidden_size=128, num_heads=4, head_dim=32, decay=0.999,
                                use_qk_norm=True).to(dev(), dtype)


def _attn_cpu_forward(m, x, state=None):
    """fp32 CPU composition of the module (attention.py:83-210): torch
    projections and LayerNorm, the restated chunked core."""
    W = {k: v.detach().float().cpu() for k, v in m.state_dict().items()}
    x = x.detach().float().cpu()
    B, L, _ = x.shape
    H, D = m.num_heads, m.head_dim
    q = (x @ W["q_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
    k = (x @ W["k_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
    v = (x @ W["v_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
    q = F.layer_norm(q, (D,), W["q_norm.weight"], W["q_norm.bias"]) / math.sqrt(D)
    k = F.layer_norm(k, (D,), W["k_norm.weight"], W["k_norm.bias"])
    y, st = TC.chunked_core(q.contiguous(), k.contiguous(), v.contiguous(), m.decay, eps=m.eps, state=state)
    return y.transpose(1, 2).reshape(B, L, H * D) @ W["o_proj.weight"].T, st


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def test_reference_prefill_output_shape_and_parity():
    m = _attn()
    x = torch.randn(2, 16, 128, device=dev())
    with torch.no_grad():
        out, state = m(x, return_state=True)
    assert out.shape == (2, 16, 128)
    S0, S1, S2, K0, K1, K2 = state
    assert S0.shape == (2, 4, 32) and S1.shape == (2, 4, 32, 32) and S2.shape == (2, 4, 32, 32)
    assert K0.shape == (2, 4, 1) and K1.shape == (2, 4, 32) and K2.shape == (2, 4, 32)
    ref, rst = _attn_cpu_forward(m, x)
    assert _rel(out, ref) < TOL_F32
    for a, b in zip(state, rst):
        assert _rel(a, b.reshape(a.shape)) < TOL_F32


def test_reference_step_decode_constant_memory_and_parity():
    m = _attn()
    with torch.no_grad():
        x0 = torch.randn(2, 4, 128, device=dev())
        _, state = m(x0, return_state=True)
        nbytes = sum(t.element_size() * t.nelement() for t in state)
        xs = [x0]
        for _ in range(20):
            tok = torch.randn(2, 1, 128, device=dev())
            out, state = m(tok, state=state, return_state=True)
            assert out.shape == (2, 1, 128)
            assert sum(t.element_size() * t.nelement() for t in state) == nbytes
            xs.append(tok)
        ref, _ = _attn_cpu_forward(m, torch.cat(xs, 1))
    assert _rel(out[:, 0], ref[:, -1]) < TOL_F32


def test_reference_gradient_flow_and_parity():
    """The module trains through the generic backward: every gradient against
    fp32 CPU autograd of the composition."""
    m = _attn()
    x = torch.randn(2, 8, 128, device=dev(), requires_grad=True)
    out, _ = m(x)
    out.sum().backward()
    assert x.grad is not None and not torch.isnan(x.grad).any()
    for p in (m.q_proj.weight, m.k_proj.weight, m.v_proj.weight):
        assert p.grad is not None
    mc = _attn().float().cpu()
    mc.load_state_dict({k: v.detach().float().cpu() for k, v in m.state_dict().items()})
    xc = x.detach().float().cpu().requires_grad_(True)
    W = dict(mc.named_parameters())
    B, L, H, D = 2, 8, 4, 32
    q = (xc @ W["q_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
    k = (xc @ W["k_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
    v = (xc @ W["v_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
    q = F.layer_norm(q, (D,), W["q_norm.weight"], W["q_norm.bias"]) / math.sqrt(D)
    k = F.layer_norm(k, (D,), W["k_norm.weight"], W["k_norm.bias"])
    y, _ = TC.chunked_core(q.contiguous(), k.contiguous(), v.contiguous(), mc.decay, eps=mc.eps)
    (y.transpose(1, 2).reshape(B, L, H * D) @ W["o_proj.weight"].T).sum().backward()
    assert _rel(x.grad, xc.grad) < TOL_F32
    for (name, p), (_, pc) in zip(m.named_parameters(), mc.named_parameters()):
        assert _rel(p.grad, pc.grad) < TOL_F32, name


def test_reference_numerical_stability():
    m = _attn()
    with torch.no_grad():
        out, _ = m(torch.randn(1, 128, 128, device=dev()) * 5.0)
    assert not torch.isnan(out).any() and not torch.isinf(out).any()


def test_reference_chunked_ssd_parity_head_dim_32():
    """tests/test_chunked_ssd_parity.py: the dense module and the chunked module
    on copied weights, fp32, B=2 L=256 H=4 D=32: outputs within 1e-5, states
    within 2e-3; and both against the fp32 CPU composition."""
    from prime_moment_attention import PrimeMomentAttention
    from prime_moment_attention.chunked_ssd import ChunkedPrimeSSD
    torch.manual_seed(0)
    dense = PrimeMomentAttention(hidden_size=128, num_heads=4, head_dim=32, decay=0.9995,
                                 use_qk_norm=True).to(dev())
    chunk = ChunkedPrimeSSD(hidden_size=128, num_heads=4, head_dim=32, chunk_size=64, decay=0.9995,
                            use_qk_norm=True).to(dev())
    chunk.load_state_dict(dense.state_dict())
    x = torch.randn(2, 256, 128, device=dev())
    with torch.no_grad():
        od, sd = dense(x, return_state=True)
        oc, sc = chunk(x, return_state=True)
    assert (od - oc).abs().max().item() < 1e-5
    for a, b in zip(sd, sc):
        assert (a.squeeze() - b.squeeze()).abs().max().item() < 2e-3
    ref, _ = _attn_cpu_forward(dense, x)
    assert _rel(od, ref) < TOL_F32


# ---- the reference's model test at head_dim 16 (tests/test_model.py) ----

def _model16():
    from prime_moment_attention import PrimeConfig, PrimeForCausalLM
    torch.manual_seed(42)
    cfg = PrimeConfig(vocab_size=100, hidden_size=64, num_layers=2, num_heads=4, head_dim=16, decay=0.999,
                      use_qk_norm=True)
    return PrimeForCausalLM(cfg).to(dev())


def test_reference_model_forward_loss_and_logits_parity():
    from test_gpu_model import _ref_forward
    model = _model16()
    ids = torch.randint(0, 100, (2, 16))
    labels = ids.clone()
    with torch.no_grad():
        out = model(ids.to(dev()), labels=labels.to(dev()))
    assert out["logits"].shape == (2, 16, 100)
    assert not torch.isnan(out["loss"]) and out["loss"].item() > 0.0
    assert _rel(out["logits"], _ref_forward(model, ids)) < TOL_F32


def test_reference_model_backward_gradients():
    model = _model16()
    ids = torch.randint(0, 100, (2, 8), device=dev())
    loss = model(ids, labels=ids.clone())["loss"]
    loss.backward()
    assert model.embed_tokens.weight.grad is not None
    assert model.layers[0].self_attn.q_proj.weight.grad is not None
    assert model.layers[0].mlp.gate_proj.weight.grad is not None
    assert not torch.isnan(model.layers[0].self_attn.q_proj.weight.grad).any()


def test_reference_model_generate():
    model = _model16()
    prompt = torch.tensor([[1, 2, 3, 4]], device=dev())
    with torch.no_grad():
        gen = model.generate(prompt, max_new_tokens=10, temperature=0.7)
    assert gen.shape == (1, 14)
    assert bool((gen >= 0).all() and (gen < 100).all())


# ---- selective PRIME at head dims below 64 (selective.py:264-444) ----

def _sel_inputs(B, H, Hkv, L, D, seed, dtype):
    q, k, v = _inputs(B, H, Hkv, L, D, dtype, seed)
    rng = np.random.default_rng(seed)
    delta = np.log1p(np.exp(rng.standard_normal((B, H, L)) - 1.0))  # softplus step sizes
    tau = rng.uniform(8.0, 400.0, H)
    beta = rng.uniform(0.6, 2.5, H).astype(np.float32)
    log_decay = (-delta / tau[None, :, None]).astype(np.float32)
    return q, k, v, log_decay, beta


def _sel_state(BH, D, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((BH, D)), rng.standard_normal((BH, D, D)) * 0.05,
            rng.standard_normal((BH, D, D)) * 0.05, np.abs(rng.standard_normal(BH)) * 5 + 1,
            rng.standard_normal((BH, D)) * 0.1, np.abs(rng.standard_normal((BH, D))) * 0.1)


@pytest.mark.parametrize("D", [32, 16])
@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, TOL_BF16), (torch.float32, TOL_F32)])
@pytest.mark.parametrize("with_state", [False, True])
def test_generic_selective_prefill_matches_oracle(D, dtype, tol, with_state):
    """Per-token decays, beta-weighted keys, the selective state convention
    (S2, K2 carry the 1/2): against oracle_selective_recurrent, with GQA."""
    B, H, Hkv, L = 2, 4, 2, 150
    q, k, v, ld, beta = _sel_inputs(B, H, Hkv, L, D, 200 + D, dtype)
    st = _sel_state(B * H, D, 7) if with_state else None
    grp = H // Hkv
    ke, ve = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    yo, so = O.selective_recurrent(q.reshape(B * H, L, D), ke.reshape(B * H, L, D), ve.reshape(B * H, L, D),
                                   np.exp(ld.astype(np.float64)).reshape(B * H, L),
                                   np.tile(beta.astype(np.float64), B), eps=1.0, state=st)
    y = torch.empty(B, H, L, D, device=dev())
    s_out = _lib.new_state(B, H, D, dev())
    _lib.selective_prefill(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(ld), to_dev(beta), 1.0,
                           state_to_dev(st, B, H, D) if with_state else None, y, s_out)
    torch.cuda.synchronize()
    assert_close(to_np(y).reshape(B * H, L, D), yo, tol, "y")
    assert_state_close(state_to_np(s_out, B * H, D), so, tol)


@pytest.mark.parametrize("gate_kind", ["decay_bh", "step"])
def test_generic_selective_decode_step(gate_kind):
    """One token through the selective step with the gate formed in the
    kernel (decays per (sequence, head), or softplus / clamp / exp of the step
    pre-activations), against the oracle; in place."""
    B, H, D = 3, 4, 32
    q, k, v, _, beta = _sel_inputs(B, H, H, 1, D, 300, torch.float32)
    rng = np.random.default_rng(301)
    pre = rng.standard_normal((B, H)).astype(np.float32)
    tau = rng.uniform(8.0, 400.0, H).astype(np.float32)
    lam = np.exp(-np.clip(np.log1p(np.exp(pre.astype(np.float64))), 1e-4, 50.0) / tau[None, :])
    st = _sel_state(B * H, D, 302)
    yo, so = O.selective_recurrent(q.reshape(B * H, 1, D), k.reshape(B * H, 1, D), v.reshape(B * H, 1, D),
                                   lam.reshape(B * H, 1), np.tile(beta.astype(np.float64), B), eps=1.0, state=st)
    s = state_to_dev(st, B, H, D)
    y = torch.empty(B, H, D, device=dev())
    if gate_kind == "decay_bh":
        lam_d = to_dev(lam.astype(np.float32))
        gate = _lib.selective_gate(B, H, decay_bh=lam_d)
    else:
        pre_d, tau_d = to_dev(pre), to_dev(tau)
        gate = _lib.selective_gate(B, H, step=pre_d, tau=tau_d)
    _lib.selective_decode_step(to_dev(q[:, :, 0]), to_dev(k[:, :, 0]), to_dev(v[:, :, 0]), gate, to_dev(beta), 1.0,
                               None, s, s, y)
    torch.cuda.synchronize()
    assert_close(to_np(y).reshape(B * H, D), yo.reshape(B * H, D), TOL_F32, "y")
    assert_state_close(state_to_np(s, B * H, D), so, TOL_F32)


@pytest.mark.parametrize("D,L", [(32, 100), (16, 70), (8, 1)])
@pytest.mark.parametrize("with_state", [False, True])
def test_generic_selective_backward_matches_fp64_autograd(D, L, with_state):
    """dq, dk, dv, the log decays' adjoint, beta's adjoint per sequence and the
    incoming state's adjoint against torch float64 autograd of
    tests/selective_ref.py (the reference's parallel branch with the step
    branch's incoming state)."""
    from selective_ref import selective_forward
    B, H = 2, 2
    q, k, v, ld, beta = _sel_inputs(B, H, H, L, D, 400 + D + L, torch.float32)
    rng = np.random.default_rng(401)
    dy = rng.standard_normal((B, H, L, D)).astype(np.float32)
    st = None
    if with_state:
        st = tuple(x.astype(np.float32) for x in _sel_state(B * H, D, 402))
        shapes = [(B, H, D), (B, H, D, D), (B, H, D, D), (B, H, 1), (B, H, D), (B, H, D)]
        st = tuple(x.reshape(sh) for x, sh in zip(st, shapes))
    ds = tuple((0.1 * rng.standard_normal(x.shape)).astype(np.float32) for x in
               (np.zeros((B, H, D)), np.zeros((B, H, D, D)), np.zeros((B, H, D, D)), np.zeros((B, H, 1)),
                np.zeros((B, H, D)), np.zeros((B, H, D))))
    t = lambda x: torch.from_numpy(np.asarray(x, dtype=np.float64)).requires_grad_(True)
    tq, tk, tv, tl = t(q), t(k), t(v), t(ld)
    tb = t(np.broadcast_to(beta, (B, H)).copy())
    ts = tuple(t(x) for x in st) if st is not None else None
    yr, so = selective_forward(tq, tk, tv, tl, tb, 1.0, ts)
    loss = (yr * torch.from_numpy(dy.astype(np.float64))).sum() + \
        sum((a * torch.from_numpy(b.astype(np.float64))).sum() for a, b in zip(so, ds))
    loss.backward()
    print(f"[generic selective bwd] D={D} L={L} state={with_state}", flush=True)
    g = [torch.empty(B, H, L, D, device=dev()) for _ in range(3)]
    dld = torch.empty(B, H, L, device=dev())
    dks = torch.empty(B, H, device=dev())
    dsi = _lib.new_state(B, H, D, dev()) if with_state else None
    _lib.selective_prefill_backward(to_dev(q), to_dev(k), to_dev(v), to_dev(ld), to_dev(beta), 1.0,
                                    tuple(to_dev(x) for x in st) if st is not None else None, to_dev(dy),
                                    tuple(to_dev(x) for x in ds), *g, dsi, dld, dks)
    torch.cuda.synchronize()
    got = {"dq": g[0], "dk": g[1], "dv": g[2], "dlog_decay": dld, "dk_scale": dks}
    ref = {"dq": tq.grad, "dk": tk.grad, "dv": tv.grad, "dlog_decay": tl.grad, "dk_scale": tb.grad}
    for n in got:
        if n == "dlog_decay" and L == 1 and not with_state:
            # one token from a zero state: its decay multiplies nothing, the
            # adjoint is exactly zero and the kernel's is the cancellation of
            # its two terms (the readout's and the final state's) -- held to
            # the scale of dv instead of its own
            err = float(got[n].abs().max().cpu()) / float(ref["dv"].abs().max())
            assert err < TOL_F32, (n, err)
            continue
        assert _rel(got[n], ref[n]) < TOL_F32, (n, _rel(got[n], ref[n]))
    if with_state:
        for i, (a, r) in enumerate(zip(dsi, ts)):
            assert _rel(a.reshape(r.grad.shape), r.grad) < TOL_F32, (i, _rel(a.reshape(r.grad.shape), r.grad))


def test_generic_selective_module_head_dim_32():
    """PrimeSelectiveMomentAttention at head_dim 32: the parallel branch and a
    carried step against an fp32 CPU composition of the module's own weights
    (selective.py:339-444), and its training gradients through the generic
    selective backward."""
    from prime_moment_attention import PrimeSelectiveMomentAttention
    from selective_ref import selective_forward
    torch.manual_seed(5)
    m = PrimeSelectiveMomentAttention(hidden_size=128, num_heads=4, head_dim=32, num_kv_heads=2).to(dev())
    with torch.no_grad():
        m.delta_proj.weight.normal_(0.0, 0.05)
        m.log_beta.uniform_(-0.3, 0.5)
    B, L = 2, 40
    x = torch.randn(B, L, 128, device=dev(), requires_grad=True)
    out, _ = m(x)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(6))
    (out * g.to(dev())).sum().backward()

    mc = PrimeSelectiveMomentAttention(hidden_size=128, num_heads=4, head_dim=32, num_kv_heads=2).double()
    mc.load_state_dict({k: v.detach().double().cpu() for k, v in m.state_dict().items()})
    xc = x.detach().double().cpu().requires_grad_(True)
    H, Hk, D = 4, 2, 32
    q = mc.q_proj(xc).view(B, L, H, D).transpose(1, 2)
    k = mc.k_proj(xc).view(B, L, Hk, D).transpose(1, 2)
    v = mc.v_proj(xc).view(B, L, Hk, D).transpose(1, 2)
    q, k = mc.q_norm(q) * mc.scaling, mc.k_norm(k)
    k, v = k.repeat_interleave(2, 1), v.repeat_interleave(2, 1)
    delta = torch.nn.functional.softplus(mc.delta_proj(xc)).clamp(min=1e-4, max=50.0)  # [B, L, H]
    ld = (-delta / mc.get_tau(xc.device)).transpose(1, 2)
    beta = mc.get_beta(xc.device).view(1, H).expand(B, H)
    y, _ = selective_forward(q, k, v, ld, beta, mc.eps)
    oc = mc.o_proj(y.transpose(1, 2).reshape(B, L, H * D))
    (oc * g.double()).sum().backward()
    assert _rel(out, oc) < TOL_F32
    assert _rel(x.grad, xc.grad) < TOL_F32
    for (name, p), (_, pc) in zip(m.named_parameters(), mc.named_parameters()):
        assert p.grad is not None, name
        assert _rel(p.grad, pc.grad) < TOL_F32, (name, _rel(p.grad, pc.grad))
    # the step branch from the parallel branch's state (no autograd)
    with torch.no_grad():
        _, st = m(x.detach(), return_state=True)
        o1, _ = m(torch.randn(B, 1, 128, device=dev()), state=st)
    assert torch.isfinite(o1).all()
