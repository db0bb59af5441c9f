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
    with pytest.raises(RuntimeError, match="selective"):
        _lib.selective_prefill(x, x, x, torch.zeros(B * H * L, device=dev()), torch.ones(H, device=dev()), 1.0,
                               None, x.clone(), _lib.new_state(B, H, D, dev()))
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
