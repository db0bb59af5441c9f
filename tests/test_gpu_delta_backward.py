"""GPU parity of the delta-rule prefill backward (prime_delta_prefill_backward)
against fp64 torch autograd of the restatement in tests/delta_ref.py (the
autograd graph of chunked_delta_prime.py:73-87, 177-283; the restatement is
pinned to the C oracle and its autograd to central differences in
tests/test_oracle.py), on the CPU with the same (bf16-rounded where bf16)
inputs.  Gradients in q, k, v, beta, alpha and the incoming state, with
dy and a gradient on the final state, ragged L, the per-chunk clamp engaged or
not, grouped k/v heads; the module's autograd through it.  The one-token step
(prime_delta_decode_step_backward) likewise, against the step restatement."""
import pytest
import torch

import delta_ref as R
from prime_moment_attention import _lib

from gpu_util import dev

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max|d| / max|ref| per gradient: the backward is fp32 arithmetic throughout


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def _case(B, H, Hkv, L, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    D = 64
    q = torch.nn.functional.normalize(torch.randn(B, H, L, D, generator=g), dim=-1) / 8
    k = torch.nn.functional.normalize(torch.randn(B, Hkv, L, D, generator=g), dim=-1)
    v = torch.randn(B, Hkv, L, D, generator=g)
    q, k, v = (t.to(dtype).float() for t in (q, k, v))  # the values both sides see
    beta = torch.sigmoid(torch.randn(B, H, L, generator=g)) * 0.5
    alpha = 0.9995 * (1 - 0.5 * torch.sigmoid(torch.randn(B, H, L, generator=g) - 2.5))
    s0 = torch.randn(B, H, D, 2 * D, generator=g) * 0.2
    dy = torch.randn(B, H, L, D, generator=g)
    ds = torch.randn(B, H, D, 2 * D, generator=g) * 0.1
    return q, k, v, beta, alpha, s0, dy, ds


def _reference(q, k, v, beta, alpha, s0, dy, ds, bound):
    """fp64 autograd of the restatement; grouped k/v heads expanded by repeat."""
    H, Hkv = q.shape[1], k.shape[1]
    xs = [t.double().clone().requires_grad_(True) for t in (q, k, v, beta, alpha, s0)]
    kk = xs[1].repeat_interleave(H // Hkv, 1)
    vv = xs[2].repeat_interleave(H // Hkv, 1)
    y, S = R.delta_chunked(xs[0], kk, vv, xs[3], xs[4], 0.9995, 1e-5, bound, 64, xs[5])
    loss = (y * dy.double()).sum() + (S * ds.double()).sum()
    return torch.autograd.grad(loss, xs)


@pytest.mark.parametrize("B,H,Hkv,L,bound,dtype", [
    (2, 2, 2, 64 * 3 + 17, 25.0, torch.float32),
    (1, 2, 2, 64 * 2 + 5, 2.0, torch.float32),    # the clamp engaged in some chunks
    (1, 4, 2, 100, 25.0, torch.bfloat16),         # grouped k/v heads, bf16 inputs
    (1, 2, 2, 2048, 3.0, torch.bfloat16),         # 32 chunks, clamp engaged
    (1, 1, 1, 1, 25.0, torch.float32),            # one token
])
def test_delta_backward_matches_fp64_autograd(B, H, Hkv, L, bound, dtype):
    q, k, v, beta, alpha, s0, dy, ds = _case(B, H, Hkv, L, L + H, dtype)
    print(f"[delta bwd] B={B} H={H} Hkv={Hkv} L={L} bound={bound} {dtype}", flush=True)
    to = lambda t, dt=torch.float32: t.to(dev(), dt).contiguous()
    got = _lib.delta_prefill_backward(to(q, dtype), to(k, dtype), to(v, dtype), to(beta), to(alpha), 0.9995, 1e-5,
                                      bound, to(s0), to(dy, dtype), to(ds))
    torch.cuda.synchronize()
    ref = _reference(q, k, v, beta, alpha, s0, dy.to(dtype).float(), ds, bound)
    for name, g, r in zip(("q", "k", "v", "beta", "alpha", "state"), got, ref):
        assert torch.isfinite(g).all(), name
        assert _rel(g, r) < TOL, (name, _rel(g, r))


def test_delta_backward_without_state_gradient_inputs():
    """No incoming state and no gradient on the final state: the adjoint starts
    at zero, dstate_in is not produced."""
    q, k, v, beta, alpha, _, dy, _ = _case(1, 2, 2, 64 + 30, 7, torch.float32)
    to = lambda t: t.to(dev()).contiguous()
    got = _lib.delta_prefill_backward(to(q), to(k), to(v), to(beta), to(alpha), 0.9995, 1e-5, 25.0, None, to(dy),
                                      None)
    torch.cuda.synchronize()
    assert got[5] is None
    xs = [t.double().clone().requires_grad_(True) for t in (q, k, v, beta, alpha)]
    y, _ = R.delta_chunked(*xs, 0.9995, 1e-5, 25.0, 64, None)
    ref = torch.autograd.grad((y * dy.double()).sum(), xs)
    for name, g, r in zip(("q", "k", "v", "beta", "alpha"), got, ref):
        assert _rel(g, r) < TOL, (name, _rel(g, r))


def test_delta_module_trains_through_the_chunked_branch():
    """ChunkedGatedDeltaPrimeAttention under autograd (the reference trains
    through this branch, chunked_delta_prime.py:177-283): gradients of every
    parameter and of the input against an fp64 CPU composition of the same
    module (torch projections, LayerNorm, gates and the restatement)."""
    from prime_moment_attention import ChunkedGatedDeltaPrimeAttention
    torch.manual_seed(3)
    hidden, H, D, L = 128, 2, 64, 150
    m = ChunkedGatedDeltaPrimeAttention(hidden, H, D, lyapunov_bound=4.0).to(dev())
    x = torch.randn(2, L, hidden, device=dev(), requires_grad=True)
    state = (torch.randn(2, H, D, 2 * D, device=dev()) * 0.1).requires_grad_(True)
    out, s = m(x, state=state, return_state=True)
    g = torch.Generator().manual_seed(4)
    ro = torch.randn(out.shape, generator=g)
    rs = torch.randn(s.shape, generator=g)
    ((out * ro.to(dev())).sum() + (s * rs.to(dev())).sum()).backward()

    mc = ChunkedGatedDeltaPrimeAttention(hidden, H, D, lyapunov_bound=4.0).double()
    mc.load_state_dict({k: v.detach().double().cpu() for k, v in m.state_dict().items()})
    xc = x.detach().double().cpu().requires_grad_(True)
    sc = state.detach().double().cpu().requires_grad_(True)
    B = 2
    q = mc.q_proj(xc).view(B, L, H, D).transpose(1, 2)
    k = mc.k_proj(xc).view(B, L, H, D).transpose(1, 2)
    v = mc.v_proj(xc).view(B, L, H, D).transpose(1, 2)
    q, k = mc.q_norm(q) * mc.scaling, mc.k_norm(k)
    bg = torch.sigmoid(mc.erase_proj(xc)).view(B, L, H, D).mean(-1).transpose(1, 2)
    wg = torch.sigmoid(mc.write_proj(xc)).view(B, L, H, D).mean(-1).transpose(1, 2)
    y, S = R.delta_chunked(q, k, v, wg * 0.5, mc.decay * (1 - bg * 0.5), mc.decay, mc.eps, 4.0, 64, sc)
    oc = mc.o_proj(y.transpose(1, 2).reshape(B, L, H * D))
    ((oc * ro.double()).sum() + (S * rs.double()).sum()).backward()
    assert _rel(out, oc) < TOL
    assert _rel(x.grad, xc.grad) < TOL and _rel(state.grad, sc.grad) < TOL
    for (name, p), (_, pc) in zip(m.named_parameters(), mc.named_parameters()):
        assert p.grad is not None, name
        assert _rel(p.grad, pc.grad) < TOL, (name, _rel(p.grad, pc.grad))


def _step_case(B, H, Hkv, D, seed, dtype, bound):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, H, D, generator=g), dim=-1) / D ** 0.5
    k = torch.randn(B, Hkv, D, generator=g)
    v = torch.randn(B, Hkv, D, generator=g)
    q, k, v = (t.to(dtype).float() for t in (q, k, v))
    beta = torch.sigmoid(torch.randn(B, H, generator=g)) * 0.5
    alpha = 0.9995 * (1 - 0.5 * torch.sigmoid(torch.randn(B, H, generator=g) - 2.5))
    s0 = torch.randn(B, H, D, 2 * D, generator=g) * (0.3 if bound < 25.0 else 0.05)
    dy = torch.randn(B, H, D, generator=g)
    ds = torch.randn(B, H, D, 2 * D, generator=g) * 0.1
    return q, k, v, beta, alpha, s0, dy, ds


@pytest.mark.parametrize("B,H,Hkv,D,bound,dtype,with_state", [
    (3, 2, 2, 64, 25.0, torch.float32, True),
    (2, 2, 2, 64, 1.5, torch.float32, True),     # the clamp engaged
    (2, 4, 2, 64, 25.0, torch.bfloat16, True),   # grouped k/v heads, bf16 inputs
    (2, 2, 2, 32, 0.8, torch.float32, True),     # the reference test's head dim, clamp engaged
    (1, 3, 3, 7, 25.0, torch.float32, False),    # odd head dim, no incoming state
])
def test_delta_step_backward_matches_fp64_autograd(B, H, Hkv, D, bound, dtype, with_state):
    """prime_delta_decode_step_backward against fp64 autograd of the step
    restatement (tests/delta_ref.py::delta_step, pinned to oracle_delta_step
    and to central differences in tests/test_oracle.py): gradients in q, k, v,
    beta, alpha and the incoming state, with dy and a gradient on the new
    state."""
    q, k, v, beta, alpha, s0, dy, ds = _step_case(B, H, Hkv, D, 31 + D + H, dtype, bound)
    if not with_state:
        s0 = None
    print(f"[delta step bwd] B={B} H={H} Hkv={Hkv} D={D} bound={bound} {dtype} state={with_state}", flush=True)
    to = lambda t, dt=torch.float32: t.to(dev(), dt).contiguous() if t is not None else None
    got = _lib.delta_decode_step_backward(to(q, dtype), to(k, dtype), to(v, dtype), to(beta), to(alpha), 1e-5,
                                          bound, to(s0), to(dy, dtype), to(ds))
    torch.cuda.synchronize()
    xs = [t.double().clone().requires_grad_(True) for t in (q, k, v, beta, alpha)]
    sx = s0.double().clone().requires_grad_(True) if s0 is not None else None
    kk = xs[1].repeat_interleave(H // Hkv, 1)
    vv = xs[2].repeat_interleave(H // Hkv, 1)
    y, S = R.delta_step(xs[0], kk, vv, xs[3], xs[4], 1e-5, bound, sx)
    loss = (y * dy.to(dtype).double()).sum() + (S * ds.double()).sum()
    ref = torch.autograd.grad(loss, xs + ([sx] if sx is not None else []))
    names = ("q", "k", "v", "beta", "alpha", "state")
    for name, g, r in zip(names, got, ref):
        assert torch.isfinite(g).all(), name
        assert _rel(g, r) < TOL, (name, _rel(g, r))
    if s0 is None:
        assert got[5] is None


def test_delta_module_trains_through_the_step_branch():
    """ChunkedGatedDeltaPrimeAttention with one token under autograd (the
    reference's L == 1 branch is plain torch and differentiable,
    chunked_delta_prime.py:140-176): gradients of every parameter, of the
    input and of the incoming state against an fp64 CPU composition of the
    same module with the step restatement."""
    from prime_moment_attention import ChunkedGatedDeltaPrimeAttention
    torch.manual_seed(5)
    hidden, H, D, B = 128, 2, 64, 3
    m = ChunkedGatedDeltaPrimeAttention(hidden, H, D, lyapunov_bound=2.0).to(dev())
    x = torch.randn(B, 1, hidden, device=dev(), requires_grad=True)
    state = (torch.randn(B, H, D, 2 * D, device=dev()) * 0.1).requires_grad_(True)
    out, s = m(x, state=state, return_state=True)
    g = torch.Generator().manual_seed(6)
    ro = torch.randn(out.shape, generator=g)
    rs = torch.randn(s.shape, generator=g)
    ((out * ro.to(dev())).sum() + (s * rs.to(dev())).sum()).backward()

    mc = ChunkedGatedDeltaPrimeAttention(hidden, H, D, lyapunov_bound=2.0).double()
    mc.load_state_dict({k: v.detach().double().cpu() for k, v in m.state_dict().items()})
    xc = x.detach().double().cpu().requires_grad_(True)
    sc = state.detach().double().cpu().requires_grad_(True)
    q = mc.q_proj(xc).view(B, 1, H, D).transpose(1, 2)
    k = mc.k_proj(xc).view(B, 1, H, D).transpose(1, 2)
    v = mc.v_proj(xc).view(B, 1, H, D).transpose(1, 2)
    q, k = mc.q_norm(q) * mc.scaling, mc.k_norm(k)
    bg = torch.sigmoid(mc.erase_proj(xc)).view(B, 1, H, D).mean(-1).transpose(1, 2)
    wg = torch.sigmoid(mc.write_proj(xc)).view(B, 1, H, D).mean(-1).transpose(1, 2)
    y, S = R.delta_step(q[:, :, 0], k[:, :, 0], v[:, :, 0], (wg * 0.5)[..., 0], (mc.decay * (1 - bg * 0.5))[..., 0],
                        mc.eps, 2.0, sc)
    oc = mc.o_proj(y.reshape(B, 1, H * D))
    ((oc * ro.double()).sum() + (S * rs.double()).sum()).backward()
    assert _rel(out, oc) < TOL
    assert _rel(x.grad, xc.grad) < TOL and _rel(state.grad, sc.grad) < TOL
    for (name, p), (_, pc) in zip(m.named_parameters(), mc.named_parameters()):
        assert p.grad is not None, name
        assert _rel(p.grad, pc.grad) < TOL, (name, _rel(p.grad, pc.grad))
