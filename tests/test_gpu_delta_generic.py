"""GPU parity of the delta rule at the shapes the token-sequential kernels
take (delta_gen.hip: head dims up to 64 with any chunk size other than the
MFMA kernels' D = 64 / chunk 64): the prefill and the step against the oracle
(oracle_delta_features / _chunked / _step, chunked_delta_prime.py:73-283,
which take any D and chunk), the backward against fp64 torch autograd of the
restatement in tests/delta_ref.py (pinned to the oracle and to central
differences in tests/test_oracle.py), and the reference's own module test at
head_dim 32 with chunk_size 32 (tests/test_chunked_delta_prime.py:9-27) with
parity checks added."""
import numpy as np
import pytest
import torch

import delta_ref as R
from oracle import oracle as O
from prime_moment_attention import _lib

from gpu_util import TOL_BF16, TOL_F32, assert_close, dev, to_dev, to_np

pytestmark = pytest.mark.gpu

FEAT_EPS = 1e-5


def _inputs(B, H, Hkv, L, D, seed, dtype):
    """q (scaled by 1/sqrt(D)), k, v as the device holds them; beta, alpha."""
    bf = dtype == torch.bfloat16
    q, _, _ = O.make_inputs((B, H, L, D), seed=seed, bf16=bf)
    _, k, v = O.make_inputs((B, Hkv, L, D), seed=seed + 1, bf16=bf)
    if bf:
        q = O.bf16_round(q)
    rng = np.random.default_rng(seed)
    beta = (0.5 / (1 + np.exp(-rng.standard_normal((B, H, L))))).astype(np.float32)
    alpha = rng.uniform(0.9, 0.999, (B, H, L)).astype(np.float32)
    return q, k, v, beta, alpha


def _oracle(q, k, v, beta, alpha, decay_pad, bound, chunk, state=None):
    B, H, L, D = q.shape
    grp = H // k.shape[1]
    ke, ve = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    BH = B * H
    psi, phi = O.delta_features(q.reshape(BH, L, D), ke.reshape(BH, L, D), eps=FEAT_EPS)
    return O.delta_chunked(psi, phi, ve.reshape(BH, L, D), beta.reshape(BH, L), alpha.reshape(BH, L),
                           decay_pad, bound=bound, chunk=chunk, state=state)


@pytest.mark.parametrize("D,chunk", [(32, 32), (16, 64), (64, 32), (32, 7), (48, 100)])
@pytest.mark.parametrize("L", [1, 13, 150])
@pytest.mark.parametrize("bound", [25.0, 2.0])
def test_delta_generic_prefill_matches_oracle(D, chunk, L, bound):
    B, H, Hkv = 2, 4, 2
    dt = torch.float32 if D == 64 else torch.bfloat16
    q, k, v, beta, alpha = _inputs(B, H, Hkv, L, D, D + L + chunk, dt)
    st = np.random.default_rng(L).standard_normal((B * H, D, 2 * D)) * 0.05
    print(f"[delta generic] D={D} chunk={chunk} L={L} bound={bound} {dt}", flush=True)
    yo, so = _oracle(q, k, v, beta, alpha, 0.995, bound, chunk, st)
    y = torch.empty(B, H, L, D, device=dev())
    s_in = to_dev(st.reshape(B, H, D, 2 * D))
    s_out = torch.empty(B, H, D, 2 * D, device=dev())
    _lib.delta_prefill(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), to_dev(beta), to_dev(alpha), 0.995, FEAT_EPS,
                       bound, s_in, y, s_out, chunk=chunk)
    torch.cuda.synchronize()
    tol = TOL_F32
    assert_close(to_np(y).reshape(B * H, L, D), yo, tol, "y")
    assert_close(to_np(s_out).reshape(B * H, D, 2 * D), so, tol, "S")
    if bound == 2.0 and L == 150:
        nrm = np.linalg.norm(to_np(s_out).reshape(B * H, -1), axis=1)
        assert nrm.max() <= 2.0 * (1 + 1e-5)  # the clamp engaged


def test_delta_generic_prefill_in_place_no_state_strided_output():
    B, H, L, D, chunk = 1, 3, 90, 32, 32
    q, k, v, beta, alpha = _inputs(B, H, H, L, D, 5, torch.float32)
    yo, so = _oracle(q, k, v, beta, alpha, 0.99, 25.0, chunk)
    y_bl = torch.empty(B, L, H, D, device=dev(), dtype=torch.bfloat16)
    s = torch.zeros(B, H, D, 2 * D, device=dev())
    _lib.delta_prefill(to_dev(q), to_dev(k), to_dev(v), to_dev(beta), to_dev(alpha), 0.99, FEAT_EPS, 25.0, s,
                       y_bl.transpose(1, 2), s, chunk=chunk)
    torch.cuda.synchronize()
    assert_close(to_np(y_bl.transpose(1, 2)).reshape(B * H, L, D), yo, TOL_BF16, "y")
    assert_close(to_np(s).reshape(B * H, D, 2 * D), so, TOL_F32, "S")


@pytest.mark.parametrize("D", [32, 16])
@pytest.mark.parametrize("bound", [25.0, 0.5])
def test_delta_generic_step_matches_oracle(D, bound):
    """The step branch (predict with the undecayed state, clamp before the
    readout), in place and with GQA."""
    B, H, Hkv = 3, 4, 2
    q, k, v, beta, alpha = _inputs(B, H, Hkv, 1, D, 70 + D, torch.float32)
    st = np.random.default_rng(D).standard_normal((B * H, D, 2 * D)) * 0.1
    grp = H // Hkv
    ke, ve = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    psi, phi = O.delta_features(q.reshape(B * H, 1, D), ke.reshape(B * H, 1, D), eps=FEAT_EPS)
    yo, so = O.delta_step(psi[:, 0], phi[:, 0], ve.reshape(B * H, D), beta.reshape(B * H), alpha.reshape(B * H),
                          bound=bound, state=st)
    s = to_dev(st.reshape(B, H, D, 2 * D))
    y = torch.empty(B, H, D, device=dev())
    _lib.delta_decode_step(to_dev(q[:, :, 0]), to_dev(k[:, :, 0]), to_dev(v[:, :, 0]), to_dev(beta[:, :, 0]),
                           to_dev(alpha[:, :, 0]), FEAT_EPS, bound, s, s, y)
    torch.cuda.synchronize()
    assert_close(to_np(y).reshape(B * H, D), yo, TOL_F32, "y")
    assert_close(to_np(s).reshape(B * H, D, 2 * D), so, TOL_F32, "S")


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("D,chunk,L,bound,Hkv", [
    (32, 32, 100, 25.0, 2),
    (32, 32, 100, 2.0, 2),    # the clamp engaged at chunk ends
    (16, 64, 130, 1.0, 1),
    (64, 32, 70, 3.0, 2),
    (8, 5, 23, 25.0, 1),      # chunks of 5, a ragged last chunk
])
def test_delta_generic_backward_matches_fp64_autograd(D, chunk, L, bound, Hkv):
    B, H = 1, 2
    g = torch.Generator().manual_seed(D + L)
    q = torch.nn.functional.normalize(torch.randn(B, H, L, D, generator=g), dim=-1) / D ** 0.5
    k = torch.nn.functional.normalize(torch.randn(B, Hkv, L, D, generator=g), dim=-1)
    v = torch.randn(B, Hkv, L, D, generator=g)
    beta = torch.sigmoid(torch.randn(B, H, L, generator=g)) * 0.5
    alpha = 0.9995 * (1 - 0.5 * torch.sigmoid(torch.randn(B, H, L, generator=g) - 2.5))
    s0 = torch.randn(B, H, D, 2 * D, generator=g) * 0.2
    dy = torch.randn(B, H, L, D, generator=g)
    ds = torch.randn(B, H, D, 2 * D, generator=g) * 0.1
    print(f"[delta generic bwd] D={D} chunk={chunk} L={L} bound={bound} Hkv={Hkv}", flush=True)
    to = lambda t: t.to(dev()).contiguous()
    got = _lib.delta_prefill_backward(to(q), to(k), to(v), to(beta), to(alpha), 0.9995, FEAT_EPS, bound, to(s0),
                                      to(dy), to(ds), chunk=chunk)
    torch.cuda.synchronize()
    xs = [t.double().clone().requires_grad_(True) for t in (q, k, v, beta, alpha, s0)]
    kk = xs[1].repeat_interleave(H // Hkv, 1)
    vv = xs[2].repeat_interleave(H // Hkv, 1)
    y, S = R.delta_chunked(xs[0], kk, vv, xs[3], xs[4], 0.9995, FEAT_EPS, bound, chunk, xs[5])
    ref = torch.autograd.grad((y * dy.double()).sum() + (S * ds.double()).sum(), xs)
    for name, gg, r in zip(("q", "k", "v", "beta", "alpha", "state"), got, ref):
        assert torch.isfinite(gg).all(), name
        assert _rel(gg, r) < 1e-3, (name, _rel(gg, r))


def test_delta_generic_backward_without_state_inputs():
    B, H, L, D, chunk = 2, 2, 40, 32, 32
    g = torch.Generator().manual_seed(9)
    q = torch.nn.functional.normalize(torch.randn(B, H, L, D, generator=g), dim=-1) / D ** 0.5
    k = torch.nn.functional.normalize(torch.randn(B, H, L, D, generator=g), dim=-1)
    v = torch.randn(B, H, L, D, generator=g)
    beta = torch.sigmoid(torch.randn(B, H, L, generator=g)) * 0.5
    alpha = 0.99 * torch.ones(B, H, L)
    dy = torch.randn(B, H, L, D, generator=g)
    to = lambda t: t.to(dev()).contiguous()
    got = _lib.delta_prefill_backward(to(q), to(k), to(v), to(beta), to(alpha), 0.99, FEAT_EPS, 25.0, None, to(dy),
                                      None, chunk=chunk)
    torch.cuda.synchronize()
    assert got[5] is None
    xs = [t.double().clone().requires_grad_(True) for t in (q, k, v, beta, alpha)]
    y, _ = R.delta_chunked(*xs, 0.99, FEAT_EPS, 25.0, chunk, None)
    ref = torch.autograd.grad((y * dy.double()).sum(), xs)
    for name, gg, r in zip(("q", "k", "v", "beta", "alpha"), got, ref):
        assert _rel(gg, r) < 1e-3, (name, _rel(gg, r))


def _module(D_model, H, D_head, chunk, bound, seed):
    from prime_moment_attention import ChunkedGatedDeltaPrimeAttention
    torch.manual_seed(seed)
    return ChunkedGatedDeltaPrimeAttention(hidden_size=D_model, num_heads=H, head_dim=D_head, chunk_size=chunk,
                                           lyapunov_bound=bound)


def _module_cpu(m, x, state, chunk, bound):
    """fp64 CPU composition of the module (chunked_delta_prime.py:105-283)."""
    mc = _module(m.hidden_size, m.num_heads, m.head_dim, chunk, bound, 0).double()
    mc.load_state_dict({k: v.detach().double().cpu() for k, v in m.state_dict().items()})
    B, L, _ = x.shape
    H, D = m.num_heads, m.head_dim
    xc = x.detach().double().cpu()
    q = mc.q_proj(xc).view(B, L, H, D).transpose(1, 2)
    k = mc.k_proj(xc).view(B, L, H, D).transpose(1, 2)
    v = mc.v_proj(xc).view(B, L, H, D).transpose(1, 2)
    q, k = mc.q_norm(q) * mc.scaling, mc.k_norm(k)
    bg = torch.sigmoid(mc.erase_proj(xc)).view(B, L, H, D).mean(-1).transpose(1, 2)
    wg = torch.sigmoid(mc.write_proj(xc)).view(B, L, H, D).mean(-1).transpose(1, 2)
    y, S = R.delta_chunked(q, k, v, wg * 0.5, mc.decay * (1 - bg * 0.5), mc.decay, mc.eps, bound, chunk,
                           None if state is None else state.double().cpu())
    return mc.o_proj(y.transpose(1, 2).reshape(B, L, H * D)), S


def test_reference_chunked_gated_delta_prime_prefill_and_step():
    """tests/test_chunked_delta_prime.py:9-27: B=2, L=256, hidden 128, 4 heads
    of 32, chunk_size 32, lyapunov_bound 20 -- shapes, and the prefill and the
    carried step against the oracle composition."""
    B, L, Dm, H, Dh = 2, 256, 128, 4, 32
    m = _module(Dm, H, Dh, 32, 20.0, 1).to(dev())
    x = torch.randn(B, L, Dm, device=dev())
    with torch.no_grad():
        out, state = m(x, return_state=True)
    assert out.shape == (B, L, Dm) and state.shape == (B, H, Dh, 2 * Dh)
    ref, rs = _module_cpu(m, x, None, 32, 20.0)
    assert _rel(out, ref) < TOL_F32 and _rel(state, rs) < TOL_F32
    xs = torch.randn(B, 1, Dm, device=dev())
    with torch.no_grad():
        o1, s1 = m(xs, state=state, return_state=True)
    assert o1.shape == (B, 1, Dm) and s1.shape == (B, H, Dh, 2 * Dh)
    # the step branch in fp64 through the oracle (predict with the undecayed state)
    mc = m.double().cpu()
    with torch.no_grad():
        xc = xs.double().cpu()
        q = mc.q_proj(xc).view(B, 1, H, Dh).transpose(1, 2)
        k = mc.k_proj(xc).view(B, 1, H, Dh).transpose(1, 2)
        v = mc.v_proj(xc).view(B, 1, H, Dh).transpose(1, 2)
        q, k = mc.q_norm(q) * mc.scaling, mc.k_norm(k)
        bg = torch.sigmoid(mc.erase_proj(xc)).view(B, 1, H, Dh).mean(-1)
        wg = torch.sigmoid(mc.write_proj(xc)).view(B, 1, H, Dh).mean(-1)
    psi, phi = O.delta_features(q.reshape(B * H, 1, Dh).numpy(), k.reshape(B * H, 1, Dh).numpy(), eps=mc.eps)
    yo, so = O.delta_step(psi[:, 0], phi[:, 0], v.reshape(B * H, Dh).numpy(), (wg * 0.5).reshape(-1).numpy(),
                          (mc.decay * (1 - bg * 0.5)).reshape(-1).numpy(), bound=20.0,
                          state=state.double().cpu().numpy())
    oo = mc.o_proj(torch.from_numpy(yo).view(B, 1, H * Dh))
    assert _rel(s1, torch.from_numpy(so).view(B, H, Dh, 2 * Dh)) < TOL_F32
    assert _rel(o1, oo) < TOL_F32


def test_delta_module_trains_at_head_dim_32_chunk_32():
    """The chunked branch under autograd at head_dim 32, chunk 32, with a state
    and the clamp engaged: every gradient against fp64 CPU autograd of the
    composition."""
    B, L, Dm, H, Dh = 2, 100, 64, 2, 32
    m = _module(Dm, H, Dh, 32, 3.0, 2).to(dev())
    x = torch.randn(B, L, Dm, device=dev(), requires_grad=True)
    state = (torch.randn(B, H, Dh, 2 * Dh, device=dev()) * 0.1).requires_grad_(True)
    out, s = m(x, state=state, return_state=True)
    g = torch.Generator().manual_seed(4)
    ro, rs = torch.randn(out.shape, generator=g), torch.randn(s.shape, generator=g)
    ((out * ro.to(dev())).sum() + (s * rs.to(dev())).sum()).backward()
    mc = _module(Dm, H, Dh, 32, 3.0, 0).double()
    mc.load_state_dict({k: v.detach().double().cpu() for k, v in m.state_dict().items()})
    xc = x.detach().double().cpu().requires_grad_(True)
    sc = state.detach().double().cpu().requires_grad_(True)
    q = mc.q_proj(xc).view(B, L, H, Dh).transpose(1, 2)
    k = mc.k_proj(xc).view(B, L, H, Dh).transpose(1, 2)
    v = mc.v_proj(xc).view(B, L, H, Dh).transpose(1, 2)
    q, k = mc.q_norm(q) * mc.scaling, mc.k_norm(k)
    bg = torch.sigmoid(mc.erase_proj(xc)).view(B, L, H, Dh).mean(-1).transpose(1, 2)
    wg = torch.sigmoid(mc.write_proj(xc)).view(B, L, H, Dh).mean(-1).transpose(1, 2)
    y, S = R.delta_chunked(q, k, v, wg * 0.5, mc.decay * (1 - bg * 0.5), mc.decay, mc.eps, 3.0, 32, sc)
    oc = mc.o_proj(y.transpose(1, 2).reshape(B, L, H * Dh))
    ((oc * ro.double()).sum() + (S * rs.double()).sum()).backward()
    assert _rel(out, oc) < TOL_F32
    assert _rel(x.grad, xc.grad) < TOL_F32 and _rel(state.grad, sc.grad) < TOL_F32
    for (name, p), (_, pc) in zip(m.named_parameters(), mc.named_parameters()):
        assert _rel(p.grad, pc.grad) < TOL_F32, (name, _rel(p.grad, pc.grad))
