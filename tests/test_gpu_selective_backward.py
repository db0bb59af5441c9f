"""GPU parity of the selective-PRIME backward (prime_selective_prefill_backward)
against torch autograd, in float64 on the CPU, of the reference's selective
formula (tests/selective_ref.py: selective.py:414-440 with the step branch's
incoming state, :384-409; pinned against oracle_selective_recurrent by the
CPU tests).  This is the derivative the reference gets when it trains its
selective module: in q, k, v, the per-token log decays (through which
delta_proj and log_tau train), beta (log_beta) and the incoming state.

fp32 inputs, the fp32 tolerance 1e-3 (max|d| / max|ref| per tensor)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import PrimeSelectiveMomentAttention, _lib
from selective_ref import selective_forward

from gpu_util import TOL_F32, assert_close, dev, state_to_dev, to_dev, to_np

pytestmark = pytest.mark.gpu

D = 64


def _state_shapes(B, H):
    return [(B, H, D), (B, H, D, D), (B, H, D, D), (B, H, 1), (B, H, D), (B, H, D)]


def _case(B, H, L, seed, with_state, with_dstate, eps=1.0):
    q, k, v = O.make_inputs((B, H, L, D), seed=seed, bf16=False)
    rng = np.random.default_rng(seed + 1)
    delta = np.log1p(np.exp(rng.standard_normal((B, H, L)) - 1.0))
    tau = rng.uniform(8.0, 400.0, H)
    ld = (-delta / tau[None, :, None]).astype(np.float32)
    beta = rng.uniform(0.6, 2.5, H).astype(np.float32)
    dy = rng.standard_normal((B, H, L, D)).astype(np.float32)
    st = None
    if with_state:
        st = (rng.standard_normal((B, H, D)), 0.05 * rng.standard_normal((B, H, D, D)),
              0.05 * rng.standard_normal((B, H, D, D)), 1.0 + 5.0 * np.abs(rng.standard_normal((B, H, 1))),
              0.1 * rng.standard_normal((B, H, D)), 0.1 * np.abs(rng.standard_normal((B, H, D))))
        st = tuple(x.astype(np.float32) for x in st)
    ds = tuple((0.1 * rng.standard_normal(sh)).astype(np.float32) for sh in _state_shapes(B, H)) \
        if with_dstate else None
    return q, k, v, ld, beta, dy, st, ds


def _reference(q, k, v, ld, beta, dy, st, ds, eps):
    """torch float64 autograd of the composition; beta per sequence [B, H]
    so that its gradient is the per-sequence d_k_scale."""
    B, H = q.shape[:2]
    t = lambda x: torch.from_numpy(np.asarray(x, dtype=np.float64)).requires_grad_(True)
    tq, tk, tv, tl = t(q), t(k), t(v), t(ld)
    tb = t(np.broadcast_to(beta, (B, H)).copy())
    ts = tuple(t(x) for x in st) if st is not None else None
    y, so = selective_forward(tq, tk, tv, tl, tb, eps, ts)
    loss = (y * torch.from_numpy(dy.astype(np.float64))).sum()
    if ds is not None:
        loss = loss + sum((a * torch.from_numpy(b.astype(np.float64))).sum() for a, b in zip(so, ds))
    loss.backward()
    grads = {"dq": tq.grad, "dk": tk.grad, "dv": tv.grad, "dlog_decay": tl.grad, "dk_scale": tb.grad}
    if ts is not None:
        grads["dstate_in"] = tuple(x.grad for x in ts)
    return {n: (tuple(x.numpy() for x in g) if isinstance(g, tuple) else g.numpy()) for n, g in grads.items()}


def _run(q, k, v, ld, beta, dy, st, ds, eps):
    B, H, L, _ = q.shape
    g = [torch.empty(B, H, L, D, device=dev()) for _ in range(3)]
    dld = torch.empty(B, H, L, device=dev())
    dks = torch.empty(B, H, device=dev())
    dsi = _lib.new_state(B, H, D, dev()) if st is not None else None
    _lib.selective_prefill_backward(to_dev(q), to_dev(k), to_dev(v), to_dev(ld), to_dev(beta), eps,
                                    state_to_dev(st, B, H, D) if st is not None else None, to_dev(dy),
                                    state_to_dev(ds, B, H, D) if ds is not None else None, *g, dsi, dld, dks)
    torch.cuda.synchronize()
    out = {"dq": g[0], "dk": g[1], "dv": g[2], "dlog_decay": dld, "dk_scale": dks}
    out = {n: to_np(x) for n, x in out.items()}
    if dsi is not None:
        out["dstate_in"] = tuple(to_np(x) for x in dsi)
    return out


def _compare(got, ref, tol=TOL_F32, floor_from_dv=False):
    """max|d| / max|ref| per tensor.  One token from a zero state has dq,
    dk, d log_decay and d beta tiny or exactly zero (y = v while the
    denominator stays above eps); only then is their error measured against
    the scale of dv."""
    floor = 0.1 * np.abs(ref["dv"]).max() if floor_from_dv else 0.0
    for name in ("dq", "dk", "dv", "dlog_decay", "dk_scale"):
        x, r = got[name], ref[name]
        assert np.isfinite(x).all(), name
        e = np.abs(x - r).max() / max(np.abs(r).max(), floor, 1e-300)
        assert e < tol, f"{name}: rel err {e:.3e} >= {tol}"
    if "dstate_in" in ref:
        for i, (x, r) in enumerate(zip(got["dstate_in"], ref["dstate_in"])):
            e = np.abs(x.reshape(-1) - r.reshape(-1)).max() / max(np.abs(r).max(), 1e-300)
            assert e < tol, f"dstate_in[{i}]: rel err {e:.3e} >= {tol}"


@pytest.mark.parametrize("B,H,L", [(1, 1, 1), (1, 2, 13), (2, 3, 64), (2, 2, 200), (1, 2, 1000)])
@pytest.mark.parametrize("with_state", [False, True])
def test_selective_backward_matches_autograd(B, H, L, with_state):
    """Ragged last chunks (13, 200, 1000) and several chunks carried; with a
    state, the final state's adjoint enters too."""
    args = _case(B, H, L, 900 + L, with_state, with_state)
    ref = _reference(*args, 1.0)
    got = _run(*args, 1.0)
    _compare(got, ref, floor_from_dv=(L == 1 and not with_state))


@pytest.mark.parametrize("L", [70, 300])
def test_selective_backward_final_state_adjoint_only(L):
    """dy = 0 and only the final state's adjoint: the gradient flows through
    the end-of-call state (selective.py:432-440), including the log decay
    of the last token."""
    q, k, v, ld, beta, dy, st, ds = _case(1, 2, L, 930 + L, False, True)
    dy = np.zeros_like(dy)
    _compare(_run(q, k, v, ld, beta, dy, st, ds, 1.0), _reference(q, k, v, ld, beta, dy, st, ds, 1.0))


@pytest.mark.parametrize("eps", [6.0, 20.0])
def test_selective_backward_clamp_active(eps):
    """eps above many tokens' denominators: the clamp's zero derivative in
    the denominator for those tokens."""
    args = _case(2, 2, 150, 940, True, True, eps=eps)
    ref = _reference(*args, eps)
    _compare(_run(*args, eps), ref)


def test_selective_backward_bf16_gradients():
    """bf16 dy and gradient outputs over fp32 q/k/v: each gradient rounded
    once (the bf16 tolerance)."""
    B, H, L = 1, 2, 130
    q, k, v, ld, beta, dy, st, ds = _case(B, H, L, 950, True, True)
    dy = O.bf16_round(dy)
    ref = _reference(q, k, v, ld, beta, dy, st, ds, 1.0)
    g = [torch.empty(B, H, L, D, device=dev(), dtype=torch.bfloat16) for _ in range(3)]
    dld = torch.empty(B, H, L, device=dev())
    dks = torch.empty(B, H, device=dev())
    _lib.selective_prefill_backward(to_dev(q), to_dev(k), to_dev(v), to_dev(ld), to_dev(beta), 1.0,
                                    state_to_dev(st, B, H, D), to_dev(dy, torch.bfloat16),
                                    state_to_dev(ds, B, H, D), *g, None, dld, dks)
    torch.cuda.synchronize()
    for name, x in (("dq", g[0]), ("dk", g[1]), ("dv", g[2]), ("dlog_decay", dld), ("dk_scale", dks)):
        assert_close(to_np(x), ref[name], 2e-2, name)


def test_selective_backward_rejects_bad_arguments():
    B, H, L = 1, 2, 70
    x = torch.zeros(B, H, L, D, device=dev())
    g = [torch.empty(B, H, L, D, device=dev()) for _ in range(3)]
    ld = torch.zeros(B, H, L, device=dev())
    beta = torch.ones(H, device=dev())
    dld, dks = torch.empty(B, H, L, device=dev()), torch.empty(B, H, device=dev())
    with pytest.raises(RuntimeError, match="F32"):
        xb = x.bfloat16()
        _lib.selective_prefill_backward(xb, xb, xb, ld, beta, 1.0, None, x, None, *g, None, dld, dks)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.selective_prefill_backward(x, x, x, ld, beta, 1.0, None, x, None, *g, None, dld, dks,
                                        workspace=torch.empty(64, dtype=torch.uint8, device=dev()))
    with pytest.raises(ValueError, match="d_log_decay"):
        _lib.selective_prefill_backward(x, x, x, ld, beta, 1.0, None, x, None, *g, None, dld[:, :, :-1], dks)


# ---------------------------------------------------------------- the module under autograd
def _module_reference(mod, x, state=None):
    """float64 CPU composition of the reference's selective forward
    (selective.py:339-444) from the module's parameters: the parallel branch
    for L > 1 (zero state), the step branch for L == 1 (from `state`).
    Returns (out, next_state, x, params)."""
    m = {n: p.detach().double().cpu().requires_grad_(True) for n, p in mod.named_parameters()}
    xd = x.detach().double().cpu().requires_grad_(True)
    B, L, _ = x.shape
    H, Hk = mod.num_heads, mod.num_kv_heads
    q = (xd @ m["q_proj.weight"].t()).view(B, L, H, D).transpose(1, 2)
    k = (xd @ m["k_proj.weight"].t()).view(B, L, Hk, D).transpose(1, 2)
    v = (xd @ m["v_proj.weight"].t()).view(B, L, Hk, D).transpose(1, 2)
    if H != Hk:
        k, v = k.repeat_interleave(H // Hk, 1), v.repeat_interleave(H // Hk, 1)
    q = torch.nn.functional.layer_norm(q, (D,), m["q_norm.weight"], m["q_norm.bias"], 1e-5)
    k = torch.nn.functional.layer_norm(k, (D,), m["k_norm.weight"], m["k_norm.bias"], 1e-5)
    q = q * mod.scaling
    tau = torch.clamp(torch.exp(m["log_tau"]), min=mod.min_tau, max=mod.max_tau)
    beta = torch.clamp(torch.exp(m["log_beta"]), min=0.1, max=15.0)
    delta = torch.nn.functional.softplus(xd @ m["delta_proj.weight"].t() + m["delta_proj.bias"]).clamp(1e-4, 50.0)
    log_decay = (-delta / tau.view(1, 1, H)).transpose(1, 2)
    st = None
    if L == 1 and state is not None:
        st = tuple(s.detach().double().cpu() for s in state)
    y, ns = selective_forward(q, k, v, log_decay, beta.view(1, H), mod.eps, st)
    out = y.transpose(1, 2).reshape(B, L, H * D) @ m["o_proj.weight"].t()
    return out, ns, xd, m


def _module(Hkv, seed):
    torch.manual_seed(seed)
    mod = PrimeSelectiveMomentAttention(hidden_size=128, num_heads=2, head_dim=D, num_kv_heads=Hkv,
                                        decay=0.995).to(dev())
    with torch.no_grad():
        for ln in (mod.q_norm, mod.k_norm):
            ln.weight.uniform_(0.5, 1.5)
            ln.bias.uniform_(-0.2, 0.2)
        mod.delta_proj.weight.normal_(0.0, 0.05)
        mod.log_tau.uniform_(2.5, 5.5)
        mod.log_beta.uniform_(-0.5, 0.8)
    return mod


@pytest.mark.parametrize("L,Hkv", [(130, 2), (300, 1)])
def test_selective_module_gradients_match_float64_composition(L, Hkv):
    """PrimeSelectiveMomentAttention trained through: x and every parameter's
    gradient (projections, QK LayerNorms, delta_proj, log_tau, log_beta)
    against the float64 composition of the reference formula."""
    mod = _module(Hkv, 960 + L)
    x = torch.randn(2, L, 128, device=dev()).requires_grad_(True)
    out, _ = mod(x)
    g = torch.randn_like(out)
    (out * g).sum().backward()
    ref_out, _, xd, m = _module_reference(mod, x)
    (ref_out * g.double().cpu()).sum().backward()
    torch.cuda.synchronize()
    assert_close(to_np(out), ref_out.detach().numpy(), TOL_F32, "out")
    assert_close(to_np(x.grad), xd.grad.numpy(), TOL_F32, "x.grad")
    for n, p in mod.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n
        assert_close(to_np(p.grad), m[n].grad.numpy(), TOL_F32, n + ".grad")


def test_selective_module_prefill_then_step_gradients():
    """A prefill returning its state, then an L == 1 step from that state,
    under autograd: the gradients of x of both calls and of the parameters
    equal those of the reference composition of the same two calls."""
    mod = _module(2, 970)
    x = torch.randn(1, 41, 128, device=dev())
    x1, x2 = x[:, :40].clone().requires_grad_(True), x[:, 40:].clone().requires_grad_(True)
    o1, s = mod(x1, return_state=True)
    o2, _ = mod(x2, state=s)
    g = torch.randn(1, 41, 128, device=dev())
    (torch.cat([o1, o2], 1) * g).sum().backward()
    r1, rs, xd1, m = _module_reference(mod, x1)
    # the step reuses the same float64 parameters and takes the composed state
    mod2 = {n: p for n, p in m.items()}
    xd2 = x2.detach().double().cpu().requires_grad_(True)
    B, H = 1, mod.num_heads
    q = torch.nn.functional.layer_norm((xd2 @ mod2["q_proj.weight"].t()).view(B, 1, H, D).transpose(1, 2), (D,),
                                       mod2["q_norm.weight"], mod2["q_norm.bias"], 1e-5) * mod.scaling
    k = torch.nn.functional.layer_norm((xd2 @ mod2["k_proj.weight"].t()).view(B, 1, H, D).transpose(1, 2), (D,),
                                       mod2["k_norm.weight"], mod2["k_norm.bias"], 1e-5)
    v = (xd2 @ mod2["v_proj.weight"].t()).view(B, 1, H, D).transpose(1, 2)
    tau = torch.clamp(torch.exp(mod2["log_tau"]), min=mod.min_tau, max=mod.max_tau)
    beta = torch.clamp(torch.exp(mod2["log_beta"]), min=0.1, max=15.0)
    delta = torch.nn.functional.softplus(xd2 @ mod2["delta_proj.weight"].t() + mod2["delta_proj.bias"]).clamp(
        1e-4, 50.0)
    y2, _ = selective_forward(q, k, v, (-delta / tau.view(1, 1, H)).transpose(1, 2), beta.view(1, H), mod.eps,
                              rs)
    r2 = y2.transpose(1, 2).reshape(B, 1, H * D) @ mod2["o_proj.weight"].t()
    (torch.cat([r1, r2], 1) * g.double().cpu()).sum().backward()
    torch.cuda.synchronize()
    assert_close(to_np(o2), r2.detach().numpy(), TOL_F32, "step out")
    assert_close(to_np(x1.grad), xd1.grad.numpy(), TOL_F32, "x1.grad")
    assert_close(to_np(x2.grad), xd2.grad.numpy(), TOL_F32, "x2.grad")
    for n, p in mod.named_parameters():
        assert_close(to_np(p.grad), m[n].grad.numpy(), TOL_F32, n + ".grad")


def test_selective_model_trains():
    """A selective PrimeForCausalLM: finite gradients reach the selective
    parameters and a few AdamW steps lower the loss on a fixed batch."""
    from prime_moment_attention import PrimeConfig, PrimeForCausalLM
    torch.manual_seed(980)
    cfg = PrimeConfig(vocab_size=100, hidden_size=128, num_layers=2, num_heads=2, head_dim=D, decay=0.995,
                      use_qk_norm=True, use_selective=True)
    model = PrimeForCausalLM(cfg).to(dev())
    ids = torch.randint(0, 100, (4, 96), device=dev())
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3)
    losses = []
    for _ in range(8):
        opt.zero_grad()
        loss = model(ids, labels=ids)["loss"]
        loss.backward()
        losses.append(float(loss.detach()))
        params = dict(model.named_parameters())
        for n in ("layers.0.self_attn.log_tau", "layers.0.self_attn.log_beta",
                  "layers.0.self_attn.delta_proj.weight", "layers.1.self_attn.q_proj.weight"):
            assert params[n].grad is not None and torch.isfinite(params[n].grad).all(), n
        opt.step()
    assert losses[-1] < losses[0] - 0.1, losses
