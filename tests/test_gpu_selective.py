"""GPU parity of selective PRIME (selective.py:264-444): prime_selective_prefill
and prime_selective_decode_step against the fp64 oracle restatements
(oracle_selective_recurrent, oracle_selective_parallel), the module against an
fp64 composition of its own weights, and the selective PRIME-125M-shaped model
through the greedy decoder."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from prime_moment_attention import (GreedyDecoder, PrimeConfig, PrimeForCausalLM,
                                    PrimeSelectiveMomentAttention, _lib)

from gpu_util import TOL_BF16, TOL_F32, assert_close, dev, state_to_dev, state_to_np, to_dev, to_np

pytestmark = pytest.mark.gpu

D = 64


def _inputs(B, H, L, seed, Hkv=None, bf16=True):
    Hkv = Hkv or H
    q, _, _ = O.make_inputs((B, H, L, D), seed=seed, bf16=bf16)
    _, k, v = O.make_inputs((B, Hkv, L, D), seed=seed + 1, bf16=bf16)
    rng = np.random.default_rng(seed)
    delta = np.log1p(np.exp(rng.standard_normal((B, H, L)) - 1.0))  # softplus step sizes
    tau = rng.uniform(8.0, 400.0, H)
    beta = rng.uniform(0.6, 2.5, H).astype(np.float32)
    log_decay = (-delta / tau[None, :, None]).astype(np.float32)
    return q, k, v, log_decay, beta


def _oracle(q, k, v, log_decay, beta, eps, state=None):
    B, H, L, _ = q.shape
    grp = H // k.shape[1]
    ke, ve = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    BH = B * H
    return O.selective_recurrent(q.reshape(BH, L, D), ke.reshape(BH, L, D), ve.reshape(BH, L, D),
                                 np.exp(log_decay.astype(np.float64)).reshape(BH, L),
                                 np.tile(beta.astype(np.float64), B), eps=eps, state=state)


def _rand_state(BH, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((BH, D)), rng.standard_normal((BH, D, D)) * 0.05,
            rng.standard_normal((BH, D, D)) * 0.05, np.abs(rng.standard_normal(BH)) * 5 + 1,
            rng.standard_normal((BH, D)) * 0.1, np.abs(rng.standard_normal((BH, D))) * 0.1)


def _run_prefill(q, k, v, log_decay, beta, eps, state=None, workspace=None, dt=torch.bfloat16):
    B, H, L, _ = q.shape
    y = torch.empty(B, H, L, D, device=dev())
    st_in = state_to_dev(state, B, H, D) if state is not None else None
    st_out = _lib.new_state(B, H, D, dev())
    _lib.selective_prefill(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt),
                           to_dev(log_decay), to_dev(beta), eps, st_in, y, st_out, workspace=workspace)
    torch.cuda.synchronize()
    return to_np(y).reshape(B * H, L, D), state_to_np(st_out, B * H, D)


@pytest.mark.parametrize("L", [1, 13, 64, 100, 200, 300, 1000])
@pytest.mark.parametrize("with_state", [False, True])
def test_selective_prefill_matches_oracle(L, with_state):
    """Ragged last chunks where only some of a thread's second rows are valid
    (L = 100, 300) exercise the decay weights of partial chunks."""
    B, H = 2, 3
    q, k, v, ld, beta = _inputs(B, H, L, seed=30 + L)
    st = _rand_state(B * H, 31) if with_state else None
    yo, so = _oracle(q, k, v, ld, beta, 1.0, st)
    y, s = _run_prefill(q, k, v, ld, beta, 1.0, st)
    assert_close(y, yo, TOL_BF16, "y")
    for i, (a, b) in enumerate(zip(s, so)):
        assert_close(a, b.reshape(a.shape), TOL_BF16, f"state[{i}]")


@pytest.mark.parametrize("L", [1, 13, 64, 100, 300, 1000])
@pytest.mark.parametrize("with_state", [False, True])
def test_selective_prefill_f32_matches_oracle(L, with_state):
    """fp32 inputs run the fp32 prefill kernel: the fp32 tolerance applies."""
    B, H = 2, 3
    q, k, v, ld, beta = _inputs(B, H, L, seed=130 + L, bf16=False)
    st = _rand_state(B * H, 131) if with_state else None
    yo, so = _oracle(q, k, v, ld, beta, 1.0, st)
    y, s = _run_prefill(q, k, v, ld, beta, 1.0, st, dt=torch.float32)
    assert_close(y, yo, TOL_F32, "y")
    for i, (a, b) in enumerate(zip(s, so)):
        assert_close(a, b.reshape(a.shape), TOL_F32, f"state[{i}]")


def test_selective_prefill_f32_parallel_branch_gqa_and_eps():
    """fp32 against the reference's own parallel form (the [L, L] decay matrix
    from the softplus step sizes, selective.py:414-440), with GQA and an eps
    small enough for the denominator clamp to be reachable."""
    B, H, Hkv, L = 1, 4, 2, 1500
    q, k, v, _, beta = _inputs(B, H, L, seed=140, Hkv=Hkv, bf16=False)
    rng = np.random.default_rng(141)
    delta = np.log1p(np.exp(rng.standard_normal((B * H, L)) - 1.0))
    tau = rng.uniform(8.0, 400.0, H)
    ld = (-delta / np.tile(tau, B)[:, None]).astype(np.float32).reshape(B, H, L)
    ke, ve = np.repeat(k, H // Hkv, axis=1), np.repeat(v, H // Hkv, axis=1)
    yo, so = O.selective_parallel(q.reshape(B * H, L, D), ke.reshape(B * H, L, D), ve.reshape(B * H, L, D),
                                  delta, np.tile(tau, B), np.tile(beta.astype(np.float64), B), eps=1e-3)
    y, s = _run_prefill(q, k, v, ld, beta, 1e-3, dt=torch.float32)
    assert_close(y, yo, TOL_F32, "y")
    for i, (a, b) in enumerate(zip(s, so)):
        assert_close(a, b.reshape(a.shape), TOL_F32, f"state[{i}]")


def test_selective_prefill_segments_gqa_and_eps():
    """A long sequence split into parallel segments (each segment's own decay
    carried by the scan), GQA, and a small eps with the clamp reachable."""
    B, H, L = 1, 4, 4096 + 37
    q, k, v, ld, beta = _inputs(B, H, L, seed=40, Hkv=2)
    assert _lib.workspace_size(B, H, L) > 0  # the segmented path runs
    yo, so = _oracle(q, k, v, ld, beta, 1e-3)
    y, s = _run_prefill(q, k, v, ld, beta, 1e-3)
    assert_close(y, yo, TOL_BF16, "y")
    for i, (a, b) in enumerate(zip(s, so)):
        assert_close(a, b.reshape(a.shape), TOL_BF16, f"state[{i}]")
    y1, s1 = _run_prefill(q, k, v, ld, beta, 1e-3, workspace=torch.empty(0, dtype=torch.uint8, device=dev()))
    assert_close(y1, y, 2e-3, "y one segment vs segments")


@pytest.mark.parametrize("with_state", [False, True])
def test_selective_prefill_f32_segments(with_state):
    """fp32 inputs split into segments (the fp32 kernel's state-only pass, the
    scan with each segment's own decay, one workgroup per segment) against the
    oracle and against one workgroup per sequence."""
    B, H, L = 1, 4, 4096 + 37
    q, k, v, ld, beta = _inputs(B, H, L, seed=42, Hkv=2, bf16=False)
    st = _rand_state(B * H, 43) if with_state else None
    assert _lib.workspace_size(B, H, L) > 0  # the segmented path runs
    yo, so = _oracle(q, k, v, ld, beta, 1.0, st)
    y, s = _run_prefill(q, k, v, ld, beta, 1.0, st, dt=torch.float32)
    assert_close(y, yo, TOL_F32, "y")
    for i, (a, b) in enumerate(zip(s, so)):
        assert_close(a, b.reshape(a.shape), TOL_F32, f"state[{i}]")
    y1, s1 = _run_prefill(q, k, v, ld, beta, 1.0, st, dt=torch.float32,
                          workspace=torch.empty(0, dtype=torch.uint8, device=dev()))
    assert_close(y1, y, 1e-4, "y one segment vs segments")
    for i, (a, b) in enumerate(zip(s1, s)):
        assert_close(a, b, 1e-4, f"state[{i}] one segment vs segments")


def test_selective_reduces_to_base_prefill():
    """beta = 1 and log_decay = log(lambda_h) per head: the base chunked
    prefill's y, and its state with S2, K2 halved."""
    B, H, L = 2, 3, 300
    q, k, v, _, _ = _inputs(B, H, L, seed=45)
    lam = np.array([0.99, 0.995, 0.9999], np.float32)
    ld = np.broadcast_to(np.log(lam)[None, :, None], (B, H, L)).astype(np.float32).copy()
    y, s = _run_prefill(q, k, v, ld, np.ones(H, np.float32), 1.0)
    yb = torch.empty(B, H, L, D, device=dev())
    sb = _lib.new_state(B, H, D, dev())
    _lib.chunked_prefill(to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16),
                         to_dev(lam), 1.0, 64, None, yb, sb)
    torch.cuda.synchronize()
    assert_close(y, to_np(yb).reshape(B * H, L, D), 2e-3, "y")
    for i, (a, b) in enumerate(zip(s, state_to_np(sb, B * H, D))):
        assert_close(a, b * (0.5 if i in (2, 5) else 1.0), 2e-3, f"state[{i}]")


@pytest.mark.parametrize("qk_norm", [False, True])
def test_selective_decode_step_matches_oracle(qk_norm):
    B, H = 3, 4
    q, k, v, ld, beta = _inputs(B, H, 1, seed=50)
    q, k, v, ld = q[:, :, 0], k[:, :, 0], v[:, :, 0], ld[:, :, 0]
    st = _rand_state(B * H, 51)
    qd, kd = to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16)
    norm = None
    if qk_norm:
        ln_q, ln_k = torch.nn.LayerNorm(D).to(dev()).bfloat16(), torch.nn.LayerNorm(D).to(dev()).bfloat16()
        with torch.no_grad():
            for m in (ln_q, ln_k):
                m.weight.uniform_(0.5, 1.5)
                m.bias.uniform_(-0.2, 0.2)
            qn = (ln_q(qd * 8.0) * 0.125)  # raw projections whose normed, scaled rows the oracle sees
            kn = ln_k(kd)
        norm = _lib.qk_norm(ln_q, ln_k, 0.125, torch.bfloat16)
        q_in, k_in = qd * 8.0, kd
        q_ref, k_ref = to_np(qn.float()), to_np(kn.float())
    else:
        q_in, k_in, q_ref, k_ref = qd, kd, to_np(qd.float()), to_np(kd.float())
    yo, so = _oracle(q_ref[:, :, None], k_ref[:, :, None], to_np(to_dev(v, torch.bfloat16).float())[:, :, None],
                     ld[:, :, None], beta, 1.0, st)
    s = state_to_dev(st, B, H, D)
    y = torch.empty(B, H, D, device=dev())
    lam = to_dev(np.exp(ld).astype(np.float32))
    _lib.selective_decode_step(q_in, k_in, to_dev(v, torch.bfloat16), _lib.selective_gate(B, H, decay_bh=lam),
                               to_dev(beta), 1.0, norm, s, s, y)
    torch.cuda.synchronize()
    # fp32 arithmetic; with the LayerNorm prologue the normed rows may differ
    # from torch's by one bf16 rounding
    tol = 5e-3 if qk_norm else 1e-4
    assert_close(to_np(y).reshape(B * H, D), yo.reshape(B * H, D), tol, "y")
    for i, (a, b) in enumerate(zip(state_to_np(s, B * H, D), so)):
        assert_close(a, b.reshape(a.shape), tol, f"state[{i}]")


def _module(seed=0, H=2, dtype=torch.bfloat16):
    torch.manual_seed(seed)
    m = PrimeSelectiveMomentAttention(128, H, D, decay=0.99).to(dev())
    with torch.no_grad():  # move off the identity initialisation
        m.delta_proj.weight.normal_(0.0, 0.05)
        m.log_tau.add_(torch.randn(H, device=dev()) * 0.5)
        m.log_beta.add_(torch.randn(H, device=dev()) * 0.3)
    return m.to(dtype)


def _module_ref(m, x, state=None):
    """fp64 composition of the module (selective.py:334-444): torch layers for
    projections, LayerNorm and the step size, the oracle for the core (the
    parallel branch for L > 1, the step for L == 1)."""
    import torch.nn.functional as F
    W = {k: v.detach().double().cpu() for k, v in m.state_dict().items()}
    xd = x.detach().double().cpu()
    B, L, _ = xd.shape
    H = m.num_heads
    lin = lambda n: xd @ W[n + ".weight"].T + (W[n + ".bias"] if n + ".bias" in W else 0)
    q = lin("q_proj").view(B, L, H, D).transpose(1, 2)
    k = lin("k_proj").view(B, L, H, D).transpose(1, 2)
    v = lin("v_proj").view(B, L, H, D).transpose(1, 2)
    q = F.layer_norm(q, (D,), W["q_norm.weight"], W["q_norm.bias"]) / 8.0
    k = F.layer_norm(k, (D,), W["k_norm.weight"], W["k_norm.bias"])
    delta = F.softplus(lin("delta_proj")).clamp(1e-4, 50.0).transpose(1, 2).reshape(B * H, L)
    tau = torch.exp(W["log_tau"]).clamp(m.min_tau, m.max_tau)
    beta = torch.exp(W["log_beta"]).clamp(0.1, 15.0)
    r = lambda t: t.reshape(B * H, L, D).numpy()
    tb, bb = np.tile(tau.numpy(), B), np.tile(beta.numpy(), B)
    if L == 1:
        y, S = O.selective_recurrent(r(q), r(k), r(v), np.exp(-delta.numpy() / tb[:, None]), bb, eps=m.eps,
                                     state=state)
    else:
        y, S = O.selective_parallel(r(q), r(k), r(v), delta.numpy(), tb, bb, eps=m.eps)
    y = torch.from_numpy(y).view(B, H, L, D).transpose(1, 2).reshape(B, L, H * D)
    return (y @ W["o_proj.weight"].T).numpy(), S


def test_selective_module_prefill_then_step():
    m = _module()
    x = torch.randn(2, 101, 128, device=dev()).bfloat16()
    with torch.no_grad():
        out, st = m(x[:, :100], return_state=True)
        out1, st1 = m(x[:, 100:], state=st, return_state=True)
    ref, S = _module_ref(m, x[:, :100])
    assert_close(to_np(out.float()), ref, TOL_BF16, "prefill out")
    for i, (a, b) in enumerate(zip(state_to_np(st, 4, D), S)):
        assert_close(a, b.reshape(a.shape), TOL_BF16, f"prefill state[{i}]")
    ref1, S1 = _module_ref(m, x[:, 100:], state=S)
    assert_close(to_np(out1.float()), ref1, TOL_BF16, "step out")
    for i, (a, b) in enumerate(zip(state_to_np(st1, 4, D), S1)):
        assert_close(a, b.reshape(a.shape), TOL_BF16, f"step state[{i}]")


def test_selective_module_f32_prefill_then_step():
    """An fp32 module: the prefill runs the fp32 kernel, the step the decode
    kernel in fp32; both within the fp32 tolerance of the fp64 composition."""
    m = _module(seed=3, dtype=torch.float32)
    x = torch.randn(2, 301, 128, device=dev())
    with torch.no_grad():
        out, st = m(x[:, :300], return_state=True)
        out1, st1 = m(x[:, 300:], state=st, return_state=True)
    ref, S = _module_ref(m, x[:, :300])
    assert_close(to_np(out), ref, TOL_F32, "prefill out")
    for i, (a, b) in enumerate(zip(state_to_np(st, 4, D), S)):
        assert_close(a, b.reshape(a.shape), TOL_F32, f"prefill state[{i}]")
    ref1, _ = _module_ref(m, x[:, 300:], state=S)
    assert_close(to_np(out1), ref1, TOL_F32, "step out")


def _sel_model(seed=0):
    torch.manual_seed(seed)
    cfg = PrimeConfig(vocab_size=384, hidden_size=128, num_layers=2, num_heads=2, head_dim=64, decay=0.99,
                      use_selective=True, mlp_type="gelu", intermediate_size=256)
    model = PrimeForCausalLM(cfg).to(dev())
    with torch.no_grad():
        for layer in model.layers:
            at = layer.self_attn
            at.delta_proj.weight.normal_(0.0, 0.05)
            at.log_beta.add_(torch.randn(2, device=dev()) * 0.3)
    return model.bfloat16().eval()


def test_selective_model_steps_continue_prefill_and_greedy_decoder():
    model = _sel_model()
    ids = torch.randint(0, 384, (3, 40), generator=torch.Generator().manual_seed(5)).to(dev())
    with torch.no_grad():
        full = model(ids)["logits"]
        out = model(ids[:, :35], return_states=True)
        states = out["states"]
        for t in range(35, 40):
            step = model(ids[:, t:t + 1], states=states, return_states=True)
            states = step["states"]
            d = (step["logits"][:, -1].float() - full[:, t].float()).abs().max() / full[:, t].float().abs().max()
            assert d.item() < 3e-2, d.item()
    n = 10
    ref = model.generate(ids[:, :30], max_new_tokens=n, temperature=0.0)
    eager = GreedyDecoder(model, use_graph=False).generate(ids[:, :30], n)
    graph = GreedyDecoder(model, use_graph=True).generate(ids[:, :30], n)
    assert torch.equal(eager, ref), (eager, ref)
    assert torch.equal(graph, ref), (graph, ref)


def test_selective_gate_from_step_preactivations():
    """The in-kernel gate (softplus, clamp and rounding in bf16, then
    exp(-Delta / tau)) gives the decays the module's torch ops give
    (selective.py:368, 386): the steps agree with the explicit-decay call."""
    B, H = 5, 4
    q, k, v, _, beta = _inputs(B, H, 1, seed=60)
    q, k, v = (to_dev(x[:, :, 0], torch.bfloat16) for x in (q, k, v))
    g = torch.Generator(device=dev()).manual_seed(61)
    pre = (torch.randn(B, H + 3, device=dev(), generator=g) * 4).bfloat16()[:, :H]  # row stride H + 3
    pre[0, 0], pre[0, 1], pre[1, 0] = -30.0, 60.0, 25.0  # clamp low, clamp high, softplus identity branch
    tau = torch.tensor([3.0, 50.0, 700.0, 1999.0], device=dev())
    lam = torch.exp(-torch.nn.functional.softplus(pre).clamp(min=1e-4, max=50.0).float() / tau.view(1, H))
    st = state_to_dev(_rand_state(B * H, 62), B, H, D)
    outs = []
    for gate in (_lib.selective_gate(B, H, decay_bh=lam.contiguous()), _lib.selective_gate(B, H, step=pre, tau=tau)):
        s_out = _lib.new_state(B, H, D, dev())
        y = torch.empty(B, H, D, device=dev())
        _lib.selective_decode_step(q, k, v, gate, to_dev(beta), 1.0, None, st, s_out, y)
        outs.append((y, s_out))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0])
    for a, b in zip(outs[0][1], outs[1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_selective_log_decay_matches_module_ops(dtype):
    """prime_selective_log_decay equals the module's torch ops bit for bit:
    -(softplus(s).clamp(1e-4, 50.0)).float() / tau, transposed to [B, H, L]
    (selective.py:368, 414-416), on pre-activations that cover softplus's
    linear branch (s > 20), both clamps and ordinary values, read through a
    strided view (a column range of a wider projection, as the model's)."""
    torch.manual_seed(5)
    B, L, H = 3, 777, 12
    wide = torch.randn(B, L, H + 20, device="cuda") * 6.0
    wide[0, :40, 20:] = 30.0 + torch.rand(40, H, device="cuda") * 40.0  # linear branch, upper clamp
    wide[1, :40, 20:] = -20.0 - torch.rand(40, H, device="cuda") * 5.0  # softplus < 1e-4: lower clamp
    s = wide.to(dtype)[:, :, 20:]
    tau = torch.linspace(2.0, 2000.0, H, device="cuda")
    got = _lib.selective_log_decay(s, tau)
    want = (-(F.softplus(s).clamp(min=1e-4, max=50.0)).float() / tau.view(1, 1, H)).transpose(1, 2).contiguous()
    assert got.shape == (B, H, L) and got.dtype == torch.float32
    assert torch.equal(got, want), (got - want).abs().max().item()
