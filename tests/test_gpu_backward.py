"""GPU parity of the chunked-prefill backward (prime_chunked_prefill_backward)
against the oracle's reverse mode of the recurrence (oracle_recurrent_vjp,
the derivative of attention.py:119-143 that torch autograd gives the
reference when it trains through its prefill, tests/test_attention.py:50-62).

bf16 inputs run the bf16-MFMA passes and are held to the bf16 tolerance,
2e-2; fp32 inputs run the fp32 passes and are held to the fp32 tolerance,
1e-3 (max|d| / max|ref| per tensor)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib

from gpu_util import (TOL_BF16, TOL_F32, assert_close, assert_state_close, random_state, state_to_dev, state_to_np,
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


def _check(ref, got, dsi, tol=TOL_BF16, one_token_from_zero=False):
    """max|d| / max|ref| per gradient tensor.  For one token from a zero
    state y = v * min(1, den / eps), so dq and dk are tiny or zero (exactly
    zero where den >= eps); only in that case is their error measured
    against the gradient scale of dv instead of their own."""
    floor = 0.1 * np.abs(ref[2]).max() if one_token_from_zero else 0.0
    for name, r, x in zip(("dq", "dk", "dv"), ref[:3], got):
        assert np.isfinite(x).all(), name
        e = np.abs(x - r).max() / max(np.abs(r).max(), floor, 1e-300)
        assert e < tol, f"{name}: rel err {e:.3e} >= {tol}"
    if dsi is not None:
        assert_state_close(dsi, ref[3], tol, "dstate_in")


@pytest.mark.parametrize("B,H,L", [(1, 1, 1), (1, 2, 13), (2, 3, 64), (2, 2, 200), (1, 2, 1000)])
@pytest.mark.parametrize("with_state", [False, True])
def test_backward_bf16_matches_oracle(B, H, L, with_state):
    ref, got, dsi = _run(B, H, L, torch.bfloat16, with_state, with_state, seed=400 + L)
    _check(ref, got, dsi, one_token_from_zero=(L == 1 and not with_state))


@pytest.mark.parametrize("B,H,L", [(1, 1, 1), (1, 2, 13), (2, 2, 77), (1, 3, 130), (1, 2, 1000)])
@pytest.mark.parametrize("with_state", [False, True])
def test_backward_f32_inputs(B, H, L, with_state):
    ref, got, dsi = _run(B, H, L, torch.float32, with_state, with_state, seed=410 + L)
    _check(ref, got, dsi, TOL_F32, one_token_from_zero=(L == 1 and not with_state))


def test_backward_f32_inputs_bf16_dy_and_grads():
    """fp32 q/k/v with a bf16 output adjoint and bf16 gradients: the fp32
    passes, each gradient rounded once to bf16 (the bf16 tolerance)."""
    ref, got, dsi = _run(2, 2, 150, torch.float32, True, True, seed=415, gdtype=torch.bfloat16)
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
    """Unnormalised fp32 q/k: some denominators fall below eps (clamped tokens
    pass no denominator gradient).  With eps = 1e-3 the unclamped denominators
    reach ~1e-3 and dq = (dnum - y dden) / den cancels between two large
    terms; the fp32 passes keep that within the fp32 tolerance (bf16 operands
    measured 2.6e-2 there)."""
    ref, got, dsi = _run(2, 2, 100, torch.float32, False, False, seed=430, normalize=False, eps=eps)
    _check(ref, got, dsi, TOL_F32)


def test_backward_clamp_active_bf16():
    """The same unnormalised case with bf16 inputs and eps = 1: the bf16 passes."""
    ref, got, dsi = _run(2, 2, 100, torch.bfloat16, False, False, seed=431, normalize=False, eps=1.0)
    _check(ref, got, dsi)


def test_backward_dense_flag_without_state_and_bf16_grads():
    ref, got, dsi = _run(1, 3, 300, torch.bfloat16, False, False, seed=440, dense_clamp=True,
                         gdtype=torch.bfloat16)
    _check(ref, got, dsi)


def _dense_case(B, H, L, dtype, seed, eps, k0=None):
    """Inputs for the dense branch's double clamp with an incoming state, and
    oracle_dense_vjp's result (dq, dk, dv, dstate_in) and the single clamp's."""
    BH = B * H
    bf = dtype == torch.bfloat16
    q, k, v = O.make_inputs((B, H, L, D), seed=seed, bf16=bf)
    rng = np.random.default_rng(seed + 1)
    lam = rng.uniform(0.99, 0.9999, H).astype(np.float32)
    dy = rng.standard_normal((B, H, L, D)).astype(np.float32)
    if bf:
        dy = O.bf16_round(dy)
    st0 = random_state(BH, D, seed + 2)
    if k0 is not None:  # a negative K0: the outer clamp active on the first tokens
        st0 = tuple(np.full_like(x, k0) if i == 3 else x for i, x in enumerate(st0))
    ds = tuple(0.1 * rng.standard_normal(x.shape) for x in O.zero_state(BH, D))
    args = (q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D), np.tile(lam.astype(np.float64), B),
            dy.reshape(BH, L, D))
    ref = O.dense_vjp(*args, eps=eps, state=st0, dstate=ds)
    single = O.recurrent_vjp(*args, eps=eps, state=st0, dstate=ds)
    return (q, k, v, lam, dy, st0, ds), ref, single


@pytest.mark.parametrize("dtype,B,H,L,k0", [(torch.float32, 1, 2, 13, None), (torch.float32, 2, 2, 200, None),
                                            (torch.float32, 1, 2, 150, -1.5), (torch.bfloat16, 2, 2, 200, None),
                                            (torch.bfloat16, 1, 3, 70, -1.5)])
def test_backward_dense_clamp_with_state(dtype, B, H, L, k0):
    """The dense branch's double clamp with an incoming state
    (attention.py:177-185; eps = 2.5 puts the inner clamp on the first
    tokens) against oracle_dense_vjp; without a negative K0 the case is one
    whose derivative differs from the single clamp's by more than the
    tolerance."""
    eps = 2.5
    tol = TOL_BF16 if dtype == torch.bfloat16 else TOL_F32
    (q, k, v, lam, dy, st0, ds), ref, single = _dense_case(B, H, L, dtype, 700 + L, eps, k0)
    if k0 is None:
        assert max(np.abs(a - b).max() / np.abs(a).max() for a, b in zip(ref[:3], single[:3])) > 2 * tol
    g = [torch.empty(B, H, L, D, device=dev(), dtype=torch.float32) for _ in range(3)]
    dsi = _lib.new_state(B, H, D, dev())
    _lib.chunked_prefill_backward(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(lam), eps,
                                  state_to_dev(st0, B, H, D), to_dev(dy, dtype), state_to_dev(ds, B, H, D), *g, dsi,
                                  flags=1)
    torch.cuda.synchronize()
    BH = B * H
    _check(ref, [to_np(t).reshape(BH, L, D) for t in g], state_to_np(dsi, BH, D), tol)


def test_core_autograd_dense_clamp_with_state():
    """prime_prefill's dense branch (the module's path for L <= chunk_threshold)
    with an incoming state, trained through: q, k, v and the state's gradients
    against oracle_dense_vjp."""
    from prime_moment_attention.chunked_ssd import prime_prefill
    B, H, L, eps = 2, 2, 90, 2.5
    BH = B * H
    (q, k, v, lam, dy, st0, ds), ref, _ = _dense_case(B, H, L, torch.float32, 720, eps)
    tq, tk, tv = (to_dev(x).requires_grad_(True) for x in (q, k, v))
    ts = [t.requires_grad_(True) for t in state_to_dev(st0, B, H, D)]
    y, st = prime_prefill(tq, tk, tv, state=tuple(ts), decay=to_dev(lam), eps=eps, return_state=True,
                          dense_clamp=True)
    loss = (y * to_dev(dy)).sum() + sum((a * to_dev(b).reshape(a.shape)).sum() for a, b in zip(st, ds))
    loss.backward()
    torch.cuda.synchronize()
    for name, t, r in (("dq", tq, ref[0]), ("dk", tk, ref[1]), ("dv", tv, ref[2])):
        assert_close(to_np(t.grad).reshape(BH, L, D), r, TOL_F32, name)
    assert_state_close(tuple(to_np(t.grad) for t in ts), ref[3], TOL_F32, "dstate_in")


def test_backward_rejects_bad_arguments():
    B, H, L = 1, 2, 70
    x = torch.zeros(B, H, L, D, device=dev(), dtype=torch.bfloat16)
    g = [torch.empty(B, H, L, D, device=dev()) for _ in range(3)]
    lam = to_dev(np.full(H, 0.99, np.float32))
    st = _lib.new_state(B, H, D, dev(), zero=True)
    token_bytes = (B * H * L * 8 + 255) // 256 * 256
    with pytest.raises(RuntimeError, match="workspace"):  # the double clamp with a state needs its correction too
        _lib.chunked_prefill_backward(x, x, x, lam, 1.0, st, x, None, *g, None, flags=1,
                                      workspace=torch.empty(token_bytes, dtype=torch.uint8, device=dev()))
    with pytest.raises(RuntimeError, match="unknown flags"):
        _lib.chunked_prefill_backward(x, x, x, lam, 1.0, None, x, None, *g, None, flags=4)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.chunked_prefill_backward(x, x, x, lam, 1.0, None, x, None, *g, None,
                                      workspace=torch.empty(64, dtype=torch.uint8, device=dev()))
    with pytest.raises(RuntimeError, match="share dtype"):
        _lib.chunked_prefill_backward(x, x, x, lam, 1.0, None, x, None, g[0], g[1], g[2].bfloat16(), None)


# ---------------------------------------------------------------- autograd
def test_core_autograd_matches_oracle_vjp():
    """chunked_prime_ssd_core under autograd (q, k, v and the incoming state
    requiring grad, the final state used in the loss) against the oracle."""
    from prime_moment_attention import chunked_prime_ssd_core
    B, H, L = 2, 2, 300
    BH = B * H
    q, k, v = O.make_inputs((B, H, L, D), seed=450, bf16=False)
    rng = np.random.default_rng(451)
    lam = rng.uniform(0.99, 0.9999, H).astype(np.float32)
    st0 = random_state(BH, D, 452)
    dy = rng.standard_normal((B, H, L, D))
    ds = tuple(0.1 * rng.standard_normal(x.shape) for x in O.zero_state(BH, D))
    ref = O.recurrent_vjp(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D),
                          np.tile(lam.astype(np.float64), B), dy.reshape(BH, L, D), state=st0, dstate=ds)
    tq, tk, tv = (to_dev(x).requires_grad_(True) for x in (q, k, v))
    ts = [t.requires_grad_(True) for t in state_to_dev(st0, B, H, D)]
    y, st = chunked_prime_ssd_core(tq, tk, tv, state=tuple(ts), decay=to_dev(lam), return_state=True)
    loss = (y * to_dev(dy)).sum() + sum((a * to_dev(b).reshape(a.shape)).sum() for a, b in zip(st, ds))
    loss.backward()
    torch.cuda.synchronize()
    for name, t, r in (("dq", tq, ref[0]), ("dk", tk, ref[1]), ("dv", tv, ref[2])):
        assert_close(to_np(t.grad).reshape(BH, L, D), r, TOL_F32, name)
    assert_state_close(tuple(to_np(t.grad) for t in ts), ref[3], TOL_F32, "dstate_in")


def _module_reference(mod, x, L):
    """float64 CPU composition of PrimeMomentAttention.forward (attention.py:77-210,
    no state: the dense and chunked branches compute the same recurrence)."""
    m = {n: p.detach().double().cpu().requires_grad_(True) for n, p in mod.named_parameters()}
    xd = x.detach().double().cpu().requires_grad_(True)
    B = x.shape[0]
    H, Hk = mod.num_heads, mod.num_kv_heads
    q = (xd @ m["q_proj.weight"].t()).view(B, L, H, D).transpose(1, 2)
    k = (xd @ m["k_proj.weight"].t()).view(B, L, Hk, D).transpose(1, 2)
    v = (xd @ m["v_proj.weight"].t()).view(B, L, Hk, D).transpose(1, 2)
    if H != Hk:
        k, v = k.repeat_interleave(H // Hk, 1), v.repeat_interleave(H // Hk, 1)
    if mod.use_qk_norm:
        q = torch.nn.functional.layer_norm(q, (D,), m["q_norm.weight"], m["q_norm.bias"], 1e-5)
        k = torch.nn.functional.layer_norm(k, (D,), m["k_norm.weight"], m["k_norm.bias"], 1e-5)
    q = q / 8.0
    idx = torch.arange(L, dtype=torch.float64)
    diff = idx.view(L, 1) - idx.view(1, L)
    dm = torch.where(diff >= 0, mod.decay ** diff.clamp(min=0), torch.zeros(()))
    A = dm * (1.0 + q @ k.transpose(-1, -2) + 0.5 * (q * q) @ (k * k).transpose(-1, -2))
    y = (A @ v) / A.sum(-1, keepdim=True).clamp(min=mod.eps)
    out = y.transpose(1, 2).reshape(B, L, H * D) @ m["o_proj.weight"].t()
    return out, xd, m


@pytest.mark.parametrize("L,Hkv", [(200, 2), (600, 2), (130, 1)])
def test_module_gradients_match_float64_composition(L, Hkv):
    """PrimeMomentAttention trained through (out.sum()-style loss, as
    tests/test_attention.py:50-62): x and every weight gradient against the
    float64 composition of the reference formula."""
    from prime_moment_attention import PrimeMomentAttention
    torch.manual_seed(460)
    mod = PrimeMomentAttention(hidden_size=128, num_heads=2, head_dim=D, num_kv_heads=Hkv, decay=0.999,
                               use_qk_norm=True).to(dev())
    with torch.no_grad():
        for ln in (mod.q_norm, mod.k_norm):
            ln.weight.uniform_(0.5, 1.5)
            ln.bias.uniform_(-0.2, 0.2)
    x = torch.randn(2, L, 128, device=dev()).requires_grad_(True)
    out, _ = mod(x)
    g = torch.randn_like(out)
    (out * g).sum().backward()
    ref_out, xd, m = _module_reference(mod, x, L)
    (ref_out * g.double().cpu()).sum().backward()
    torch.cuda.synchronize()
    assert_close(to_np(out), ref_out.detach().numpy(), TOL_F32, "out")
    assert_close(to_np(x.grad), xd.grad.numpy(), TOL_F32, "x.grad")
    for n, p in mod.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n
        assert_close(to_np(p.grad), m[n].grad.numpy(), TOL_F32, n + ".grad")


def test_module_state_gradient_flows_through_steps():
    """A prefill followed by two L == 1 steps with the state carried, all
    under autograd: gradients reach x of every call and equal those of one
    prefill over the concatenated input."""
    from prime_moment_attention import PrimeMomentAttention
    torch.manual_seed(470)
    mod = PrimeMomentAttention(hidden_size=128, num_heads=2, head_dim=D, decay=0.995, use_qk_norm=True,
                               chunk_threshold=16).to(dev())
    x = torch.randn(1, 40, 128, device=dev())
    x1, x2, x3 = (t.clone().requires_grad_(True) for t in (x[:, :38], x[:, 38:39], x[:, 39:]))
    o1, s = mod(x1, return_state=True)
    o2, s = mod(x2, state=s, return_state=True)
    o3, _ = mod(x3, state=s)
    g = torch.randn(1, 40, 128, device=dev())
    (torch.cat([o1, o2, o3], 1) * g).sum().backward()
    xa = x.clone().requires_grad_(True)
    oa, _ = mod(xa)
    (oa * g).sum().backward()
    torch.cuda.synchronize()
    assert_close(to_np(torch.cat([x1.grad, x2.grad, x3.grad], 1)), to_np(xa.grad), TOL_F32, "x.grad")


def test_model_trains():
    """PrimeForCausalLM (tests/test_model.py:32-43 of the reference): the loss
    backward gives finite gradients to the embedding, attention and MLP
    weights, and a few AdamW steps lower the loss on a fixed batch."""
    from prime_moment_attention import PrimeConfig, PrimeForCausalLM
    torch.manual_seed(480)
    cfg = PrimeConfig(vocab_size=100, hidden_size=128, num_layers=2, num_heads=2, head_dim=D, decay=0.999,
                      use_qk_norm=True)
    model = PrimeForCausalLM(cfg).to(dev())
    ids = torch.randint(0, 100, (4, 96), device=dev())
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3)
    losses = []
    for _ in range(8):
        opt.zero_grad()
        loss = model(ids, labels=ids)["loss"]
        loss.backward()
        losses.append(float(loss.detach()))
        for n in ("embed_tokens.weight", "layers.0.self_attn.q_proj.weight", "layers.0.mlp.gate_proj.weight"):
            gr = dict(model.named_parameters())[n].grad
            assert gr is not None and torch.isfinite(gr).all(), n
        opt.step()
    assert losses[-1] < losses[0] - 0.1, losses


@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_segmented_equals_one_segment(with_state, dtype):
    """Few long sequences: the segment-parallel plan (forward state-only pass
    and scan for the segment-entry states, per-segment dual contributions and
    a reverse scan) against one segment per sequence (minimum workspace) and
    the oracle, with a ragged last chunk, an incoming state and a final-state
    adjoint; bf16 inputs (the bf16 passes) and fp32 inputs (the fp32 passes,
    one workgroup per CU, so fewer segments)."""
    B, H, L = 1, 2, 64 * 37 + 5
    BH = B * H
    bf = dtype == torch.bfloat16
    print(f"[backward segments] {dtype} state={with_state}", flush=True)
    q, k, v = O.make_inputs((B, H, L, D), seed=490, bf16=bf)
    rng = np.random.default_rng(491)
    lam = np.array([0.995, 0.9995], np.float32)
    dy = rng.standard_normal((B, H, L, D)).astype(np.float32)
    if bf:
        dy = O.bf16_round(dy)
    st0 = random_state(BH, D, 492) if with_state else None
    ds = tuple(0.1 * rng.standard_normal(x.shape) for x in O.zero_state(BH, D))
    full = _lib.backward_workspace_size(B, H, L)
    small = (BH * L * 8 + 255) // 256 * 256  # per-token denominators only
    assert full > small, "this shape should split into segments"
    outs = []
    for nbytes in (full, small):
        g = [torch.empty(B, H, L, D, device=dev()) for _ in range(3)]
        dsi = _lib.new_state(B, H, D, dev()) if with_state else None
        _lib.chunked_prefill_backward(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                      to_dev(lam), 1.0, state_to_dev(st0, B, H, D) if with_state else None,
                                      to_dev(dy, dtype), state_to_dev(ds, B, H, D), *g, dsi,
                                      workspace=torch.empty(nbytes, dtype=torch.uint8, device=dev()))
        torch.cuda.synchronize()
        outs.append(([to_np(t).reshape(BH, L, D) for t in g], state_to_np(dsi, BH, D) if with_state else None))
    tol_seg = 5e-3 if bf else 1e-4
    for x, y, n in zip(outs[0][0], outs[1][0], ("dq", "dk", "dv")):
        assert_close(x, y, tol_seg, n + " segmented vs one segment")
    if with_state:
        assert_state_close(outs[0][1], outs[1][1], tol_seg, "dstate_in")
    ref = O.recurrent_vjp(q.reshape(BH, L, D), k.reshape(BH, L, D), v.reshape(BH, L, D),
                          np.tile(lam.astype(np.float64), B), dy.reshape(BH, L, D), state=st0, dstate=ds)
    _check(ref, outs[0][0], outs[0][1], TOL_BF16 if bf else TOL_F32)
