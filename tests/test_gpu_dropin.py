"""GPU tests of the reference's drop-in module classes beyond
PrimeMomentAttention: ChunkedPrimeSSD (chunked_ssd.py:187-251) and
PrimeMomentCache (cache.py:15-56) driving a real decode loop.

The ChunkedPrimeSSD parity test follows the reference's only numeric test,
tests/test_chunked_ssd_parity.py:13-42 (weights copied from a
PrimeMomentAttention into a ChunkedPrimeSSD, B=2, L=256 so the module takes
its dense branch, H=4, decay 0.9995, LayerNorm QK-norm; outputs within 1e-5,
states within 2e-3), at head_dim 64 (the reference test's own head_dim 32
runs in tests/test_gpu_generic_d.py).  Both classes are then checked against a
float64 composition of their own weights through the oracle recurrence.  The
module's inference projection (q, k and v as one GEMM over stacked weights) is
checked against the three nn.Linear calls autograd records through."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from prime_moment_attention import ChunkedPrimeSSD, PrimeMomentAttention, PrimeMomentCache, PrimeSelectiveMomentAttention

from gpu_util import TOL_BF16, TOL_F32, assert_close, assert_state_close, dev, state_to_np, to_np

pytestmark = pytest.mark.gpu

D = 64


def _copy_weights(src, dst):
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
        for p in ("weight", "bias"):
            a = getattr(getattr(src, name), p, None)
            if a is not None:
                getattr(getattr(dst, name), p).data.copy_(a.data)


def _random_ln(mod, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for ln in (mod.q_norm, mod.k_norm):
            ln.weight.copy_(torch.empty(D).uniform_(0.5, 1.5, generator=g))
            ln.bias.copy_(torch.empty(D).uniform_(-0.2, 0.2, generator=g))


def _oracle_module(mod, x, state=None):
    """float64 composition of the module's forward (chunked_ssd.py:225-251 /
    attention.py:83-210): projections, LayerNorm QK-norm, q / sqrt(D), the
    recurrence (the oracle), o_proj.  Returns (out [B, L, hidden], state)."""
    W = {n: p.detach().double().cpu() for n, p in mod.named_parameters()}
    xd = x.detach().double().cpu()
    B, L, _ = xd.shape
    H = mod.num_heads
    proj = lambda n: (xd @ W[n + ".weight"].T).view(B, L, H, D).transpose(1, 2)
    q, k, v = proj("q_proj"), proj("k_proj"), proj("v_proj")
    q = F.layer_norm(q, (D,), W["q_norm.weight"], W["q_norm.bias"], 1e-5)
    k = F.layer_norm(k, (D,), W["k_norm.weight"], W["k_norm.bias"], 1e-5)
    q = q / np.sqrt(D)
    y, st = O.recurrent(q.reshape(B * H, L, D).numpy(), k.reshape(B * H, L, D).numpy(),
                        v.reshape(B * H, L, D).numpy(), np.full(B * H, float(mod.decay)), eps=mod.eps, state=state)
    y = torch.from_numpy(y).view(B, H, L, D).transpose(1, 2).reshape(B, L, H * D)
    return (y @ W["o_proj.weight"].T).numpy(), st


def test_chunked_ssd_parity_with_module():
    """tests/test_chunked_ssd_parity.py:13-42 at D = 64: ChunkedPrimeSSD (the
    chunked core) == PrimeMomentAttention (its dense branch, L = 256 <= 512)
    on the same weights, outputs within 1e-5 and states within 2e-3."""
    B, L, hidden, H = 2, 256, 128, 4
    torch.manual_seed(0)
    dense = PrimeMomentAttention(hidden_size=hidden, num_heads=H, head_dim=D, decay=0.9995, use_qk_norm=True)
    chunk = ChunkedPrimeSSD(hidden_size=hidden, num_heads=H, head_dim=D, chunk_size=64, decay=0.9995,
                            use_qk_norm=True)
    _random_ln(dense, 1)
    _copy_weights(dense, chunk)
    dense, chunk = dense.to(dev()), chunk.to(dev())
    x = torch.randn(B, L, hidden, device=dev())
    with torch.no_grad():
        out_d, st_d = dense(x, return_state=True)
        out_c, st_c = chunk(x, return_state=True)
    torch.cuda.synchronize()
    assert float((out_d - out_c).abs().max()) < 1e-5
    for i, (a, b) in enumerate(zip(st_d, st_c)):
        assert float((a.squeeze() - b.squeeze()).abs().max()) < 2e-3, i
    # and both against the float64 composition of the same weights
    ref, st_ref = _oracle_module(chunk, x)
    assert_close(to_np(out_c), ref, TOL_F32, "ChunkedPrimeSSD out")
    assert_state_close(state_to_np(st_c, B * H, D), st_ref, TOL_F32, "ChunkedPrimeSSD")


@pytest.mark.parametrize("dtype,tol", [(torch.float32, TOL_F32), (torch.bfloat16, TOL_BF16)])
def test_chunked_ssd_carries_state(dtype, tol):
    """ChunkedPrimeSSD over 700 tokens, then 300 more with the state carried,
    against the float64 composition over all 1000 (the reference core raises on
    a 6-tuple state, chunked_ssd.py:129-137; here the state is carried)."""
    B, hidden, H = 2, 192, 3
    torch.manual_seed(5)
    mod = ChunkedPrimeSSD(hidden_size=hidden, num_heads=H, head_dim=D, decay=0.999, use_qk_norm=True)
    _random_ln(mod, 6)
    mod = mod.to(dev(), dtype)
    x = torch.randn(B, 1000, hidden, device=dev()).to(dtype)
    with torch.no_grad():
        o1, s1 = mod(x[:, :700], return_state=True)
        o2, s2 = mod(x[:, 700:], state=s1, return_state=True)
    torch.cuda.synchronize()
    ref, st_ref = _oracle_module(mod, x)
    assert_close(to_np(torch.cat([o1, o2], 1)), ref, tol, "ChunkedPrimeSSD out")
    assert_state_close(state_to_np(s2, B * H, D), st_ref, tol, "ChunkedPrimeSSD")


def test_cache_feeds_decode_loop():
    """PrimeMomentCache (cache.py:15-56) as the state store of a layer stack:
    a prefill of 40 tokens, then 6 single-token steps, each layer reading its
    state with get_state and writing the next with set_state, update() counting
    tokens.  The outputs equal one prefill over all 46 tokens, the held bytes
    stay constant, and reset() empties the cache."""
    torch.manual_seed(7)
    hidden, H, layers, B = 128, 2, 3, 2
    mods = [PrimeMomentAttention(hidden_size=hidden, num_heads=H, head_dim=D, decay=0.995, use_qk_norm=True,
                                 chunk_threshold=16).to(dev()) for _ in range(layers)]
    x = torch.randn(B, 46, hidden, device=dev())

    def stack(h, cache):
        for i, m in enumerate(mods):
            out, st = m(h, state=cache.get_state(i) if cache is not None else None, return_state=True)
            if cache is not None:
                cache.set_state(i, st)
                kv = h.new_empty(B, H, h.shape[1], D)  # update() only counts the tokens
                ret = cache.update(kv, kv, i)
                assert ret[0] is kv and ret[1] is kv
            h = h + out
        return h

    with torch.no_grad():
        full = stack(x, None)
        cache = PrimeMomentCache()
        assert cache.get_state(0) is None and cache.get_seq_length() == 0
        outs = [stack(x[:, :40], cache)]
        held = cache.state_bytes()
        assert held == layers * B * H * (2 * D * D + 3 * D + 1) * 4
        for t in range(40, 46):
            outs.append(stack(x[:, t:t + 1], cache))
            assert cache.state_bytes() == held
        assert cache.get_seq_length() == 46
    torch.cuda.synchronize()
    assert_close(to_np(torch.cat(outs, 1)), to_np(full), TOL_F32, "cached steps vs one prefill")
    s0 = cache.get_state(0)
    assert len(s0) == 6 and s0[3].shape == (B, H, 1)
    cache.reset()
    assert cache.get_state(0) is None and cache.get_seq_length() == 0


@pytest.mark.parametrize("selective", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_stacked_qkv_projection_matches_three_linears(dtype, selective):
    """attention.py:83-85 (selective.py:358-360): inference projects q, k and v
    with one GEMM over the stacked weights; the result is that of the three
    projections autograd records through, the stacked copy follows in-place
    weight updates, and training keeps the three nn.Linear calls."""
    torch.manual_seed(11)
    if selective:
        m = PrimeSelectiveMomentAttention(hidden_size=256, num_heads=4, head_dim=D, num_kv_heads=2, decay=0.99)
        with torch.no_grad():  # per-token decays that vary
            m.delta_proj.weight.normal_(0.0, 0.05)
    else:
        m = PrimeMomentAttention(hidden_size=256, num_heads=4, head_dim=D, num_kv_heads=2, decay=0.999,
                                 use_qk_norm=True)
    m = m.to(dev(), dtype)
    x = torch.randn(2, 300, 256, device=dev(), dtype=dtype)
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    for rep in range(2):
        with torch.no_grad():
            y_inf, st_inf = m(x, return_state=True)
        assert m.__dict__.get("_qkv_cache") is not None
        y_tr, st_tr = m(x, return_state=True)  # autograd records: three projections
        assert y_tr.requires_grad
        assert_close(to_np(y_inf), to_np(y_tr.detach()), tol)
        assert_state_close(state_to_np(st_inf, 8, D), state_to_np(st_tr, 8, D), tol)
        with torch.no_grad():
            m.k_proj.weight.mul_(0.5)  # the next inference call restacks
    y_tr.float().square().mean().backward()
    assert m.q_proj.weight.grad is not None and m.v_proj.weight.grad is not None
