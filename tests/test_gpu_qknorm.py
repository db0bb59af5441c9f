"""GPU parity of the QK LayerNorm applied as the prefill kernels load q and k
(prime_chunked_prefill_qknorm / prime_selective_prefill_qknorm): bit-identical
to prime_head_layernorm on the projections (attention.py:96-101,
selective.py:358-362) followed by the plain prefill, whose own parity with the
oracle the other prefill tests pin."""
import pytest
import torch

from prime_moment_attention import _lib

from gpu_util import dev, random_state, state_to_dev

pytestmark = pytest.mark.gpu

D = 64


def _norms(seed, affine):
    if not affine:
        return None, None
    g = torch.Generator().manual_seed(seed)
    lns = []
    for _ in range(2):
        ln = torch.nn.LayerNorm(D)
        with torch.no_grad():
            ln.weight.copy_(1 + 0.3 * torch.randn(D, generator=g))
            ln.bias.copy_(0.2 * torch.randn(D, generator=g))
        lns.append(ln.to(device=dev(), dtype=torch.bfloat16))
    return lns


def _projections(B, H, Hkv, L, seed):
    """Raw q/k/v projections as the module holds them: [B, H, L, D] views of
    [B, L, H, D] buffers, with an offset and a spread the LayerNorm removes."""
    g = torch.Generator().manual_seed(seed)
    mk = lambda h, s, o: (torch.randn(B, L, h, D, generator=g) * s + o).to(dev(), torch.bfloat16).transpose(1, 2)
    return mk(H, 2.0, 0.3), mk(Hkv, 1.5, -0.2), mk(Hkv, 1.0, 0.0)


def _normalised(q, k, q_norm, k_norm, scale):
    qn, kn = q.clone(), k.clone()
    _lib.head_layernorm(qn, qn, q_norm, scale)
    if k_norm is not None:
        _lib.head_layernorm(kn, kn, k_norm, 1.0)
    return qn, kn


def _assert_same(a, b):
    ya, sa = a
    yb, sb = b
    assert torch.equal(ya, yb), f"y differs: max |d| {(ya.float() - yb.float()).abs().max().item()}"
    if sa is not None:
        for i, (x, z) in enumerate(zip(sa, sb)):
            assert torch.equal(x, z), f"state component {i} differs"


@pytest.mark.parametrize("affine", [True, False])
@pytest.mark.parametrize("segmented", [True, False])
@pytest.mark.parametrize("with_state", [False, True])
def test_prefill_qknorm_on_load_equals_normalising_first(affine, segmented, with_state):
    B, H, Hkv, L = 2, 4, 2, 64 * 9 + 7
    q, k, v = _projections(B, H, Hkv, L, 11)
    q_norm, k_norm = _norms(12, affine)
    lam = torch.tensor([0.99, 0.995, 0.999, 0.9999], device=dev())
    st0 = state_to_dev(random_state(B * H, D, 13), B, H, D) if with_state else None
    norm = _lib.qk_norm(q_norm, k_norm, 0.125, torch.bfloat16)
    ws = None if segmented else torch.empty(0, dtype=torch.uint8, device=dev())
    if segmented:
        assert _lib.workspace_size(B, H, L) > 0

    def run(qq, kk, nrm):
        y = torch.empty(B, H, L, D, device=dev(), dtype=torch.bfloat16)
        st = _lib.new_state(B, H, D, dev())
        _lib.chunked_prefill(qq, kk, v, lam, 1.0, 64, st0, y, st, 0, workspace=ws, qk_norm=nrm)
        return y, st

    fused = run(q, k, norm)
    qn, kn = _normalised(q, k, q_norm, k_norm, 0.125)
    first = run(qn, kn, None)
    torch.cuda.synchronize()
    _assert_same(fused, first)


def test_prefill_qknorm_dense_clamp():
    B, H, L = 2, 3, 300
    q, k, v = _projections(B, H, H, L, 21)
    q_norm, k_norm = _norms(22, True)
    lam = torch.tensor([0.99, 0.995, 0.9995], device=dev())
    norm = _lib.qk_norm(q_norm, k_norm, 0.125, torch.bfloat16)
    outs = []
    for qq, kk, nrm in ((q, k, norm), (*_normalised(q, k, q_norm, k_norm, 0.125), None)):
        y = torch.empty(B, H, L, D, device=dev(), dtype=torch.float32)
        st = _lib.new_state(B, H, D, dev())
        _lib.chunked_prefill(qq, kk, v, lam, 1.0, 64, None, y, st, _lib.PRIME_FLAG_DENSE_CLAMP, qk_norm=nrm)
        outs.append((y, st))
    torch.cuda.synchronize()
    _assert_same(*outs)


@pytest.mark.parametrize("segmented", [True, False])
def test_selective_prefill_qknorm_on_load(segmented):
    B, H, L = 2, 3, 64 * 7 + 19
    q, k, v = _projections(B, H, H, L, 31)
    q_norm, k_norm = _norms(32, True)
    g = torch.Generator().manual_seed(33)
    log_decay = (-torch.rand(B, H, L, generator=g) * 0.05).to(dev())
    beta = (0.5 + torch.rand(H, generator=g)).to(dev())
    norm = _lib.qk_norm(q_norm, k_norm, 0.125, torch.bfloat16)
    ws = None if segmented else torch.empty(0, dtype=torch.uint8, device=dev())
    outs = []
    for qq, kk, nrm in ((q, k, norm), (*_normalised(q, k, q_norm, k_norm, 0.125), None)):
        y = torch.empty(B, H, L, D, device=dev(), dtype=torch.bfloat16)
        st = _lib.new_state(B, H, D, dev())
        _lib.selective_prefill(qq, kk, v, log_decay, beta, 1.0, None, y, st, workspace=ws, qk_norm=nrm)
        outs.append((y, st))
    torch.cuda.synchronize()
    _assert_same(*outs)


def test_prefill_qknorm_rejects_fp32_inputs():
    B, H, L = 1, 2, 70
    q, k, v = (t.float() for t in _projections(B, H, H, L, 41))
    norm = _lib.qk_norm(None, None, 0.125, torch.float32)
    y = torch.empty(B, H, L, D, device=dev())
    with pytest.raises(RuntimeError, match="BF16"):
        _lib.chunked_prefill(q, k, v, torch.full((H,), 0.99, device=dev()), 1.0, 64, None, y, None,
                             qk_norm=norm)


def test_module_prefill_uses_the_load_norm():
    """The attention module's bf16 prefill passes its QK-norm to the kernels,
    and its output matches normalising first."""
    from prime_moment_attention import PrimeMomentAttention
    torch.manual_seed(51)
    m = PrimeMomentAttention(hidden_size=256, num_heads=4, head_dim=D, use_qk_norm=True).to(dev(), torch.bfloat16).eval()
    with torch.no_grad():
        for ln in (m.q_norm, m.k_norm):
            ln.weight.copy_(1 + 0.3 * torch.randn(D, device=dev()))
            ln.bias.copy_(0.2 * torch.randn(D, device=dev()))
    x = torch.randn(2, 700, 256, device=dev(), dtype=torch.bfloat16)
    with torch.no_grad():
        q, k, _ = m.project(x, normalize=False)
        assert m._load_norm(q) is not None
        y1, s1 = m(x, return_state=True)
        m._load_norm = lambda q: None  # force normalising first
        y2, s2 = m(x, return_state=True)
    torch.cuda.synchronize()
    _assert_same((y1, s1), (y2, s2))
