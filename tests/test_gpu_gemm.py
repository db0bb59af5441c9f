"""GPU parity of the projection kernels of the PRIME-125M blocks
(prime_linear / prime_linear_residual, model.py:59-68, 101-118) against fp32
products of the same bf16 operands: many-row shapes (the prefill's 256 x 256
tile kernel) and few-row shapes (the decode step's skinny kernel), with the
GELU and residual epilogues."""
import pytest
import torch
import torch.nn.functional as F

from prime_moment_attention import _lib

from gpu_util import dev

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-30)).item()


def _operands(M, N, K, seed, ldx=None):
    g = torch.Generator().manual_seed(seed)
    xs = torch.randn(M, ldx or K, generator=g)
    x = xs.to(dev(), torch.bfloat16)[:, :K]
    w = (torch.randn(N, K, generator=g) * 0.05).to(dev(), torch.bfloat16)
    return x, w


# (M, N, K, ldx): the prefill's projections (q/k/v and o 768, stacked q/k/v 2304,
# up 3072, down from 3072), ragged M, strided x rows, and decode-sized M
SHAPES = [(4096, 768, 768, None), (2048 + 37, 2304, 768, None), (4096, 3072, 768, None), (4096, 768, 3072, None),
          (3000, 768, 768, 832), (256, 768, 768, None), (37, 768, 768, None)]


@pytest.mark.parametrize("M,N,K,ldx", SHAPES)
def test_linear_matches_fp32_product(M, N, K, ldx):
    x, w = _operands(M, N, K, seed=M + N + K, ldx=ldx)
    y = torch.empty(M, N, device=dev(), dtype=torch.bfloat16)
    _lib.linear(x, w, y)
    ref = x.float() @ w.float().T
    assert _rel(y, ref) < 8e-3, _rel(y, ref)  # one bf16 rounding of the output
    assert _rel(y, F.linear(x, w)) < 8e-3


@pytest.mark.parametrize("M,N,K,ldx", SHAPES[:4] + SHAPES[-1:])
def test_linear_gelu_epilogue(M, N, K, ldx):
    x, w = _operands(M, N, K, seed=7 + M, ldx=ldx)
    y = torch.empty(M, N, device=dev(), dtype=torch.bfloat16)
    _lib.linear(x, w, y, _lib.EPILOGUE_GELU)
    ref = F.gelu(x.float() @ w.float().T)
    assert _rel(y, ref) < 8e-3
    assert _rel(y, F.gelu(F.linear(x, w))) < 8e-3


@pytest.mark.parametrize("M,N,K,ldx", SHAPES)
@pytest.mark.parametrize("inplace", [True, False])
def test_linear_residual_epilogue(M, N, K, ldx, inplace):
    x, w = _operands(M, N, K, seed=11 + K, ldx=ldx)
    g = torch.Generator().manual_seed(3)
    r = (torch.randn(M, N, generator=g) * 4).to(dev(), torch.bfloat16)
    want = (r.float() + F.linear(x, w).float()).to(torch.bfloat16)  # the block's two bf16 ops
    out = r if inplace else torch.empty_like(r)
    r0 = r.clone()
    _lib.linear_residual(x, w, r, out)
    torch.cuda.synchronize()
    assert _rel(out, want) < 8e-3
    exact = r0.float() + (x.float() @ w.float().T)
    assert _rel(out, exact) < 8e-3
    if not inplace:
        assert torch.equal(r, r0)


def test_linear_residual_rejects_partial_overlap():
    x, w = _operands(512, 768, 768, seed=1)
    buf = torch.empty(513, 768, device=dev(), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="overlap"):
        _lib.linear_residual(x, w, buf[1:], buf[:512])


# prime_linear_fused: the decode step's projections with the RMSNorm folded in
# (model.py:47-56 then 59-68) and the GELU / residual epilogues
FUSED = [(256, 2304, 768), (256, 768, 768), (256, 3072, 768), (256, 768, 3072), (37, 768, 768), (1000, 1536, 768),
         (32, 50304, 768), (130, 640, 384), (64, 352, 512)]


@pytest.mark.parametrize("M,N,K", FUSED)
@pytest.mark.parametrize("epi", ["none", "gelu", "residual"])
@pytest.mark.parametrize("rms", [True, False])
def test_linear_fused_matches_fp32(M, N, K, epi, rms):
    x, w = _operands(M, N, K, seed=M + N + K + (1 if rms else 0))
    x = x * 3 + 0.5  # rows with their own scale, as the residual stream has
    g = torch.Generator().manual_seed(N)
    gamma = (1 + 0.2 * torch.randn(K, generator=g)).to(dev(), torch.bfloat16)
    eps = 1e-6
    wg = (w.float() * gamma.float()).to(torch.bfloat16) if rms else w  # the norm's weight in w's columns
    ref = x.float() @ wg.float().T
    if rms:
        ref = ref * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps)
    r = (torch.randn(M, N, generator=g) * 2).to(dev(), torch.bfloat16)
    out = torch.empty(M, N, device=dev(), dtype=torch.bfloat16)
    code = {"none": _lib.EPILOGUE_NONE, "gelu": _lib.EPILOGUE_GELU, "residual": _lib.EPILOGUE_RESIDUAL}[epi]
    _lib.linear_fused(x, wg, out, code, eps if rms else 0.0, r if epi == "residual" else None)
    if epi == "gelu":
        ref = F.gelu(ref)
    elif epi == "residual":
        ref = r.float() + ref
    torch.cuda.synchronize()
    assert _rel(out, ref) < 8e-3, _rel(out, ref)
    if rms and epi == "none":
        # against the block's own two steps: RMSNorm (rounded) then the projection
        n = torch.empty_like(x)
        _lib.add_rmsnorm(x.contiguous(), None, gamma, n, eps)
        assert _rel(out, F.linear(n, w)) < 1.5e-2


def test_linear_fused_residual_in_place():
    x, w = _operands(256, 768, 3072, seed=5)
    r = torch.randn(256, 768, device=dev()).to(torch.bfloat16)
    want = (r.float() + F.linear(x, w).float()).to(torch.bfloat16)
    _lib.linear_fused(x, w, r, _lib.EPILOGUE_RESIDUAL, 0.0, r)
    torch.cuda.synchronize()
    assert _rel(r, want) < 8e-3


def test_linear_fused_rejects_bad_shapes():
    x, w = _operands(256, 768, 768, seed=1)
    with pytest.raises(RuntimeError, match="multiple"):
        _lib.linear_fused(x[:, :704], w[:, :704], torch.empty(256, 768, device=dev(), dtype=torch.bfloat16))
    big = torch.empty(1025, 768, device=dev(), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="1024"):
        _lib.linear_fused(big, w, torch.empty(1025, 768, device=dev(), dtype=torch.bfloat16))
