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
