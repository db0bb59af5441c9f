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


# ---------------------------------------------------------------- GELU pass
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n", [1, 7, 8, 9, 4096 * 3 + 5, 3 * 2**20 + 11])
def test_gelu_matches_torch(dtype, n):
    """prime_gelu (the prefill MLP's activation, nn.GELU's exact form) against
    the float64 GELU of the same values: within one unit in the last place of
    the dtype plus the fp32 formula's cancellation in 1 + erf for x below
    about -3 (the fp32 erf of the device library may also differ from another
    build's by an ulp, which moves a rounding at a halfway point), and equal to
    torch's F.gelu on the GPU in all but a few elements; the 16-byte body, the
    per-element tail and the special values (signed zeros, infinities, NaN,
    large magnitudes) covered; out of place and in place."""
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(n, generator=g) * 3).to(dev(), dtype)
    special = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 30.0, -30.0, 1e-30, -5.5],
                           dtype=dtype)[:n]
    x[:special.numel()] = special.to(dev())
    torch_gelu = F.gelu(x)
    x64 = x.double().cpu()
    want = F.gelu(x64)
    ulp = {torch.bfloat16: 2.0**-7, torch.float16: 2.0**-10, torch.float32: 2.0**-22}[dtype]
    tiny = {torch.bfloat16: 1e-38, torch.float16: 6e-8, torch.float32: 1e-44}[dtype]

    def check(y):
        yc = y.double().cpu()
        assert torch.equal(yc.isnan(), want.isnan())
        ok = ~want.isnan()
        fin = ok & want.isfinite()
        assert torch.equal(yc[ok & ~fin], want[ok & ~fin])
        err = (yc[fin] - want[fin]).abs()
        # one ulp of the result, plus the fp32 formula's own error where 1 + erf
        # cancels (x below about -3: an ulp or two of erf near -1, times x / 2)
        bound = ulp * want[fin].abs() + x64[fin].abs() * 2.0**-22 + tiny
        assert bool((err <= bound).all()), (err - bound).max().item()
        same = (y == torch_gelu) | (y.isnan() & torch_gelu.isnan())
        assert (~same).sum().item() <= max(2, n // 1000)

    y = torch.empty_like(x)
    _lib.gelu(x, y)
    torch.cuda.synchronize()
    check(y)
    _lib.gelu(x)  # in place
    torch.cuda.synchronize()
    check(x)


def test_gelu_rejects_overlap_and_misalignment():
    x = torch.randn(64, device=dev(), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="overlap"):
        _lib.gelu(x[8:], x[:56])
    with pytest.raises(RuntimeError, match="aligned"):
        _lib.gelu(x[1:9], torch.empty(8, device=dev(), dtype=torch.bfloat16))


# ---------------------------------------------------------------- fragment layout
def _frag_index(R, K, device):
    """Flat index of element (r, k) of an R x K matrix in the fragment layout
    (16 x 32 blocks, block-row-major; slot r%16 + 16 ((k%32)/8), element k%8)."""
    r = torch.arange(R, device=device).view(-1, 1)
    k = torch.arange(K, device=device).view(1, -1)
    return ((r // 16) * (K // 32) + k // 32) * 512 + ((r % 16) + 16 * ((k % 32) // 8)) * 8 + k % 8


def _unfrag(flat, R, K):
    return flat[_frag_index(R, K, flat.device)]


def test_pack_frag_layout_and_gather():
    """prime_pack_frag puts (r, k) where the layout formula says, pads rows to
    a multiple of 32 with zeros, gathers rows by index (ids out of range give
    zero rows) and reads strided rows."""
    g = torch.Generator(device=dev()).manual_seed(3)
    src = torch.randn(50, 320, device=dev(), generator=g).to(torch.bfloat16)[:, :256]
    f = _lib.pack_frag(src, M=50)
    assert f.numel() == 64 * 256
    full = _unfrag(f, 64, 256)
    assert torch.equal(full[:50], src) and not full[50:].any()
    rows = torch.tensor([7, 0, 49, 3, -1, 50, 7], device=dev(), dtype=torch.int64)
    f2 = _lib.pack_frag(src, rows=rows)
    got = _unfrag(f2, 32, 256)
    for i, r in enumerate(rows.tolist()):
        exp = src[r] if 0 <= r < 50 else torch.zeros(256, device=dev(), dtype=torch.bfloat16)
        assert torch.equal(got[i], exp), i
    assert not got[len(rows):].any()


def _frag_ref(x, w, rms_eps=None, bias=None, epi=_lib.EPILOGUE_NONE, r=None, with_product=False):
    """fp32 product of the bf16 operands, row RMS scale, bias, one rounding,
    then the GELU / residual epilogue with its rounding (and the rounded
    product, whose own ulp bounds what an epilogue passes on)."""
    acc = x.float() @ w.float().T
    if rms_eps is not None:
        acc = acc * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + rms_eps)
    if bias is not None:
        acc = acc + bias
    o = acc.to(torch.bfloat16).float()
    prod = o
    if epi == _lib.EPILOGUE_GELU:
        o = F.gelu(o).to(torch.bfloat16).float()
    elif epi == _lib.EPILOGUE_RESIDUAL:
        o = o + r.float()
    o = o.to(torch.bfloat16)
    return (o, prod) if with_product else o


def _close_bf16(out, ref, what, prod=None):
    """Within one bf16 ulp (2^-7 relative) of the result, plus one ulp of the
    rounded product where an epilogue follows it (a product that flips by one
    ulp passes that ulp on through the GELU, slope <= 1.13, or the residual
    add, where r may cancel the product), plus 1e-3 of the largest value: the
    fp32 sums differ from the reference's in order only."""
    d = (out.float() - ref.float()).abs()
    bound = ref.float().abs() * 2 ** -7 + 1e-3 * ref.float().abs().max()
    if prod is not None:
        bound = bound + 1.13 * prod.abs() * 2 ** -7
    assert bool((d <= bound).all()), f"{what}: max |d| {float(d.max()):.3e}"


# the decode step's projections at B=256 and B=32 (q/k/v 2304 and the selective
# 2368, o and down into 768, up 3072), small and ragged shapes
FRAG_SHAPES = [(256, 2304, 768), (256, 768, 768), (256, 3072, 768), (256, 768, 3072), (32, 2368, 768),
               (32, 768, 3072), (37, 512, 256), (5, 96, 512), (300, 1024, 1536)]


@pytest.mark.parametrize("M,N,K", FRAG_SHAPES)
@pytest.mark.parametrize("kind", ["rows_rms_bias", "frag_gelu_rms", "frag_residual", "rows_plain"])
def test_linear_frag_matches_fp32_product(M, N, K, kind):
    g = torch.Generator(device=dev()).manual_seed(M * 31 + N + K)
    x = (torch.randn(M, K, device=dev(), generator=g) * 0.7).to(torch.bfloat16)
    w = (torch.randn(N, K, device=dev(), generator=g) * K ** -0.5).to(torch.bfloat16)
    xf, wf = _lib.pack_frag(x), _lib.pack_frag(w)
    Mp = _lib.frag_rows(M)
    if kind.startswith("rows"):
        rms = 1e-6 if "rms" in kind else None
        bias = torch.randn(N, device=dev(), generator=g) * 0.1 if "bias" in kind else None
        ldy = N + 64
        yb = torch.full((M, ldy), float("nan"), device=dev(), dtype=torch.bfloat16)
        _lib.linear_frag(xf, wf, M, N, K, yb, flags=_lib.LINEAR_RMS if rms else 0, rms_eps=rms or 0.0, bias=bias,
                         ldy=ldy)
        torch.cuda.synchronize()
        out = yb[:, :N]
        assert torch.isnan(yb[:, N:].float()).all(), "wrote past the row"
        ref = _frag_ref(x, w, rms, bias)
    else:
        if N % 32:
            pytest.skip("fragment-layout outputs need N % 32 == 0")
        y = torch.empty(Mp * N, device=dev(), dtype=torch.bfloat16)
        if kind == "frag_gelu_rms":
            _lib.linear_frag(xf, wf, M, N, K, y, _lib.EPILOGUE_GELU, _lib.LINEAR_RMS | _lib.LINEAR_OUT_FRAG,
                             rms_eps=1e-5)
            ref, prod = _frag_ref(x, w, 1e-5, epi=_lib.EPILOGUE_GELU, with_product=True)
        else:
            r = (torch.randn(M, N, device=dev(), generator=g)).to(torch.bfloat16)
            _lib.pack_frag(r, out=y)  # residual in place: y holds r on entry
            _lib.linear_frag(xf, wf, M, N, K, y, _lib.EPILOGUE_RESIDUAL, _lib.LINEAR_OUT_FRAG, r=y)
            ref, prod = _frag_ref(x, w, epi=_lib.EPILOGUE_RESIDUAL, r=r, with_product=True)
        torch.cuda.synchronize()
        out = _unfrag(y, Mp, N)[:M]
    _close_bf16(out, ref, f"{kind} {M}x{N}x{K}", None if kind.startswith("rows") else prod)


@pytest.mark.parametrize("M,V", [(256, 50304), (32, 50304), (7, 384), (100, 4096), (300, 8192), (130, 50304)])
def test_linear_frag_argmax_equals_argmax_of_its_logits(M, V):
    """The fused greedy token (prime_linear_frag with tokens) equals
    torch.argmax of the logits the same call writes (first index of the
    largest, so ties resolve as torch does), with and without the logits."""
    K = 768 if V > 1000 else 256
    if V == 8192:
        K = 512
    g = torch.Generator(device=dev()).manual_seed(M + V)
    x = torch.randn(M, K, device=dev(), generator=g).to(torch.bfloat16)
    w = (torch.randn(V, K, device=dev(), generator=g) * 0.02).to(torch.bfloat16)
    w[V // 3] = w[V // 5]  # duplicated rows: exact ties between two columns
    xf, wf = _lib.pack_frag(x), _lib.pack_frag(w)
    ws = torch.empty(_lib.linear_frag_workspace_size(M, V, K), device=dev(), dtype=torch.uint8)
    logits = torch.empty(M, V, device=dev(), dtype=torch.bfloat16)
    t1 = torch.full((M,), -1, device=dev(), dtype=torch.int64)
    t2 = torch.full((M,), -1, device=dev(), dtype=torch.int64)
    _lib.linear_frag(xf, wf, M, V, K, logits, flags=_lib.LINEAR_RMS, rms_eps=1e-6, tokens=t1, workspace=ws)
    _lib.linear_frag(xf, wf, M, V, K, None, flags=_lib.LINEAR_RMS, rms_eps=1e-6, tokens=t2, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(t1, torch.argmax(logits, dim=-1))
    assert torch.equal(t1, t2)
    _close_bf16(logits, _frag_ref(x, w, 1e-6), "lm_head logits")


def test_decode_step_frag_output_equals_strided():
    """The decode kernel's y in the fragment layout holds exactly the values of
    its strided output (same kernel, same arithmetic)."""
    B, H, D = 37, 12, 64
    g = torch.Generator(device=dev()).manual_seed(8)
    q, k, v = (torch.randn(B, H, D, device=dev(), generator=g).to(torch.bfloat16) for _ in range(3))
    lam = torch.full((H,), 0.999, device=dev())
    st = _lib.new_state(B, H, D, dev(), zero=True)
    for t in st:
        t.normal_(generator=g)
    st[3].abs_().add_(1.0)
    y1 = torch.empty(B, H, D, device=dev(), dtype=torch.bfloat16)
    y2 = torch.empty(_lib.frag_rows(B) * H * D, device=dev(), dtype=torch.bfloat16)
    norm = _lib.qk_norm(None, None, 0.125, torch.bfloat16)
    o1, o2 = _lib.new_state(B, H, D, dev()), _lib.new_state(B, H, D, dev())
    _lib.decode_step_qknorm(q, k, v, lam, 1.0, norm, st, o1, y1)
    _lib.decode_step_qknorm(q, k, v, lam, 1.0, norm, st, o2, y2, y_frag=True)
    torch.cuda.synchronize()
    assert torch.equal(_unfrag(y2, _lib.frag_rows(B), H * D)[:B], y1.view(B, H * D))
    assert all(torch.equal(a, b) for a, b in zip(o1, o2))


def test_linear_frag_rejects_bad_arguments():
    x = torch.zeros(32 * 256, device=dev(), dtype=torch.bfloat16)
    w = torch.zeros(64 * 256, device=dev(), dtype=torch.bfloat16)
    y = torch.zeros(32 * 64, device=dev(), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="K must be"):
        _lib.linear_frag(x, w, 32, 64, 128, y)
    with pytest.raises(RuntimeError, match="overlaps"):
        _lib.linear_frag(x, w, 32, 64, 256, x, flags=_lib.LINEAR_OUT_FRAG)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.linear_frag(x, w, 32, 64, 256, y, tokens=torch.zeros(32, device=dev(), dtype=torch.int64))
