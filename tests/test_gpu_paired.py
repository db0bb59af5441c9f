"""GPU parity of the paired split of the bf16 prefill (more sequences than CUs:
some sequences run as two workgroups, the second starting from the first's
end state handed over through the workspace).  The split must not change a
single bit against one workgroup per sequence (no workspace): the hand-off
carries the exact fp32 state.  Shapes are the PRIME-125M prefill's (B=32 x
H=12 = 384 sequences of 2048 tokens, model.py:163-181 calling
attention.py:145-158) and ragged / GQA / selective / QK-norm variants."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib

from gpu_util import TOL_BF16, assert_close, assert_state_close, dev, random_state, state_to_dev, state_to_np, to_np

pytestmark = pytest.mark.gpu

D = 64
NO_WS = None  # set per call: an empty tensor forces one workgroup per sequence


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _inputs(B, H, Hkv, L, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda h: torch.nn.functional.normalize(torch.randn(B, h, L, D, generator=g), dim=-1).to(dev(), torch.bfloat16)
    return mk(H), mk(Hkv), mk(Hkv)


def _run_base(q, k, v, lam, st_in, workspace, y_dtype=torch.float32, qk_norm=None):
    B, H, L, _ = q.shape
    y = torch.empty(B, H, L, D, device=dev(), dtype=y_dtype)
    st = _lib.new_state(B, H, D, dev())
    _lib.chunked_prefill(q, k, v, lam, 1.0, 64, st_in, y, st, 0, workspace=workspace, qk_norm=qk_norm)
    torch.cuda.synchronize()
    return y, st


def _same(a, b, what):
    ya, sa = a
    yb, sb = b
    assert torch.equal(ya, yb), f"{what}: y differs, max |d| {(ya.float() - yb.float()).abs().max().item():.3e}"
    for i, (x, z) in enumerate(zip(sa, sb)):
        assert torch.equal(x, z), f"{what}: state component {i} differs"


def _need_pairs(B, H, L):
    if B * H <= _cus():
        pytest.skip(f"{B * H} sequences do not exceed the {_cus()} CUs")
    nbytes = _lib.workspace_size(B, H, L)
    assert nbytes > 0, "the paired split should be planned for more sequences than CUs"
    return nbytes


@pytest.mark.parametrize("B,H,Hkv,L,with_state", [(32, 12, 12, 2048, False), (32, 12, 12, 2048, True),
                                                  (25, 12, 4, 64 * 19 + 37, True)])
def test_paired_split_bit_identical_to_one_workgroup(B, H, Hkv, L, with_state):
    _need_pairs(B, H, L)
    q, k, v = _inputs(B, H, Hkv, L, seed=B + L)
    lam = torch.from_numpy(np.random.default_rng(L).uniform(0.99, 0.9999, H).astype(np.float32)).to(dev())
    st_in = state_to_dev(random_state(B * H, D, 5), B, H, D) if with_state else None
    paired = _run_base(q, k, v, lam, st_in, None)
    whole = _run_base(q, k, v, lam, st_in, torch.empty(0, dtype=torch.uint8, device=dev()))
    _same(paired, whole, "paired vs one workgroup")
    # a second paired call on a reused workspace (flags consumed and reset)
    ws = torch.empty(_lib.workspace_size(B, H, L), dtype=torch.uint8, device=dev())
    for _ in range(2):
        _same(_run_base(q, k, v, lam, st_in, ws), whole, "paired, reused workspace")
    # the oracle on the first (paired) and the last (whole) sequences
    grp = H // Hkv
    sel = [0, 1, B * H - 1]
    qn, kn, vn = (to_np(x) for x in (q, k.repeat_interleave(grp, 1), v.repeat_interleave(grp, 1)))
    pick = lambda x: x.reshape(B * H, L, D)[sel]
    lam_bh = np.tile(lam.cpu().numpy().astype(np.float64), B)[sel]
    st0 = None if st_in is None else tuple(s[sel] for s in state_to_np(st_in, B * H, D))
    yo, so = O.chunked(pick(qn), pick(kn), pick(vn), lam_bh, eps=1.0, chunk=64, state=st0)
    assert_close(to_np(paired[0]).reshape(B * H, L, D)[sel], yo, TOL_BF16, "y vs oracle")
    assert_state_close(tuple(s[sel] for s in state_to_np(paired[1], B * H, D)), so, TOL_BF16, "paired")


def test_paired_split_qknorm_and_bf16_y():
    """The model's form: raw projections normalised on load, bf16 y."""
    B, H, L = 32, 12, 2048
    _need_pairs(B, H, L)
    q, k, v = _inputs(B, H, H, L, seed=3)
    g = torch.Generator().manual_seed(4)
    lns = []
    for _ in range(2):
        ln = torch.nn.LayerNorm(D)
        with torch.no_grad():
            ln.weight.copy_(1 + 0.3 * torch.randn(D, generator=g))
            ln.bias.copy_(0.2 * torch.randn(D, generator=g))
        lns.append(ln.to(device=dev(), dtype=torch.bfloat16))
    norm = _lib.qk_norm(lns[0], lns[1], D ** -0.5, torch.bfloat16)
    lam = torch.full((H,), 0.9995, device=dev())
    paired = _run_base(q, k, v, lam, None, None, torch.bfloat16, norm)
    whole = _run_base(q, k, v, lam, None, torch.empty(0, dtype=torch.uint8, device=dev()), torch.bfloat16, norm)
    _same(paired, whole, "QK-norm paired vs one workgroup")


def test_paired_split_selective():
    B, H, L = 32, 12, 1024 + 5
    _need_pairs(B, H, L)
    q, k, v = _inputs(B, H, H, L, seed=9)
    g = torch.Generator().manual_seed(10)
    ld = (-torch.rand(B, H, L, generator=g) * 0.02).to(dev())
    beta = (0.5 + torch.rand(H, generator=g)).to(dev())
    outs = []
    for ws in (None, torch.empty(0, dtype=torch.uint8, device=dev())):
        y = torch.empty(B, H, L, D, device=dev())
        st = _lib.new_state(B, H, D, dev())
        _lib.selective_prefill(q, k, v, ld, beta, 1e-3, None, y, st, workspace=ws)
        torch.cuda.synchronize()
        outs.append((y, st))
    _same(outs[0], outs[1], "selective paired vs one workgroup")


def test_paired_split_graph_replays():
    """A paired prefill captured in a HIP graph: every replay (eager work and
    synchronisations between them) equals the eager call."""
    B, H, L = 32, 12, 512 + 64
    _need_pairs(B, H, L)
    q, k, v = _inputs(B, H, H, L, seed=21)
    lam = torch.full((H,), 0.999, device=dev())
    ref = _run_base(q, k, v, lam, None, torch.empty(0, dtype=torch.uint8, device=dev()))
    ws = torch.empty(_lib.workspace_size(B, H, L), dtype=torch.uint8, device=dev())
    y = torch.empty(B, H, L, D, device=dev())
    st = _lib.new_state(B, H, D, dev())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _lib.chunked_prefill(q, k, v, lam, 1.0, 64, None, y, st, 0, workspace=ws)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.chunked_prefill(q, k, v, lam, 1.0, 64, None, y, st, 0, workspace=ws)
    for i in range(3):
        y.zero_()
        for t in st:
            t.zero_()
        _run_base(q, k, v, lam, None, ws)  # eager paired call between replays, same workspace
        graph.replay()
        torch.cuda.synchronize()
        _same((y, st), ref, f"replay {i}")


@pytest.mark.parametrize("pattern", ["small_ints", "bf16_one", "int64_ids"])
def test_paired_split_leftover_workspace_data(pattern):
    """The hand-off flags sit in a workspace nobody clears: whatever earlier
    tensors left there (small integers, a bf16 run [1, 0, 0, 0] = 0x3F80 as a
    64-bit word, token ids) must not read as the call's hand-off value, so the
    result stays bit-identical to one workgroup per sequence."""
    B, H, L = 32, 12, 512 + 64
    nbytes = _need_pairs(B, H, L)
    q, k, v = _inputs(B, H, H, L, seed=33)
    lam = torch.full((H,), 0.9993, device=dev())
    whole = _run_base(q, k, v, lam, None, torch.empty(0, dtype=torch.uint8, device=dev()))
    words = (nbytes + 7) // 8
    if pattern == "small_ints":
        fill = torch.arange(words, device=dev(), dtype=torch.int64) % 4096
    elif pattern == "bf16_one":
        fill = torch.full((words,), 0x3F80, device=dev(), dtype=torch.int64)
    else:
        fill = torch.randint(0, 50304, (words,), device=dev(), dtype=torch.int64,
                             generator=torch.Generator(device=dev()).manual_seed(5))
    ws8 = torch.empty(words * 8, dtype=torch.uint8, device=dev())
    for _ in range(2):  # the pattern again before a second call on the same workspace
        ws8.view(torch.int64).copy_(fill)
        _same(_run_base(q, k, v, lam, None, ws8[:nbytes]), whole, f"paired over leftover {pattern}")
