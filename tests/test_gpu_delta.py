"""GPU parity of the delta-rule PRIME kernels (prime_delta_prefill,
prime_delta_decode_step) against the oracle restatement of
chunked_delta_prime.py:73-283 (oracle/prime_oracle.c: oracle_delta_features,
oracle_delta_chunked, oracle_delta_step)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib

from gpu_util import TOL_BF16, TOL_F32, assert_close, dev, to_dev, to_np

pytestmark = pytest.mark.gpu

D = 64
FEAT_EPS = 1e-5


def _inputs(B, H, L, seed, Hkv=None, bf16=True, beta_scale=0.5):
    Hkv = Hkv or H
    q, _, _ = O.make_inputs((B, H, L, D), seed=seed, bf16=bf16)
    _, k, v = O.make_inputs((B, Hkv, L, D), seed=seed + 1, bf16=bf16)
    rng = np.random.default_rng(seed)
    beta = (beta_scale / (1 + np.exp(-rng.standard_normal((B, H, L))))).astype(np.float32)
    alpha = rng.uniform(0.95, 0.999, (B, H, L)).astype(np.float32)
    return q, k, v, beta, alpha


def _oracle(q, k, v, beta, alpha, decay_pad, bound, state=None):
    B, H, L, _ = q.shape
    grp = H // k.shape[1]
    ke, ve = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    BH = B * H
    psi, phi = O.delta_features(q.reshape(BH, L, D), ke.reshape(BH, L, D), eps=FEAT_EPS)
    return O.delta_chunked(psi, phi, ve.reshape(BH, L, D), beta.reshape(BH, L), alpha.reshape(BH, L),
                           decay_pad, bound=bound, chunk=64, state=state)


def _run(q, k, v, beta, alpha, decay_pad, bound, state=None, dt=torch.bfloat16, workspace=None, inplace=False):
    B, H, L, _ = q.shape
    y = torch.empty(B, H, L, D, device=dev())
    s_in = None if state is None else to_dev(state.reshape(B, H, D, 2 * D))
    s_out = s_in if (inplace and s_in is not None) else torch.empty(B, H, D, 2 * D, device=dev())
    _lib.delta_prefill(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), to_dev(beta), to_dev(alpha), decay_pad,
                       FEAT_EPS, bound, s_in, y, s_out, workspace=workspace)
    torch.cuda.synchronize()
    return to_np(y).reshape(B * H, L, D), to_np(s_out).reshape(B * H, D, 2 * D)


@pytest.mark.parametrize("L", [1, 13, 64, 200, 700])
@pytest.mark.parametrize("with_state", [False, True])
def test_delta_prefill_matches_oracle(L, with_state):
    B, H = 2, 3
    q, k, v, beta, alpha = _inputs(B, H, L, seed=50 + L)
    st = np.random.default_rng(51).standard_normal((B * H, D, 2 * D)) * 0.05 if with_state else None
    yo, so = _oracle(q, k, v, beta, alpha, 0.995, 25.0, st)
    y, s = _run(q, k, v, beta, alpha, 0.995, 25.0, st)
    assert_close(y, yo, TOL_BF16, "y")
    assert_close(s, so, TOL_BF16, "S")


def test_delta_prefill_clamp_active_and_gqa():
    """A small Lyapunov bound clamps every chunk; k/v shared by head pairs."""
    B, H, L = 1, 4, 300
    q, k, v, beta, alpha = _inputs(B, H, L, seed=60, Hkv=2, beta_scale=1.0)
    yo, so = _oracle(q, k, v, beta, alpha, 0.99, 0.5)
    nrm = np.sqrt((so ** 2).sum(axis=(1, 2)))
    assert np.all(nrm <= 0.5 + 1e-6) and np.all(nrm > 0.49)  # the clamp is active in the oracle
    y, s = _run(q, k, v, beta, alpha, 0.99, 0.5)
    assert_close(y, yo, TOL_BF16, "y")
    assert_close(s, so, TOL_BF16, "S")


def test_delta_prefill_without_clamp_equals_tokenwise():
    """bound <= 0: the chunked form is the per-token gated delta rule with the
    decay applied before the prediction (decay^pad on the final state)."""
    B, H, L = 1, 2, 150
    q, k, v, beta, alpha = _inputs(B, H, L, seed=61)
    y, s = _run(q, k, v, beta, alpha, 0.99, 0.0)
    BH = B * H
    psi, phi = O.delta_features(q.reshape(BH, L, D), k.reshape(BH, L, D), eps=FEAT_EPS)
    yt, stk = O.delta_tokenwise(psi, phi, v.reshape(BH, L, D), beta.reshape(BH, L), alpha.reshape(BH, L))
    pad = (64 - L % 64) % 64
    assert_close(y, yt, TOL_BF16, "y")
    assert_close(s, stk * 0.99 ** pad, TOL_BF16, "S")


@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("ws_chunks", [1, 4])
def test_delta_prefill_windows_agree(with_state, ws_chunks):
    """Workspaces for one chunk (one-chunk windows in order) and for four
    chunks (two-chunk windows whose prep runs on the side stream, overlapped
    with the previous window's scan), the state carried between windows
    through the workspace and updated in place, give the one-window result."""
    B, H, L = 1, 2, 64 * 5 + 17
    q, k, v, beta, alpha = _inputs(B, H, L, seed=62)
    st = np.random.default_rng(63).standard_normal((B * H, D, 2 * D)) * 0.05 if with_state else None
    y1, s1 = _run(q, k, v, beta, alpha, 0.995, 25.0, st)
    small = torch.empty(_lib.delta_workspace_size(B, H, 64 * ws_chunks), dtype=torch.uint8, device=dev())
    y2, s2 = _run(q, k, v, beta, alpha, 0.995, 25.0, st, workspace=small, inplace=True)
    assert_close(y2, y1, 1e-5, "y")
    assert_close(s2, s1, 1e-5, "S")


@pytest.mark.parametrize("L", [1, 64, 130, 700])
@pytest.mark.parametrize("with_state", [False, True])
def test_delta_prefill_f32_inputs(L, with_state):
    """fp32 inputs take the fp32 path (fp32 MFMA operands and records): the
    fp32 tolerance applies."""
    B, H = 2, 3
    q, k, v, beta, alpha = _inputs(B, H, L, seed=64 + L, bf16=False)
    st = np.random.default_rng(65).standard_normal((B * H, D, 2 * D)) * 0.05 if with_state else None
    yo, so = _oracle(q, k, v, beta, alpha, 0.995, 25.0, st)
    y, s = _run(q, k, v, beta, alpha, 0.995, 25.0, st, dt=torch.float32)
    assert_close(y, yo, TOL_F32, "y")
    assert_close(s, so, TOL_F32, "S")


def test_delta_prefill_f32_clamp_active_and_gqa():
    B, H, L = 1, 4, 300
    q, k, v, beta, alpha = _inputs(B, H, L, seed=66, Hkv=2, beta_scale=1.0, bf16=False)
    yo, so = _oracle(q, k, v, beta, alpha, 0.99, 0.5)
    nrm = np.sqrt((so ** 2).sum(axis=(1, 2)))
    assert np.all(nrm <= 0.5 + 1e-6) and np.all(nrm > 0.49)
    y, s = _run(q, k, v, beta, alpha, 0.99, 0.5, dt=torch.float32)
    assert_close(y, yo, TOL_F32, "y")
    assert_close(s, so, TOL_F32, "S")


def test_delta_prefill_f32_long_sequence_and_bf16_output():
    """64 chunks of fp32 inputs, y written as bf16 (the state stays fp32)."""
    B, H, L = 1, 2, 4096
    q, k, v, beta, alpha = _inputs(B, H, L, seed=67, beta_scale=1.0, bf16=False)
    yo, so = _oracle(q, k, v, beta, alpha, 0.995, 25.0)
    y = torch.empty(B, H, L, D, device=dev(), dtype=torch.bfloat16)
    s = torch.empty(B, H, D, 2 * D, device=dev())
    _lib.delta_prefill(to_dev(q), to_dev(k), to_dev(v), to_dev(beta), to_dev(alpha), 0.995, FEAT_EPS, 25.0,
                       None, y, s)
    torch.cuda.synchronize()
    assert_close(to_np(s).reshape(B * H, D, 2 * D), so, TOL_F32, "S")
    assert_close(to_np(y).reshape(B * H, L, D), yo, 4e-3, "y (bf16 output)")


@pytest.mark.parametrize("ws_chunks", [1, 4])
def test_delta_prefill_f32_windows_agree(ws_chunks):
    """fp32 records in workspaces of one and four chunks (the latter double
    buffered on the side stream) give the one-window result."""
    B, H, L = 1, 2, 64 * 5 + 17
    q, k, v, beta, alpha = _inputs(B, H, L, seed=68, bf16=False)
    st = np.random.default_rng(69).standard_normal((B * H, D, 2 * D)) * 0.05
    y1, s1 = _run(q, k, v, beta, alpha, 0.995, 25.0, st, dt=torch.float32)
    small = torch.empty(_lib.delta_workspace_size(B, H, 64 * ws_chunks, torch.float32), dtype=torch.uint8,
                        device=dev())
    y2, s2 = _run(q, k, v, beta, alpha, 0.995, 25.0, st, dt=torch.float32, workspace=small, inplace=True)
    assert_close(y2, y1, 1e-6, "y")
    assert_close(s2, s1, 1e-6, "S")


def test_delta_prefill_f32_rejects_bf16_sized_workspace():
    """A workspace sized for one bf16 chunk holds no fp32 record: the call fails
    with an error naming the flag, before any launch."""
    B, H, L = 1, 2, 64
    q, k, v, beta, alpha = _inputs(B, H, L, seed=70, bf16=False)
    ws = torch.empty(_lib.delta_workspace_size(B, H, 64), dtype=torch.uint8, device=dev())
    with pytest.raises(RuntimeError, match="PRIME_FLAG_F32_INPUTS"):
        _run(q, k, v, beta, alpha, 0.995, 25.0, dt=torch.float32, workspace=ws)


def test_delta_prefill_long_sequence_subset():
    """4096 tokens (64 chunks, two windows of the default size would need more):
    the scan stays within tolerance over many chunks and the state stays bounded."""
    B, H, L = 1, 2, 4096
    q, k, v, beta, alpha = _inputs(B, H, L, seed=65, beta_scale=1.0)
    yo, so = _oracle(q, k, v, beta, alpha, 0.995, 25.0)
    y, s = _run(q, k, v, beta, alpha, 0.995, 25.0)
    assert np.isfinite(y).all() and np.isfinite(s).all()
    assert_close(y, yo, TOL_BF16, "y")
    assert_close(s, so, TOL_BF16, "S")


def test_delta_prefill_concurrent_calls_on_two_streams():
    """Two prime_delta_prefill calls enqueued at the same time from two host
    threads, each on its own stream with a four-chunk workspace (so both run
    the double-buffered path, prep on a side stream overlapped with the scan),
    three times each: every result equals the one-window result of the same
    inputs.  The calls share no side stream or event (one set per caller
    stream, its lock held across the whole enqueue sequence)."""
    import threading
    B, H, L = 1, 2, 64 * 21 + 9
    cases = [_inputs(B, H, L, seed=95 + i) for i in range(2)]
    refs = [_run(*c, 0.995, 25.0) for c in cases]
    results = [[], []]
    errors = []
    start = threading.Barrier(2)

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                q, k, v, beta, alpha = cases[i]
                ins = (to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16), to_dev(beta),
                       to_dev(alpha))
                ws = torch.empty(_lib.delta_workspace_size(B, H, 64 * 4), dtype=torch.uint8, device=dev())
                outs = [(torch.empty(B, H, L, D, device=dev()), torch.empty(B, H, D, 2 * D, device=dev()))
                        for _ in range(3)]
                s.synchronize()
                start.wait()
                for y, st in outs:
                    _lib.delta_prefill(*ins, 0.995, FEAT_EPS, 25.0, None, y, st, workspace=ws)
                s.synchronize()
            results[i] = [(to_np(y).reshape(B * H, L, D), to_np(st).reshape(B * H, D, 2 * D)) for y, st in outs]
        except Exception as exc:  # reported by the main thread
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    for i in range(2):
        assert len(results[i]) == 3
        for y, st in results[i]:
            assert_close(y, refs[i][0], 1e-5, f"call {i} y")
            assert_close(st, refs[i][1], 1e-5, f"call {i} S")


@pytest.mark.parametrize("bound", [25.0, 0.3])
def test_delta_decode_step_matches_oracle(bound):
    B, H = 3, 4
    q, _, _ = O.make_inputs((B, H, D), seed=70)
    _, k, v = O.make_inputs((B, H, D), seed=71)
    rng = np.random.default_rng(72)
    beta = rng.uniform(0.1, 0.5, (B, H)).astype(np.float32)
    alpha = rng.uniform(0.9, 0.999, (B, H)).astype(np.float32)
    st = rng.standard_normal((B * H, D, 2 * D)) * 0.05
    BH = B * H
    psi, phi = O.delta_features(q.reshape(BH, 1, D), k.reshape(BH, 1, D), eps=FEAT_EPS)
    yo, so = O.delta_step(psi[:, 0], phi[:, 0], v.reshape(BH, D), beta.reshape(BH), alpha.reshape(BH),
                          bound=bound, state=st)
    s = to_dev(st.reshape(B, H, D, 2 * D))
    y = torch.empty(B, H, D, device=dev())
    _lib.delta_decode_step(to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16),
                           to_dev(beta), to_dev(alpha), FEAT_EPS, bound, s, s, y)  # in place
    torch.cuda.synchronize()
    assert_close(to_np(y).reshape(BH, D), yo, 1e-4, "y")
    assert_close(to_np(s).reshape(BH, D, 2 * D), so, 1e-4, "S")


def _module_ref(mod, x, state=None):
    """fp64 CPU composition of the module (chunked_delta_prime.py:89-283):
    torch layers for projections, gates and LayerNorm, the oracle for the core."""
    import torch.nn.functional as F
    W = {k: v.detach().double().cpu() for k, v in mod.state_dict().items()}
    xd = x.detach().double().cpu()
    B, L, _ = xd.shape
    H, Dh = mod.num_heads, mod.head_dim
    proj = lambda n: (xd @ W[n + ".weight"].T + (W[n + ".bias"] if n + ".bias" in W else 0))
    q = proj("q_proj").view(B, L, H, Dh).transpose(1, 2)
    k = proj("k_proj").view(B, L, H, Dh).transpose(1, 2)
    v = proj("v_proj").view(B, L, H, Dh).transpose(1, 2)
    bg = torch.sigmoid(proj("erase_proj")).view(B, L, H, Dh).transpose(1, 2)
    wg = torch.sigmoid(proj("write_proj")).view(B, L, H, Dh).transpose(1, 2)
    q = F.layer_norm(q, (Dh,), W["q_norm.weight"], W["q_norm.bias"]) / 8.0
    k = F.layer_norm(k, (Dh,), W["k_norm.weight"], W["k_norm.bias"])
    beta = (wg.mean(-1) * 0.5).numpy()
    alpha = (mod.decay * (1.0 - bg.mean(-1) * 0.5)).numpy()
    BH = B * H
    psi, phi = O.delta_features(q.reshape(BH, L, Dh).numpy(), k.reshape(BH, L, Dh).numpy(), eps=mod.eps)
    if L == 1:
        y, S = O.delta_step(psi[:, 0], phi[:, 0], v.reshape(BH, Dh).numpy(), beta.reshape(BH), alpha.reshape(BH),
                            bound=mod.lyapunov_bound, state=state)
        y = y[:, None]
    else:
        y, S = O.delta_chunked(psi, phi, v.reshape(BH, L, Dh).numpy(), beta.reshape(BH, L), alpha.reshape(BH, L),
                               mod.decay, bound=mod.lyapunov_bound, chunk=64, state=state)
    y = torch.from_numpy(y).view(B, H, L, Dh).transpose(1, 2).reshape(B, L, H * Dh)
    return (y @ W["o_proj.weight"].T).numpy(), S


def test_delta_module_prefill_then_step_matches_composition():
    """The module's chunked (L = 100) and step (L = 1) branches against the fp64
    composition of the same weights, the step continuing the prefill state."""
    from prime_moment_attention import ChunkedGatedDeltaPrimeAttention
    torch.manual_seed(0)
    mod = ChunkedGatedDeltaPrimeAttention(128, 2, 64, decay=0.99).to(dev())
    x = torch.randn(2, 101, 128, device=dev())
    with torch.no_grad():
        out, st = mod(x[:, :100], return_state=True)
        out1, st1 = mod(x[:, 100:], state=st, return_state=True)
    ref, S = _module_ref(mod, x[:, :100])
    assert_close(to_np(out), ref, TOL_BF16, "prefill out")
    assert_close(to_np(st).reshape(S.shape), S, TOL_BF16, "prefill state")
    ref1, S1 = _module_ref(mod, x[:, 100:], state=S)
    assert_close(to_np(out1), ref1, TOL_BF16, "step out")
    assert_close(to_np(st1).reshape(S1.shape), S1, TOL_BF16, "step state")
