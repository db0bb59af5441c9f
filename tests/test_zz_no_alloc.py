"""GPU test of prime_accumulate_noalloc, the variant of prime_accumulate that
allocates nothing (its segment slots live in the library's fixed device
scratch).  Two calls in a row through the C-ABI, the second smaller, each
against prime_accumulate with a workspace of the recommended size (same
segment plan, so the states must be bit-identical) and against the oracle
recurrence's final state (the bf16-input tolerance)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from prime_moment_attention import _lib

from gpu_util import TOL_BF16, assert_state_close, dev, random_state, state_to_dev, state_to_np, to_dev

pytestmark = pytest.mark.gpu

D = 64


def _case(B, H, Hkv, L, seed, with_state):
    BH = B * H
    _, k, v = O.make_inputs((B, Hkv, L, D), seed=seed, bf16=True)
    lam = np.random.default_rng(seed + 1).uniform(0.99, 0.9999, H).astype(np.float32)
    st0 = random_state(BH, D, seed + 2) if with_state else None
    grp = H // Hkv
    kr = np.repeat(k, grp, axis=1).reshape(BH, L, D)
    vr = np.repeat(v, grp, axis=1).reshape(BH, L, D)
    # the final state of the recurrence over these tokens (q does not enter it)
    _, ref = O.recurrent(np.zeros_like(kr), kr, vr, np.tile(lam.astype(np.float64), B), state=st0)
    return (to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16), to_dev(lam),
            state_to_dev(st0, B, H, D) if with_state else None, ref)


def test_accumulate_noalloc_matches_accumulate_on_two_calls():
    assert _lib.accumulate_workspace_size(4, 12, 3000) <= _lib.NOALLOC_SCRATCH_BYTES
    cases = [(4, 12, 12, 3000, 700, False), (2, 3, 1, 500, 710, True)]  # the second smaller, GQA, in place
    for B, H, Hkv, L, seed, with_state in cases:
        print(f"[no-alloc] B={B} H={H} Hkv={Hkv} L={L} state={with_state}", flush=True)
        k, v, lam, st0, ref = _case(B, H, Hkv, L, seed, with_state)
        # the existing entry point, recommended workspace
        out_ref = _lib.new_state(B, H, D, dev())
        _lib.accumulate(k, v, lam, st0, out_ref, H=H)
        # the no-allocation entry point; with a state it updates that state in place
        if with_state:
            out = tuple(t.clone() for t in st0)
            _lib.accumulate_noalloc(k, v, lam, out, out, H=H)
        else:
            out = _lib.new_state(B, H, D, dev())
            _lib.accumulate_noalloc(k, v, lam, None, out, H=H)
        torch.cuda.synchronize()
        for a, b, n in zip(out, out_ref, ("S0", "S1", "S2", "K0", "K1", "K2")):
            assert torch.equal(a, b), f"{n}: no-alloc differs from prime_accumulate"
        assert_state_close(state_to_np(out, B * H, D), ref, TOL_BF16, "no-alloc accumulate")


def test_accumulate_noalloc_refuses_too_many_sequences():
    k = torch.zeros(1, 993, 64, D, device=dev(), dtype=torch.bfloat16)
    lam = torch.full((993,), 0.99, device=dev())
    out = _lib.new_state(1, 993, D, dev())
    with pytest.raises(RuntimeError, match="scratch"):
        _lib.accumulate_noalloc(k, k, lam, None, out)
