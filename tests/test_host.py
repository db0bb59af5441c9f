"""CPU tests of host-side logic that needs no GPU: PrimeMomentCache's
container semantics (the reference's tests/test_cache.py:6-33) and the
argument checks the Python layer makes before any kernel call."""
import pytest
import torch

from prime_moment_attention import PrimeMomentCache
from prime_moment_attention.chunked_ssd import prime_prefill


def test_cache_set_get_identity():
    """tests/test_cache.py:6-25: a stored 6-tuple comes back as the same
    tensors."""
    cache = PrimeMomentCache()
    assert cache.get_state(0) is None
    B, H, D = 2, 4, 32
    state = (torch.randn(B, H, D), torch.randn(B, H, D, D), torch.randn(B, H, D, D), torch.randn(B, H, 1),
             torch.randn(B, H, D), torch.randn(B, H, D))
    cache.set_state(layer_idx=0, state=state)
    got = cache.get_state(layer_idx=0)
    assert got is not None and len(got) == 6
    assert all(a is b for a, b in zip(got, state))
    assert torch.equal(got[0], state[0])
    assert cache.state_bytes() == sum(t.numel() * 4 for t in state)


def test_cache_reset():
    """tests/test_cache.py:27-33."""
    cache = PrimeMomentCache()
    cache.set_state(layer_idx=1, state=tuple(torch.zeros(1) for _ in range(6)))
    assert cache.get_state(1) is not None
    cache.update(torch.zeros(1, 1, 5, 8), torch.zeros(1, 1, 5, 8), 0)
    assert cache.get_seq_length() == 5
    cache.reset()
    assert cache.get_state(1) is None
    assert cache.get_seq_length() == 0


def test_cache_update_counts_layer0_only():
    """update() keeps no history: it returns its inputs and counts the tokens
    of layer 0 only (cache.py:36-46)."""
    cache = PrimeMomentCache()
    k, v = torch.zeros(2, 3, 7, 16), torch.ones(2, 3, 7, 16)
    for layer in range(4):
        rk, rv = cache.update(k, v, layer)
        assert rk is k and rv is v
    assert cache.get_seq_length() == 7
    assert cache.get_max_length() is None and cache.get_max_cache_shape() is None


def test_cache_is_a_transformers_cache():
    transformers = pytest.importorskip("transformers")
    from transformers.cache_utils import Cache
    assert isinstance(PrimeMomentCache(), Cache)
    del transformers


def test_learnable_decay_refused_under_autograd():
    """A per-head decay tensor that requires grad would train without a
    gradient (the kernels give none in decay): refused before any launch."""
    q = torch.zeros(1, 2, 8, 64)
    decay = torch.nn.Parameter(torch.full((2,), 0.99))
    with pytest.raises(NotImplementedError, match="decay"):
        prime_prefill(q, q, q, decay=decay)
