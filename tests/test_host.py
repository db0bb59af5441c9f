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


@pytest.mark.parametrize("config_as_dict", [False, True])
def test_base_to_selective_warm_start(tmp_path, config_as_dict):
    """from_pretrained_base_to_selective (model.py:269-310): a base checkpoint
    warm-starts a selective model that keeps every pretrained tensor; only
    the selective parameters are new, at their identity initialisation; the
    checkpoint is read without unpickling anything but PrimeConfig."""
    import dataclasses
    from prime_moment_attention import PrimeConfig, PrimeForCausalLM
    cfg = PrimeConfig(vocab_size=96, hidden_size=128, num_layers=2, num_heads=2, head_dim=64, decay=0.99)
    torch.manual_seed(0)
    base = PrimeForCausalLM(cfg)
    path = tmp_path / "base.pt"
    torch.save({"config": dataclasses.asdict(cfg) if config_as_dict else cfg,
                "model_state_dict": base.state_dict()}, path)
    sel = PrimeForCausalLM.from_pretrained_base_to_selective(str(path))
    assert sel.config.use_selective and sel.config.decay == 0.99
    sd_b, sd_s = base.state_dict(), sel.state_dict()
    for k, v in sd_b.items():
        assert torch.equal(sd_s[k], v), k
    new = set(sd_s) - set(sd_b)
    assert new and all(k.split(".")[-2] in ("delta_proj",) or k.endswith(("log_tau", "log_beta")) for k in new), new
    for layer in sel.layers:
        at = layer.self_attn
        assert not at.delta_proj.weight.any()
        lam = torch.exp(-torch.nn.functional.softplus(at.delta_proj.bias) / at.get_tau(at.log_tau.device))
        assert torch.allclose(lam, torch.full_like(lam, 0.99), rtol=1e-5)
        assert torch.equal(at.get_beta(at.log_beta.device), torch.ones_like(at.log_beta))


def test_base_to_selective_needs_a_config(tmp_path):
    from prime_moment_attention import PrimeForCausalLM
    path = tmp_path / "noconf.pt"
    torch.save({"model_state_dict": {}}, path)
    with pytest.raises(ValueError, match="no saved config"):
        PrimeForCausalLM.from_pretrained_base_to_selective(str(path))


def test_stacked_qkv_cache_follows_weights_and_modes():
    """The attention module's stacked q/k/v copy (one inference GEMM instead
    of three, attention.py:83-85): rebuilt after an in-place weight update and
    outside inference_mode when it was made inside it, absent while autograd
    records through the weights; host logic only (no kernel runs)."""
    from prime_moment_attention.attention import PrimeMomentAttention, _stacked_qkv
    m = PrimeMomentAttention(64, 2, 32, num_kv_heads=1)
    assert _stacked_qkv(m) is None  # weights require grad, grad mode on
    with torch.no_grad():
        w = _stacked_qkv(m)
        assert w.shape == (64 + 2 * 32, 64) and _stacked_qkv(m) is w
        assert torch.equal(w, torch.cat([m.q_proj.weight, m.k_proj.weight, m.v_proj.weight]))
        m.v_proj.weight.mul_(2.0)
        w2 = _stacked_qkv(m)
        assert w2 is not w and torch.equal(w2[96:], m.v_proj.weight)
    with torch.inference_mode():
        assert _stacked_qkv(m) is w2  # an ordinary tensor serves inference_mode too
        del m.__dict__["_qkv_cache"]
        wi = _stacked_qkv(m)
        assert wi.is_inference() and _stacked_qkv(m) is wi
    for p in m.parameters():
        p.requires_grad_(False)
    wo = _stacked_qkv(m)  # grad mode on, frozen weights: usable, not an inference tensor
    assert wo is not None and not wo.is_inference()
    m.k_proj.bias = torch.nn.Parameter(torch.zeros(32), requires_grad=False)
    with torch.no_grad():
        assert _stacked_qkv(m) is None  # a bias: the three projections run


def test_selective_gate_constants_follow_parameters():
    """The selective module's cached tau and beta (fp32 [H] for the kernels;
    selective.py:367-368): the module's own get_tau / get_beta values, rebuilt
    after an in-place update of log_tau or log_beta; host logic only."""
    from prime_moment_attention import PrimeSelectiveMomentAttention
    m = PrimeSelectiveMomentAttention(hidden_size=64, num_heads=4, head_dim=16)
    tau, beta = m._gate_constants(torch.device("cpu"))
    assert torch.equal(tau, m.get_tau(torch.device("cpu")).float()) and tau.dtype == torch.float32
    assert torch.equal(beta, m.get_beta(torch.device("cpu")).float())
    assert m._gate_constants(torch.device("cpu"))[0] is tau
    with torch.no_grad():
        m.log_tau.add_(0.5)
        m.log_beta.sub_(0.25)
    tau2, beta2 = m._gate_constants(torch.device("cpu"))
    assert tau2 is not tau and torch.equal(tau2, m.get_tau(torch.device("cpu")).float())
    assert torch.equal(beta2, m.get_beta(torch.device("cpu")).float())
    assert not tau2.requires_grad
