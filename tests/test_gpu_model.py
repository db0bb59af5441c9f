"""GPU tests of the PRIME-125M-shaped causal LM host path (model.py:20-242 of the
reference) on the HIP kernels: logits against an fp32 CPU composition of the
same weights (textbook layers + the fp32 PyTorch-CPU restatement of the PRIME
core from oracle/torch_cpu.py), prefill/decode continuity, and the HIP-graph
greedy decoder against eager generation."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import torch_cpu as TC
from prime_moment_attention import GreedyDecoder, PrimeConfig, PrimeForCausalLM

from gpu_util import dev

pytestmark = pytest.mark.gpu

TOL_LOGITS = 3e-2  # max|d| / max|ref| for bf16 weights/activations vs the fp32 composition


def _small(mlp="swiglu", layers=2, heads=2, decay=0.995):
    return PrimeConfig(vocab_size=384, hidden_size=128, num_layers=layers, num_heads=heads, head_dim=64,
                       decay=decay, mlp_type=mlp, intermediate_size=256 if mlp == "gelu" else None)


def _model(cfg, seed=0):
    torch.manual_seed(seed)
    return PrimeForCausalLM(cfg).to(device=dev(), dtype=torch.bfloat16).eval()


def _ref_forward(model, ids, L_threshold=512):
    """fp32 CPU forward of the same weights: model.py:163-199 with the attention
    of attention.py:83-210 (dense below the threshold = chunked without state)."""
    cfg = model.config
    W = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    x = W["embed_tokens.weight"][ids.cpu()]
    B, L = ids.shape
    H, D = cfg.num_heads, cfg.head_dim

    def rms(x, w):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.rms_norm_eps) * w

    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        hN = rms(x, W[p + "input_layernorm.weight"])
        q = (hN @ W[p + "self_attn.q_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
        k = (hN @ W[p + "self_attn.k_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
        v = (hN @ W[p + "self_attn.v_proj.weight"].T).view(B, L, H, D).transpose(1, 2)
        if cfg.use_qk_norm:
            q = F.layer_norm(q, (D,), W[p + "self_attn.q_norm.weight"], W[p + "self_attn.q_norm.bias"])
            k = F.layer_norm(k, (D,), W[p + "self_attn.k_norm.weight"], W[p + "self_attn.k_norm.bias"])
        q = q / math.sqrt(D)
        y, _ = TC.chunked_core(q.contiguous(), k.contiguous(), v.contiguous(), cfg.decay, eps=cfg.eps)
        y = y.transpose(1, 2).reshape(B, L, H * D)
        x = x + y @ W[p + "self_attn.o_proj.weight"].T
        hN = rms(x, W[p + "post_attention_layernorm.weight"])
        if cfg.mlp_type == "gelu":
            m = F.gelu(hN @ W[p + "mlp.up_proj.weight"].T) @ W[p + "mlp.down_proj.weight"].T
        else:
            m = (F.silu(hN @ W[p + "mlp.gate_proj.weight"].T) * (hN @ W[p + "mlp.up_proj.weight"].T)) \
                @ W[p + "mlp.down_proj.weight"].T
        x = x + m
    return rms(x, W["norm.weight"]) @ W["embed_tokens.weight"].T


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).abs().max() / b.abs().max()).item()


@pytest.mark.parametrize("mlp,L", [("swiglu", 70), ("gelu", 600)])
def test_model_logits_match_fp32_composition(mlp, L):
    """Dense branch (L <= 512) and chunked branch (L > 512)."""
    model = _model(_small(mlp))
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, model.config.vocab_size, (2, L), generator=g)
    with torch.no_grad():
        out = model(ids.to(dev()))["logits"]
    ref = _ref_forward(model, ids)
    assert torch.isfinite(out).all()
    assert _rel(out, ref) < TOL_LOGITS, _rel(out, ref)


def test_prefill_then_steps_equal_longer_prefill():
    """States carried by the decode kernel continue the prefill exactly (up to
    bf16 rounding): logits of step-decoded tokens == logits of one long prefill."""
    model = _model(_small())
    ids = torch.randint(0, 384, (2, 45), generator=torch.Generator().manual_seed(2)).to(dev())
    with torch.no_grad():
        full = model(ids)["logits"]
        out = model(ids[:, :40], return_states=True)
        states = out["states"]
        for t in range(40, 45):
            step = model(ids[:, t:t + 1], states=states, return_states=True)
            states = step["states"]
            assert _rel(step["logits"][:, -1], full[:, t]) < TOL_LOGITS


def _gelu_cfg(hidden):
    """GELU-MLP configurations whose one-token step is folded: hidden 128 takes
    the row kernels (prime_linear_fused), hidden 256 the fragment-layout
    kernels (prime_linear_frag, K = 256 and 768)."""
    return PrimeConfig(vocab_size=512, hidden_size=hidden, num_layers=2, num_heads=hidden // 64, head_dim=64,
                       decay=0.995, mlp_type="gelu", intermediate_size=2 * hidden if hidden == 128 else 3 * hidden)


@pytest.mark.parametrize("hidden", [128, 256])
@pytest.mark.parametrize("L0", [40, 600])
def test_folded_gelu_step_matches_fp32_composition(L0, hidden):
    """The folded one-token step the headline decode runs (GELU MLP, bf16:
    each RMSNorm's weight in the next projection's columns, the row scale and
    the GELU / residual add inside the projection kernels; hidden 256: the
    fragment-layout step with the lm_head's own kernel) against the fp32 CPU
    composition of the same weights over the whole sequence, for prompts on the
    dense (L <= 512) and the chunked branch."""
    from prime_moment_attention import model as M
    model = _model(_gelu_cfg(hidden))
    consts = M._step_constants(model)
    assert all(c.folded for c in consts), "the folded step must be taken for this configuration"
    assert M._frag_step_ready(consts) == (hidden == 256)
    ids = torch.randint(0, 512, (3, L0 + 4), generator=torch.Generator().manual_seed(12))
    with torch.no_grad():
        out = model(ids[:, :L0].to(dev()), return_states=True)
        states = out["states"]
        for t in range(L0, L0 + 4):
            step = model(ids[:, t:t + 1].to(dev()), states=states, return_states=True)
            states = step["states"]
            ref = _ref_forward(model, ids[:, :t + 1])[:, -1]
            assert torch.isfinite(step["logits"]).all()
            assert _rel(step["logits"][:, -1], ref) < TOL_LOGITS, (t, _rel(step["logits"][:, -1], ref))


@pytest.mark.parametrize("cfg", ["swiglu", "gelu_frag", "selective_frag"])
def test_greedy_decoder_graph_equals_eager_generate(cfg):
    """Greedy tokens: HIP-graph decoder == eager decoder == generate(temperature=0);
    graph replays are interleaved with eager work and synchronisations, and the
    states stay in place.  For the fragment-layout step the decoder takes the
    lm_head kernel's own argmax while generate takes torch.argmax of its logits."""
    if cfg == "swiglu":
        model = _model(_small(layers=2, heads=2, decay=0.99))
    else:
        c = _gelu_cfg(256)
        c.use_selective = cfg == "selective_frag"
        model = _model(c)
        if c.use_selective:
            with torch.no_grad():
                g = torch.Generator().manual_seed(5)
                for layer in model.layers:
                    layer.self_attn.delta_proj.weight.copy_(torch.randn(layer.self_attn.delta_proj.weight.shape,
                                                                        generator=g) * 0.02)
                    layer.self_attn.log_beta.copy_(torch.rand(layer.self_attn.log_beta.shape, generator=g) - 0.5)
    ids = torch.randint(0, model.config.vocab_size, (3, 30), generator=torch.Generator().manual_seed(3)).to(dev())
    n = 12
    ref = model.generate(ids, max_new_tokens=n, temperature=0.0)
    eager = GreedyDecoder(model, use_graph=False).generate(ids, n)
    dec = GreedyDecoder(model, use_graph=True)
    toks = [dec.prefill(ids).clone()]
    ptrs = [t.data_ptr() for st in dec.states for t in st]
    for i in range(n - 1):
        toks.append(dec.step().clone())
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=dev()).sum().item()  # unrelated eager work between replays
    graph = torch.cat([ids] + toks, dim=-1)
    assert [t.data_ptr() for st in dec.states for t in st] == ptrs
    assert torch.equal(eager, ref), (eager, ref)
    assert torch.equal(graph, ref), (graph, ref)


def test_greedy_decoder_leaves_module_states_functional():
    """Building and running a GreedyDecoder changes no module setting: a later
    model.forward with a saved state still returns new state tensors and leaves
    the passed-in ones untouched (the reference's functional contract,
    attention.py:126-132), so a saved prefix can be branched from."""
    model = _model(_small())
    ids = torch.randint(0, 384, (2, 20), generator=torch.Generator().manual_seed(8)).to(dev())
    with torch.no_grad():
        saved = model(ids, return_states=True)["states"]
        dec = GreedyDecoder(model, use_graph=True)
        dec.prefill(ids)
        for _ in range(3):
            dec.step()
        snap = [tuple(t.clone() for t in st) for st in saved]
        tok = ids[:, -1:]
        a = model(tok, states=saved, return_states=True)
        b = model(tok, states=saved, return_states=True)
    torch.cuda.synchronize()
    for st, sn, new in zip(saved, snap, a["states"]):
        assert all(torch.equal(x, y) for x, y in zip(st, sn))
        assert all(x.data_ptr() != y.data_ptr() for x, y in zip(st, new))
    assert torch.equal(a["logits"], b["logits"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("n,vocab,pad",[(256, 50304, 0), (3, 1000, 0), (5, 50257, 0), (4, 37, 3), (1, 9000, 1)])
def test_argmax_matches_torch(dtype, n, vocab, pad):
    """prime_argmax == torch.argmax (first index of the largest), on padded
    (strided, unaligned) rows and ragged vocabularies."""
    from prime_moment_attention import _lib
    g = torch.Generator(device=dev()).manual_seed(n + vocab)
    full = torch.randn(n, vocab + pad, device=dev(), generator=g).to(dtype)
    x = full[:, :vocab]
    out = torch.empty(n, dtype=torch.int64, device=dev())
    _lib.argmax(x, out)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.argmax(x, dim=-1))


def test_argmax_ties_nan_and_signed_zero():
    from prime_moment_attention import _lib
    x = torch.full((5, 3000), -1.0, device=dev(), dtype=torch.bfloat16)
    x[0, 7] = x[0, 2500] = 3.0            # tie: first index
    x[1, 11] = float("nan"); x[1, 12] = float("inf")  # NaN counts as largest
    x[2, :] = 0.0; x[2, :1000] = -0.0     # -0 == +0: first index (0)
    x[3, 2999] = float("inf")             # last element
    x[4, :] = float("-inf")               # all -inf: index 0
    out = torch.empty(5, dtype=torch.int64, device=dev())
    _lib.argmax(x, out)
    torch.cuda.synchronize()
    assert out.tolist() == [7, 11, 0, 2999, 0]
    assert torch.equal(out, torch.argmax(x, dim=-1))


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 0), (torch.float32, 1e-5)])
@pytest.mark.parametrize("with_ln", [True, False])
def test_head_layernorm_matches_module_ops(dtype, tol, with_ln):
    """prime_head_layernorm in place on the projection layout ([B, L, H, D]
    storage seen as [B, H, L, D]) == nn.LayerNorm then * scale (attention.py:96-101);
    bf16: equal up to one bf16 ulp (the kernel's rsqrt vs torch's)."""
    from prime_moment_attention import _lib
    B, L, H, D = 3, 37, 5, 64
    torch.manual_seed(4)
    ln = torch.nn.LayerNorm(D).to(dev()).to(dtype)
    with torch.no_grad():
        ln.weight.uniform_(0.5, 1.5)
        ln.bias.uniform_(-0.3, 0.3)
    raw = (torch.randn(B, L, H * D, device=dev()) * 3 + 0.5).to(dtype)
    x = raw.view(B, L, H, D).transpose(1, 2)
    with torch.no_grad():
        ref = (ln(x) if with_ln else x) * 0.125
    _lib.head_layernorm(x, x, ln if with_ln else None, 0.125)
    torch.cuda.synchronize()
    d = (x.float() - ref.float()).abs()
    bound = ref.float().abs() * (2 ** -7) + 1e-6 if dtype == torch.bfloat16 else tol * (1 + ref.float().abs())
    assert bool((d <= bound).all()), float(d.max())
    if not with_ln:
        assert torch.equal(x, ref)  # a power-of-two scale is exact


@pytest.mark.parametrize("M,N,K", [(256, 2304, 768), (256, 768, 3072), (3, 100, 64), (37, 3072, 768), (1, 8, 128),
                                   (300, 3000, 64), (256, 3072, 768),
                                   (300, 52, 192)])
@pytest.mark.parametrize("gelu", [False, True])
def test_linear_matches_torch(M, N, K, gelu):
    """prime_linear (skinny bf16 GEMM, fp32 accumulation) == F.linear in fp32
    then the exact GELU, rounded once to bf16; x a strided row view."""
    from prime_moment_attention import _lib
    g = torch.Generator(device=dev()).manual_seed(M * 7 + N + K)
    xb = torch.randn(M, K + 64, device=dev(), generator=g).bfloat16()
    x = xb[:, 32:32 + K]  # row stride K + 64, 64-byte offset
    w = (torch.randn(N, K, device=dev(), generator=g) * K ** -0.5).bfloat16()
    out = torch.full((M, N), float("nan"), device=dev(), dtype=torch.bfloat16)
    _lib.linear(x, w, out, _lib.EPILOGUE_GELU if gelu else _lib.EPILOGUE_NONE)
    torch.cuda.synchronize()
    ref = x.float() @ w.float().T
    if gelu:
        ref = torch.nn.functional.gelu(ref)
    d = (out.float() - ref).abs()
    assert bool((d <= ref.abs() * 2 ** -7 + 1e-3 * ref.abs().max()).all()), float(d.max())


def test_linear_rejects_bad_shapes():
    from prime_moment_attention import _lib
    x = torch.zeros(4, 100, device=dev(), dtype=torch.bfloat16)
    w = torch.zeros(8, 100, device=dev(), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        _lib.linear(x, w, torch.empty(4, 8, device=dev(), dtype=torch.bfloat16))
