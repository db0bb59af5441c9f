"""PrimeForCausalLM: drop-in for the reference's model.py, on the HIP kernels.

Same configuration fields, module tree and parameter names as the reference
(model.py:20-149), so its state dicts load unchanged; the forward contract
``forward(input_ids, labels=None, states=None, return_states=False) -> dict``
and ``generate`` follow model.py:163-242.  Every PRIME attention layer runs the
library's decode step or chunked prefill (PrimeMomentAttention); projections,
norms and the MLP are torch layers (library GEMMs).

Additions for serving:
  * ``PrimeConfig.mlp_type = "gelu"`` selects an up/GELU/down MLP of width
    ``intermediate_size`` (the PRIME-125M benchmark shape); the default
    "swiglu" is the reference's PrimeMLP (model.py:59-68).
  * ``forward(..., logits_to_keep=n)`` computes logits for the last n
    positions only (generation needs one).
  * One token per sequence (the generate loop) runs a fused step: each
    residual add folded into the next RMSNorm (same rounding as the separate
    add), one stacked q/k/v GEMM, the QK-norm and scale inside the decode
    kernel, and the skinny HIP GEMM (exact GELU applied to its fp32
    accumulator) where it beats the library GEMM.  Its rounding differs from
    the blocks' separate torch ops only in those GEMMs.
  * ``GreedyDecoder`` runs that same step with per-layer states updated in
    place, the whole step (embedding, 12 layers, final norm, lm_head, argmax)
    captured in one HIP graph and replayed per token, so its tokens equal
    ``generate``'s at temperature 0.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .attention import PrimeMomentAttention
from .selective import PrimeSelectiveMomentAttention


@dataclass
class PrimeConfig:
    """model.py:20-44, plus ``mlp_type``."""
    vocab_size: int = 32000
    hidden_size: int = 512
    num_layers: int = 6
    num_heads: int = 8
    head_dim: int = 64
    num_kv_heads: Optional[int] = None
    intermediate_size: Optional[int] = None
    decay: float = 0.9995
    use_qk_norm: bool = True
    rms_norm_eps: float = 1e-6
    eps: float = 1.0
    tie_word_embeddings: bool = True
    initializer_range: float = 0.02
    use_selective: bool = False
    min_tau: float = 2.0
    max_tau: float = 2000.0
    mlp_type: str = "swiglu"

    def __post_init__(self):
        if self.num_kv_heads is None:
            self.num_kv_heads = self.num_heads
        if self.intermediate_size is None:
            self.intermediate_size = int(2 * (4 * self.hidden_size) / 3)
        if self.mlp_type not in ("swiglu", "gelu"):
            raise ValueError(f"mlp_type must be 'swiglu' or 'gelu', not {self.mlp_type!r}")


def prime_125m_config(mlp_type: str = "gelu", vocab_size: int = 50304, use_selective: bool = False) -> PrimeConfig:
    """The PRIME-125M benchmark shape: 12 layers, d_model 768, 12 x 64 heads,
    MLP 3072 (GELU) or the reference's SwiGLU width, tied 50304-token vocab;
    use_selective for the selective attention of the shipped PRIME-125M."""
    return PrimeConfig(vocab_size=vocab_size, hidden_size=768, num_layers=12, num_heads=12, head_dim=64,
                       intermediate_size=3072 if mlp_type == "gelu" else None, mlp_type=mlp_type,
                       use_selective=use_selective)


class RMSNorm(nn.Module):
    """model.py:47-56, one HIP kernel (prime_add_rmsnorm): x * rsqrt(mean(x^2)
    + eps) * weight, computed in fp32 and rounded once to x's dtype."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad):
            # training: the reference's ops (model.py:54-56), differentiable
            return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight
        xc = x.contiguous()
        out = torch.empty_like(xc)
        w = self.weight if self.weight.dtype == xc.dtype else self.weight.to(xc.dtype)
        _lib.add_rmsnorm(xc, None, w, out, self.eps)
        return out


class PrimeMLP(nn.Module):
    """SwiGLU feed-forward, model.py:59-68."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class PrimeGeluMLP(nn.Module):
    """up -> GELU -> down feed-forward (the PRIME-125M benchmark's MLP)."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(F.gelu(self.up_proj(x)))


def _mlp_inner(mlp: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """The MLP up to its down projection (inference path): gelu(up x), the
    GELU by prime_gelu in place on the projection (the exact form of nn.GELU,
    the same bits as F.gelu), or silu(gate x) * up x."""
    if isinstance(mlp, PrimeGeluMLP):
        return _lib.gelu(mlp.up_proj(x))
    return F.silu(mlp.gate_proj(x)) * mlp.up_proj(x)


class PrimeBlock(nn.Module):
    """Pre-norm block, model.py:71-118: x + Attn(RMSNorm x); x + MLP(RMSNorm x)."""

    def __init__(self, config: PrimeConfig):
        super().__init__()
        self.input_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        if config.use_selective:
            self.self_attn = PrimeSelectiveMomentAttention(
                hidden_size=config.hidden_size, num_heads=config.num_heads, head_dim=config.head_dim,
                num_kv_heads=config.num_kv_heads, decay=config.decay, use_qk_norm=config.use_qk_norm,
                eps=config.eps, min_tau=config.min_tau, max_tau=config.max_tau)
        else:
            self.self_attn = PrimeMomentAttention(
                hidden_size=config.hidden_size, num_heads=config.num_heads, head_dim=config.head_dim,
                num_kv_heads=config.num_kv_heads, decay=config.decay, use_qk_norm=config.use_qk_norm,
                eps=config.eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        mlp = PrimeGeluMLP if config.mlp_type == "gelu" else PrimeMLP
        self.mlp = mlp(config.hidden_size, config.intermediate_size)

    def forward(self, hidden_states, state=None, return_state=False):
        residual = hidden_states
        h, next_state = self.self_attn(self.input_layernorm(hidden_states), state=state,
                                       return_state=return_state)
        hidden_states = residual + h
        hidden_states = hidden_states + self.mlp(self.post_attention_layernorm(hidden_states))
        return hidden_states, next_state


class PrimeForCausalLM(nn.Module):
    """model.py:121-242 on the HIP attention kernels."""

    def __init__(self, config: PrimeConfig):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([PrimeBlock(config) for _ in range(config.num_layers)])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight
        self.apply(self._init_weights)
        # output projections re-drawn with std / sqrt(2 * layers) (model.py:141-147)
        scale = config.initializer_range / math.sqrt(2 * config.num_layers)
        for layer in self.layers:
            layer.self_attn.o_proj.weight.data.normal_(mean=0.0, std=scale)
            layer.mlp.down_proj.weight.data.normal_(mean=0.0, std=scale)
            if hasattr(layer.self_attn, "init_selective_weights"):  # model.py:148-149
                layer.self_attn.init_selective_weights()

    @classmethod
    def from_pretrained_base_to_selective(cls, checkpoint_path: str,
                                          device: Any = "cpu") -> "PrimeForCausalLM":
        """Identity-preserving warm start of a selective model from a base PRIME
        checkpoint (model.py:269-310): every pretrained tensor (embeddings,
        projections, norms, MLP, lm_head) is kept; the selective parameters the
        checkpoint lacks keep their initialisation (init_selective_weights:
        zero step weights and a step bias that reproduces the base decay, so
        the warm-started model computes the base model at step 0).

        The checkpoint holds "config" (a PrimeConfig or a dict of its fields)
        and "model_state_dict".  It is read with torch.load(weights_only=True),
        PrimeConfig being the only class allowed besides tensors (the
        reference unpickles the whole file)."""
        with torch.serialization.safe_globals([PrimeConfig]):
            ckpt = torch.load(checkpoint_path, map_location=device, weights_only=True)
        base = ckpt.get("config", None)
        if base is None:
            raise ValueError(f"Checkpoint at {checkpoint_path} has no saved config.")
        get = (lambda k, d=None: base.get(k, d)) if isinstance(base, dict) else (lambda k, d=None: getattr(base, k, d))
        sel_config = PrimeConfig(
            vocab_size=get("vocab_size"), hidden_size=get("hidden_size"), num_layers=get("num_layers"),
            num_heads=get("num_heads"), head_dim=get("head_dim"), num_kv_heads=get("num_kv_heads"),
            intermediate_size=get("intermediate_size"), decay=get("decay"), use_qk_norm=get("use_qk_norm"),
            rms_norm_eps=get("rms_norm_eps"), eps=get("eps"), tie_word_embeddings=get("tie_word_embeddings"),
            initializer_range=get("initializer_range"), use_selective=True, mlp_type=get("mlp_type", "swiglu"))
        model = cls(sel_config).to(device)
        sd = ckpt["model_state_dict"]
        missing_keys, unexpected_keys = model.load_state_dict(sd, strict=False)
        print(f"[Selective Warm-Start] Loaded {len(sd)} pretrained tensors from {checkpoint_path}")
        print(f"    Missing keys initialized to identity: {len(missing_keys)}")
        print(f"    Unexpected keys: {len(unexpected_keys)}")
        return model

    def _init_weights(self, module: nn.Module):
        if isinstance(module, (nn.Linear, nn.Embedding)):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)
            if getattr(module, "bias", None) is not None:
                nn.init.zeros_(module.bias)

    def get_input_embeddings(self) -> nn.Embedding:
        return self.embed_tokens

    def set_input_embeddings(self, value: nn.Embedding):
        self.embed_tokens = value

    def forward(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
                states: Optional[List[Tuple[torch.Tensor, ...]]] = None, return_states: bool = False,
                logits_to_keep: int = 0) -> Dict[str, Any]:
        if torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters()):
            return self._forward_graph(input_ids, labels, states, return_states, logits_to_keep)
        if input_ids.shape[-1] == 1 and _fused_step_supported(self):
            # one token per sequence (the generate loop, model.py:238): the fused
            # step GreedyDecoder runs, with functional states
            consts = _step_constants(self)
            if _frag_step_ready(consts):
                logits, ns = _frag_step(self, input_ids, states, consts, inplace=False)
            else:
                logits, ns = _fused_step(self, input_ids, states, consts, inplace=False)
            logits = logits.unsqueeze(1)
            loss = None
            if labels is not None:
                shift_logits = logits[..., :-1, :].contiguous().to(torch.float32)
                loss = F.cross_entropy(shift_logits.view(-1, self.config.vocab_size),
                                       labels[..., 1:].contiguous().view(-1), ignore_index=-100)
            return {"loss": loss, "logits": logits, "states": ns if return_states else None}
        # x is this call's own residual stream, updated in place: each block's
        # output projection and its residual add are one GEMM with beta = 1
        # (x += y W^T, the sum rounded once), followed by the RMSNorm
        # (prime_add_rmsnorm without a delta).
        x = self.embed_tokens(input_ids)
        hidden = x.shape[-1]
        x2 = x.view(-1, hidden)
        next_states = [] if return_states else None
        for i, layer in enumerate(self.layers):
            at = layer.self_attn
            n1 = torch.empty_like(x)
            _lib.add_rmsnorm(x, None, layer.input_layernorm.weight, n1, layer.input_layernorm.eps)
            y, ns = at.mix(n1, state=states[i] if states is not None else None, return_state=return_states)
            x2.addmm_(y.reshape(x2.shape[0], -1), at.o_proj.weight.t())
            n2 = torch.empty_like(x)
            _lib.add_rmsnorm(x, None, layer.post_attention_layernorm.weight, n2, layer.post_attention_layernorm.eps)
            x2.addmm_(_mlp_inner(layer.mlp, n2).reshape(x2.shape[0], -1), layer.mlp.down_proj.weight.t())
            if return_states:
                next_states.append(ns)
        if logits_to_keep:
            x = x[:, -logits_to_keep:].contiguous()
        nf = torch.empty_like(x)
        _lib.add_rmsnorm(x.view(-1, hidden), None, self.norm.weight, nf.view(-1, hidden), self.norm.eps)
        logits = self.lm_head(nf)
        loss = None
        if labels is not None:
            shift_logits = logits[..., :-1, :].contiguous().to(torch.float32)
            loss = F.cross_entropy(shift_logits.view(-1, self.config.vocab_size),
                                   labels[..., 1:].contiguous().view(-1), ignore_index=-100)
        return {"loss": loss, "logits": logits, "states": next_states}

    def _forward_graph(self, input_ids, labels, states, return_states, logits_to_keep):
        """The reference's composition (model.py:175-200) for autograd: each
        block's residual adds and RMSNorms as torch ops, the attention through
        the differentiable prefill."""
        x = self.embed_tokens(input_ids)
        next_states = [] if return_states else None
        for i, layer in enumerate(self.layers):
            x, ns = layer(x, state=states[i] if states is not None else None, return_state=return_states)
            if return_states:
                next_states.append(ns)
        if logits_to_keep:
            x = x[:, -logits_to_keep:]
        logits = self.lm_head(self.norm(x))
        loss = None
        if labels is not None:
            shift_logits = logits[..., :-1, :].contiguous().to(torch.float32)
            loss = F.cross_entropy(shift_logits.view(-1, self.config.vocab_size),
                                   labels[..., 1:].contiguous().view(-1), ignore_index=-100)
        return {"loss": loss, "logits": logits, "states": next_states}

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 50, temperature: float = 1.0,
                 top_k: int = 50, eos_token_id: Optional[int] = None) -> torch.Tensor:
        """model.py:202-242: prefill, then one recurrent step per token."""
        self.eval()
        out = self.forward(input_ids, return_states=True, logits_to_keep=1)
        states = out["states"]
        next_logits = out["logits"][:, -1, :]
        generated = input_ids
        for _ in range(max_new_tokens):
            next_logits = torch.nan_to_num(next_logits, nan=0.0, posinf=50.0, neginf=-50.0)
            if temperature > 0.0:
                logits = next_logits / max(temperature, 1e-4)
                if top_k > 0:
                    v, _ = torch.topk(logits, min(top_k, logits.size(-1)))
                    logits[logits < v[:, [-1]]] = -float("Inf")
                probs = torch.nan_to_num(F.softmax(logits, dim=-1), nan=1.0 / self.config.vocab_size)
                next_token = torch.multinomial(probs, num_samples=1)
            else:
                next_token = torch.argmax(next_logits, dim=-1, keepdim=True)
            generated = torch.cat([generated, next_token], dim=-1)
            if eos_token_id is not None and (next_token == eos_token_id).all():
                break
            step = self.forward(next_token, states=states, return_states=True)
            states = step["states"]
            next_logits = step["logits"][:, -1, :]
        return generated


def _decode_linear(x: torch.Tensor, w: torch.Tensor, gelu: bool = False) -> torch.Tensor:
    """x @ w.T (then the exact GELU) for the decode step's few rows: the skinny
    HIP kernel (prime_linear) on the shapes where it beats the library GEMM
    on MI355X (up to 64 rows, or K and N both at most 1024), the library GEMM
    otherwise."""
    M, K = x.shape
    N = w.shape[0]
    if (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and K % 64 == 0 and N % 4 == 0 and K <= 1024
            and (M <= 64 or N <= 1024)):
        return _lib.linear(x, w, torch.empty(M, N, device=x.device, dtype=x.dtype),
                           _lib.EPILOGUE_GELU if gelu else _lib.EPILOGUE_NONE)
    y = F.linear(x, w)
    return _lib.gelu(y) if gelu else y


class _LayerStep:
    """Per-layer constants of the fused one-token step: the q/k/v projection
    weights stacked into one [Hq*D + 2*Hkv*D, hidden] matrix (one GEMM), the
    QK-norm descriptor, and the decay tensor (base attention) or (tau, beta)
    (selective attention), all taken from the module as it is now."""

    def __init__(self, layer: "PrimeBlock", dtype: torch.dtype, device: torch.device):
        at = layer.self_attn
        self.qkv = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight], dim=0)
        self.norm = _lib.qk_norm(at.q_norm if at.use_qk_norm else None, at.k_norm if at.use_qk_norm else None,
                                 at.scaling, dtype)
        if isinstance(at, PrimeSelectiveMomentAttention):
            self.decay = None
            self.sel = (at.get_tau(device).float().contiguous(), at.get_beta(device).float().contiguous())
        else:
            self.decay = _lib.decay_tensor(at.decay, at.num_heads, device)
            self.sel = None
        # the folded form (base attention, GELU MLP, bf16): each RMSNorm's weight
        # multiplied into the columns of the projection after it, so that the
        # projection kernel applies the norm as a per-row scale (prime_linear_fused,
        # which applies it for rms_eps > 0 only: a norm eps of 0 keeps the unfolded
        # form; the fragment-layout step below takes "apply the norm" as a flag)
        self.qkv_g = self.up_g = None
        if (self.sel is None and isinstance(layer.mlp, PrimeGeluMLP) and dtype == torch.bfloat16
                and self.qkv.shape[1] % 128 == 0 and self.qkv.shape[0] % 32 == 0
                and layer.mlp.up_proj.weight.shape[0] % 128 == 0
                and layer.input_layernorm.eps > 0 and layer.post_attention_layernorm.eps > 0):
            g1 = layer.input_layernorm.weight.to(torch.float32)
            g2 = layer.post_attention_layernorm.weight.to(torch.float32)
            self.qkv_g = (self.qkv.to(torch.float32) * g1).to(dtype)
            self.up_g = (layer.mlp.up_proj.weight.to(torch.float32) * g2).to(dtype)
        # the fragment-layout step (prime_linear_frag): the same folded form with
        # every weight packed once into MFMA-operand blocks
        self.frag = None
        at_dims = (at.num_heads * at.head_dim, layer.mlp.up_proj.weight.shape[0] if isinstance(layer.mlp, PrimeGeluMLP)
                   else 0)
        if (isinstance(layer.mlp, PrimeGeluMLP) and dtype == torch.bfloat16 and at.head_dim == 64 and self.qkv.is_cuda
                and _lib.frag_supported(self.qkv.shape[1]) and _lib.frag_supported(at_dims[0])
                and _lib.frag_supported(at_dims[1]) and self.qkv.shape[1] % 32 == 0 and at_dims[1] % 32 == 0):
            self.frag = _FragLayer(layer, self, dtype)
        self.folded = self.qkv_g is not None or self.frag is not None


class _FragLayer:
    """One block's weights for the fragment-layout step: the stacked q/k/v
    weight (and, for selective attention, the step projection's rows, its bias
    kept apart) with the input RMSNorm's weight in its columns, padded to a
    multiple of 64 rows; o_proj; up_proj with the post-attention RMSNorm's
    weight in its columns; down_proj -- each packed into the fragment layout."""

    def __init__(self, layer: "PrimeBlock", ls: "_LayerStep", dtype: torch.dtype):
        at = layer.self_attn
        g1 = layer.input_layernorm.weight.to(torch.float32)
        g2 = layer.post_attention_layernorm.weight.to(torch.float32)
        w = ls.qkv.to(torch.float32) * g1
        self.nq0 = w.shape[0]
        bias = None
        if ls.sel is not None:
            H = at.num_heads
            w = torch.cat([w, at.delta_proj.weight.to(torch.float32) * g1])
            bias = torch.zeros(w.shape[0], dtype=torch.float32, device=w.device)
            bias[self.nq0:self.nq0 + H] = at.delta_proj.bias.to(torch.float32)
        n = w.shape[0]
        self.nq = -(-n // 64) * 64
        if self.nq > n:
            w = torch.cat([w, w.new_zeros(self.nq - n, w.shape[1])])
            if bias is not None:
                bias = torch.cat([bias, bias.new_zeros(self.nq - n)])
        self.bq = bias.contiguous() if bias is not None else None
        self.wq = _lib.pack_frag(w.to(dtype).contiguous())
        self.wo = _lib.pack_frag(at.o_proj.weight.contiguous())
        self.wu = _lib.pack_frag((layer.mlp.up_proj.weight.to(torch.float32) * g2).to(dtype).contiguous())
        self.wd = _lib.pack_frag(layer.mlp.down_proj.weight.contiguous())
        self.inter = layer.mlp.up_proj.weight.shape[0]


class _StepConstants(list):
    """Per-layer step constants, plus the lm_head with the final RMSNorm's
    weight in its columns in the fragment layout (``head``; None when the
    fragment step does not apply)."""
    head = None


def _constants_key(model: "PrimeForCausalLM"):
    """What the step constants are derived from: every parameter's storage and
    version counter (an in-place update or a new tensor changes it)."""
    return tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in model.parameters())


def _step_constants(model: "PrimeForCausalLM") -> List[_LayerStep]:
    """The per-layer step constants, rebuilt only when a parameter changed
    since they were last built (the stacked and norm-folded weights are tens
    of MB at the PRIME-125M shape; the generate loop calls this per token)."""
    key = _constants_key(model)
    cached = model.__dict__.get("_step_cache")
    if cached is not None and cached[0] == key:
        return cached[1]
    w = model.embed_tokens.weight
    consts = _StepConstants(_LayerStep(layer, w.dtype, w.device) for layer in model.layers)
    V, hidden = model.lm_head.weight.shape
    if (all(c.frag is not None for c in consts) and w.is_cuda and V % 16 == 0 and hidden % 32 == 0
            and model.lm_head.weight.dtype == torch.bfloat16):
        g = model.norm.weight.to(torch.float32)
        consts.head = _lib.pack_frag((model.lm_head.weight.to(torch.float32) * g).to(w.dtype).contiguous())
    model.__dict__["_step_cache"] = (key, consts)
    return consts


def _frag_step_ready(consts) -> bool:
    return getattr(consts, "head", None) is not None


def _fused_step_supported(model: "PrimeForCausalLM") -> bool:
    """The fused step takes the QK LayerNorm parameters in the activations'
    dtype, on the model's device (the kernels read them directly)."""
    w = model.embed_tokens.weight
    if not w.is_cuda:
        return False
    for layer in model.layers:
        at = layer.self_attn
        if at.use_qk_norm:
            for t in (at.q_norm.weight, at.q_norm.bias, at.k_norm.weight, at.k_norm.bias):
                if t is None or t.dtype != w.dtype or t.device != w.device or not t.is_contiguous():
                    return False
    return True


@torch.no_grad()
def _fused_step(model: "PrimeForCausalLM", tokens: torch.Tensor, states, consts: List[_LayerStep],
                inplace: bool):
    """One token per sequence through the whole model (the blocks of
    model.py:107-118, then the final norm and lm_head): embedding -> per layer
    add_rmsnorm -> one stacked q/k/v GEMM -> the decode kernel with the QK-norm
    and 1/sqrt(D) inside (attention.py:96-143, or selective.py:384-409) -> o_proj
    -> add_rmsnorm -> MLP; each residual add is fused into the following RMSNorm
    with the block's rounding.  For base attention with the GELU MLP in bf16
    the folded form runs instead: per layer RMSNorm + stacked q/k/v as one
    kernel (the norm's weight in the stacked weight's columns, its row scale
    applied to the products), the decode kernel, o_proj + residual add as one
    kernel, RMSNorm + up projection + GELU as one kernel, and down_proj with
    its residual add in the library GEMM (beta = 1); the norms' outputs are
    then not rounded on their own (prime_linear_fused).  Returns (logits
    [B, V], next states).

    inplace: the kernels update `states` in place (every layer's state must be
    given).  Otherwise the states are functional, as in the reference: new
    6-tuples are returned and the given ones are not written (unless the
    module was built with inplace_state and the given tensors are its own
    layout)."""
    cfg = model.config
    x = model.embed_tokens(tokens).reshape(-1, cfg.hidden_size)  # the residual stream, updated in place
    B = x.shape[0]
    dev = x.device
    # folded form: RMSNorm -> projection and projection -> residual add /
    # GELU as one kernel each (prime_linear_fused), the down projection's
    # residual add in the library GEMM (beta = 1)
    folded = B <= 1024 and all(c.qkv_g is not None for c in consts)
    pending = None
    next_states = []
    for i, (layer, c) in enumerate(zip(model.layers, consts)):
        at = layer.self_attn
        H, Hk, D = at.num_heads, at.num_kv_heads, at.head_dim
        if folded:
            qkv = _lib.linear_fused(x, c.qkv_g, torch.empty(B, c.qkv_g.shape[0], device=dev, dtype=x.dtype),
                                    _lib.EPILOGUE_NONE, layer.input_layernorm.eps)
        else:
            n1 = torch.empty_like(x)
            _lib.add_rmsnorm(x, pending, layer.input_layernorm.weight, n1, layer.input_layernorm.eps)
            qkv = _decode_linear(n1, c.qkv)
        q = qkv[:, :H * D].view(B, H, D)
        k = qkv[:, H * D:(H + Hk) * D].view(B, Hk, D)
        v = qkv[:, (H + Hk) * D:].view(B, Hk, D)
        st = states[i] if states is not None else None
        if inplace:
            st_in = st_out = st
        else:
            st_in = _lib.as_state(st, B, H, D, dev) if st is not None else None
            if at.inplace_state and st_in is not None and all(a.data_ptr() == b.data_ptr()
                                                              for a, b in zip(st_in, st)):
                st_out = st_in
            else:
                st_out = _lib.new_state(B, H, D, dev)
        y = torch.empty(B, H, D, device=dev, dtype=x.dtype)
        if c.sel is not None:
            # lambda_t = exp(-Delta_t / tau_h) formed in the kernel (selective.py:368, 385-386)
            tau, beta = c.sel
            gate = _lib.selective_gate(B, H, step=at.delta_proj(n1), tau=tau)
            _lib.selective_decode_step(q, k, v, gate, beta, at.eps, c.norm, st_in, st_out, y)
        else:
            _lib.decode_step_qknorm(q, k, v, c.decay, at.eps, c.norm, st_in, st_out, y)
        next_states.append(st_out)
        if folded:
            _lib.linear_fused(y.view(B, -1), at.o_proj.weight, x, _lib.EPILOGUE_RESIDUAL, 0.0, x)
            t = _lib.linear_fused(x, c.up_g, torch.empty(B, c.up_g.shape[0], device=dev, dtype=x.dtype),
                                  _lib.EPILOGUE_GELU, layer.post_attention_layernorm.eps)
            x.addmm_(t, layer.mlp.down_proj.weight.t())
            continue
        a = _decode_linear(y.view(B, -1), at.o_proj.weight)
        n2 = torch.empty_like(x)
        _lib.add_rmsnorm(x, a, layer.post_attention_layernorm.weight, n2, layer.post_attention_layernorm.eps)
        if isinstance(layer.mlp, PrimeGeluMLP):
            pending = _decode_linear(_decode_linear(n2, layer.mlp.up_proj.weight, gelu=True),
                                     layer.mlp.down_proj.weight)
        else:
            pending = layer.mlp(n2)
    nf = torch.empty_like(x)
    _lib.add_rmsnorm(x, pending, model.norm.weight, nf, model.norm.eps)
    return model.lm_head(nf), next_states


def _step_states(at, st, B, H, D, dev, inplace):
    """(state_in, state_out) of one layer's decode step: in place, or the
    reference's functional contract (new tensors unless the module keeps its
    own layout in place)."""
    if inplace:
        return st, st
    st_in = _lib.as_state(st, B, H, D, dev) if st is not None else None
    if at.inplace_state and st_in is not None and all(a.data_ptr() == b.data_ptr() for a, b in zip(st_in, st)):
        return st_in, st_in
    return st_in, _lib.new_state(B, H, D, dev)


@torch.no_grad()
def _frag_step(model: "PrimeForCausalLM", tokens: torch.Tensor, states, consts: "_StepConstants", inplace: bool,
               want_logits: bool = True, tokens_out: Optional[torch.Tensor] = None):
    """One token per sequence through the whole model on the fragment-layout
    kernels (the blocks of model.py:107-118, the final norm and lm_head of
    model.py:160, the greedy choice of model.py:230-231).  The residual stream
    x, the attention output y and the MLP's hidden layer stay in the fragment
    layout from the embedding gather to the lm_head:
      x  <- embed_tokens[tokens]                      (prime_pack_frag)
      per layer:
        qkv <- RMS(x) . Wqkv'^T (+ step bias)         (prime_linear_frag, row-major)
        y   <- decode step (QK-norm, 1/sqrt(D) inside; selective gate from qkv)
        x   <- x + y . Wo^T                           (residual epilogue, in place)
        t   <- GELU(RMS(x) . Wup'^T)
        x   <- x + t . Wdown^T
      logits <- RMS(x) . Wlm'^T, and/or the argmax of each row into tokens_out
    (W' carries the RMSNorm weight before the projection in its columns, so
    the norm's output is never rounded on its own).  Returns (logits [B, V] or
    None, next states); `states` as in _fused_step."""
    cfg = model.config
    K = cfg.hidden_size
    tok = tokens.reshape(-1)
    if tok.dtype != torch.int64:
        tok = tok.to(torch.int64)
    tok = tok.contiguous()
    B = tok.numel()
    dev = tok.device
    Mp = _lib.frag_rows(B)
    x = _lib.pack_frag(model.embed_tokens.weight, rows=tok)
    at0 = model.layers[0].self_attn
    y = torch.empty(Mp * at0.num_heads * at0.head_dim, device=dev, dtype=x.dtype)
    t = torch.empty(Mp * consts[0].frag.inter, device=dev, dtype=x.dtype)
    next_states = []
    for i, (layer, c) in enumerate(zip(model.layers, consts)):
        f, at = c.frag, layer.self_attn
        H, Hk, D = at.num_heads, at.num_kv_heads, at.head_dim
        qkv = torch.empty(B, f.nq, device=dev, dtype=x.dtype)
        _lib.linear_frag(x, f.wq, B, f.nq, K, qkv, flags=_lib.LINEAR_RMS, rms_eps=layer.input_layernorm.eps,
                         bias=f.bq)
        q = qkv[:, :H * D].view(B, H, D)
        k = qkv[:, H * D:(H + Hk) * D].view(B, Hk, D)
        v = qkv[:, (H + Hk) * D:(H + 2 * Hk) * D].view(B, Hk, D)
        st_in, st_out = _step_states(at, states[i] if states is not None else None, B, H, D, dev, inplace)
        if c.sel is not None:
            tau, beta = c.sel
            gate = _lib.selective_gate(B, H, step=qkv[:, f.nq0:f.nq0 + H], tau=tau)
            _lib.selective_decode_step(q, k, v, gate, beta, at.eps, c.norm, st_in, st_out, y, y_frag=True)
        else:
            _lib.decode_step_qknorm(q, k, v, c.decay, at.eps, c.norm, st_in, st_out, y, y_frag=True)
        next_states.append(st_out)
        _lib.linear_frag(y, f.wo, B, K, H * D, x, _lib.EPILOGUE_RESIDUAL, _lib.LINEAR_OUT_FRAG, r=x)
        _lib.linear_frag(x, f.wu, B, f.inter, K, t, _lib.EPILOGUE_GELU, _lib.LINEAR_RMS | _lib.LINEAR_OUT_FRAG,
                         rms_eps=layer.post_attention_layernorm.eps)
        _lib.linear_frag(t, f.wd, B, K, f.inter, x, _lib.EPILOGUE_RESIDUAL, _lib.LINEAR_OUT_FRAG, r=x)
    V = model.lm_head.weight.shape[0]
    logits = torch.empty(B, V, device=dev, dtype=x.dtype) if want_logits else None
    ws = None
    if tokens_out is not None:
        ws = torch.empty(_lib.linear_frag_workspace_size(B, V, K), device=dev, dtype=torch.uint8)
    _lib.linear_frag(x, consts.head, B, V, K, logits, flags=_lib.LINEAR_RMS, rms_eps=model.norm.eps,
                     tokens=tokens_out, workspace=ws)
    return logits, next_states


class GreedyDecoder:
    """Greedy decoding with in-place states and a HIP-graph-captured step.

    ``prefill(input_ids)`` runs the prompt through the chunked kernels and
    keeps one state 6-tuple per layer; ``step()`` appends one token per
    sequence with the model's fused one-token step (the one
    ``PrimeForCausalLM.forward`` runs for a single token, so the tokens equal
    those of ``generate`` at temperature 0, model.py:230-231), states updated
    in place, then argmax.  With ``use_graph`` the step is captured once after
    the prefill and replayed; every buffer it touches is fixed.
    """

    def __init__(self, model: PrimeForCausalLM, use_graph: bool = True):
        # the modules keep their functional state contract: no module flag is
        # changed here; the decoder's own prefill starts from no state and its
        # step hands the kernels the same buffers as input and output
        if not _fused_step_supported(model):
            raise ValueError("GreedyDecoder needs the model on a HIP device with QK LayerNorm parameters in the "
                             "activations' dtype")
        self.model = model.eval()
        self.use_graph = use_graph
        self.graph = None
        self.states = None
        self.consts = None

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Run the prompt; returns the first generated token [B, 1]."""
        m = self.model
        out = m.forward(input_ids, return_states=True, logits_to_keep=1)
        self.states = [tuple(s) for s in out["states"]]
        self.token = torch.empty(input_ids.shape[0], 1, dtype=torch.int64, device=input_ids.device)
        _lib.argmax(out["logits"][:, -1, :], self.token)
        # the step's per-layer constants, taken from the modules now
        self.consts = _step_constants(m)
        self.graph = None
        return self.token

    @torch.no_grad()
    def _step_eager(self) -> torch.Tensor:
        if _frag_step_ready(self.consts):
            # the lm_head kernel writes the greedy tokens itself (no logits);
            # the embedding gather at the start of the step has consumed the old ones
            _frag_step(self.model, self.token, self.states, self.consts, inplace=True, want_logits=False,
                       tokens_out=self.token.view(-1))
            return self.token
        logits, _ = _fused_step(self.model, self.token, self.states, self.consts, inplace=True)
        _lib.argmax(logits, self.token)  # the embedding above has consumed the old token
        return self.token

    @torch.no_grad()
    def step(self) -> torch.Tensor:
        """One decode step for every sequence; returns the new tokens [B, 1]."""
        if not self.use_graph:
            return self._step_eager()
        if self.graph is None:
            self._capture()
        self.graph.replay()
        return self.token

    def _capture(self):
        # warm up on a side stream (allocator pools, cached decay tensors), on a
        # copy of the states so that the real states advance only by replays
        saved = [tuple(t.clone() for t in st) for st in self.states]
        tok = self.token.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._step_eager()
        torch.cuda.current_stream().wait_stream(s)
        for st, sv in zip(self.states, saved):
            for t, x in zip(st, sv):
                t.copy_(x)
        self.token.copy_(tok)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._step_eager()
        # capture does not execute: states and token are as after the prefill
        self.graph = g

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        toks = [self.prefill(input_ids).clone()]
        for _ in range(max_new_tokens - 1):
            toks.append(self.step().clone())
        return torch.cat([input_ids] + toks, dim=-1)
