"""PrimeMomentAttention: drop-in for the reference's attention.py.

Same constructor, same ``forward(hidden_states, state=None, return_state=False)
-> (out, next_state)`` and the same 6-tuple fp32 state (S0, S1, S2, K0, K1, K2)
(attention.py:42-210).  Projections, the optional LayerNorm QK-norm and o_proj
are ordinary torch layers; everything between them -- the moment recurrence in
all three regimes the reference dispatches on L (attention.py:120, 146, 161) --
is one HIP kernel launch through the C ABI:

  L == 1                     prime_decode_step (attention.py:119-143)
  L >  chunk_threshold       prime_chunked_prefill (attention.py:145-158)
  1 < L <= chunk_threshold   prime_chunked_prefill with PRIME_FLAG_DENSE_CLAMP,
                             which reproduces the dense branch's clamp of the
                             intra denominator before the incoming-state carry
                             is added (attention.py:177, 185)

The state is functional by default, as in the reference (a new 6-tuple is
returned, the incoming one is untouched).  ``inplace_state=True`` updates the
incoming tensors instead, with the same HBM traffic.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
from .chunked_ssd import needs_grad, prime_prefill


def _same_storage(a, b) -> bool:
    """True when the validated state views alias the caller's tensors (so an
    in-place update reaches them)."""
    return all(x.data_ptr() == y.data_ptr() for x, y in zip(a, b))


def _stacked_qkv(mod: nn.Module) -> Optional[torch.Tensor]:
    """The q, k and v weights of an attention module stacked into one
    [(H + 2 Hk) D, hidden] matrix, so that inference projects with one GEMM
    instead of three (the same products: each output column is the same dot
    product).  Cached on the module outside its state dict and rebuilt when a
    weight's storage or version counter changes; None while autograd records
    through the weights (training keeps the three nn.Linear calls) or when the
    three differ in dtype or device or carry a bias."""
    lins = (mod.q_proj, mod.k_proj, mod.v_proj)
    ws = tuple(m.weight for m in lins)
    if torch.is_grad_enabled() and any(w.requires_grad for w in ws):
        return None
    if any(m.bias is not None for m in lins) or len({(w.dtype, w.device) for w in ws}) != 1:
        return None
    # the cache holds the weight tensors themselves, so their storage
    # cannot be freed and reused by a new weight at the same address
    key = tuple((w.data_ptr(), w._version) for w in ws)
    cached = mod.__dict__.get("_qkv_cache")
    # (a copy made under inference_mode is rebuilt outside it: autograd could
    # not save an inference tensor for a backward through hidden_states)
    if (cached is not None and all(a is b for a, b in zip(cached[0], ws)) and cached[1] == key
            and (not cached[2].is_inference() or torch.is_inference_mode_enabled())):
        return cached[2]
    w = torch.cat(ws, 0)
    mod.__dict__["_qkv_cache"] = (ws, key, w)
    return w


def project_qkv(mod: nn.Module, hidden_states: torch.Tensor):
    """q, k, v projections of [B, L, hidden] as [B, H(kv), L, D] views
    (attention.py:83-85): one GEMM into [B, L, (H + 2 Hk) D] over the stacked
    weights where _stacked_qkv allows it (q, k, v are then column ranges of
    that result), else the module's three nn.Linear layers."""
    B, L, _ = hidden_states.shape
    H, Hk, D = mod.num_heads, mod.num_kv_heads, mod.head_dim
    w = _stacked_qkv(mod)
    if w is None:
        return (mod.q_proj(hidden_states).view(B, L, H, D).transpose(1, 2),
                mod.k_proj(hidden_states).view(B, L, Hk, D).transpose(1, 2),
                mod.v_proj(hidden_states).view(B, L, Hk, D).transpose(1, 2))
    qkv = torch.nn.functional.linear(hidden_states, w)
    return (qkv[..., :H * D].view(B, L, H, D).transpose(1, 2),
            qkv[..., H * D:(H + Hk) * D].view(B, L, Hk, D).transpose(1, 2),
            qkv[..., (H + Hk) * D:].view(B, L, Hk, D).transpose(1, 2))


class PrimeMomentAttention(nn.Module):
    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        head_dim: int,
        num_kv_heads: Optional[int] = None,
        decay=0.9995,
        use_qk_norm: bool = False,
        eps: float = 1.0,
        chunk_size: int = 64,
        chunk_threshold: int = 512,
        inplace_state: bool = False,
    ):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads or num_heads
        self.num_kv_groups = num_heads // self.num_kv_heads
        self.decay = decay
        self.scaling = 1.0 / math.sqrt(head_dim)
        self.eps = eps
        self.use_qk_norm = use_qk_norm
        self.chunk_size = chunk_size
        self.chunk_threshold = chunk_threshold
        self.inplace_state = inplace_state

        self.q_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.num_kv_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.num_kv_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(num_heads * head_dim, hidden_size, bias=False)
        if self.use_qk_norm:
            self.q_norm = nn.LayerNorm(head_dim)
            self.k_norm = nn.LayerNorm(head_dim)

    def project(self, hidden_states: torch.Tensor, normalize: bool = True):
        """q (scaled), k, v as [B, H(kv), L, D] views (attention.py:83-101);
        normalize=False returns the raw projections (QK-norm and scale left
        to the decode kernel)."""
        q, k, v = project_qkv(self, hidden_states)
        if not normalize:
            return q, k, v
        self._normalize(q, k)
        return q, k, v

    def _normalize(self, q: torch.Tensor, k: torch.Tensor) -> None:
        """QK-norm and the 1/sqrt(D) scale in place on the fresh projections
        (prime_head_layernorm, the module's rounding), read by the prefill
        kernel through the [B, L, H, D] strides."""
        _lib.head_layernorm(q, q, self.q_norm if self.use_qk_norm else None, self.scaling)
        if self.use_qk_norm:
            _lib.head_layernorm(k, k, self.k_norm, 1.0)

    def _load_norm(self, q: torch.Tensor):
        """The QK-norm for the prefill kernels to apply as they load q and k
        (bf16 projections with LayerNorm parameters of that dtype and one eps),
        or None when q and k are to be normalised first."""
        return _lib.qk_norm_on_load(self.q_norm if self.use_qk_norm else None,
                                    self.k_norm if self.use_qk_norm else None, self.scaling, q)

    def forward(
        self,
        hidden_states: torch.Tensor,
        state: Optional[Tuple[torch.Tensor, ...]] = None,
        return_state: bool = False,
    ):
        B, L, _ = hidden_states.shape
        orig_dtype = hidden_states.dtype
        H, D = self.num_heads, self.head_dim

        if torch.is_grad_enabled() and (hidden_states.requires_grad or any(p.requires_grad for p in self.parameters())):
            # training: QK-norm and scale as torch ops, the recurrence through the
            # differentiable prefill (for L == 1 its chunked form is the step,
            # attention.py:119-143; for 1 < L <= chunk_threshold the dense
            # branch's double clamp, attention.py:177-185, with or without a state)
            q, k, v = self.project(hidden_states, normalize=False)
            if self.use_qk_norm:
                q, k = self.q_norm(q), self.k_norm(k)
            q = q * self.scaling
            dense = 1 < L <= self.chunk_threshold
            y, next_state = prime_prefill(q, k, v, state=state, decay=self.decay, eps=self.eps,
                                          chunk_size=self.chunk_size, return_state=return_state,
                                          dense_clamp=dense)
            y = y.to(orig_dtype).transpose(1, 2).reshape(B, L, H * D)
            return self.o_proj(y), (next_state if return_state else None)
        y, next_state = self.mix(hidden_states, state, return_state)
        return self.o_proj(y), (next_state if return_state else None)

    def mix(self, hidden_states: torch.Tensor, state: Optional[Tuple[torch.Tensor, ...]] = None,
            return_state: bool = False):
        """The attention up to its output projection, without autograd:
        (y [B, L, H*D] in the input dtype, next state or None), so that
        ``forward`` is ``o_proj`` of it (attention.py:83-208) and a caller can
        fold o_proj into its residual add (PrimeForCausalLM)."""
        B, L, _ = hidden_states.shape
        orig_dtype = hidden_states.dtype
        H, D = self.num_heads, self.head_dim
        dev = hidden_states.device
        y_dtype = orig_dtype if orig_dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        if L == 1:
            # the QK LayerNorm and the 1/sqrt(D) scale run inside the decode kernel
            q, k, v = self.project(hidden_states, normalize=False)
            norm = _lib.qk_norm(self.q_norm if self.use_qk_norm else None,
                                self.k_norm if self.use_qk_norm else None, self.scaling, q.dtype)
            dec = _lib.decay_tensor(self.decay, H, dev)
            st_in = _lib.as_state(state, B, H, D, dev) if state is not None else None
            if self.inplace_state and st_in is not None and _same_storage(st_in, state):
                st_out = st_in
            else:
                st_out = _lib.new_state(B, H, D, dev)
            y = torch.empty(B, H, D, device=dev, dtype=y_dtype)
            _lib.decode_step_qknorm(q[:, :, 0], k[:, :, 0], v[:, :, 0], dec, self.eps, norm, st_in, st_out, y)
            y = y.unsqueeze(2)
            next_state = st_out
        else:
            q, k, v = self.project(hidden_states, normalize=False)
            norm = self._load_norm(q)
            if norm is None:
                self._normalize(q, k)
            dense = L <= self.chunk_threshold
            st_out = None
            if return_state and self.inplace_state and state is not None:
                st_in = _lib.as_state(state, B, H, D, dev)
                if _same_storage(st_in, state):
                    st_out = st_in
            # y written in the o_proj input layout [B, L, H, D] through strides
            y_bl = torch.empty(B, L, H, D, device=dev, dtype=y_dtype)
            y, next_state = prime_prefill(q, k, v, state=state, decay=self.decay, eps=self.eps,
                                          chunk_size=self.chunk_size, return_state=return_state,
                                          out_dtype=y_dtype, dense_clamp=dense, state_out=st_out,
                                          y=y_bl.transpose(1, 2), qk_norm=norm)

        y = y.to(orig_dtype).transpose(1, 2).reshape(B, L, H * D)
        return y, (next_state if return_state else None)
