"""Chunked PRIME prefill: drop-in for the reference's chunked_ssd.py.

``chunked_prime_ssd_core`` keeps the reference signature and contract
(chunked_ssd.py:48-61): q, k, v are projected, normalised [B, H, L, D] tensors
with q already scaled by 1/sqrt(D); it returns (y fp32 [B, H, L, D], state or
None).  All of it runs in one HIP kernel launch (prime_chunked_prefill); see
csrc/prefill.hip for the algorithm.

Differences from the reference, by design:
  * ``decay`` may also be an [H] tensor (one decay per head).
  * q/k/v may be bf16 (read as-is) or fp32; k/v may carry fewer heads (GQA:
    head h uses k/v head h // (H // H_kv), like attention.py:92-94).
  * an incoming ``state`` is carried as the recurrence defines it.  The
    reference core raises a shape error for a 6-tuple state (its 3-D state
    components broadcast against a 5-D decay table, chunked_ssd.py:129-137).
  * the result does not depend on ``chunk_size`` beyond rounding (the chunked
    form is exact for every chunk size); the kernel tiles 64 tokens.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib


def _prep(x: torch.Tensor) -> torch.Tensor:
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    if x.stride(-1) != 1 or x.data_ptr() % 16 or any((s * x.element_size()) % 16 for s in x.stride()[:-1]):
        x = x.contiguous()
    return x


def needs_grad(*xs) -> bool:
    """True when autograd records: grad mode on and some input requires grad."""
    return torch.is_grad_enabled() and any(torch.is_tensor(x) and x.requires_grad for x in xs)


class _NoBackward(torch.autograd.Function):
    """Ties a HIP result to the inputs it was computed from, so that a
    backward through it fails loudly instead of leaving their gradients
    silently empty."""

    @staticmethod
    def forward(ctx, what, y, *inputs):
        ctx.what = what
        return y.view_as(y)

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(f"{ctx.what} has no backward in this library (the base chunked prefill does); "
                                  "run it under torch.no_grad()")


def no_backward(what: str, y: torch.Tensor, *inputs) -> torch.Tensor:
    """y, marked as not differentiable with respect to `inputs` (a backward raises)."""
    if needs_grad(*inputs):
        return _NoBackward.apply(what, y, *[x for x in inputs if torch.is_tensor(x)])
    return y


class _PrefillFn(torch.autograd.Function):
    """prime_chunked_prefill with its backward (prime_chunked_prefill_backward):
    the derivative torch autograd takes through the reference's prefill
    (attention.py:77-210, chunked_ssd.py:48-184) when it trains."""

    @staticmethod
    def forward(ctx, q, k, v, dec, eps, flags, return_state, out_dtype, *state):
        B, H, L, D = q.shape
        st_in = tuple(state) if state else None
        y = torch.empty(B, H, L, D, device=q.device, dtype=out_dtype)
        st_out = _lib.new_state(B, H, D, q.device) if return_state else None
        _lib.chunked_prefill(q, k, v, dec, eps, 64, st_in, y, st_out, flags)
        ctx.save_for_backward(q, k, v, dec, *(st_in or ()))
        ctx.eps, ctx.flags, ctx.has_state = eps, flags, st_in is not None
        ctx.set_materialize_grads(False)
        return (y, *st_out) if return_state else y

    @staticmethod
    def backward(ctx, dy, *dstate):
        q, k, v, dec, *st = ctx.saved_tensors
        B, H, L, D = q.shape
        Hkv = k.shape[1]
        grp = H // Hkv
        if grp > 1:  # the kernel takes one k/v head per query head (attention.py:92-94 expands them too)
            k, v = k.repeat_interleave(grp, dim=1), v.repeat_interleave(grp, dim=1)
        dev = q.device
        dy = torch.zeros(B, H, L, D, device=dev, dtype=torch.float32) if dy is None else _prep(dy)
        dso = None
        if any(t is not None for t in dstate):
            zs = _lib.new_state(B, H, D, dev, zero=True)
            dso = tuple(z if t is None else t.to(torch.float32).reshape(z.shape).contiguous()
                        for z, t in zip(zs, dstate))
        dq, dk, dv = (torch.empty(B, H, L, D, device=dev, dtype=q.dtype) for _ in range(3))
        dsi = _lib.new_state(B, H, D, dev) if ctx.has_state else None
        _lib.chunked_prefill_backward(q, k, v, dec, ctx.eps, tuple(st) if st else None, dy, dso, dq, dk, dv, dsi,
                                      flags=ctx.flags)
        if grp > 1:
            dk, dv = dk.view(B, Hkv, grp, L, D).sum(2), dv.view(B, Hkv, grp, L, D).sum(2)
        return (dq, dk, dv, None, None, None, None, None, *(dsi or ()))


def prime_prefill(q, k, v, state=None, decay=0.9995, eps=1.0, chunk_size=64, return_state=False,
                  out_dtype=torch.float32, dense_clamp=False, state_out=None, y=None, qk_norm=None):
    """Core launcher shared by the modules.  Returns (y, next_state | None);
    ``y`` may be a caller-provided [B, H, L, D] view (any strides with a
    contiguous D and 16-byte aligned rows).  When autograd records (an input
    requires grad), the call is differentiable -- in q, k, v and the incoming
    state -- through the HIP backward; ``y`` and ``state_out`` are then not
    used (fresh outputs are returned).  ``qk_norm`` (``_lib.qk_norm(...)``,
    bf16 only, no autograd): q and k are the raw projections and the module's
    QK LayerNorm and q scale are applied by the kernels as they load them."""
    B, H, L, D = q.shape
    if needs_grad(decay):
        # a per-head decay tensor is this library's extension; the backward
        # kernels give no derivative in it, so a learnable decay would train
        # with a silently missing gradient
        raise NotImplementedError("the prefill has no gradient with respect to decay; pass a decay that does not "
                                  "require grad (e.g. decay.detach()) or run under torch.no_grad()")
    q, k, v = _prep(q), _prep(k), _prep(v)
    if k.dtype != q.dtype or v.dtype != q.dtype:
        k, v = k.to(q.dtype), v.to(q.dtype)
    dev = q.device
    dec = _lib.decay_tensor(decay, H, dev)
    st_in = _lib.as_state(state, B, H, D, dev) if state is not None else None
    if needs_grad(q, k, v, *(st_in or ())):
        if qk_norm is not None:
            raise NotImplementedError("the QK-norm on load has no backward; normalise q and k with torch ops")
        flags = _lib.PRIME_FLAG_DENSE_CLAMP if dense_clamp else 0
        outs = _PrefillFn.apply(q, k, v, dec, float(eps), flags, bool(return_state), out_dtype, *(st_in or ()))
        if return_state:
            return outs[0], tuple(outs[1:])
        return outs, None
    if y is None:
        y = torch.empty(B, H, L, D, device=dev, dtype=out_dtype)
    st_out = None
    if return_state:
        st_out = state_out if state_out is not None else _lib.new_state(B, H, D, dev)
    _lib.chunked_prefill(q, k, v, dec, eps, chunk_size, st_in, y, st_out,
                         _lib.PRIME_FLAG_DENSE_CLAMP if dense_clamp else 0, qk_norm=qk_norm)
    return y, st_out


def chunked_prime_ssd_core(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    state: Optional[Tuple[torch.Tensor, ...]] = None,
    decay: float = 0.9995,
    eps: float = 1.0,
    chunk_size: int = 64,
    return_state: bool = False,
) -> Tuple[torch.Tensor, Optional[Tuple[torch.Tensor, ...]]]:
    """Drop-in for chunked_ssd.py:48-184 (same arguments, same outputs)."""
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    return prime_prefill(q, k, v, state=state, decay=decay, eps=eps, chunk_size=chunk_size,
                         return_state=return_state, out_dtype=torch.float32)


class ChunkedPrimeSSD(nn.Module):
    """Module twin that always runs the chunked core (chunked_ssd.py:187-251)."""

    def __init__(self, hidden_size: int, num_heads: int, head_dim: int, chunk_size: int = 64,
                 decay: float = 0.9995, eps: float = 1.0, use_qk_norm: bool = True):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.chunk_size = chunk_size
        self.decay = decay
        self.eps = eps
        self.scaling = 1.0 / math.sqrt(head_dim)
        self.use_qk_norm = use_qk_norm
        self.q_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(num_heads * head_dim, hidden_size, bias=False)
        if self.use_qk_norm:
            self.q_norm = nn.LayerNorm(head_dim)
            self.k_norm = nn.LayerNorm(head_dim)

    def forward(self, hidden_states: torch.Tensor, state=None, return_state: bool = False):
        B, L, _ = hidden_states.shape
        dtype = hidden_states.dtype
        q = self.q_proj(hidden_states).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        if needs_grad(q, k, v):
            # training: QK-norm and scale as torch ops (chunked_ssd.py:225-236), the core differentiable
            if self.use_qk_norm:
                q, k = self.q_norm(q), self.k_norm(k)
            q = q * self.scaling
            y, next_state = prime_prefill(q, k, v, state=state, decay=self.decay, eps=self.eps,
                                          chunk_size=self.chunk_size, return_state=return_state)
            y = y.to(dtype).transpose(1, 2).reshape(B, L, self.num_heads * self.head_dim)
            return self.o_proj(y), next_state
        # QK-norm and scale in place on the projections (chunked_ssd.py:225-236)
        _lib.head_layernorm(q, q, self.q_norm if self.use_qk_norm else None, self.scaling)
        if self.use_qk_norm:
            _lib.head_layernorm(k, k, self.k_norm, 1.0)
        y_dtype = dtype if dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        y_bl = torch.empty(B, L, self.num_heads, self.head_dim, device=q.device, dtype=y_dtype)
        y, next_state = prime_prefill(q, k, v, state=state, decay=self.decay, eps=self.eps,
                                      chunk_size=self.chunk_size, return_state=return_state,
                                      out_dtype=y_dtype, y=y_bl.transpose(1, 2))
        y = y.to(dtype).transpose(1, 2).reshape(B, L, self.num_heads * self.head_dim)
        return self.o_proj(y), next_state
