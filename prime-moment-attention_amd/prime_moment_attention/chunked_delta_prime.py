"""ChunkedGatedDeltaPrimeAttention: drop-in for the reference's chunked_delta_prime.py.

Same constructor, parameters and ``forward(hidden_states, state=None,
return_state=False) -> (out, next_state)`` as chunked_delta_prime.py:25-283,
with the state an fp32 [B, H, D, 2D] tensor.  Projections, the erase/write
gates, the LayerNorm QK-norm and o_proj are torch layers; the recurrence runs
in the HIP kernels through the C ABI:

  L == 1   prime_delta_decode_step  (the reference's step branch, :140-176,
           which predicts with the undecayed state)
  L >  1   prime_delta_prefill      (the chunked branch, :177-283)

The per-token scalars the kernels take are the reference's: beta =
0.5 mean(sigmoid(write)) and alpha = decay (1 - 0.5 mean(sigmoid(erase)))
(:133-137).  The chunked branch clamps once per chunk, so its result depends
on ``chunk_size``: head_dim 64 with chunk_size 64 (the reference default)
runs the MFMA chunk kernels, any other head_dim up to 64 or chunk size the
token-sequential kernels.

Training: with autograd recording, the chunked branch runs through
prime_delta_prefill_backward (gradients in q, k, v, beta, alpha and the
incoming state), and the projections, QK LayerNorm and gates are the
reference's differentiable torch ops.  The step branch has no backward.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
from .chunked_ssd import no_backward


class _DeltaPrefillFn(torch.autograd.Function):
    """The chunked delta-rule prefill with its HIP backward."""

    @staticmethod
    def forward(ctx, q, k, v, beta, alpha, s_in, decay, feat_eps, bound, y_dtype, chunk):
        B, H, L, D = q.shape
        y = torch.empty(B, H, L, D, device=q.device, dtype=y_dtype)
        s_out = torch.empty(B, H, D, 2 * D, device=q.device, dtype=torch.float32)
        _lib.delta_prefill(q, k, v, beta, alpha, decay, feat_eps, bound, s_in, y, s_out, chunk=chunk)
        ctx.save_for_backward(q, k, v, beta, alpha, s_in)
        ctx.consts = (decay, feat_eps, bound, chunk)
        return y, s_out

    @staticmethod
    def backward(ctx, dy, ds_out):
        q, k, v, beta, alpha, s_in = ctx.saved_tensors
        decay, feat_eps, bound, chunk = ctx.consts
        if dy is None:
            dy = torch.zeros(q.shape, device=q.device, dtype=torch.float32)
        dy = dy.contiguous()
        if dy.dtype not in (torch.float32, torch.bfloat16):
            dy = dy.float()
        ds = ds_out.contiguous().float() if ds_out is not None else None
        dq, dk, dv, dbeta, dalpha, dstate = _lib.delta_prefill_backward(q, k, v, beta, alpha, decay, feat_eps,
                                                                          bound, s_in, dy, ds, chunk=chunk)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dbeta, dalpha, dstate, None, None, None, None, None)


class _DeltaStepFn(torch.autograd.Function):
    """The delta-rule decode step (one token) with its HIP backward."""

    @staticmethod
    def forward(ctx, q, k, v, beta, alpha, s_in, feat_eps, bound, y_dtype):
        B, H, D = q.shape
        y = torch.empty(B, H, D, device=q.device, dtype=y_dtype)
        s_out = torch.empty(B, H, D, 2 * D, device=q.device, dtype=torch.float32)
        _lib.delta_decode_step(q, k, v, beta, alpha, feat_eps, bound, s_in, s_out, y)
        ctx.save_for_backward(q, k, v, beta, alpha, s_in)
        ctx.consts = (feat_eps, bound)
        return y, s_out

    @staticmethod
    def backward(ctx, dy, ds_out):
        q, k, v, beta, alpha, s_in = ctx.saved_tensors
        feat_eps, bound = ctx.consts
        if dy is None:
            dy = torch.zeros(q.shape, device=q.device, dtype=torch.float32)
        dy = dy.contiguous()
        if dy.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            dy = dy.float()
        ds = ds_out.contiguous().float() if ds_out is not None else None
        dq, dk, dv, dbeta, dalpha, dstate = _lib.delta_decode_step_backward(q, k, v, beta, alpha, feat_eps, bound,
                                                                              s_in, dy, ds)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dbeta.view_as(beta), dalpha.view_as(alpha), dstate,
                None, None, None)


class ChunkedGatedDeltaPrimeAttention(nn.Module):
    def __init__(self, hidden_size: int, num_heads: int, head_dim: int, num_kv_heads: Optional[int] = None,
                 chunk_size: int = 64, decay: float = 0.9995, use_qk_norm: bool = True,
                 lyapunov_bound: float = 25.0, eps: float = 1e-5):
        super().__init__()
        if chunk_size < 1:
            raise ValueError("chunk_size must be positive")
        if head_dim > 64:
            raise ValueError("head_dim above 64 is not supported")
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads or num_heads
        self.num_kv_groups = num_heads // self.num_kv_heads
        self.chunk_size = chunk_size
        self.decay = decay
        self.scaling = 1.0 / math.sqrt(head_dim)
        self.use_qk_norm = use_qk_norm
        self.lyapunov_bound = lyapunov_bound
        self.eps = eps
        self.q_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.num_kv_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.num_kv_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(num_heads * head_dim, hidden_size, bias=False)
        self.erase_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=True)
        self.write_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=True)
        if use_qk_norm:
            self.q_norm = nn.LayerNorm(head_dim)
            self.k_norm = nn.LayerNorm(head_dim)
        self._init_weights()

    def _init_weights(self):
        # gate biases as chunked_delta_prime.py:67-71 (erase ~ 0.05, write ~ 0.25)
        nn.init.constant_(self.erase_proj.bias, -2.5)
        nn.init.constant_(self.write_proj.bias, -1.0)

    def gates(self, hidden_states: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """(beta, alpha) fp32 [B, H, L] (chunked_delta_prime.py:110-111, 133-137)."""
        B, L, _ = hidden_states.shape
        H, D = self.num_heads, self.head_dim
        b = torch.sigmoid(self.erase_proj(hidden_states)).view(B, L, H, D).float().mean(-1)
        w = torch.sigmoid(self.write_proj(hidden_states)).view(B, L, H, D).float().mean(-1)
        beta = (w * 0.5).transpose(1, 2).contiguous()
        alpha = (self.decay * (1.0 - b * 0.5)).transpose(1, 2).contiguous()
        return beta, alpha

    def project(self, hidden_states: torch.Tensor):
        """q (scaled), k, v as [B, H(kv), L, D] (chunked_delta_prime.py:105-126)."""
        B, L, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(B, L, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(B, L, self.num_kv_heads, self.head_dim).transpose(1, 2)
        # QK-norm and scale in place on the fresh projections (prime_head_layernorm)
        _lib.head_layernorm(q, q, self.q_norm if self.use_qk_norm else None, self.scaling)
        if self.use_qk_norm:
            _lib.head_layernorm(k, k, self.k_norm, 1.0)
        return q, k, v

    def forward(self, hidden_states: torch.Tensor, state: Optional[torch.Tensor] = None,
                return_state: bool = False) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        B, L, _ = hidden_states.shape
        H, D = self.num_heads, self.head_dim
        dtype, dev = hidden_states.dtype, hidden_states.device
        if torch.is_grad_enabled() and (hidden_states.requires_grad or
                                                  any(p.requires_grad for p in self.parameters()) or
                                                  (state is not None and state.requires_grad)):
            return self._forward_train(hidden_states, state, return_state)
        q, k, v = self.project(hidden_states)
        beta, alpha = self.gates(hidden_states)
        if q.dtype not in (torch.bfloat16, torch.float32):
            q, k, v = q.float(), k.float(), v.float()
        y_dtype = dtype if dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        s_in = None
        if state is not None:
            s_in = state.to(device=dev, dtype=torch.float32).reshape(B, H, D, 2 * D).contiguous()
        s_out = torch.empty(B, H, D, 2 * D, device=dev, dtype=torch.float32)
        if L == 1:
            y = torch.empty(B, H, D, device=dev, dtype=y_dtype)
            _lib.delta_decode_step(q[:, :, 0], k[:, :, 0], v[:, :, 0], beta, alpha, self.eps,
                                   self.lyapunov_bound, s_in, s_out, y)
            y = y.unsqueeze(2)
        else:
            q, k, v = (t if (t.stride(-1) == 1 and all((s * t.element_size()) % 16 == 0 for s in t.stride()[:-1]))
                       else t.contiguous() for t in (q, k, v))
            y = torch.empty(B, H, L, D, device=dev, dtype=y_dtype)
            _lib.delta_prefill(q, k, v, beta, alpha, self.decay, self.eps, self.lyapunov_bound, s_in, y, s_out,
                               chunk=self.chunk_size)
        y = no_backward("the delta-rule PRIME (inference path)", y, q, k, v, beta, alpha, s_in)
        y = y.to(dtype).transpose(1, 2).reshape(B, L, H * D)
        return self.o_proj(y), (s_out if return_state else None)

    def _forward_train(self, hidden_states, state, return_state):
        """The chunked branch under autograd: the reference's torch ops for the
        projections, QK LayerNorm, scale and gates (chunked_delta_prime.py:
        105-137), the HIP prefill and its backward for the recurrence."""
        B, L, _ = hidden_states.shape
        H, D = self.num_heads, self.head_dim
        dtype, dev = hidden_states.dtype, hidden_states.device
        q = self.q_proj(hidden_states).view(B, L, H, D).transpose(1, 2)
        k = self.k_proj(hidden_states).view(B, L, self.num_kv_heads, D).transpose(1, 2)
        v = self.v_proj(hidden_states).view(B, L, self.num_kv_heads, D).transpose(1, 2)
        if self.use_qk_norm:
            q = self.q_norm(q)
            k = self.k_norm(k)
        q = q * self.scaling
        beta, alpha = self.gates(hidden_states)
        if q.dtype not in (torch.bfloat16, torch.float32):
            q, k, v = q.float(), k.float(), v.float()
        q, k, v = (t.contiguous() for t in (q, k, v))
        y_dtype = dtype if dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        s_in = None
        if state is not None:
            s_in = state.to(device=dev, dtype=torch.float32).reshape(B, H, D, 2 * D).contiguous()
        if L == 1:
            # the step branch (chunked_delta_prime.py:140-176) and its backward
            y, s_out = _DeltaStepFn.apply(q[:, :, 0], k[:, :, 0], v[:, :, 0], beta.contiguous(),
                                          alpha.contiguous(), s_in, self.eps, self.lyapunov_bound, y_dtype)
            y = y.unsqueeze(2)
        else:
            y, s_out = _DeltaPrefillFn.apply(q, k, v, beta, alpha, s_in, self.decay, self.eps, self.lyapunov_bound,
                                             y_dtype, self.chunk_size)
        y = y.to(dtype).transpose(1, 2).reshape(B, L, H * D)
        return self.o_proj(y), (s_out if return_state else None)
