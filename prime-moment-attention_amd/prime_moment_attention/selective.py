"""PrimeSelectiveMomentAttention: drop-in for the reference's native selective
PRIME module (selective.py:264-444).

Same constructor, parameters (q/k/v/o projections, q_norm/k_norm, delta_proj,
log_tau, log_beta), identity-preserving initialisation and ``forward(
hidden_states, state=None, return_state=False) -> (out, next_state)``.  The
recurrence is the base PRIME moment recurrence with

  * a decay per token and head, lambda_t = exp(-Delta_t / tau_h) with
    Delta_t = softplus(W_delta x_t + b_delta) clamped to [1e-4, 50];
  * the key weighted by an inverse temperature beta_h (beta for the first
    order, beta^2 / 2 for the second), folded into the state, so that S2 and
    K2 carry the 1/2 (the reference's state convention, selective.py:395-400).

L == 1 runs prime_selective_decode_step (selective.py:384-409; the QK
LayerNorm and 1/sqrt(D) inside the kernel); L > 1 runs prime_selective_prefill
in place of the parallel branch's [L, L] decay matrix (selective.py:414-440).
As in the reference, the parallel branch starts from a zero state: an incoming
``state`` is used by the L == 1 step only, and the returned state of an L > 1
call covers that call's tokens.  bf16 projections run the bf16-MFMA prefill;
fp32 projections (fp16 ones are widened to fp32) run the fp32 prefill kernel,
as the reference computes this branch in fp32 (selective.py:363-365).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .chunked_ssd import no_backward


class PrimeSelectiveMomentAttention(nn.Module):
    def __init__(self, hidden_size: int, num_heads: int, head_dim: int, num_kv_heads: Optional[int] = None,
                 decay: float = 0.995, use_qk_norm: bool = True, eps: float = 1.0, min_tau: float = 2.0,
                 max_tau: float = 2000.0):
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
        self.min_tau = min_tau
        self.max_tau = max_tau
        self.inplace_state = False  # True: L == 1 updates the incoming state tensors in place
        self.q_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.num_kv_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.num_kv_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(num_heads * head_dim, hidden_size, bias=False)
        if use_qk_norm:
            self.q_norm = nn.LayerNorm(head_dim)
            self.k_norm = nn.LayerNorm(head_dim)
        self.delta_proj = nn.Linear(hidden_size, num_heads, bias=True)
        base_tau = -1.0 / math.log(max(1e-5, min(0.9999, decay)))
        self.log_tau = nn.Parameter(torch.full((num_heads,), math.log(base_tau), dtype=torch.float32))
        self.log_beta = nn.Parameter(torch.zeros(num_heads, dtype=torch.float32))
        self.init_selective_weights()

    def init_selective_weights(self):
        """selective.py:324-332: W_delta = 0, softplus(b_delta) = 1, tau from
        `decay`, beta = 1 -- the base module's recurrence exactly."""
        with torch.no_grad():
            self.delta_proj.weight.zero_()
            self.delta_proj.bias.fill_(math.log(math.exp(1.0) - 1.0))
            self.log_tau.fill_(math.log(-1.0 / math.log(max(1e-5, min(0.9999, self.decay)))))
            self.log_beta.zero_()

    def get_tau(self, device: torch.device) -> torch.Tensor:
        return torch.clamp(torch.exp(self.log_tau.to(device)), min=self.min_tau, max=self.max_tau)

    def get_beta(self, device: torch.device) -> torch.Tensor:
        return torch.clamp(torch.exp(self.log_beta.to(device)), min=0.1, max=15.0)

    def step_size(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """Delta [B, L, H] (selective.py:368)."""
        return F.softplus(self.delta_proj(hidden_states)).clamp(min=1e-4, max=50.0)

    def forward(self, hidden_states: torch.Tensor, state: Optional[Tuple[torch.Tensor, ...]] = None,
                return_state: bool = False):
        y, next_state = self.mix(hidden_states, state, return_state)
        return self.o_proj(y), next_state

    def mix(self, hidden_states: torch.Tensor, state: Optional[Tuple[torch.Tensor, ...]] = None,
            return_state: bool = False):
        """The attention up to its output projection: (y [B, L, H*D] in the
        input dtype, next state or None); ``forward`` is ``o_proj`` of it."""
        B, L, _ = hidden_states.shape
        H, D = self.num_heads, self.head_dim
        orig_dtype, dev = hidden_states.dtype, hidden_states.device
        y_dtype = orig_dtype if orig_dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        q = self.q_proj(hidden_states).view(B, L, H, D).transpose(1, 2)
        k = self.k_proj(hidden_states).view(B, L, self.num_kv_heads, D).transpose(1, 2)
        v = self.v_proj(hidden_states).view(B, L, self.num_kv_heads, D).transpose(1, 2)
        tau = self.get_tau(dev).float().contiguous()
        beta = self.get_beta(dev).float().contiguous()
        if L == 1:
            norm = _lib.qk_norm(self.q_norm if self.use_qk_norm else None,
                                self.k_norm if self.use_qk_norm else None, self.scaling, q.dtype)
            # the kernel forms Delta and lambda from the pre-activations (selective.py:368, 386)
            pre = self.delta_proj(hidden_states)[:, 0, :]
            gate = _lib.selective_gate(B, H, step=pre, tau=tau)
            st_in = _lib.as_state(state, B, H, D, dev) if state is not None else None
            if self.inplace_state and st_in is not None and all(
                    a.data_ptr() == b.data_ptr() for a, b in zip(st_in, state)):
                st_out = st_in
            else:
                st_out = _lib.new_state(B, H, D, dev)
            y = torch.empty(B, H, D, device=dev, dtype=y_dtype)
            _lib.selective_decode_step(q[:, :, 0], k[:, :, 0], v[:, :, 0], gate, beta, self.eps, norm, st_in,
                                       st_out, y)
            y = y.unsqueeze(2)
            next_state = st_out
        else:
            if q.dtype not in (torch.bfloat16, torch.float32):
                q, k, v = q.float(), k.float(), v.float()
            # the QK LayerNorm and scale as the kernels load q and k (or first,
            # in place, where the parameters do not allow that)
            norm = _lib.qk_norm_on_load(self.q_norm if self.use_qk_norm else None,
                                        self.k_norm if self.use_qk_norm else None, self.scaling, q)
            if norm is None:
                _lib.head_layernorm(q, q, self.q_norm if self.use_qk_norm else None, self.scaling)
                if self.use_qk_norm:
                    _lib.head_layernorm(k, k, self.k_norm, 1.0)
            # per-token log decays -(Delta / tau), [B, H, L]
            delta = self.step_size(hidden_states)  # [B, L, H]
            log_decay = (-delta.float() / tau.view(1, 1, H)).transpose(1, 2).contiguous()
            y_bl = torch.empty(B, L, H, D, device=dev, dtype=y_dtype)
            next_state = _lib.new_state(B, H, D, dev) if return_state else None
            _lib.selective_prefill(q, k, v, log_decay, beta, self.eps, None, y_bl.transpose(1, 2), next_state,
                                   qk_norm=norm)
            y = y_bl.transpose(1, 2)
        y = no_backward("selective PRIME", y, q, k, v, tau, beta, hidden_states,
                        *(state if state is not None else ()))
        y = y.to(orig_dtype).transpose(1, 2).reshape(B, L, H * D)
        return y, (next_state if return_state else None)
