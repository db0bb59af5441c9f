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

When autograd records (a parameter or the input requires grad), the module
differentiates as torch autograd does through the reference: the QK
LayerNorm, the q scale, the grouped-head expansion, softplus/clamp of the
step sizes and the tau and beta clamps run as torch ops, and the recurrence
runs through ``_SelectivePrefillFn`` (the fp32 prefill forward, the HIP
backward prime_selective_prefill_backward), which gives the gradients in q,
k, v, the per-token log decays, beta and the incoming state.  L == 1 with a
state then runs as a one-token prefill from that state: the reference's step
branch (selective.py:384-409) computes the same function.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .attention import project_qkv
from .chunked_ssd import _prep, needs_grad


class _SelectivePrefillFn(torch.autograd.Function):
    """prime_selective_prefill (fp32 q/k/v with H heads) with its backward
    (prime_selective_prefill_backward): differentiable in q, k, v, log_decay
    [B, H, L], beta [H] and the incoming state (selective convention)."""

    @staticmethod
    def forward(ctx, q, k, v, log_decay, beta, eps, return_state, *state):
        B, H, L, D = q.shape
        st_in = tuple(state) if state else None
        y = torch.empty(B, H, L, D, device=q.device, dtype=torch.float32)
        st_out = _lib.new_state(B, H, D, q.device) if return_state else None
        _lib.selective_prefill(q, k, v, log_decay, beta, eps, st_in, y, st_out)
        ctx.save_for_backward(q, k, v, log_decay, beta, *(st_in or ()))
        ctx.eps, ctx.has_state = eps, st_in is not None
        ctx.set_materialize_grads(False)
        return (y, *st_out) if return_state else y

    @staticmethod
    def backward(ctx, dy, *dstate):
        q, k, v, log_decay, beta, *st = ctx.saved_tensors
        B, H, L, D = q.shape
        dev = q.device
        dy = torch.zeros(B, H, L, D, device=dev, dtype=torch.float32) if dy is None else _prep(dy)
        dso = None
        if any(t is not None for t in dstate):
            zs = _lib.new_state(B, H, D, dev, zero=True)
            dso = tuple(z if t is None else t.to(torch.float32).reshape(z.shape).contiguous()
                        for z, t in zip(zs, dstate))
        dq, dk, dv = (torch.empty(B, H, L, D, device=dev, dtype=torch.float32) for _ in range(3))
        dld = torch.empty(B, H, L, device=dev, dtype=torch.float32)
        dbeta = torch.empty(B, H, device=dev, dtype=torch.float32)
        dsi = _lib.new_state(B, H, D, dev) if ctx.has_state else None
        _lib.selective_prefill_backward(q, k, v, log_decay, beta, ctx.eps, tuple(st) if st else None, dy, dso,
                                        dq, dk, dv, dsi, dld, dbeta)
        return (dq, dk, dv, dld, dbeta.sum(0), None, None, *(dsi or ()))


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

    def _gate_constants(self, device: torch.device):
        """tau and beta as contiguous fp32 [H] on `device` for the kernels
        (inference: no autograd through them), cached outside the state dict
        and rebuilt when log_tau or log_beta changes (storage or version), so
        that a prefill or a step does not relaunch their elementwise ops."""
        ps = (self.log_tau, self.log_beta)
        key = tuple((p.data_ptr(), p._version) for p in ps) + (str(device), self.min_tau, self.max_tau)
        cached = self.__dict__.get("_gate_cache")
        if cached is not None and all(a is b for a, b in zip(cached[0], ps)) and cached[1] == key:
            return cached[2]
        with torch.no_grad():
            consts = (self.get_tau(device).float().contiguous(), self.get_beta(device).float().contiguous())
        self.__dict__["_gate_cache"] = (ps, key, consts)
        return consts

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
        q, k, v = project_qkv(self, hidden_states)
        if needs_grad(hidden_states, *self.parameters(), *(state or ())):
            tau = self.get_tau(dev).float().contiguous()
            beta = self.get_beta(dev).float().contiguous()
            return self._mix_autograd(hidden_states, q, k, v, tau, beta, state, return_state)
        tau, beta = self._gate_constants(dev)
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
            # per-token log decays -(Delta / tau), [B, H, L], from delta_proj(x)
            # in one kernel (the stages of step_size, each rounded as there)
            log_decay = _lib.selective_log_decay(self.delta_proj(hidden_states), tau)
            y_bl = torch.empty(B, L, H, D, device=dev, dtype=y_dtype)
            next_state = _lib.new_state(B, H, D, dev) if return_state else None
            _lib.selective_prefill(q, k, v, log_decay, beta, self.eps, None, y_bl.transpose(1, 2), next_state,
                                   qk_norm=norm)
            y = y_bl.transpose(1, 2)
        y = y.to(orig_dtype).transpose(1, 2).reshape(B, L, H * D)
        return y, (next_state if return_state else None)

    def _mix_autograd(self, hidden_states, q, k, v, tau, beta, state, return_state):
        """``mix`` under autograd (selective.py:354-440 as torch differentiates
        it): torch ops up to the recurrence, _SelectivePrefillFn for it."""
        B, L, _ = hidden_states.shape
        H, D = self.num_heads, self.head_dim
        if self.num_kv_groups > 1:
            k = k.repeat_interleave(self.num_kv_groups, dim=1)
            v = v.repeat_interleave(self.num_kv_groups, dim=1)
        if self.use_qk_norm:
            q, k = self.q_norm(q), self.k_norm(k)
        q = q * self.scaling
        q, k, v = (t.to(torch.float32).contiguous() for t in (q, k, v))
        log_decay = (-self.step_size(hidden_states).float() / tau.view(1, 1, H)).transpose(1, 2).contiguous()
        # the parallel branch (L > 1) starts from a zero state, the step branch from `state`
        st = _lib.as_state(state, B, H, D, q.device) if (state is not None and L == 1) else ()
        outs = _SelectivePrefillFn.apply(q, k, v, log_decay, beta, float(self.eps), bool(return_state), *st)
        y, next_state = (outs[0], tuple(outs[1:])) if return_state else (outs, None)
        return y.to(hidden_states.dtype).transpose(1, 2).reshape(B, L, H * D), next_state
