"""Hybrid window-PRIME kernels: the object the reference's hybrid attention
obtains from ``get_cpp_kernel()`` (hybrid.py:28-43), with the same four
methods, argument order and return values as its JIT extension
(prime_cpp_kernel.cpp:6-124), run by the HIP library instead of a sequential
torch-op loop:

  prime_prefill_cpp(q, k, v, decay)            -> [out, S0, S1, S2, K0, K1, K2]
  prime_accumulate_evicted_cpp(k, v, decay)    -> [S0, S1, S2, K0, K1, K2]
  prime_query_step_cpp(q, S0, S1, S2, K0, K1, K2) -> y [B, H, D]
  prime_step_evict_update_cpp(kt, vt, S0, S1, S2, K0, K1, K2, decay)  (in place)

Tensors live on the HIP device: q/k/v [B, H, L, D] (or [B, H, D] for the
steps) in fp32 (bf16 and fp16 are accepted too), states fp32 with K0 [B, H, 1]
as in the reference.  The denominator clamp is the reference's 1e-3.  A
missing library raises instead of falling back to a CPU loop.
"""
from __future__ import annotations

from typing import List

import torch

from . import _lib

EPS = 1e-3  # prime_cpp_kernel.cpp:40, :96


def _contig_rows(x: torch.Tensor) -> torch.Tensor:
    return x if x.stride(-1) == 1 else x.contiguous()


def _state6(S0, S1, S2, K0, K1, K2):
    st = (S0, S1, S2, K0, K1, K2)
    for t in st:
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("state tensors must be contiguous fp32 (the reference updates them in place)")
    return st


class HybridKernels:
    """Drop-in for the reference's ``prime_cpp_hybrid`` extension module."""

    @staticmethod
    def prime_prefill_cpp(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, decay: float) -> List[torch.Tensor]:
        """prime_cpp_kernel.cpp:6-46: outputs of all L tokens and the final
        state, from a zero state; y in q's dtype."""
        q, k, v = _contig_rows(q), _contig_rows(k), _contig_rows(v)
        B, H, L, D = q.shape
        y = torch.empty(B, H, L, D, device=q.device, dtype=q.dtype)
        st = _lib.new_state(B, H, D, q.device)
        _lib.chunked_prefill(q, k, v, _lib.decay_tensor(float(decay), H, q.device), EPS, 64, None, y, st)
        return [y, *st]

    @staticmethod
    def prime_accumulate_evicted_cpp(k: torch.Tensor, v: torch.Tensor, decay: float) -> List[torch.Tensor]:
        """prime_cpp_kernel.cpp:48-83: the state of the evicted tokens, from zero."""
        k, v = _contig_rows(k), _contig_rows(v)
        B, H, L, D = k.shape
        st = _lib.new_state(B, H, D, k.device, zero=L == 0)
        if L > 0:
            _lib.accumulate(k, v, _lib.decay_tensor(float(decay), H, k.device), None, st)
        return list(st)

    @staticmethod
    def prime_query_step_cpp(q: torch.Tensor, S0, S1, S2, K0, K1, K2) -> torch.Tensor:
        """prime_cpp_kernel.cpp:85-100: readout of q [B, H, D] against the state."""
        q = _contig_rows(q)
        st = _state6(S0, S1, S2, K0, K1, K2)
        y = torch.empty_like(q)
        _lib.decode_readout(q, EPS, st, y)
        return y

    @staticmethod
    def prime_step_evict_update_cpp(kt: torch.Tensor, vt: torch.Tensor, S0, S1, S2, K0, K1, K2,
                                    decay: float) -> None:
        """prime_cpp_kernel.cpp:102-117: the state absorbs one token, in place."""
        kt, vt = _contig_rows(kt), _contig_rows(vt)
        st = _state6(S0, S1, S2, K0, K1, K2)
        H = kt.shape[1]
        _lib.decode_update(kt, vt, _lib.decay_tensor(float(decay), H, kt.device), st, st)


_kernels = None


def get_cpp_kernel() -> HybridKernels:
    """hybrid.py:28-43.  The reference returns None when its JIT build fails
    and then runs a Python loop; here the HIP library is required."""
    global _kernels
    if _kernels is None:
        _lib.load()
        _kernels = HybridKernels()
    return _kernels
