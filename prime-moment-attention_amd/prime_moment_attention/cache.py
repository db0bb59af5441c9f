"""PrimeMomentCache: constant-size recurrent state container (drop-in for the
reference's cache.py:15-56).  Holds one (S0, S1, S2, K0, K1, K2) fp32 6-tuple
per layer and never stores key/value history; ``update`` only counts tokens.

The base class is transformers' ``Cache`` when transformers is importable (as
in the reference), else ``object``.  ``Cache.__init__`` changed signature
across transformers releases (newer ones require ``layers`` or
``layer_class_to_replicate``); the keyword arguments this class hands it are
worked out once, from the signature, when the module is imported.
"""
from __future__ import annotations

import inspect
from typing import Any, Dict, Optional, Tuple

import torch

try:  # transformers is optional: without it the cache is a plain object
    from transformers.cache_utils import Cache as _Base
except Exception:  # pragma: no cover - depends on the environment
    _Base = object


def _base_init_kwargs() -> Optional[Dict[str, Any]]:
    """Keyword arguments for the base constructor: an empty layer list where
    the base takes one, nothing otherwise; None when the base is ``object``
    (nothing to call)."""
    if _Base is object:
        return None
    try:
        params = inspect.signature(_Base.__init__).parameters
    except (TypeError, ValueError):  # pragma: no cover - builtin without a signature
        return {}
    return {"layers": []} if "layers" in params else {}


_BASE_KWARGS = _base_init_kwargs()


class PrimeMomentCache(_Base):
    def __init__(self):
        if _BASE_KWARGS is not None:
            super().__init__(**_BASE_KWARGS)
        self.prime_states: Dict[int, Tuple[torch.Tensor, ...]] = {}
        self._seen_tokens = 0

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self._seen_tokens

    def get_max_cache_shape(self) -> Optional[int]:
        return None

    def get_max_length(self) -> Optional[int]:
        return None

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[Dict[str, Any]] = None):
        """Counts the tokens on layer 0 and hands the inputs back unchanged
        (no key/value history is kept, cache.py:36-46)."""
        if layer_idx == 0:
            self._seen_tokens += key_states.shape[-2]
        return key_states, value_states

    def get_state(self, layer_idx: int) -> Optional[Tuple[torch.Tensor, ...]]:
        return self.prime_states.get(layer_idx)

    def set_state(self, layer_idx: int, state: Tuple[torch.Tensor, ...]):
        self.prime_states[layer_idx] = state

    def reset(self):
        self.prime_states.clear()
        self._seen_tokens = 0

    def state_bytes(self) -> int:
        """Bytes held by all layer states (constant in sequence length)."""
        return sum(t.element_size() * t.nelement() for s in self.prime_states.values() for t in s)
