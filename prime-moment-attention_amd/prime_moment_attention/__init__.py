"""MI355X (gfx950) PRIME moment attention.

Drop-in host API mirroring the reference package ``prime_moment_attention``
(PrimeMomentAttention, chunked_prime_ssd_core, ChunkedPrimeSSD,
PrimeMomentCache) over the HIP library libprime_mi355x.so.
"""
from .attention import PrimeMomentAttention
from .cache import PrimeMomentCache
from .chunked_ssd import ChunkedPrimeSSD, chunked_prime_ssd_core

__version__ = "0.1.0"

__all__ = ["PrimeMomentAttention", "PrimeMomentCache", "ChunkedPrimeSSD", "chunked_prime_ssd_core"]
