"""MI355X (gfx950) PRIME moment attention.

Drop-in host API mirroring the reference package ``prime_moment_attention``
(PrimeMomentAttention, chunked_prime_ssd_core, ChunkedPrimeSSD,
PrimeMomentCache, PrimeConfig / PrimeForCausalLM,
ChunkedGatedDeltaPrimeAttention, PrimeSelectiveMomentAttention) over the HIP library
libprime_mi355x.so.
"""
from .attention import PrimeMomentAttention
from .cache import PrimeMomentCache
from .chunked_delta_prime import ChunkedGatedDeltaPrimeAttention
from .chunked_ssd import ChunkedPrimeSSD, chunked_prime_ssd_core
from .model import GreedyDecoder, PrimeConfig, PrimeForCausalLM, prime_125m_config
from .selective import PrimeSelectiveMomentAttention

__version__ = "0.1.0"

__all__ = ["PrimeMomentAttention", "PrimeMomentCache", "ChunkedPrimeSSD", "chunked_prime_ssd_core",
           "PrimeConfig", "PrimeForCausalLM", "GreedyDecoder", "prime_125m_config",
           "ChunkedGatedDeltaPrimeAttention", "PrimeSelectiveMomentAttention"]
