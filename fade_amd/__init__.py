"""fade_amd -- FADE's tiered-KV hot path on AMD Instinct MI355X (gfx950).

Public API mirrors the reference package ``fade`` (Omodaka9375/fade):
``FadeConfig``, ``create_tiered_cache``, ``TieredKVCache``, ``get_backend``
and the ``quant_backend`` names, with the quantize/pack, re-RoPE and
attention work done by hand-written HIP kernels in ``libfade_hip.so``
(C ABI: ``include/fade_hip.h``).
"""

from .backends import AsymGroupBackend, QuantBackend, RotatedINT4Backend, SymmetricINT4Backend, get_backend
from .cache import TIER_EVICT, TIER_FP16, TIER_INT2, TIER_INT4, TIER_PQ, LayerState, TieredKVCache
from .config import FadeConfig
from .patch import create_tiered_cache

__version__ = "0.1.0"

__all__ = [
    "AsymGroupBackend",
    "FadeConfig",
    "LayerState",
    "QuantBackend",
    "RotatedINT4Backend",
    "SymmetricINT4Backend",
    "TIER_EVICT",
    "TIER_FP16",
    "TIER_INT2",
    "TIER_INT4",
    "TIER_PQ",
    "TieredKVCache",
    "create_tiered_cache",
    "get_backend",
]
