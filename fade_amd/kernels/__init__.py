"""Attention ops of the FADE hot path on MI355X kernels."""

from .fused_int4_attn import check_fused_parity, fused_int4_sdpa, fused_int4_sdpa_with_fallback
from .int4_attention import check_parity, int4_sdpa
from .prefill import TieredPrefillPlan, tiered_prefill_attention
from .tiered_attn import MiddleTier, TieredDecodePlan, tiered_decode_attention

__all__ = [
    "MiddleTier",
    "TieredDecodePlan",
    "TieredPrefillPlan",
    "check_fused_parity",
    "check_parity",
    "fused_int4_sdpa",
    "fused_int4_sdpa_with_fallback",
    "int4_sdpa",
    "tiered_decode_attention",
    "tiered_prefill_attention",
]
