"""HF ``generate()`` on the fused tiered kernels: the ``"fade"`` attention implementation.

The reference's cache returns the materialized ``[sink | dequantized middle |
recent]`` K/V from ``update()`` (fade/cache.py:347-379,693-699) and the
model's own attention reads that copy.  Here a model built with
``attn_implementation="fade"`` (or switched with
``model.set_attn_implementation("fade")``) gets a ``TieredKVCache`` from
``create_tiered_cache`` whose ``update()`` only appends; the attention call of
the same layer then reads the layer's tiers in place:

  * one query token per row  -> ``fade_tiered_decode_attn``;
  * a chunk of Sq > 1 tokens -> ``fade_tiered_prefill_attn`` (the chunk is the
    last Sq tokens of the fp16 tier, bottom-right causal).

Transformers dispatches attention through ``ALL_ATTENTION_FUNCTIONS`` and the
mask through ``ALL_MASK_ATTENTION_FUNCTIONS``; both get a ``"fade"`` entry
when this module is imported.  The kernels apply the causal mask themselves,
so the mask function returns ``None``; padded batches are rejected.
"""

from __future__ import annotations

import threading

import torch
from torch import Tensor

_active = threading.local()
NAME = "fade"


def set_active_cache(cache) -> None:
    """Record the cache whose ``update()`` ran last on this thread (HF calls the
    layer's attention right after it)."""
    _active.cache = cache


def active_cache():
    cache = getattr(_active, "cache", None)
    if cache is None:
        raise RuntimeError(
            "fade attention: no TieredKVCache in fused mode is active; pass the cache built by "
            "create_tiered_cache(model) as past_key_values"
        )
    return cache


def fade_attention_forward(
    module: torch.nn.Module,
    query: Tensor,
    key: Tensor,
    value: Tensor,
    attention_mask: Tensor | None,
    dropout: float = 0.0,
    scaling: float | None = None,
    **kwargs,
) -> tuple[Tensor, None]:
    """``ALL_ATTENTION_FUNCTIONS["fade"]``: attention of ``query`` [B, Hq, Sq, D] over
    the tiers of ``module.layer_idx`` in the active cache; returns [B, Sq, Hq, D]."""
    if attention_mask is not None:
        raise ValueError("fade attention: the kernels apply the causal mask; an explicit mask is not supported")
    if kwargs.get("sliding_window") is not None:
        raise ValueError("fade attention: sliding-window layers are not supported")
    cache = active_cache()
    out = cache.attend(query, module.layer_idx, sm_scale=scaling)
    return out.transpose(1, 2).contiguous(), None


def fade_mask(
    batch_size: int,
    q_length: int,
    kv_length: int,
    q_offset: int = 0,
    kv_offset: int = 0,
    mask_function=None,
    attention_mask: Tensor | None = None,
    **kwargs,
):
    """``ALL_MASK_ATTENTION_FUNCTIONS["fade"]``: ``None`` (causal in the kernel)."""
    if attention_mask is not None and not bool(attention_mask.all()):
        raise ValueError("fade attention: padded batches are not supported (every row must be full length)")
    return None


def register() -> None:
    """Register ``"fade"`` with transformers' attention and mask interfaces (idempotent)."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface

    AttentionInterface.register(NAME, fade_attention_forward)
    AttentionMaskInterface.register(NAME, fade_mask)


def uses_fade_attention(model) -> bool:
    cfg = getattr(model, "config", None)
    text_cfg = getattr(cfg, "text_config", cfg)
    impl = getattr(text_cfg, "_attn_implementation", None) or getattr(cfg, "_attn_implementation", None)
    return impl == NAME


register()

__all__ = ["NAME", "active_cache", "fade_attention_forward", "fade_mask", "register", "set_active_cache",
           "uses_fade_attention"]
