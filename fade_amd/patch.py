"""``create_tiered_cache``: build a cache from an HF model's config (fade/patch.py:125-207)."""

from __future__ import annotations

import warnings

import torch

from .cache import TieredKVCache
from .config import FadeConfig
from .hf_attention import uses_fade_attention
from .rope import extract_rope_scheme

_RECURRENT_TYPES = {"mamba", "mamba2", "rwkv", "rwkv5", "rwkv6", "xlstm"}
_DEEPSEEK_TYPES = {"deepseek", "deepseek_r1", "deepseek_r2", "deepseek_v2", "deepseek_v3"}


def create_tiered_cache(model, dtype: torch.dtype = torch.float16, config: FadeConfig | None = None, **kwargs):
    """Return a ``TieredKVCache`` configured with the model's head_dim and RoPE scheme.

    ``config`` supplies the cache knobs; explicit ``kwargs`` override them.
    Recurrent models get a plain ``DynamicCache``; DeepSeek MLA models get a
    cache whose layers are all pass-through (their K/V is already latent).
    """
    text_cfg = getattr(model.config, "text_config", model.config)
    model_type = getattr(text_cfg, "model_type", "")
    if model_type in _RECURRENT_TYPES:
        warnings.warn(
            f"Model type {model_type!r} is a recurrent architecture with no standard K/V cache. "
            "Returning a plain DynamicCache. FADE tier compression is not applicable.",
            RuntimeWarning,
            stacklevel=2,
        )
        from transformers.cache_utils import DynamicCache

        return DynamicCache()
    head_dim = getattr(text_cfg, "head_dim", None) or text_cfg.hidden_size // text_cfg.num_attention_heads
    scheme = extract_rope_scheme(text_cfg, head_dim=head_dim)
    kw: dict = {}
    if config is not None:
        kw.update(config.to_cache_kwargs())
    kw.update(kwargs)
    cache = TieredKVCache(dtype=dtype, rope_theta=scheme.theta, head_dim=head_dim, rope_scheme=scheme, **kw)
    # attn_implementation="fade": attention reads the tiers in place (no materialized K/V)
    cache.fused = uses_fade_attention(model)
    if cache.fused and dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f'attn_implementation="fade" reads float16 and bfloat16 caches; got dtype={dtype}')
    layer_types = getattr(text_cfg, "layer_types", None)
    if layer_types is not None:
        skip = {i for i, t in enumerate(layer_types) if t not in ("full_attention", "sliding_attention")}
        if skip:
            cache.set_skip_layers(skip)
    if model_type in _DEEPSEEK_TYPES:
        warnings.warn(
            f"Model type {model_type!r} uses Multi-head Latent Attention. K/V are already compressed "
            "latent vectors. FADE tier management is disabled (all layers skipped).",
            RuntimeWarning,
            stacklevel=2,
        )
        cache.set_skip_layers(set(range(getattr(text_cfg, "num_hidden_layers", 0))))
    return cache


__all__ = ["create_tiered_cache"]
