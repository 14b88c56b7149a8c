"""Tier assignment: scores -> ``tiers[S]`` (fade/policy.py:232-274).

Host-side policy logic (an argsort of at most a few thousand scores per
layer), kept in torch exactly as the reference computes it; the tiers it
returns drive ``TieredKVCache.apply_tier_assignment``.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .cache import TIER_EVICT, TIER_FP16, TIER_INT2, TIER_INT4


def _assign_one_layer(
    S: int,
    scores: Tensor,
    n_sink: int,
    recent_window: int,
    int4_budget: int | None,
    int2_budget: int,
) -> Tensor:
    """Sinks and the recent window stay FP16; the middle is ranked by score.

    ``int4_budget=None`` keeps every middle token in INT4 (no eviction).
    Otherwise the top ``int4_budget`` scores go to INT4, the next
    ``int2_budget`` to INT2 and the rest are evicted.
    """
    tiers = torch.full((S,), TIER_EVICT, dtype=torch.long, device=scores.device)
    sink_end = min(n_sink, S)
    tiers[:sink_end] = TIER_FP16
    tiers[max(sink_end, S - recent_window) :] = TIER_FP16
    middle = (tiers == TIER_EVICT).nonzero(as_tuple=False).squeeze(-1)
    if middle.numel() == 0:
        return tiers
    if int4_budget is None or int4_budget >= int(middle.numel()):
        tiers[middle] = TIER_INT4
        return tiers
    order = scores[middle].argsort(descending=True)
    tiers[middle[order[:int4_budget]]] = TIER_INT4
    if int2_budget > 0:
        k2 = min(int2_budget, int(order.shape[0]) - int4_budget)
        if k2 > 0:
            tiers[middle[order[int4_budget : int4_budget + k2]]] = TIER_INT2
    return tiers


def reassign_tiers_by_position(cache, num_layers: int) -> None:
    """Position (FIFO) policy: newer middle tokens score higher (fade/policy.py:126-159)."""
    for li in range(num_layers):
        if not cache.is_managed(li):
            continue
        S = int(cache.get_seq_length(li))
        if S == 0:
            continue
        scores = torch.arange(S, dtype=torch.float32)
        tiers = _assign_one_layer(S, scores, cache.n_sink, cache.recent_window, cache.int4_budget, cache.int2_budget)
        cache.apply_tier_assignment(li, tiers)


def reassign_tiers_with_scores(cache, layer_scores: dict[int, Tensor]) -> None:
    """Apply the rule to externally computed per-layer scores (e.g. H2O attention mass)."""
    for li, scores in layer_scores.items():
        S = cache.get_seq_length(li)
        tiers = _assign_one_layer(S, scores, cache.n_sink, cache.recent_window, cache.int4_budget, cache.int2_budget)
        cache.apply_tier_assignment(li, tiers, scores=scores)


__all__ = ["_assign_one_layer", "reassign_tiers_by_position", "reassign_tiers_with_scores"]
