"""Numpy restatement of the tier-assignment rule (test infrastructure only).

Reference: ``fade/policy.py:232-274`` (``_assign_one_layer``) and the tier
constants ``fade/cache.py:45-49``.
"""

from __future__ import annotations

import numpy as np

TIER_FP16, TIER_INT4, TIER_INT2, TIER_EVICT, TIER_PQ = 0, 1, 2, 3, 4


def assign_one_layer(S, scores, n_sink, recent_window, int4_budget, int2_budget):
    """fade/policy.py:232-274.

    Sinks ``[0, n_sink)`` and the recent window ``[max(sink_end, S-recent), S)``
    are FP16; the middle goes to INT4 when the budget is unlimited, else the
    top ``int4_budget`` scores go to INT4, the next ``int2_budget`` to INT2
    and the rest are evicted.  The reference sorts with a non-stable
    descending argsort; ties have probability zero for continuous scores.
    """
    tiers = np.full(S, TIER_EVICT, dtype=np.int64)
    sink_end = min(n_sink, S)
    tiers[:sink_end] = TIER_FP16
    recent_start = max(sink_end, S - recent_window)
    tiers[recent_start:] = TIER_FP16
    middle = np.nonzero(tiers == TIER_EVICT)[0]
    if middle.size == 0:
        return tiers
    if int4_budget is None or int4_budget >= middle.size:
        tiers[middle] = TIER_INT4
        return tiers
    order = np.argsort(-np.asarray(scores, dtype=np.float64)[middle], kind="stable")
    tiers[middle[order[:int4_budget]]] = TIER_INT4
    if int2_budget > 0:
        k2 = min(int2_budget, order.size - int4_budget)
        if k2 > 0:
            tiers[middle[order[int4_budget : int4_budget + k2]]] = TIER_INT2
    return tiers
