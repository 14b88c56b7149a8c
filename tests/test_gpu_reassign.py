"""Device-side tier reassignment (fade_reassign_plan / fade_reassign_gather) against
the host path of ``apply_tier_assignment``, which follows fade/cache.py:881-1057 op
for op and is pinned to the oracle.  Every tier field must match bit for bit."""

import numpy as np
import pytest
import torch

from fade_amd.cache import TIER_EVICT, TIER_FP16, TIER_INT2, TIER_INT4, TieredKVCache
from fade_amd.policy import _assign_one_layer

pytestmark = pytest.mark.gpu

FIELDS = ("sink_k", "sink_v", "sink_pos", "fp16_k", "fp16_v", "fp16_pos", "int4_kq", "int4_ks", "int4_vq",
          "int4_vs", "int4_pos", "int2_kq")


def _pair(**kw):
    caches = []
    for dev_path in (False, True):
        c = TieredKVCache(head_dim=128, **kw)
        c.device_reassign = dev_path
        caches.append(c)
    return caches


def _append(caches, B, H, n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(B, H, n, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).half().to(dev)
    v = torch.randn(B, H, n, 128, generator=g).half().to(dev)
    for c in caches:
        c.update(k, v, 0)


def _same(a, b, what):
    for f in FIELDS:
        x, y = getattr(a._layers[0], f), getattr(b._layers[0], f)
        assert (x is None) == (y is None), f"{what}: {f} present in one path only"
        if x is not None:
            assert x.shape == y.shape, f"{what}: {f} shape {tuple(x.shape)} vs {tuple(y.shape)}"
            assert torch.equal(x.cpu(), y.cpu()), f"{what}: {f} differs"
    for f in ("next_position", "sink_count", "int2_actual_count"):
        assert getattr(a._layers[0], f) == getattr(b._layers[0], f), f"{what}: {f}"
    assert a.get_seq_length(0) == b.get_seq_length(0)


@pytest.mark.parametrize("tiers_on", ["cpu", "cuda", "cuda+counts"])
@pytest.mark.parametrize("budget", [None, 40])
def test_reassign_device_matches_host(dev, tiers_on, budget):
    """Three rounds of append + reassign (scores seeded), eviction when budget is set."""
    print(f"case reassign tiers_on={tiers_on} budget={budget}", flush=True)
    B, H = 2, 2
    host, devc = _pair(n_sink=4, recent_window=16, int4_budget=budget, int2_budget=0)
    _append((host, devc), B, H, 150, 1, dev)
    rng = np.random.default_rng(5)
    for rnd in range(3):
        S = host.get_seq_length(0)
        scores = torch.from_numpy(rng.exponential(size=S).astype(np.float32))
        tiers = _assign_one_layer(S, scores, 4, 16, budget, 0)
        counts = tuple(int((tiers == t).sum()) for t in (TIER_FP16, TIER_INT4, TIER_INT2))
        host.apply_tier_assignment(0, tiers)
        if tiers_on == "cpu":
            devc.apply_tier_assignment(0, tiers)
        elif tiers_on == "cuda":
            devc.apply_tier_assignment(0, tiers.to(dev))
        else:
            devc.apply_tier_assignment(0, tiers.to(dev), counts=counts)
        assert devc._last_reassign_counts is not None, "device path not taken"
        c = devc._last_reassign_counts.cpu().tolist()
        assert c[:3] == [counts[0], counts[1], counts[0] + counts[1]] and c[3] == 0
        _same(host, devc, f"round {rnd}")
        devc._last_reassign_counts = None
        _append((host, devc), B, H, 37 + 11 * rnd, 10 + rnd, dev)
        _same(host, devc, f"append after round {rnd}")


def test_reassign_device_decode_matches(dev):
    """Decode attention after a device reassignment equals the one after the host path."""
    print("case reassign decode", flush=True)
    host, devc = _pair(n_sink=4, recent_window=32, int4_budget=100, int2_budget=0)
    _append((host, devc), 2, 2, 400, 3, dev)
    S = host.get_seq_length(0)
    scores = torch.from_numpy(np.random.default_rng(1).exponential(size=S).astype(np.float32))
    tiers = _assign_one_layer(S, scores, 4, 32, 100, 0)
    host.apply_tier_assignment(0, tiers)
    devc.apply_tier_assignment(0, tiers)
    q = torch.randn(2, 8, 1, 128, generator=torch.Generator().manual_seed(9)).half().to(dev)
    assert torch.equal(host.decode_attention(q, 0), devc.decode_attention(q, 0))


def test_reassign_device_no_host_sync(dev):
    """Host tiers: plan, gather and requantization run without a host synchronization."""
    print("case reassign no sync", flush=True)
    (devc,) = _pair(n_sink=4, recent_window=16, int4_budget=30, int2_budget=0)[1:]
    _append((devc,), 1, 2, 120, 4, dev)
    S = devc.get_seq_length(0)
    tiers = _assign_one_layer(S, torch.arange(S, dtype=torch.float32), 4, 16, 30, 0)
    devc._rope_tables(devc._layers[0].next_position, dev)  # table upload done up front
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        devc.apply_tier_assignment(0, tiers)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    assert devc._last_reassign_counts is not None
    assert devc.get_seq_length(0) == 4 + 16 + 30


def test_reassign_int2_falls_back(dev):
    """An assignment with INT2 tokens takes the host path (device path declines it)."""
    print("case reassign int2 fallback", flush=True)
    host, devc = _pair(n_sink=2, recent_window=8, int4_budget=10, int2_budget=5)
    _append((host, devc), 1, 2, 60, 6, dev)
    S = host.get_seq_length(0)
    tiers = _assign_one_layer(S, torch.arange(S, dtype=torch.float32), 2, 8, 10, 5)
    assert int((tiers == TIER_INT2).sum()) == 5 and int((tiers == TIER_EVICT).sum()) > 0
    host.apply_tier_assignment(0, tiers)
    devc.apply_tier_assignment(0, tiers.to(dev))
    assert devc._last_reassign_counts is None
    _same(host, devc, "int2")
    assert devc._layers[0].int2_actual_count == 5
