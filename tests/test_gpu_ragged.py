"""Per-sequence (ragged) tier assignment: the reference's pins (tests/test_ragged.py:27-128),
same shapes and tier patterns, on fp16 GPU tensors, for the reference's zero-padded mode
and for the ragged layout (``ragged_layout``: rows keep exactly their own tokens).  head_dim
is 64 instead of the reference's 32: the quantizers are built for 64, 128 and 256."""

import pytest
import torch

from fade_amd.cache import TIER_EVICT, TIER_FP16, TIER_INT4, TieredKVCache

pytestmark = pytest.mark.gpu
B, H, D = 2, 2, 64
F, I, E = TIER_FP16, TIER_INT4, TIER_EVICT


def _make_cache(ragged, **kw):
    defaults = dict(n_sink=2, recent_window=2, int4_budget=None, int2_budget=0, rope_theta=10000.0, head_dim=D)
    defaults.update(kw)
    c = TieredKVCache(**defaults)
    c.ragged_layout = ragged
    return c


def _kv(S, dev, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, H, S, D, generator=g).half().to(dev), torch.randn(B, H, S, D, generator=g).half().to(dev)


@pytest.mark.parametrize("ragged", [False, True])
def test_per_sequence_no_eviction(dev, ragged):
    """tests/test_ragged.py:27-43."""
    cache = _make_cache(ragged)
    cache.update(*_kv(8, dev), layer_idx=0)
    tiers = torch.tensor([F, F, I, I, I, I, F, F])
    cache.apply_tier_assignment_per_sequence(0, tiers.unsqueeze(0).expand(B, -1).contiguous())
    assert cache.get_seq_length(0) == 8
    k_out, _ = cache._materialize(0)
    assert k_out.shape == (B, H, 8, D)


@pytest.mark.parametrize("ragged", [False, True])
def test_per_sequence_different_eviction(dev, ragged):
    """tests/test_ragged.py:46-68: row 0 evicts two middle tokens, row 1 none."""
    cache = _make_cache(ragged)
    cache.update(*_kv(8, dev, 1), layer_idx=0)
    row0 = torch.tensor([F, F, E, E, I, I, F, F])
    row1 = torch.tensor([F, F, I, I, I, I, F, F])
    cache.apply_tier_assignment_per_sequence(0, torch.stack([row0, row1]))
    k_out, _ = cache._materialize(0)
    assert k_out.shape[0] == B
    assert k_out.shape[-2] >= 6
    if ragged:
        assert cache._layers[0].lens_host == [[2, 2, 2], [2, 4, 2]]
        assert not k_out[0, :, 6:].any()  # row 0 keeps 6 tokens, the rest is padding


@pytest.mark.parametrize("ragged", [False, True])
def test_per_sequence_all_eviction_one_row(dev, ragged):
    """tests/test_ragged.py:71-87."""
    cache = _make_cache(ragged, n_sink=1, recent_window=1)
    cache.update(*_kv(6, dev, 2), layer_idx=0)
    row0 = torch.tensor([F, E, E, E, E, F])
    row1 = torch.tensor([F, E, I, I, E, F])
    cache.apply_tier_assignment_per_sequence(0, torch.stack([row0, row1]))
    k_out, _ = cache._materialize(0)
    assert k_out.shape[0] == B
    assert torch.isfinite(k_out).all()


@pytest.mark.parametrize("ragged", [False, True])
def test_per_sequence_shape_validation(dev, ragged):
    """tests/test_ragged.py:90-104."""
    cache = _make_cache(ragged)
    cache.update(*_kv(6, dev, 3), layer_idx=0)
    bad_tiers = torch.full((3, 6), F, dtype=torch.long)
    with pytest.raises(ValueError, match="B=2"):
        cache.apply_tier_assignment_per_sequence(0, bad_tiers)


@pytest.mark.parametrize("ragged", [False, True])
def test_per_sequence_decode_after_ragged_eviction(dev, ragged):
    """tests/test_ragged.py:107-128."""
    cache = _make_cache(ragged)
    cache.update(*_kv(8, dev, 4), layer_idx=0)
    row0 = torch.tensor([F, F, E, I, I, I, F, F])
    row1 = torch.tensor([F, F, I, I, I, I, F, F])
    cache.apply_tier_assignment_per_sequence(0, torch.stack([row0, row1]))
    k2, v2 = _kv(1, dev, 5)
    k_out, _ = cache.update(k2, v2, layer_idx=0)
    assert k_out.shape[0] == B
    assert torch.isfinite(k_out).all()
    if ragged:
        assert cache._layers[0].lens_host == [[2, 3, 3], [2, 4, 3]]
        assert torch.equal(k_out[0, :, 7], k2[0, :, 0]) and torch.equal(k_out[1, :, 8], k2[1, :, 0])
