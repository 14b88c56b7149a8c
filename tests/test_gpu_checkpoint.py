"""The reference's checkpoint contract (tests/test_checkpoint.py:27-120, fade/cache.py:485-559)
on the GPU cache, plus what the build adds to it: decoding continues after a load, byte
counts survive it, and the layers the reference has no form for (backend-compressed middle
tiers, the ragged and paged layouts) round-trip through extra keys.

Differences from the reference's tests: fp16 tensors on the GPU (the reference's are fp32 on
the CPU) and head_dim 64 (the reference's 32 is below the quantizers' 64 / 128 / 256)."""

import pytest
import torch

from fade_amd.backends import AsymGroupBackend, RotatedINT4Backend
from fade_amd.cache import TIER_EVICT, TIER_FP16, TIER_INT2, TIER_INT4, TieredKVCache
from fade_amd.policy import _assign_one_layer

pytestmark = pytest.mark.gpu
B, H, D = 1, 2, 64


def _make_cache(**kw) -> TieredKVCache:
    defaults = dict(n_sink=2, recent_window=3, int4_budget=None, int2_budget=0, rope_theta=10000.0, head_dim=D)
    defaults.update(kw)
    return TieredKVCache(**defaults)


def _kv(dev, n, b=B, h=H, d=D, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(b, h, n, d, generator=g).half().to(dev), torch.randn(b, h, n, d, generator=g).half().to(dev))


def test_round_trip_fp16_only(dev):
    """tests/test_checkpoint.py:27-49."""
    cache = _make_cache()
    k, v = _kv(dev, 8)
    cache.update(k, v, layer_idx=0)
    sd = cache.cache_state_dict()
    assert sd["n_layers"] == 1 and "layer.0.fp16_k" in sd
    cache2 = _make_cache()
    cache2.load_cache_state_dict(sd, device=dev)
    assert cache2.get_seq_length(0) == 8
    for a, b in zip(cache._materialize(0), cache2._materialize(0)):
        assert torch.equal(a, b)


def test_round_trip_with_int4(dev):
    """tests/test_checkpoint.py:52-86 (the materialized cache is now bit-identical)."""
    cache = _make_cache()
    k, v = _kv(dev, 10, seed=1)
    cache.update(k, v, layer_idx=0)
    F4, I4 = TIER_FP16, TIER_INT4
    cache.apply_tier_assignment(0, torch.tensor([F4, F4, I4, I4, I4, I4, I4, F4, F4, F4]))
    sd = cache.cache_state_dict()
    assert "layer.0.int4_kq" in sd and "layer.0.int4_ks" in sd
    cache2 = _make_cache()
    cache2.load_cache_state_dict(sd, device=dev)
    assert cache2.get_seq_length(0) == 10
    for a, b in zip(cache._materialize(0), cache2._materialize(0)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_round_trip_typed_cache_with_int4_and_int2(dev, dtype):
    """tests/test_checkpoint.py:52-86 on a bfloat16 / float32 cache (the reference's
    own tests run fp32): tiers, scales and the materialized cache keep the dtype
    and come back bit-identical, after eviction and with an INT2 tier."""
    print(f"case checkpoint {dtype}", flush=True)
    kw = dict(dtype=dtype, int4_budget=4, int2_budget=64)
    cache = _make_cache(**kw)
    k, v = _kv(dev, 200, seed=5)
    cache.update(k.to(dtype), v.to(dtype), layer_idx=0)
    g = torch.Generator().manual_seed(6)
    cache.apply_tier_assignment(0, _assign_one_layer(200, torch.rand(200, generator=g), 2, 3, 4, 64))
    st = cache._layers[0]
    assert st.int2_kq is not None and st.int2_ks.dtype == dtype and st.int4_ks.dtype == dtype
    sd = cache.cache_state_dict()
    assert sd["dtype"] == str(dtype)
    cache2 = _make_cache(**kw)
    cache2.load_cache_state_dict(sd, device=dev)
    assert cache2.get_seq_length(0) == cache.get_seq_length(0)
    for a, b in zip(cache._materialize(0), cache2._materialize(0)):
        assert a.dtype == dtype and torch.equal(a, b)


def test_excludes_dequant_caches(dev):
    """tests/test_checkpoint.py:89-106."""
    cache = _make_cache()
    k, v = _kv(dev, 8, seed=2)
    cache.update(k, v, layer_idx=0)
    F4, I4 = TIER_FP16, TIER_INT4
    cache.apply_tier_assignment(0, torch.tensor([F4, F4, I4, I4, I4, I4, F4, F4]))
    cache._materialize(0)  # populates the dequant cache
    assert cache._layers[0].int4_k_deq is not None
    for key in cache.cache_state_dict():
        assert "_deq" not in key, key


def test_preserves_scalars(dev):
    """tests/test_checkpoint.py:109-120."""
    cache = _make_cache()
    k, v = _kv(dev, 6, seed=3)
    cache.update(k, v, layer_idx=0)
    sd = cache.cache_state_dict()
    assert sd["layer.0.sink_count"] == 0 and sd["layer.0.next_position"] == 6
    cache2 = _make_cache()
    cache2.load_cache_state_dict(sd, device=dev)
    assert cache2._layers[0].next_position == 6


def _continue_equal(dev, c1, c2, steps=3, hq=4, seed=9, same_bytes=True):
    """Appending the same tokens to the original and the restored cache, the decode outputs,
    the materialized tiers and the compressed byte counts stay identical."""
    b, h = c1._layers[0].fp16_k.shape[:2] if c1._layers[0].fp16_k is not None else (B, H)
    if same_bytes:
        assert c1.compressed_storage_bytes() == c2.compressed_storage_bytes()
    g = torch.Generator().manual_seed(seed)
    for _ in range(steps):
        k = torch.randn(b, h, 1, c1.head_dim, generator=g).half().to(dev)
        v = torch.randn(b, h, 1, c1.head_dim, generator=g).half().to(dev)
        q = torch.randn(b, hq, 1, c1.head_dim, generator=g).half().to(dev)
        c1.update(k, v, 0)
        c2.update(k, v, 0)
        o1, o2 = c1.decode_attention(q, 0), c2.decode_attention(q, 0)
        if not (torch.equal(o1, o2) or (o1.float() - o2.float()).abs().max() <= 1e-3):
            # which (row, head) differs, and which cache's output changes when decoded again
            d = (o1.float() - o2.float()).abs().amax(dim=(2, 3)).cpu()
            r1, r2 = c1.decode_attention(q, 0), c2.decode_attention(q, 0)
            raise AssertionError(
                f"decode outputs differ; per (row, head) max diff {d.tolist()}; "
                f"decoded again: |o1 - r1| {(o1.float() - r1.float()).abs().max().item()}, "
                f"|o2 - r2| {(o2.float() - r2.float()).abs().max().item()}, "
                f"|r1 - r2| {(r1.float() - r2.float()).abs().max().item()}"
            )
    for a, b_ in zip(c1._materialize(0), c2._materialize(0)):
        assert torch.equal(a, b_)


def test_decode_continues_after_load_with_int4_and_int2(dev):
    """A cache with sink, INT4, INT2 and recent tiers (D=128 for the fused decode): saved,
    restored, then both continue decoding with the same new tokens."""
    c1 = _make_cache(head_dim=128, int4_budget=40, int2_budget=64, recent_window=16, n_sink=4)
    k, v = _kv(dev, 200, h=2, d=128, seed=4)
    c1.update(k, v, 0)
    scores = torch.rand(200, generator=torch.Generator().manual_seed(5))
    c1.apply_tier_assignment(0, _assign_one_layer(200, scores, 4, 16, 40, 64))
    st = c1._layers[0]
    assert st.int2_kq is not None and st.int4_kq is not None
    sd = c1.cache_state_dict()
    assert "layer.0.int2_kq" in sd and sd["layer.0.int2_actual_count"] == 64
    c2 = _make_cache(head_dim=128, int4_budget=40, int2_budget=64, recent_window=16, n_sink=4)
    c2.load_cache_state_dict(sd, device=dev)
    _continue_equal(dev, c1, c2)


@pytest.mark.parametrize("backend", ["rotated", "asym"])
def test_backend_middle_round_trip(dev, backend):
    """Backend-compressed middle tiers (no reference key) survive a round trip."""
    be = RotatedINT4Backend(head_dim=128, bits=4) if backend == "rotated" else AsymGroupBackend(head_dim=128)
    mk = lambda: _make_cache(head_dim=128, recent_window=16, n_sink=4, quant_backend=be)  # noqa: E731
    c1 = mk()
    k, v = _kv(dev, 150, h=2, d=128, seed=6)
    c1.update(k, v, 0)
    c1.apply_tier_assignment(0, _assign_one_layer(150, torch.zeros(150), 4, 16, None, 0))
    assert c1._layers[0].backend_k is not None
    sd = c1.cache_state_dict()
    assert any(key.startswith("layer.0.backend_k.") for key in sd)
    c2 = mk()
    c2.load_cache_state_dict(sd, device=dev)
    _continue_equal(dev, c1, c2)


@pytest.mark.parametrize("paged", [False, True])
def test_ragged_layout_round_trip(dev, paged):
    """The ragged layout (per-row tier lengths; optionally a paged middle tier) is saved as
    padded tensors plus layer.{i}.lens, restored unpaged, and decodes the same."""
    from fade_amd.pages import MiddlePagePool

    mk = lambda: _make_cache(head_dim=128, recent_window=16, n_sink=4, int4_budget=60)  # noqa: E731
    c1 = mk()
    c1.ragged_layout = True
    if paged:
        c1.page_pool = MiddlePagePool(n_pages=64, n_kv_heads=2, head_dim=128, device=dev)
    k, v = _kv(dev, 300, b=3, h=2, d=128, seed=7)
    c1.update(k, v, 0)
    g = torch.Generator().manual_seed(8)
    tiers = torch.stack([_assign_one_layer(300, torch.rand(300, generator=g), 4, 16, 60 - 10 * r, 0) for r in range(3)])
    c1.apply_tier_assignment_per_sequence(0, tiers)
    assert c1._layers[0].lens is not None and (c1._layers[0].mid_table is not None) == paged
    sd = c1.cache_state_dict()
    assert "layer.0.lens" in sd
    c2 = mk()
    c2.load_cache_state_dict(sd, device=dev)
    # a paged middle tier is restored as padded tensors: its byte count is the padded one
    assert c2._layers[0].mid_table is None
    if paged:
        st2 = c2._layers[0]
        padded = sum(int(t.numel() * t.element_size()) for t in (st2.int4_kq, st2.int4_vq, st2.int4_vs))
        assert c2.compressed_storage_bytes() - c1.compressed_storage_bytes() == padded - c1._layers[0].mid_page_bytes
    _continue_equal(dev, c1, c2, hq=8, same_bytes=not paged)
