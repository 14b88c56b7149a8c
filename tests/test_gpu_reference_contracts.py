"""The reference's own contract tests for this path, run against the HIP build:
fade tests/test_quant.py, tests/test_backends.py, tests/test_cache.py, tests/test_cache_batched.py,
tests/test_attn_impl.py and tests/test_perf.py (file:line on each test).  Same
calls, shapes and bounds, with one difference: the build's caches and kernels are
float16 on the GPU (the reference tests use float32 on the CPU), so every tensor
here is fp16 on cuda:0, except in the INT4 quantizer tests that the reference
runs on bfloat16 and float32 (those dtypes are quantized natively).  The one
fp32-precision bar (K of fp16 survivors within 1e-4) holds as it is: without an
eviction nothing is re-RoPE'd.  Bit-level parity is pinned elsewhere against the
oracle; these pin the contracts."""

import pytest
import torch

from fade_amd.cache import TIER_EVICT, TIER_FP16, TIER_INT2, TIER_INT4, TieredKVCache
from fade_amd.kernels import int4_sdpa
from fade_amd.quant import (
    dequant_int4,
    dequant_k_int2,
    dequant_v_int2,
    pad_to_group,
    quant_k_int2,
    quant_k_int4,
    quant_v_int2,
    quant_v_int4,
)

pytestmark = pytest.mark.gpu

B, H, S, D = 1, 4, 128, 64  # tests/test_quant.py:25
F16 = torch.float16


def _rel(a, b):  # tests/test_quant.py:29-30
    a, b = a.float(), b.float()
    return (a - b).abs().mean().item() / a.abs().mean().item()


def _randn(*shape, dev):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(sum(shape))).to(F16).to(dev)


# ---------------------------------------------------------------- tests/test_quant.py
def test_quant_k_int4_roundtrip(dev):  # :33-44
    k = _randn(B, H, S, D, dev=dev)
    q, scale = quant_k_int4(k)
    assert q.shape == (B, H, S, D // 2) and q.dtype == torch.uint8
    assert scale.shape == (B, H, 1, D)
    k_hat = dequant_int4(q, scale, dtype=F16)
    assert k_hat.shape == k.shape and _rel(k, k_hat) < 0.15


def test_quant_v_int4_roundtrip(dev):  # :47-55
    v = _randn(B, H, S, D, dev=dev)
    q, scale = quant_v_int4(v)
    assert q.shape == (B, H, S, D // 2) and q.dtype == torch.uint8
    assert scale.shape == (B, H, S, 1)
    v_hat = dequant_int4(q, scale, dtype=F16)
    assert v_hat.shape == v.shape and _rel(v, v_hat) < 0.15


def test_int4_odd_last_dim_rejected(dev):  # :58-65
    with pytest.raises(ValueError):
        quant_k_int4(_randn(B, H, S, 15, dev=dev))


@pytest.mark.parametrize("which", ["k", "v"])
def test_quant_int2_roundtrip(dev, which):  # :68-80, :92-100
    x = _randn(B, H, S, D, dev=dev)
    quant, deq = (quant_k_int2, dequant_k_int2) if which == "k" else (quant_v_int2, dequant_v_int2)
    q, scale = quant(x, group_size=64)
    assert q.shape == x.shape and scale.shape == (B, H, S // 64, D)
    x_hat = deq(q, scale, group_size=64, dtype=F16)
    assert torch.isfinite(x_hat).all() and _rel(x, x_hat) < 1.1


@pytest.mark.parametrize("which", ["k", "v"])
def test_quant_int2_requires_divisible_group(dev, which):  # :83-89, :103-108
    quant = quant_k_int2 if which == "k" else quant_v_int2
    with pytest.raises(ValueError):
        quant(_randn(B, H, 100, D, dev=dev), group_size=64)


def test_quant_k_int4_bf16_roundtrip(dev):  # :110-124
    k = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(110)).to(torch.bfloat16).to(dev)
    q, scale = quant_k_int4(k)
    assert q.dtype == torch.uint8
    assert scale.dtype == torch.bfloat16
    k_hat = dequant_int4(q, scale, dtype=torch.bfloat16)
    assert k_hat.dtype == torch.bfloat16
    assert torch.isfinite(k_hat).all()
    assert _rel(k.float(), k_hat.float()) < 0.2


def test_quant_v_int4_bf16_roundtrip(dev):  # :127-132
    v = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(127)).to(torch.bfloat16).to(dev)
    q, scale = quant_v_int4(v)
    v_hat = dequant_int4(q, scale, dtype=torch.bfloat16)
    assert torch.isfinite(v_hat).all()
    assert _rel(v.float(), v_hat.float()) < 0.2


def test_quant_handles_tiny_absmax_without_nan(dev):  # :135-141
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        k = torch.zeros(B, H, S, D, dtype=dtype, device=dev)
        q, scale = quant_k_int4(k)
        k_hat = dequant_int4(q, scale, dtype=dtype)
        assert torch.isfinite(k_hat).all(), f"NaN in {dtype} zero round-trip"


def test_quant_rejects_non_float_kv_dtypes(dev):  # no reference counterpart: dtypes outside fp16/bf16/fp32
    for dtype in (torch.float64, torch.int8):
        with pytest.raises(ValueError):
            quant_k_int4(torch.zeros(B, H, S, D, dtype=dtype, device=dev))


def test_pad_to_group(dev):  # :144-154
    x = _randn(B, H, 50, D, dev=dev)
    padded, actual = pad_to_group(x, 64)
    assert actual == 50 and padded.shape[-2] == 64 and torch.equal(padded[..., :50, :], x)
    y = _randn(B, H, 128, D, dev=dev)
    padded2, actual2 = pad_to_group(y, 64)
    assert actual2 == 128 and padded2.shape[-2] == 128


# ------------------------------------------------------------- tests/test_backends.py
def test_int4_backend_round_trip(dev):  # :19-38 (float32 K/V, as the reference's DTYPE)
    from fade_amd.backends import SymmetricINT4Backend

    backend = SymmetricINT4Backend()
    gen = torch.Generator().manual_seed(19)
    k = torch.randn(1, 2, 16, 64, generator=gen).to(dev)
    v = torch.randn(1, 2, 16, 64, generator=gen).to(dev)
    ck, cv = backend.compress_k(k), backend.compress_v(v)
    assert "packed" in ck and "scale" in ck and "packed" in cv and "scale" in cv
    k_hat = backend.decompress_k(ck, dtype=torch.float32)
    v_hat = backend.decompress_v(cv, dtype=torch.float32)
    assert k_hat.shape == k.shape and v_hat.shape == v.shape
    assert ((k - k_hat).abs().mean() / k.abs().mean()).item() < 0.15
    assert ((v - v_hat).abs().mean() / v.abs().mean()).item() < 0.15


def test_rotated_backend_round_trip_float32_and_bf16(dev):  # no reference test: the same bar for the rotated backend
    from fade_amd.backends import get_backend

    be = get_backend("rotated", head_dim=64, bits=4)
    for dtype in (torch.float32, torch.bfloat16):
        k = torch.randn(1, 2, 16, 64, generator=torch.Generator().manual_seed(7)).to(dtype).to(dev)
        ck = be.compress_k(k)
        assert ck["scale"].dtype == dtype
        k_hat = be.decompress_k(ck, dtype=dtype)
        assert k_hat.dtype == dtype and torch.isfinite(k_hat).all()
        assert ((k.float() - k_hat.float()).abs().mean() / k.float().abs().mean()).item() < 0.15


def test_backend_registry_and_cache_field(dev):  # :41-52, :55-63, :87-100
    from fade_amd.backends import SymmetricINT4Backend, get_backend
    from fade_amd.config import FadeConfig

    assert SymmetricINT4Backend().name == "symmetric_int4"
    assert isinstance(get_backend("int4"), SymmetricINT4Backend)
    with pytest.raises(ValueError, match="Unknown"):
        get_backend("nonexistent")
    with pytest.raises(ImportError):  # turboquant-kv is not installed: the reference's test skips
        get_backend("turbo", head_dim=64, bits=4).compress_k(torch.zeros(1, 2, 16, 64, device=dev))
    c = FadeConfig.safe()
    assert c.quant_backend == "int4" and "quant_backend" in c.to_cache_kwargs()
    assert TieredKVCache(head_dim=64, quant_backend="int4")._quant_backend.name == "symmetric_int4"


# ---------------------------------------------------------------- tests/test_cache.py
CH, CD = 2, 32  # tests/test_cache.py:22


def _cache(**kw):  # tests/test_cache.py:27-36
    args = dict(n_sink=2, recent_window=3, int4_budget=None, int2_budget=0, rope_theta=10000.0, head_dim=CD)
    args.update(kw)
    return TieredKVCache(**args)


def _cos_sin(positions, dev):  # the model's [1, S, D] RoPE tables (textbook RoPE, theta 1e4)
    inv = 1.0 / (10000.0 ** (torch.arange(0, CD, 2, dtype=torch.float32) / CD))
    emb = positions.float()[:, None] * inv[None]
    emb = torch.cat((emb, emb), dim=-1)
    return emb.cos()[None].to(dev), emb.sin()[None].to(dev)


def _rope(x, cos, sin):
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return (x.float() * cos[:, None] + rot.float() * sin[:, None]).to(F16)


def _filled(n, dev, batch=1):
    k = _randn(batch, CH, n, CD, dev=dev)
    v = _randn(batch, CH, n + 1, CD, dev=dev)[:, :, :n].contiguous()
    cos, sin = _cos_sin(torch.arange(n), dev)
    k_rope = _rope(k, cos, sin)
    return k_rope, v, {"cos": cos, "sin": sin}


def test_tier_assignment_splits_storage(dev):  # tests/test_cache.py:90-117
    cache = _cache()
    k, v, kw = _filled(10, dev)
    cache.update(k, v, 0, kw)
    t = [TIER_FP16] * 2 + [TIER_INT4] * 5 + [TIER_FP16] * 3
    cache.apply_tier_assignment(0, torch.tensor(t))
    st = cache._layers[0]
    n_sink = 0 if st.sink_k is None else st.sink_k.shape[-2]
    n_recent = 0 if st.fp16_k is None else st.fp16_k.shape[-2]
    assert n_sink + n_recent == 5 and st.int4_kq.shape[-2] == 5 and cache.get_seq_length(0) == 10


def test_materialize_preserves_fp16_positions(dev):  # tests/test_cache.py:119-142
    cache = _cache()
    k_rope, v, kw = _filled(8, dev)
    cache.update(k_rope, v, 0, kw)
    cache.apply_tier_assignment(0, torch.tensor([TIER_FP16] * 2 + [TIER_INT4] * 4 + [TIER_FP16] * 2))
    k_out, v_out = cache._materialize(0)
    assert k_out.shape == (1, CH, 8, CD)
    assert torch.equal(v_out[:, :, :2], v[:, :, :2]) and torch.equal(v_out[:, :, -2:], v[:, :, -2:])
    # nothing is evicted: the fp16 survivors keep their positions and come back as stored
    assert (k_out[:, :, :2].float() - k_rope[:, :, :2].float()).abs().max().item() < 1e-4


def test_eviction_shrinks_then_appends(dev):  # tests/test_cache.py:199-227
    cache = _cache()
    k_rope, v, kw = _filled(8, dev)
    cache.update(k_rope, v, 0, kw)
    cache.apply_tier_assignment(0, torch.tensor([TIER_FP16] * 2 + [TIER_EVICT] * 2 + [TIER_INT4] * 2 + [TIER_FP16] * 2))
    assert cache.get_seq_length(0) == 6
    cos, sin = _cos_sin(torch.tensor([6]), dev)
    k_new = _rope(_randn(1, CH, 1, CD, dev=dev), cos, sin)
    k_out, _ = cache.update(k_new, _randn(1, CH, 1, CD + 1, dev=dev)[..., :CD].contiguous(), 0, {"cos": cos, "sin": sin})
    assert k_out.shape == (1, CH, 7, CD) and cache.get_seq_length(0) == 7


def test_mixed_int4_int2_middle_ordering(dev):  # tests/test_cache.py:264-305
    cache = _cache(n_sink=1, recent_window=1)
    n = 130
    k_rope, v, kw = _filled(n, dev)
    cache.update(k_rope, v, 0, kw)
    tiers = torch.full((n,), TIER_INT4, dtype=torch.long)
    tiers[0] = tiers[-1] = TIER_FP16
    tiers[2 : n - 1 : 2] = TIER_INT2
    cache.apply_tier_assignment(0, tiers)
    st = cache._layers[0]
    assert st.int4_kq is not None and st.int2_kq is not None and cache.get_seq_length(0) == n
    k_out, _ = cache._materialize(0)
    assert k_out.shape == (1, CH, n, CD)
    _, _, pos = cache._all_in_position_order(0)
    assert ((pos[1:] - pos[:-1]) > 0).all()


# ------------------------------------------------------- tests/test_cache_batched.py
def test_tier_assignment_batched_splits_storage(dev):  # tests/test_cache_batched.py:87-123
    cache = _cache()
    k, v, kw = _filled(10, dev, batch=3)
    cache.update(k, v, 0)
    cache.apply_tier_assignment(0, torch.tensor([TIER_FP16] * 2 + [TIER_INT4] * 5 + [TIER_FP16] * 3))
    st = cache._layers[0]
    n_sink = 0 if st.sink_k is None else st.sink_k.shape[-2]
    n_recent = 0 if st.fp16_k is None else st.fp16_k.shape[-2]
    assert n_sink + n_recent == 5 and st.fp16_k.shape[0] == 3
    assert st.int4_kq.shape == (3, CH, 5, CD // 2)
    assert st.int4_ks.shape == (3, CH, 1, CD) and st.int4_vs.shape == (3, CH, 5, 1)
    assert cache.get_seq_length(0) == 10


def test_batch_size_pinned_and_input_checks(dev):  # tests/test_cache_batched.py:230-272
    cache = _cache()
    assert cache.batch_size is None
    cache.update(_randn(2, CH, 4, CD, dev=dev), _randn(2, CH, 4, CD, dev=dev), 0)
    assert cache.batch_size == 2
    with pytest.raises(ValueError, match="batch size mismatch"):
        _cache(batch_size=2).update(_randn(3, CH, 4, CD, dev=dev), _randn(3, CH, 4, CD, dev=dev), 0)
    with pytest.raises(ValueError, match="K/V shape mismatch"):
        _cache().update(_randn(2, CH, 4, CD, dev=dev), _randn(2, CH, 5, CD, dev=dev), 0)
    with pytest.raises(ValueError, match=r"\[B, H, S, D\]"):
        _cache().update(_randn(CH, 4, CD, dev=dev), _randn(CH, 4, CD, dev=dev), 0)


# ---------------------------------------------------------- tests/test_attn_impl.py
def test_position_budget_arithmetic(dev):  # tests/test_attn_impl.py:67-102 (cache side)
    from fade_amd.policy import reassign_tiers_by_position

    cache = _cache(n_sink=2, recent_window=4, int4_budget=4, int2_budget=0)
    k, v, _ = _filled(20, dev)
    cache.update(k, v, 0)
    reassign_tiers_by_position(cache, 1)
    # 20 - 2 sinks - 4 recent = 14 middle: 4 INT4, 10 evicted
    assert cache._layers[0].int4_kq.shape[-2] == 4 and cache.get_seq_length(0) == 2 + 4 + 4


# --------------------------------------------------------------- tests/test_perf.py
def test_int4_sdpa_matches_full_precision_attention(dev):  # tests/test_perf.py:163-180
    q = _randn(1, 4, 1, 128, dev=dev)
    k = _randn(1, 4, 32, 128, dev=dev)
    v = _randn(1, 4, 33, 128, dev=dev)[:, :, :32].contiguous()
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    kp, ks = quant_k_int4(k)
    vp, vs = quant_v_int4(v)
    out = int4_sdpa(q, kp, ks, vp, vs, dtype=F16)
    rel = ((out.float() - ref).abs().mean() / ref.abs().mean()).item()
    assert rel < 0.3
