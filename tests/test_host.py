"""Host-side logic that runs without a GPU: config, backends registry, RoPE
scheme detection and tables, tier policy, cache contracts, and the rule that
the kernels refuse CPU tensors instead of falling back."""

import types

import numpy as np
import pytest
import torch

import fade_amd
from fade_amd import FadeConfig, TieredKVCache, get_backend
from fade_amd import rope as frope
from fade_amd.policy import _assign_one_layer
from oracle import policy as opol
from oracle import rope as orope


def test_config_presets_and_validation():
    assert FadeConfig.safe().int4_budget is None
    b = FadeConfig.balanced()
    assert (b.phase, b.int4_budget, b.recent_window) == ("2", 400, 64)
    assert FadeConfig.aggressive().int4_budget == 200
    with pytest.raises(ValueError, match="requires int4_budget=None"):
        FadeConfig(phase="1a", int4_budget=10)
    with pytest.raises(ValueError, match="at least one of"):
        FadeConfig(phase="2")
    with pytest.raises(ValueError, match="n_sink must be >= 0"):
        FadeConfig(n_sink=-1)
    with pytest.raises(ValueError, match="middle_v_bits must be 4 or 2"):
        FadeConfig(middle_v_bits=3)
    assert b.with_overrides(int4_budget=100).int4_budget == 100
    kw = b.to_cache_kwargs()
    assert kw["int4_budget"] == 400 and kw["quant_backend"] == "int4"


def test_backend_registry():
    assert get_backend("int4").name == "symmetric_int4"
    assert get_backend("rotated", head_dim=128, bits=2).name == "rotated_int2"
    assert get_backend("int4_asym_g32").name == "int4_asym_g32"
    with pytest.raises(ValueError, match="Unknown quant backend"):
        get_backend("nope")
    with pytest.raises(ImportError, match="turboquant"):
        get_backend("turbo").compress_k(torch.zeros(1, 1, 1, 8))
    assert isinstance(get_backend("int4"), fade_amd.QuantBackend)


def test_rope_scheme_detection():
    ns = types.SimpleNamespace
    assert isinstance(frope.extract_rope_scheme(ns(rope_theta=1e6, hidden_size=128, num_attention_heads=1)), frope.Vanilla)
    s = frope.extract_rope_scheme(
        ns(rope_theta=5e5, head_dim=128, rope_scaling={"rope_type": "llama3", "factor": 8.0,
                                                        "original_max_position_embeddings": 8192})
    )
    assert isinstance(s, frope.Llama3) and s.factor == 8.0
    assert isinstance(frope.extract_rope_scheme(ns(alibi=True, head_dim=64)), frope.NoRope)
    assert isinstance(
        frope.extract_rope_scheme(ns(head_dim=64, rope_scaling={"type": "linear", "factor": 2.0})), frope.LinearScaled
    )
    assert isinstance(frope.extract_rope_scheme(ns(head_dim=64, rope_scaling={"type": "yarn", "factor": 4.0})), frope.Yarn)


def test_llama3_bands_match_closed_form():
    """High-frequency band unchanged, low-frequency band divided by factor (fade/rope.py:127-157)."""
    s = frope.Llama3(theta=5e5, head_dim=128, factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                     original_max_position_embeddings=8192)
    base = frope._vanilla_inv_freq(128, 5e5)
    inv = s.inv_freq()
    wl = 2 * np.pi / base.numpy()
    hi = wl < 8192 / 4.0
    lo = wl > 8192 / 1.0
    assert torch.equal(inv[torch.from_numpy(hi)], base[torch.from_numpy(hi)])
    assert torch.allclose(inv[torch.from_numpy(lo)], base[torch.from_numpy(lo)] / 8.0)


def test_host_tables_match_oracle_formula():
    s = frope.Vanilla(theta=1e6, head_dim=128)
    pos = torch.arange(4096)
    cos, sin = s.host_cos_sin(pos)
    inv = s.inv_freq().numpy()
    oc, osn = orope.cos_sin_tables(pos.numpy(), inv)
    assert cos.dtype == torch.float32 and cos.shape == (4096, 128)
    assert np.mean(cos.numpy() == oc) > 0.999 and np.abs(cos.numpy() - oc).max() <= 2 ** -11
    assert np.mean(sin.numpy() == osn) > 0.999 and np.abs(sin.numpy() - osn).max() <= 2 ** -11
    nc, ns_ = frope.NoRope(head_dim=8).host_cos_sin(torch.arange(3))
    assert torch.equal(nc, torch.ones(3, 8)) and torch.equal(ns_, torch.zeros(3, 8))


def test_assign_one_layer_matches_oracle_and_reference_kat():
    scores = torch.tensor([0.1, 0.2, 5.0, 4.0, 3.0, 0.5, 0.4, 0.3])
    t = _assign_one_layer(S=8, scores=scores, n_sink=1, recent_window=1, int4_budget=2, int2_budget=0)
    assert t.tolist()[0] == fade_amd.TIER_FP16 and t.tolist()[-1] == fade_amd.TIER_FP16
    assert set((t == fade_amd.TIER_INT4).nonzero().squeeze(-1).tolist()) == {2, 3}
    g = torch.Generator().manual_seed(3)
    for S, ns, nr, b4, b2 in ((4096, 4, 64, 400, 0), (300, 4, 32, 100, 50), (10, 4, 64, None, 0)):
        sc = -torch.log(torch.rand(S, generator=g))
        mine = _assign_one_layer(S, sc, ns, nr, b4, b2).numpy()
        assert np.array_equal(mine, opol.assign_one_layer(S, sc.numpy(), ns, nr, b4, b2))


def test_cache_contracts_without_gpu():
    c = TieredKVCache(n_sink=4, recent_window=8)
    assert len(c) == 0 and c.get_seq_length() == 0
    with pytest.raises(ValueError, match=r"\[B, H, S, D\]"):
        c.update(torch.zeros(2, 3, 4), torch.zeros(2, 3, 4), 0)
    with pytest.raises(ValueError, match="K/V shape mismatch"):
        c.update(torch.zeros(1, 2, 3, 8), torch.zeros(1, 2, 4, 8), 0)
    with pytest.raises(ValueError, match="float16, bfloat16 and float32"):
        TieredKVCache(dtype=torch.float64)
    assert TieredKVCache(dtype=torch.bfloat16).dtype == torch.bfloat16
    assert c.get_mask_sizes(5, 0) == (5, 0)


def test_kernels_refuse_cpu_tensors():
    from fade_amd.quant import quant_k_int4, quant_v_int4
    from fade_amd.rope import rerope_gather

    x = torch.zeros(1, 1, 8, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        quant_k_int4(x)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        quant_v_int4(x)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        rerope_gather(x, x, torch.arange(2), torch.ones(8, 128), torch.zeros(8, 128), torch.ones(2, 128),
                      torch.zeros(2, 128))


def test_fade_attention_registration_and_fused_update():
    """The "fade" attention/mask implementations are registered, the mask
    function rejects padding, and a fused cache's update() appends without
    materializing (host plumbing only; the kernels run in the GPU tests)."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface

    from fade_amd import TieredKVCache
    from fade_amd.hf_attention import active_cache, fade_mask

    assert "fade" in AttentionInterface._global_mapping
    assert "fade" in AttentionMaskInterface._global_mapping
    assert fade_mask(2, 1, 9, attention_mask=torch.ones(2, 9, dtype=torch.bool)) is None
    with pytest.raises(ValueError, match="padded"):
        fade_mask(2, 1, 9, attention_mask=torch.tensor([[1] * 9, [0] + [1] * 8], dtype=torch.bool))
    cache = TieredKVCache(n_sink=2, recent_window=4)
    cache.fused = True
    k = torch.randn(1, 2, 5, 128).half()
    v = torch.randn(1, 2, 5, 128).half()
    rk, rv = cache.update(k, v, 0)
    assert rk is k and rv is v
    assert cache.get_seq_length(0) == 5
    assert active_cache() is cache
    # the fused kernels read float16 and bfloat16 tiers: a float32 cache refuses fused mode
    from transformers import AutoConfig

    from fade_amd import create_tiered_cache

    cfg = AutoConfig.for_model("qwen2", hidden_size=256, num_attention_heads=2, num_key_value_heads=1,
                               num_hidden_layers=2, intermediate_size=512, vocab_size=100)
    cfg._attn_implementation = "fade"
    model = types.SimpleNamespace(config=cfg)
    with pytest.raises(ValueError, match="reads float16 and bfloat16 caches"):
        create_tiered_cache(model, dtype=torch.float32)
    assert create_tiered_cache(model).fused
    assert create_tiered_cache(model, dtype=torch.bfloat16).fused
    c32 = TieredKVCache(dtype=torch.float32)
    c32.fused = True
    with pytest.raises(NotImplementedError, match="bfloat16"):
        c32.update(k.float(), v.float(), 0)
    assert c32.get_seq_length(0) == 0 and c32.batch_size is None  # refused before any state changes
    cb = TieredKVCache(dtype=torch.bfloat16)
    cb.fused = True
    rk, _ = cb.update(k.bfloat16(), v.bfloat16(), 0)
    assert rk.dtype == torch.bfloat16 and cb.get_seq_length(0) == 5


def test_paginate_middle_pools_pages_on_host():
    """paginate_middle (host logic; runs on CPU tensors): every row's 64-token tiles land in
    the pool pages its block table names, in any page order, and the SYM K scale stays per row."""
    import torch

    from fade_amd.kernels.tiered_attn import MiddleTier, paginate_middle

    B, H, S = 3, 2, 150
    g = torch.Generator().manual_seed(0)
    kc = torch.randint(0, 256, (B, H, S, 64), generator=g, dtype=torch.uint8)
    vc = torch.randint(0, 256, (B, H, S, 64), generator=g, dtype=torch.uint8)
    ks = torch.rand(B, H, 1, 128, generator=g).half()
    vs = torch.rand(B, H, S, 1, generator=g).half()
    mid = MiddleTier("int4", kc, vc, ks, vs)
    lens = [150, 64, 1]
    order = [3, 0, 4, 1, 2]  # 3 + 1 + 1 pages, placed out of order
    p = paginate_middle(mid, lens, order=order)
    assert p.k_codes.shape == (5, H, 64, 64) and p.v_scale.shape == (5, H, 64, 1)
    assert p.k_scale is ks and p.length == 150
    assert p.pages.tolist() == [[3, 0, 4], [1, 0, 0], [2, 0, 0]]
    for b, n in enumerate(lens):
        for t in range(-(-n // 64)):
            pg = int(p.pages[b, t])
            rows = min(64, n - 64 * t)
            assert torch.equal(p.k_codes[pg, :, :rows], kc[b, :, 64 * t : 64 * t + rows])
            assert torch.equal(p.v_codes[pg, :, :rows], vc[b, :, 64 * t : 64 * t + rows])
            assert torch.equal(p.v_scale[pg, :, :rows], vs[b, :, 64 * t : 64 * t + rows])


def test_host_tier_counts_and_graph_split():
    import torch

    import bench
    from fade_amd.cache import TIER_EVICT, TIER_FP16, TIER_INT2, TIER_INT4, TieredKVCache

    t = torch.tensor([TIER_FP16, TIER_INT4, TIER_INT4, TIER_EVICT, TIER_INT2, TIER_FP16])
    assert TieredKVCache._host_tier_counts(t) == (2, 2, 1)
    assert TieredKVCache._host_tier_counts(torch.tensor([0, 7])) is None
    for steps in (1, 5, 37, 64, 200, 1000):
        calls, reps = bench.graph_split(steps)
        assert calls * reps == steps and calls <= 32
    assert bench.graph_split(200) == (20, 10)
    assert bench.graph_split(20) == (20, 1)
    assert bench.STATS_REPLAYS >= 10


def test_reassign_status_check():
    """check_reassign_status reads the gather's status word and names the dropped tokens
    (a fabricated counts tensor: host logic only)."""
    import pytest
    import torch

    from fade_amd.cache import TieredKVCache

    c = TieredKVCache(head_dim=128)
    ok = torch.tensor([3, 5, 8, 0], dtype=torch.int32)
    bad = torch.tensor([[3, 5, 8, 0], [3, 5, 8, 8 | 16]], dtype=torch.int32)
    c._check_status(bad, 2)  # off by default: nothing read
    c.check_reassign_status = True
    c._check_status(ok, 1)
    with pytest.raises(RuntimeError, match="row 1.*slot past a tier's capacity.*token the row does not have"):
        c._check_status(bad, 2)
