"""GPU tests of the tiered cache: HF update protocol, eviction + re-RoPE + requant
composed exactly as fade/cache.py:881-1057 does, and fused decode vs materialize."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from fade_amd import FadeConfig, TieredKVCache, create_tiered_cache
from fade_amd.cache import TIER_EVICT, TIER_FP16, TIER_INT4
from fade_amd.policy import _assign_one_layer, reassign_tiers_by_position
from fade_amd.rope import Vanilla
from fade_amd.synthetic import exp_scores, kv_tensors
from oracle import attention as oatt
from oracle import quant as oq
from oracle import rope as orope

pytestmark = pytest.mark.gpu


_TDT = {"bf16": torch.bfloat16, "f32": torch.float32}


def _oracle_reassign(k, v, pos, tiers, scheme, n_sink, dtype="f16"):
    """The composed state change of apply_tier_assignment, restated with the oracle
    (``dtype`` "bf16" / "f32": a cache of that dtype, bf16 as uint16 bits)."""
    keep = np.nonzero(tiers != TIER_EVICT)[0]
    n = keep.size
    if n < k.shape[2]:
        tdt = _TDT.get(dtype, torch.float16)
        co, so = scheme.host_cos_sin(torch.from_numpy(pos), tdt)
        cn, sn = scheme.host_cos_sin(torch.arange(n), tdt)
        tabs = (co.numpy(), so.numpy(), cn.numpy(), sn.numpy())
        if dtype == "f16":
            k, v = orope.rerope_gather(k, v, keep, *tabs)
        else:
            k, v = orope.rerope_gather_typed(k, v, keep, *tabs, dtype)
        tiers, pos = tiers[keep], np.arange(n)
    f = np.nonzero(tiers == TIER_FP16)[0]
    i4 = np.nonzero(tiers == TIER_INT4)[0]
    if dtype == "f16":
        kq, ks = oq.quant_k_int4(k[:, :, i4])
        vq, vs = oq.quant_v_int4(v[:, :, i4])
    else:
        kq, ks = oq.quant_k_int4_typed(k[:, :, i4], dtype)
        vq, vs = oq.quant_v_int4_typed(v[:, :, i4], dtype)
    return {"fp16_k": k[:, :, f], "fp16_v": v[:, :, f], "kq": kq, "ks": ks, "vq": vq, "vs": vs,
            "int4_pos": pos[i4], "fp16_pos": pos[f], "n_sink": min(n_sink, f.size)}


def test_update_materializes_in_position_order(dev):
    print("case cache update", flush=True)
    _, k, v = kv_tensors(2, 4, 50, 128, seed=1)
    c = TieredKVCache(n_sink=4, recent_window=8)
    K, V = c.update(k[:, :, :40].to(dev), v[:, :, :40].to(dev), 0)
    K, V = c.update(k[:, :, 40:].to(dev), v[:, :, 40:].to(dev), 0)
    assert torch.equal(K.cpu(), k) and torch.equal(V.cpu(), v)
    assert c.get_seq_length(0) == 50 and c.get_mask_sizes(1, 0) == (51, 0)
    with pytest.raises(ValueError, match="batch size mismatch"):
        c.update(k[:1, :, :1].to(dev), v[:1, :, :1].to(dev), 0)


@pytest.mark.parametrize("budget", [None, 400])
def test_apply_tier_assignment_matches_oracle_composition(dev, budget):
    """Config-3 flow (Qwen2.5-7B shape, theta 1e6): eviction, re-RoPE, requant bit-exact."""
    print(f"case cache reassign budget={budget}", flush=True)
    B, Hkv, S, D = 2, 4, 1024, 128
    _, k, v = kv_tensors(B, Hkv, S, D, seed=1003)
    scheme = Vanilla(theta=1e6, head_dim=D)
    cos, sin = scheme.host_cos_sin(torch.arange(S))
    k = torch.from_numpy(orope.apply_rope(k.numpy(), cos.numpy(), sin.numpy()))
    c = TieredKVCache(n_sink=4, recent_window=64, int4_budget=budget, rope_scheme=scheme, head_dim=D)
    c.update(k.to(dev), v.to(dev), 0)
    scores = exp_scores(S, seed=2003)
    tiers = _assign_one_layer(S, scores, 4, 64, budget, 0)
    c.apply_tier_assignment(0, tiers)
    o = _oracle_reassign(k.numpy(), v.numpy(), np.arange(S), tiers.numpy(), scheme, 4)
    st = c._layers[0]
    assert np.array_equal(st.int4_kq.cpu().numpy(), o["kq"]) and np.array_equal(st.int4_vq.cpu().numpy(), o["vq"])
    assert np.array_equal(st.int4_ks.cpu().numpy().view(np.uint16), o["ks"].view(np.uint16))
    assert np.array_equal(st.int4_vs.cpu().numpy().view(np.uint16), o["vs"].view(np.uint16))
    ns = o["n_sink"]
    assert st.sink_count == ns
    assert np.array_equal(st.sink_k.cpu().numpy().view(np.uint16), o["fp16_k"][:, :, :ns].view(np.uint16))
    assert np.array_equal(st.fp16_k.cpu().numpy().view(np.uint16), o["fp16_k"][:, :, ns:].view(np.uint16))
    assert np.array_equal(st.int4_pos.cpu().numpy(), o["int4_pos"])
    n_kept = int((tiers != TIER_EVICT).sum())
    assert c.get_seq_length(0) == n_kept and st.next_position == (n_kept if budget else S)

    # decode straight from the tiers == SDPA over the materialized cache
    q = torch.randn(B, 28, 1, D, generator=torch.Generator().manual_seed(3)).to(torch.float16)
    Kn, Vn = c.update(k[:, :, :1].to(dev), v[:, :, :1].to(dev), 0)
    fused = c.decode_attention(q.to(dev), 0).float().cpu().numpy()
    ref = oatt.sdpa_fp32(q.numpy(), Kn.cpu().numpy(), Vn.cpu().numpy())
    assert np.abs(fused - ref).max() <= 2e-3

    # a second reassignment requantizes from dequantized values (fade/cache.py:976-989)
    S2 = c.get_seq_length(0)
    tiers2 = _assign_one_layer(S2, torch.arange(S2, dtype=torch.float32), 4, 64, 200, 0)
    Kp, Vp = Kn.cpu().numpy(), Vn.cpu().numpy()
    pos2 = np.concatenate([st.sink_pos.cpu().numpy(), st.int4_pos.cpu().numpy(), st.fp16_pos.cpu().numpy()])
    c.apply_tier_assignment(0, tiers2)
    o2 = _oracle_reassign(Kp, Vp, pos2, tiers2.numpy(), scheme, 4)
    st = c._layers[0]
    assert np.array_equal(st.int4_kq.cpu().numpy(), o2["kq"]) and np.array_equal(st.int4_vq.cpu().numpy(), o2["vq"])


def _dev_t(a, dtype, dev):
    if dtype == "bf16":
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _host_t(t, dtype):
    t = t.cpu().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16) if dtype == "bf16" else t.numpy()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_typed_cache_reassign_matches_oracle_composition(dev, dtype):
    """A bfloat16 / float32 cache (create_tiered_cache(dtype=...)): eviction, re-RoPE
    and INT4 requant at the cache dtype bit-exact, the materialized K/V the
    dequantized tiers in position order, a second reassignment from them, and
    an INT2 tier's grouped codes."""
    print(f"case typed cache {dtype}", flush=True)
    tdt = _TDT[dtype]
    B, Hkv, S, D = 2, 4, 700, 128
    _, k16, v16 = kv_tensors(B, Hkv, S, D, seed=31)
    scheme = Vanilla(theta=1e6, head_dim=D)
    cos, sin = scheme.host_cos_sin(torch.arange(S), tdt)
    k = orope.apply_rope_typed(oq.from_f32(k16.float().numpy() * 1.7, dtype), cos.numpy(), sin.numpy(), dtype)
    v = oq.from_f32(v16.float().numpy(), dtype)
    c = TieredKVCache(n_sink=4, recent_window=64, int4_budget=300, rope_scheme=scheme, head_dim=D, dtype=tdt)
    K0, _ = c.update(_dev_t(k, dtype, dev), _dev_t(v, dtype, dev), 0)
    assert K0.dtype == tdt
    tiers = _assign_one_layer(S, exp_scores(S, seed=32), 4, 64, 300, 0)
    c.apply_tier_assignment(0, tiers)
    o = _oracle_reassign(k, v, np.arange(S), tiers.numpy(), scheme, 4, dtype)
    st = c._layers[0]
    assert st.int4_ks.dtype == tdt and st.int4_vs.dtype == tdt and st.fp16_k.dtype == tdt
    assert np.array_equal(st.int4_kq.cpu().numpy(), o["kq"]) and np.array_equal(st.int4_vq.cpu().numpy(), o["vq"])
    assert np.array_equal(_host_t(st.int4_ks, dtype), o["ks"]) and np.array_equal(_host_t(st.int4_vs, dtype), o["vs"])
    ns = o["n_sink"]
    assert np.array_equal(_host_t(st.sink_k, dtype), o["fp16_k"][:, :, :ns])
    assert np.array_equal(_host_t(st.fp16_k, dtype), o["fp16_k"][:, :, ns:])
    assert np.array_equal(_host_t(st.fp16_v, dtype), o["fp16_v"][:, :, ns:])
    assert np.array_equal(st.int4_pos.cpu().numpy(), o["int4_pos"])

    # materialized K/V: sink | dequantized middle | recent (the middle sits between them here)
    K, V = c._materialize(0)
    assert K.dtype == tdt
    kd = oq.dequant_int4_typed(o["kq"], o["ks"], dtype)
    vd = oq.dequant_int4_typed(o["vq"], o["vs"], dtype)
    fk, fv = o["fp16_k"], o["fp16_v"]
    assert np.array_equal(_host_t(K, dtype), np.concatenate([fk[:, :, :ns], kd, fk[:, :, ns:]], 2))
    assert np.array_equal(_host_t(V, dtype), np.concatenate([fv[:, :, :ns], vd, fv[:, :, ns:]], 2))
    if dtype == "f32":
        with pytest.raises(NotImplementedError, match="bfloat16 tiers"):
            c.decode_attention(torch.zeros(B, 8, 1, D, dtype=torch.float32, device=dev), 0)
    else:
        # a bf16 cache decodes on the kernels: fp32 attention over the materialized
        # bf16 K/V (the reference's path), bf16 tolerance 4e-3 + 2^-7 |ref|
        qd = torch.randn(B, 8, 1, D, generator=torch.Generator().manual_seed(34)).to(dev, tdt)
        out = c.decode_attention(qd, 0)
        assert out.dtype == tdt
        ref = oatt.sdpa_fp32(qd.float().cpu().numpy(), K.float().cpu().numpy(), V.float().cpu().numpy())
        assert (np.abs(out.float().cpu().numpy() - ref) - 2.0**-7 * np.abs(ref)).max() <= 4e-3
        with pytest.raises(ValueError, match="query's dtype"):
            c.decode_attention(qd.half(), 0)

    # a second reassignment requantizes from the dequantized values
    S2 = c.get_seq_length(0)
    tiers2 = _assign_one_layer(S2, torch.arange(S2, dtype=torch.float32), 4, 64, 150, 0)
    pos2 = np.concatenate([st.sink_pos.cpu().numpy(), st.int4_pos.cpu().numpy(), st.fp16_pos.cpu().numpy()])
    c.apply_tier_assignment(0, tiers2)
    o2 = _oracle_reassign(_host_t(K, dtype), _host_t(V, dtype), pos2, tiers2.numpy(), scheme, 4, dtype)
    st = c._layers[0]
    assert np.array_equal(st.int4_kq.cpu().numpy(), o2["kq"]) and np.array_equal(st.int4_vq.cpu().numpy(), o2["vq"])
    assert np.array_equal(_host_t(st.int4_ks, dtype), o2["ks"])

    # an INT2 tier (three-tier policy): grouped codes at the cache dtype
    c3 = TieredKVCache(n_sink=4, recent_window=64, int4_budget=200, int2_budget=128, rope_scheme=scheme,
                       head_dim=D, dtype=tdt)
    c3.update(_dev_t(k, dtype, dev), _dev_t(v, dtype, dev), 0)
    c3.apply_tier_assignment(0, _assign_one_layer(S, exp_scores(S, seed=33), 4, 64, 200, 128))
    st3 = c3._layers[0]
    assert st3.int2_kq is not None and st3.int2_ks.dtype == tdt
    K3, _ = c3._materialize(0)
    assert K3.dtype == tdt and K3.shape[2] == c3.get_seq_length(0)


def test_k4v2_cache_decode(dev):
    print("case cache k4v2", flush=True)
    _, k, v = kv_tensors(1, 8, 700, 128, seed=4)
    c = TieredKVCache(n_sink=4, recent_window=256, middle_v_bits=2)
    c.update(k.to(dev), v.to(dev), 0)
    c.apply_tier_assignment(0, _assign_one_layer(700, torch.zeros(700), 4, 256, None, 0))
    st = c._layers[0]
    assert st.int4_vq.dtype == torch.int8 and st.int4_vq.shape[2] % 64 == 0
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(5)).to(torch.float16)
    K, V = c._materialize(0)
    fused = c.decode_attention(q.to(dev), 0).float().cpu().numpy()
    ref = oatt.sdpa_fp32(q.numpy(), K.cpu().numpy(), V.cpu().numpy())
    assert np.abs(fused - ref).max() <= 2e-3


@pytest.mark.parametrize("backend", ["rotated", "int4_asym_g32"])
def test_backend_caches_decode(dev, backend):
    print(f"case cache backend={backend}", flush=True)
    _, k, v = kv_tensors(1, 8, 600, 128, seed=6)
    cfg = FadeConfig(quant_backend=backend)
    c = TieredKVCache(head_dim=128, **cfg.to_cache_kwargs())
    c.update(k.to(dev), v.to(dev), 0)
    reassign_tiers_by_position(c, 1)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(7)).to(torch.float16)
    K, V = c._materialize(0)
    fused = c.decode_attention(q.to(dev), 0).float().cpu().numpy()
    ref = oatt.sdpa_fp32(q.numpy(), K.cpu().numpy(), V.cpu().numpy())
    assert np.abs(fused - ref).max() <= 2e-3


def test_per_sequence_assignment_and_checkpoint(dev):
    print("case cache per-sequence", flush=True)
    _, k, v = kv_tensors(2, 2, 300, 128, seed=8)
    c = TieredKVCache(n_sink=4, recent_window=32, int4_budget=100)
    c.update(k.to(dev), v.to(dev), 0)
    g = torch.Generator().manual_seed(9)
    t = torch.stack([_assign_one_layer(300, torch.rand(300, generator=g), 4, 32, 100, 0) for _ in range(2)])
    c.apply_tier_assignment_per_sequence(0, t)
    assert c._layers[0].int4_kq.shape[2] == 100
    sd = c.cache_state_dict()
    c2 = TieredKVCache(n_sink=4, recent_window=32, int4_budget=100)
    c2.load_cache_state_dict(sd, device=dev)
    K1, V1 = c._materialize(0)
    K2, V2 = c2._materialize(0)
    assert torch.equal(K1, K2) and torch.equal(V1, V2)


def test_create_tiered_cache_from_hf_config(dev):
    print("case create_tiered_cache", flush=True)
    from transformers import AutoConfig

    cfg = AutoConfig.for_model("qwen2", hidden_size=256, num_attention_heads=2, num_key_value_heads=1,
                               num_hidden_layers=2, intermediate_size=512, vocab_size=100, rope_theta=1e6)
    model = type("M", (), {"config": cfg})()
    c = create_tiered_cache(model, config=FadeConfig.balanced())
    assert c.head_dim == 128 and c.int4_budget == 400 and c.rope_scheme.theta == 1e6
    _, k, v = kv_tensors(1, 1, 10, 128, seed=1)
    K, _ = c.update(k.to(dev), v.to(dev), 0)
    assert K.shape == (1, 1, 10, 128)
    q = torch.randn(1, 2, 1, 128).to(torch.float16)
    out = c.decode_attention(q.to(dev), 0)
    ref = F.scaled_dot_product_attention(q.float(), k.float().repeat_interleave(2, 1), v.float().repeat_interleave(2, 1))
    assert (out.float().cpu() - ref).abs().max() <= 2e-3


@pytest.mark.parametrize("split_sink", [False, True])
def test_decode_plan_reuse_matches_fresh_plans(dev, split_sink):
    """decode_attention keeps one plan per layer and relaunches it while the tiers are
    the same tensors (only q, the output and the recent tier's length change).  Across
    appends, a grown fp16 buffer and a reassignment, every step equals a plan built
    afresh for that step, bit for bit (deterministic mode), and the SDPA reference."""
    print(f"case decode plan reuse split_sink={split_sink}", flush=True)
    B, H, Hq, D = 2, 4, 16, 128
    g = torch.Generator().manual_seed(7)
    c = TieredKVCache(n_sink=4, recent_window=16, int4_budget=None, int2_budget=0, head_dim=D)
    k = torch.randn(B, H, 300, D, generator=g).half().to(dev)
    v = torch.randn(B, H, 300, D, generator=g).half().to(dev)
    c.update(k, v, 0)
    t = torch.full((300,), TIER_INT4, dtype=torch.long)
    t[:4] = TIER_FP16
    t[-16:] = TIER_FP16
    c.apply_tier_assignment(0, t)
    st = c._layers[0]
    if not split_sink:  # the sink as the head of the fp16 tier
        st.fp16_k = torch.cat([st.sink_k, st.fp16_k], dim=2)
        st.fp16_v = torch.cat([st.sink_v, st.fp16_v], dim=2)
        st.fp16_pos = torch.cat([st.sink_pos, st.fp16_pos])
        st._fp16_buf_k = st._fp16_buf_v = st._fp16_buf_pos = None
        st.sink_k = st.sink_v = st.sink_pos = None
        st.sink_count = 4
    torch.use_deterministic_algorithms(True)
    try:
        plans = set()
        for step in range(140):  # crosses the fp16 buffer's first growth
            kt = torch.randn(B, H, 1, D, generator=g).half().to(dev)
            vt = torch.randn(B, H, 1, D, generator=g).half().to(dev)
            c.update(kt, vt, 0)
            q = torch.randn(B, Hq, 1, D, generator=g).half().to(dev)
            out = c.decode_attention(q, 0)
            plans.add(id(st._decode_plan[1]))
            st_plan, st._decode_plan = st._decode_plan, None
            fresh = c.decode_attention(q, 0)  # built afresh for this step
            st._decode_plan = st_plan
            assert torch.equal(out, fresh), step
            if step % 35 == 0:
                kf, vf = c._materialize(0)
                ref = F.scaled_dot_product_attention(q.float(), kf.float().repeat_interleave(Hq // H, 1),
                                                     vf.float().repeat_interleave(Hq // H, 1))
                assert (out.float() - ref).abs().max().item() <= 2e-3, step
        assert len(plans) < 10  # reused, not rebuilt per step
    finally:
        torch.use_deterministic_algorithms(False)
