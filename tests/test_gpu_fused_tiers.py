"""The fused decode and chunk prefill over every tier layout the reference's cache can hold
(fade/cache.py:715-876): an INT2 tier next to the INT4 middle tier (int2_budget > 0, read as
its fp16 dequantization joined to the sink), and chunk prefill over the K4 + literal INT2 V,
rotated and asymmetric middle tiers (read through their fp16 dequantization).  Each against
fp32 SDPA over the cache the reference materializes for the same tokens (``update()``'s
K/V), with the bottom-right mask for chunks."""

import numpy as np
import pytest
import torch

from fade_amd.backends import AsymGroupBackend, RotatedINT4Backend
from fade_amd.cache import TieredKVCache
from fade_amd.policy import _assign_one_layer
from fade_amd.synthetic import kv_tensors
from oracle import attention as oatt

pytestmark = pytest.mark.gpu
ATOL = 2e-3
B, Hq, Hkv, D, S = 2, 16, 4, 128, 700


def _cache(dev, int4_budget=None, int2_budget=0, middle_v_bits=4, backend="int4", seed=11):
    be = {"int4": "int4", "rotated": RotatedINT4Backend(head_dim=D, bits=4),
          "rotated2": RotatedINT4Backend(head_dim=D, bits=2), "asym": AsymGroupBackend(head_dim=D),
          "asym42": AsymGroupBackend(head_dim=D, bits=4, v_bits=2)}[backend]
    c = TieredKVCache(n_sink=4, recent_window=48, int4_budget=int4_budget, int2_budget=int2_budget, head_dim=D,
                      middle_v_bits=middle_v_bits, quant_backend=be, rope_theta=1e6)
    _, k, v = kv_tensors(B, Hkv, S, D, seed=seed)
    c.update(k.to(dev), v.to(dev), 0)
    scores = torch.rand(S, generator=torch.Generator().manual_seed(seed + 1))
    c.apply_tier_assignment(0, _assign_one_layer(S, scores, 4, 48, int4_budget, int2_budget))
    return c


def _decode_check(dev, c, seed):
    g = torch.Generator().manual_seed(seed)
    for step in range(2):
        k1 = torch.randn(B, Hkv, 1, D, generator=g).half().to(dev)
        v1 = torch.randn(B, Hkv, 1, D, generator=g).half().to(dev)
        q = torch.randn(B, Hq, 1, D, generator=g).half()
        K, V = c.update(k1, v1, 0)
        out = c.decode_attention(q.to(dev), 0).float().cpu().numpy()
        ref = oatt.sdpa_fp32(q.numpy(), K.cpu().numpy(), V.cpu().numpy())
        err = float(np.abs(out - ref).max())
        assert err <= ATOL, f"step {step}: decode max-abs error {err}"


def _prefill_check(dev, c, seed, Sq=40):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(B, Hkv, Sq, D, generator=g).half().to(dev)
    vc = torch.randn(B, Hkv, Sq, D, generator=g).half().to(dev)
    q = torch.randn(B, Hq, Sq, D, generator=g).half()
    K, V = c.update(kc, vc, 0)
    out = c.prefill_attention(q.to(dev), 0).float().cpu().numpy()
    Sk = int(K.shape[2])
    ref = oatt.sdpa_fp32(q.numpy(), K.cpu().numpy(), V.cpu().numpy(), mask=oatt.bottom_right_causal_mask(Sq, Sk))
    err = float(np.abs(out - ref).max())
    assert err <= ATOL, f"prefill max-abs error {err}"


@pytest.mark.parametrize("middle_v_bits", [4, 2])
def test_decode_with_int2_tier(dev, middle_v_bits):
    """int4_budget 200 + int2_budget 150 of the 648 middle candidates (the rest evicted)."""
    print(f"case decode int2 tier mvb={middle_v_bits}", flush=True)
    c = _cache(dev, int4_budget=200, int2_budget=150, middle_v_bits=middle_v_bits)
    st = c._layers[0]
    assert st.int2_kq is not None and st.int2_actual_count == 150
    _decode_check(dev, c, seed=21)


def test_prefill_with_int2_tier(dev):
    print("case prefill int2 tier", flush=True)
    c = _cache(dev, int4_budget=200, int2_budget=150)
    _prefill_check(dev, c, seed=22)


@pytest.mark.parametrize("backend,mvb", [("int4", 2), ("rotated", 4), ("rotated2", 4), ("asym", 4), ("asym42", 4)])
def test_prefill_other_middle_formats(dev, backend, mvb):
    """Chunk prefill over K4 + literal INT2 V, rotated (4- and 2-bit) and asymmetric middles."""
    print(f"case prefill middle {backend} mvb={mvb}", flush=True)
    c = _cache(dev, middle_v_bits=mvb, backend=backend)
    _prefill_check(dev, c, seed=23)
    # the next decode step reads the same tiers
    _decode_check(dev, c, seed=24)


def test_front_tier_is_reused_until_the_tiers_change(dev):
    """The joined sink + INT2 tensors are built once per tier state."""
    c = _cache(dev, int4_budget=200, int2_budget=150)
    st = c._layers[0]
    q = torch.randn(B, Hq, 1, D).half().to(dev)
    c.decode_attention(q, 0)
    first = st._front_cache[2]
    c.decode_attention(q, 0)
    assert st._front_cache[2] is first
    c.apply_tier_assignment(0, _assign_one_layer(c.get_seq_length(0), torch.rand(c.get_seq_length(0)), 4, 48, 100, 50))
    c.decode_attention(q, 0)
    assert st._front_cache[2] is not first
