"""GPU parity of the fused eviction re-RoPE against the oracle (config 3 shape)."""

import numpy as np
import pytest
import torch

from fade_amd import rope as frope
from fade_amd.policy import _assign_one_layer
from fade_amd.synthetic import ReropeConfig, exp_scores, kv_tensors
from oracle import policy as opol
from oracle import quant as oq
from oracle import rope as orope

pytestmark = pytest.mark.gpu


def _post_rope_k(cfg, seed):
    """Keys stored post-RoPE at positions 0..S-1 (theta 1e6), as the cache holds them."""
    _, k, v = kv_tensors(cfg.B, cfg.Hkv, cfg.S, cfg.D, seed=seed)
    scheme = frope.Vanilla(theta=cfg.theta, head_dim=cfg.D)
    cos, sin = scheme.host_cos_sin(torch.arange(cfg.S))
    k_post = orope.apply_rope(k.numpy(), cos.numpy(), sin.numpy())
    return scheme, k_post, v.numpy()


@pytest.mark.parametrize("B", [8, 1])
def test_rerope_config3_bit_exact(dev, B):
    cfg = ReropeConfig(B=B)
    print(f"case rerope config3 B={B}", flush=True)
    scheme, k, v = _post_rope_k(cfg, seed=1003)
    scores = exp_scores(cfg.S, seed=2003)
    tiers = _assign_one_layer(cfg.S, scores, cfg.n_sink, cfg.recent, cfg.int4_budget, 0)
    otiers = opol.assign_one_layer(cfg.S, scores.numpy(), cfg.n_sink, cfg.recent, cfg.int4_budget, 0)
    assert np.array_equal(tiers.numpy(), otiers)  # keep set bit-exact
    keep = (tiers != opol.TIER_EVICT).nonzero().squeeze(-1)
    n = int(keep.numel())
    assert n == 4 + 400 + 64
    co, so = scheme.host_cos_sin(torch.arange(cfg.S))
    cn, sn = scheme.host_cos_sin(torch.arange(n))
    ko, vo = frope.rerope_gather(
        torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev), keep.to(dev), co, so, cn, sn
    )
    rk, rv = orope.rerope_gather(k, v, keep.numpy(), co.numpy(), so.numpy(), cn.numpy(), sn.numpy())
    assert np.array_equal(vo.cpu().numpy(), rv)
    kg = ko.cpu().numpy()
    assert np.array_equal(kg.view(np.uint16), rk.view(np.uint16)), (
        f"max-abs {np.abs(kg.astype(np.float32) - rk.astype(np.float32)).max()}"
    )


def test_rerope_strided_input_and_no_v(dev):
    print("case rerope strided", flush=True)
    cfg = ReropeConfig(B=2, S=256, int4_budget=50)
    scheme, k, v = _post_rope_k(cfg, seed=7)
    big = torch.zeros(2, 4, 300, 128, dtype=torch.float16, device=dev)
    big[:, :, :256] = torch.from_numpy(k).to(dev)
    keep = torch.tensor([0, 3, 7, 100, 255], device=dev)
    co, so = scheme.host_cos_sin(torch.arange(256))
    cn, sn = scheme.host_cos_sin(torch.arange(5))
    ko, vo = frope.rerope_gather(big[:, :, :256], None, keep, co, so, cn, sn)
    assert vo is None
    rk, _ = orope.rerope_gather(k, v, keep.cpu().numpy(), co.numpy(), so.numpy(), cn.numpy(), sn.numpy())
    assert np.array_equal(ko.cpu().numpy().view(np.uint16), rk.view(np.uint16))


def test_rerope_llama3_scheme_tables(dev):
    """Any scheme works: the kernel consumes host tables (Llama-3 band interpolation here)."""
    print("case rerope llama3", flush=True)
    scheme = frope.Llama3(theta=5e5, head_dim=128, factor=8.0)
    _, k, v = kv_tensors(1, 2, 128, 128, seed=11)
    keep = torch.arange(0, 128, 3)
    co, so = scheme.host_cos_sin(torch.arange(128))
    cn, sn = scheme.host_cos_sin(torch.arange(int(keep.numel())))
    ko, _ = frope.rerope_gather(k.to(dev), v.to(dev), keep.to(dev), co, so, cn, sn)
    rk, _ = orope.rerope_gather(k.numpy(), v.numpy(), keep.numpy(), co.numpy(), so.numpy(), cn.numpy(), sn.numpy())
    assert np.array_equal(ko.cpu().numpy().view(np.uint16), rk.view(np.uint16))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("D", [128, 64, 32, 256, 24, 20])  # 20: D/2 not a multiple of 4 (one element pair per thread)
def test_rerope_typed_bit_exact(dev, dtype, D):
    """A bfloat16 / float32 cache: fp32 math, un-RoPE and re-RoPE each rounded
    to the cache dtype; bf16 tables are not rounded (fade/rope.py:83-93)."""
    print(f"case rerope {dtype} D={D}", flush=True)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    rng = np.random.default_rng(21)
    S = 300
    k = oq.from_f32((rng.standard_normal((2, 4, S, D)) * 3).astype(np.float32), dtype)
    v = oq.from_f32(rng.standard_normal((2, 4, S, D)).astype(np.float32), dtype)
    scheme = frope.Vanilla(theta=1e6, head_dim=D)
    keep = torch.tensor(sorted(rng.choice(S, 120, replace=False)))
    co, so = scheme.host_cos_sin(torch.arange(S) + 500, tdt)
    cn, sn = scheme.host_cos_sin(torch.arange(120), tdt)

    def dev_t(a):
        if dtype == "bf16":
            return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)
        return torch.from_numpy(a).to(dev)

    def host(t):
        t = t.cpu().contiguous()
        return t.view(torch.int16).numpy().view(np.uint16) if dtype == "bf16" else t.numpy()

    ko, vo = frope.rerope_gather(dev_t(k), dev_t(v), keep.to(dev), co, so, cn, sn)
    assert ko.dtype == tdt and vo.dtype == tdt
    rk, rv = orope.rerope_gather_typed(k, v, keep.numpy(), co.numpy(), so.numpy(), cn.numpy(), sn.numpy(), dtype)
    assert np.array_equal(host(vo), rv)
    assert np.array_equal(host(ko), rk)
    with pytest.raises(ValueError, match="dtypes differ"):
        frope.rerope_gather(dev_t(k), dev_t(v).half(), keep.to(dev), co, so, cn, sn)
