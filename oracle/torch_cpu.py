"""Torch-CPU restatement of the reference's decode step (TEST INFRASTRUCTURE: the
timed CPU baseline of bench.py and its pin in tests; the product never imports it).

One decode call of the reference over a tiered cache with a packed INT4 middle
tier is: unpack the nibbles and dequantize (``dequant_int4``,
fade/quant.py:46-58,124-127), concatenate sink | middle | recent along S
(fade/cache.py:715-808), expand the KV heads for GQA (``repeat_interleave``,
fade/kernels/fused_int4_attn.py:306-312) and run
``F.scaled_dot_product_attention`` (fade/kernels/int4_attention.py:179-202).

Two working dtypes, as the CPU baseline reports them:
  ``"fp16"``  dequantize and concatenate in fp16 (the cache's dtype), SDPA in fp32
  ``"fp32"``  everything in fp32 (the reference's own CPU default dtype,
              benchmarks/tps.py:22-24)
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """uint8 [..., D/2] -> int8 [..., D]: high nibble = even channel, two's complement."""
    hi = (packed >> 4).to(torch.int16)
    lo = (packed & 0xF).to(torch.int16)
    hi = hi - ((hi & 8) << 1)
    lo = lo - ((lo & 8) << 1)
    return torch.stack((hi, lo), dim=-1).flatten(-2).to(torch.int8)


def dequant_int4(packed: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``codes.to(dtype) * scale.to(dtype)`` (one rounding per op in ``dtype``)."""
    return unpack_int4(packed).to(dtype) * scale.to(dtype)


def decode_step(q, sink, mid, recent, mode: str = "fp16") -> torch.Tensor:
    """Attention of q [B, Hq, 1, D] over sink | INT4 middle | recent; returns fp32 [B, Hq, 1, D].

    ``sink``/``recent``: (K, V) fp16 [B, Hkv, n, D]; ``mid``: (k_packed, k_scale, v_packed,
    v_scale) in the reference INT4 layout."""
    dt = torch.float16 if mode == "fp16" else torch.float32
    kq, ks, vq, vs = mid
    K = torch.cat([sink[0].to(dt), dequant_int4(kq, ks, dt), recent[0].to(dt)], dim=-2)
    V = torch.cat([sink[1].to(dt), dequant_int4(vq, vs, dt), recent[1].to(dt)], dim=-2)
    rep = q.shape[1] // K.shape[1]
    K = K.float().repeat_interleave(rep, dim=1)
    V = V.float().repeat_interleave(rep, dim=1)
    return F.scaled_dot_product_attention(q.float(), K, V)


__all__ = ["decode_step", "dequant_int4", "unpack_int4"]
