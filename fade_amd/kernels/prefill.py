"""Ragged tiered prefill attention (``fade_tiered_prefill_attn``).

The reference has no prefill kernel: a chunk goes through
``TieredKVCache.update`` (fade/cache.py:347-379), which returns the
materialized ``[sink | dequantized middle | recent | chunk]`` K/V
(fade/cache.py:683-842), and the model runs causal SDPA over it with the
mask aligned bottom-right (the chunk is the last ``Sq`` keys).  This op reads
the tiers in place, per batch row with its own tier lengths.
"""

from __future__ import annotations

import ctypes
import math

import torch
from torch import Tensor

from .. import _lib
from .tiered_attn import MiddleTier, _attn_dtype, _fp16_tier, _mid_tier

_MASKS = {"bottom_right": _lib.MASK_BOTTOM_RIGHT, "top_left": _lib.MASK_TOP_LEFT, "none": _lib.MASK_NONE}


class TieredPrefillPlan:
    """Validated launch for fixed tensors; ``run()`` enqueues one kernel.

    Args:
        q: [B, Hq, Sq, D] fp16 or bf16 queries of the chunk; D a multiple of 8 up to 256.
            Every other 16-bit tensor (tiers, scales, the output) is of q's dtype.
        chunk: (K, V) [B, Hkv, Sq, D] fp16, the chunk's own keys/values
            (with ``mask`` ``"top_left"`` / ``"none"``: any length, or None).
        sink, recent: (K, V) [B, Hkv, cap, D] fp16 padded along S, or None.
        mid: reference INT4 middle tier (``MiddleTier("int4", ...)``) with
            codes padded to a common row count, an fp16 one (``MiddleTier("fp16",
            k, v)``, rows [B, Hkv, S, D]), or None.
        lens: int32 [B, 3] (sink, middle, recent tokens used by each row);
            default: every row uses the full capacities.
        order: optional int32 [B] dispatch order of the batch rows (longest first).
        mask: ``"bottom_right"`` (default: the cache fully visible, chunk key
            i visible to chunk queries j >= i), ``"top_left"`` (query j sees
            keys 0..j of the row's sequence [sink | middle | recent | chunk],
            the reference fused kernel's ``is_causal``) or ``"none"``.
    """

    def __init__(
        self,
        q: Tensor,
        chunk: tuple[Tensor, Tensor],
        sink: tuple[Tensor, Tensor] | None = None,
        mid: MiddleTier | None = None,
        recent: tuple[Tensor, Tensor] | None = None,
        lens: Tensor | None = None,
        order: Tensor | None = None,
        sm_scale: float | None = None,
        out: Tensor | None = None,
        mask: str = "bottom_right",
    ) -> None:
        if q.dim() != 4:
            raise ValueError(f"q must be [B, Hq, Sq, D], got {tuple(q.shape)}")
        if mask not in _MASKS:
            raise ValueError(f"mask must be one of {sorted(_MASKS)}, got {mask!r}")
        if chunk is None and mask == "bottom_right":
            raise ValueError("the bottom-right mask needs the chunk's own K/V")
        tensors = [q] + ([*chunk] if chunk else []) + ([*sink] if sink else []) + ([*recent] if recent else []) \
            + (mid.tensors() if mid else [])
        _lib.require_gpu(*tensors, op="tiered_prefill_attention")
        dtc = _attn_dtype(q, "tiered_prefill_attention")
        B, Hq, Sq, D = q.shape
        ref = chunk[0] if chunk else (sink[0] if sink else (recent[0] if recent else (mid.k_codes if mid else None)))
        if ref is None:
            raise ValueError("tiered_prefill_attention: no keys")
        Hkv = int(ref.shape[1])
        if chunk is not None:
            n_c = Sq if mask == "bottom_right" else int(chunk[0].shape[2])
            if tuple(chunk[0].shape) != (B, Hkv, n_c, D) or chunk[1].shape != chunk[0].shape:
                raise ValueError(f"chunk K/V must be [B, Hkv, {'Sq=' if mask == 'bottom_right' else ''}{n_c}, D]")
        if mid is not None and mid.fmt not in ("int4", "sym", "fp16"):
            raise ValueError("the prefill kernel reads the reference INT4 middle tier or an fp16 one")
        if mid is not None and mid.fmt in ("int4", "sym") and D % 32:
            # the kernel stages packed rows in 32-channel units: at other head dims it
            # reads the middle tier as its fp16 dequantization (the reference's
            # rounding, fade/quant.py:124-127)
            if mid.pages is not None:
                raise ValueError("a paged INT4 middle tier needs head_dim % 32 == 0 in the prefill kernel")
            from ..quant import dequant_int4

            mid = MiddleTier("fp16", dequant_int4(mid.k_codes, mid.k_scale, dtype=q.dtype),
                             dequant_int4(mid.v_codes, mid.v_scale, dtype=q.dtype), length=mid.length)
        if mid is not None and mid.fmt == "fp16" and (mid.k_codes.dtype != q.dtype or mid.k_codes.shape[-1] != D):
            raise ValueError(f"an fp16-layout middle tier holds {q.dtype} rows [B, Hkv, S, D] (the query's dtype)")
        if q.stride(-1) != 1:
            q = q.contiguous()
        caps = [int(sink[0].shape[2]) if sink else 0, mid.n_tokens if mid else 0, int(recent[0].shape[2]) if recent else 0]
        if lens is None:
            lens = torch.tensor([caps] * B, dtype=torch.int32, device=q.device)
        lens = lens.to(device=q.device, dtype=torch.int32).contiguous()
        if tuple(lens.shape) != (B, 3):
            raise ValueError(f"lens must be int32 [B={B}, 3]")
        if order is not None:
            order = order.to(device=q.device, dtype=torch.int32).contiguous()
        if out is None:
            out = torch.empty(B, Hq, Sq, D, dtype=q.dtype, device=q.device)
        if out.dtype != q.dtype:
            raise ValueError(f"out must be {q.dtype} (the query's dtype), got {out.dtype}")
        self._keep = (q, chunk, sink, mid, recent, lens, order, out)
        a = _lib.PrefillArgs()
        a.B, a.Hq, a.Hkv, a.D, a.Sq = B, Hq, Hkv, D, Sq
        a.q, a.q_sb, a.q_sh, a.q_ss = q.data_ptr(), q.stride(0), q.stride(1), q.stride(2)
        a.out, a.o_sb, a.o_sh, a.o_ss = out.data_ptr(), out.stride(0), out.stride(1), out.stride(2)
        a.sm_scale = float(1.0 / math.sqrt(D) if sm_scale is None else sm_scale)
        a.lens = lens.data_ptr()
        a.order = order.data_ptr() if order is not None else None
        dt = q.dtype
        a.sink, a.mid = _fp16_tier(sink, dt), _mid_tier(mid, dt)
        a.recent, a.chunk = _fp16_tier(recent, dt), _fp16_tier(chunk, dt)
        a.mask_mode = _MASKS[mask]
        a.dtype = dtc
        self.args = a
        self.out = out
        self._fn = _lib.load().fade_tiered_prefill_attn
        self._argp = ctypes.byref(a)

    def run(self, stream: int | None = None) -> Tensor:
        s = torch.cuda.current_stream(self.out.device).cuda_stream if stream is None else stream
        _lib.check(self._fn(self._argp, s), "fade_tiered_prefill_attn")
        return self.out


def tiered_prefill_attention(q, chunk, sink=None, mid=None, recent=None, lens=None, order=None, sm_scale=None,
                             mask: str = "bottom_right") -> Tensor:
    """Causal attention of a chunk over each row's tiered cache; returns [B, Hq, Sq, D] of q's dtype."""
    return TieredPrefillPlan(q, chunk, sink, mid, recent, lens, order, sm_scale, mask=mask).run()


__all__ = ["TieredPrefillPlan", "tiered_prefill_attention"]
