"""``fused_int4_sdpa``: attention straight from packed INT4 K/V (fade/kernels/fused_int4_attn.py).

Same signature, shapes and GQA mapping as the reference's Triton op
(fade/kernels/fused_int4_attn.py:277-342).  Single-token queries run the
tiered decode kernel with the whole packed tensor as its middle tier; several
query rows (or a top-left causal mask) run the MFMA prefill kernel over it in
one launch.  GQA is resolved inside the kernels (no ``repeat_interleave``
copies).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from .. import _lib
from .prefill import tiered_prefill_attention
from .tiered_attn import MiddleTier, tiered_decode_attention


def fused_int4_sdpa(
    q: Tensor,
    k_packed: Tensor,
    k_scale: Tensor,
    v_packed: Tensor,
    v_scale: Tensor,
    is_causal: bool = False,
) -> Tensor:
    """Fused INT4 attention.

    Args:
        q: [B, H_q, S_q, D] fp16.
        k_packed / v_packed: [B, H_kv, S_k, D//2] uint8 (fade/quant.py layout).
        k_scale: [B, H_kv, 1, D] fp16; v_scale: [B, H_kv, S_k, 1] fp16.
        is_causal: top-left aligned causal mask, as the reference's kernel
            applies it (query row i sees keys j <= i).
    Returns:
        [B, H_q, S_q, D] fp16.
    """
    _lib.require_gpu(q, k_packed, k_scale, v_packed, v_scale, op="fused_int4_sdpa")
    B, Hq, Sq, D = q.shape
    if k_packed.shape[-1] * 2 != D or v_packed.shape != k_packed.shape:
        raise ValueError(f"packed K/V must be [B, H_kv, S_k, {D // 2}]")
    Sk = int(k_packed.shape[2])
    mid = MiddleTier(
        fmt="int4",
        k_codes=k_packed.contiguous(),
        v_codes=v_packed.contiguous(),
        k_scale=k_scale.to(torch.float16).contiguous(),
        v_scale=v_scale.to(torch.float16).contiguous(),
    )
    q16 = q.to(torch.float16)
    if Sq == 1 and not is_causal:
        return tiered_decode_attention(q16, None, mid, None)
    # several query rows, or top-left causal: one launch of the MFMA prefill kernel with the
    # packed tensor as every row's middle tier and no keys of the queries' own
    B = int(q.shape[0])
    lens = torch.tensor([[0, Sk, 0]] * B, dtype=torch.int32).to(q.device, non_blocking=True)
    return tiered_prefill_attention(q16, None, None, mid, None, lens=lens,
                                    mask="top_left" if is_causal else "none")


def fused_int4_sdpa_with_fallback(q, k_packed, k_scale, v_packed, v_scale, force_fused: bool = False) -> Tensor:
    """fade/kernels/fused_int4_attn.py:345-365.

    ``force_fused=False`` is the reference's "dequantize then SDPA" path: the
    dequantization runs on the HIP kernel and SDPA on torch (GPU only).
    """
    if force_fused:
        return fused_int4_sdpa(q, k_packed, k_scale, v_packed, v_scale)
    from ..quant import dequant_int4

    k = dequant_int4(k_packed, k_scale)
    v = dequant_int4(v_packed, v_scale)
    Hq, Hkv = q.shape[1], k.shape[1]
    if Hq != Hkv:
        k = k.repeat_interleave(Hq // Hkv, dim=1)
        v = v.repeat_interleave(Hq // Hkv, dim=1)
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float()).to(q.dtype)


def check_fused_parity(B: int = 1, H: int = 4, S_q: int = 1, S_k: int = 256, D: int = 128, atol: float = 1e-2) -> dict:
    """fade/kernels/fused_int4_attn.py:368-402: fused kernel vs dequantize + SDPA."""
    if not torch.cuda.is_available():
        return {"passed": False, "error": "no GPU available"}
    try:
        _lib.load()
    except RuntimeError as e:
        return {"passed": False, "error": str(e)}
    from ..quant import quant_k_int4, quant_v_int4

    torch.manual_seed(42)
    dev = "cuda"
    q = torch.randn(B, H, S_q, D, dtype=torch.float16, device=dev)
    k = torch.randn(B, H, S_k, D, dtype=torch.float16, device=dev)
    v = torch.randn(B, H, S_k, D, dtype=torch.float16, device=dev)
    kp, ks = quant_k_int4(k)
    vp, vs = quant_v_int4(v)
    ref = fused_int4_sdpa_with_fallback(q, kp, ks, vp, vs, force_fused=False)
    out = fused_int4_sdpa(q, kp, ks, vp, vs)
    err = (ref.float() - out.float()).abs()
    return {
        "passed": bool(err.max().item() < atol),
        "max_abs_error": err.max().item(),
        "mean_abs_error": err.mean().item(),
        "atol": atol,
    }


__all__ = ["check_fused_parity", "fused_int4_sdpa", "fused_int4_sdpa_with_fallback"]
