"""``int4_sdpa``: INT4 attention entry point of fade/kernels/int4_attention.py:206-225.

The reference dequantizes (torch or an uncoalesced Triton unpack) and calls
SDPA without expanding GQA heads.  Here the packed tensors feed the fused
kernels (decode for single-token queries, the MFMA prefill kernel without a
mask for longer ones), which also resolve GQA.  ``force_triton`` is accepted
for signature compatibility and ignored (there is no Triton in this build).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from .. import _lib
from ..quant import dequant_int4
from .fused_int4_attn import fused_int4_sdpa

USE_TRITON_KERNEL = False


def _int4_sdpa_hip(q, k_packed, k_scale, v_packed, v_scale, dtype=torch.float16) -> Tensor:
    return fused_int4_sdpa(q, k_packed, k_scale, v_packed, v_scale).to(dtype)


def int4_sdpa(
    q: Tensor,
    k_packed: Tensor,
    k_scale: Tensor,
    v_packed: Tensor,
    v_scale: Tensor,
    dtype: torch.dtype = torch.float16,
    force_triton: bool = False,
) -> Tensor:
    """Attention over packed INT4 K/V; ``q`` and K/V must have the same head count here."""
    del force_triton
    _lib.require_gpu(q, k_packed, k_scale, v_packed, v_scale, op="int4_sdpa")
    return _int4_sdpa_hip(q, k_packed, k_scale, v_packed, v_scale, dtype)


def check_parity(B=1, H=4, S_q=1, S_k=32, D=128, atol=1e-2, rtol=0.05) -> dict:
    """fade/kernels/int4_attention.py:228-269: fused HIP path vs dequantize + SDPA."""
    if not torch.cuda.is_available():
        return {"passed": False, "error": "no GPU available"}
    from ..quant import quant_k_int4, quant_v_int4

    torch.manual_seed(42)
    q = torch.randn(B, H, S_q, D, dtype=torch.float16, device="cuda")
    k = torch.randn(B, H, S_k, D, dtype=torch.float16, device="cuda")
    v = torch.randn(B, H, S_k, D, dtype=torch.float16, device="cuda")
    kp, ks = quant_k_int4(k)
    vp, vs = quant_v_int4(v)
    ref = F.scaled_dot_product_attention(
        q.float(), dequant_int4(kp, ks).float(), dequant_int4(vp, vs).float()
    )
    out = int4_sdpa(q, kp, ks, vp, vs)
    err = (ref - out.float()).abs()
    return {
        "passed": bool(err.max().item() < atol and err.mean().item() < atol * 0.5),
        "max_abs_error": err.max().item(),
        "mean_abs_error": err.mean().item(),
        "atol": atol,
        "rtol": rtol,
    }


__all__ = ["USE_TRITON_KERNEL", "check_parity", "int4_sdpa"]
