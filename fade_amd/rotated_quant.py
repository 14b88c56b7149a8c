"""Rotation-then-quantize for K/V (fade/rotated_quant.py), on MI355X kernels.

``x_rot = x.float() @ R.T`` is a plain fp32 GEMM (rocBLAS through torch);
the quantizer that follows (fp32 absmax, ``inv = reciprocal(absmax) * qmax``,
round-half-even, clamp, bit-pack) runs in ``fade_quant_rotated`` and is
bit-exact given ``x_rot``.  Dequantize is ``fp16(code * scale)`` in
``fade_dequant_sym`` followed by the fp32 ``@ R`` GEMM.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from .quant import _pack_codes, _unpack_codes, dequant_sym

DEFAULT_SEED: int = 42
EPS: float = 1e-8
_BIT_PARAMS: dict[int, tuple[int, int]] = {4: (-8, 7), 3: (-4, 3), 2: (-2, 1)}


def _pack_int2_last_dim(q: Tensor) -> Tensor:
    """fade/rotated_quant.py:35-48: four 2-bit codes per byte, first in bits 7:6."""
    if q.shape[-1] % 4 != 0:
        raise ValueError(f"last dim must be divisible by 4 for INT2 packing, got {q.shape[-1]}")
    return _pack_codes(q, 2)


def _unpack_int2_last_dim(packed: Tensor) -> Tensor:
    """fade/rotated_quant.py:51-69."""
    return _unpack_codes(packed, 2)


def _random_orthogonal(dim: int, seed: int = DEFAULT_SEED) -> Tensor:
    """fade/rotated_quant.py:91-96: Q of the QR of a seeded CPU Gaussian matrix."""
    gen = torch.Generator().manual_seed(seed)
    q, _ = torch.linalg.qr(torch.randn(dim, dim, generator=gen))
    return q


def _rotate(x: Tensor, R: Tensor) -> Tensor:
    return (x.float() @ R.to(x.device, dtype=torch.float32).T).contiguous()


def _quant_rotated(x: Tensor, R: Tensor, bits: int, axis: int, op: str):
    if bits not in _BIT_PARAMS:
        raise ValueError(f"bits must be 2, 3 or 4, got {bits}")
    if x.dim() != 4:
        raise ValueError(f"{op}: expected [B, H, S, D], got shape {tuple(x.shape)}")
    _lib.require_gpu(x, op=op)
    B, H, S, D = x.shape
    x_rot = _rotate(x, R)
    row = D if bits == 3 else D * bits // 8
    packed = torch.empty(B, H, S, row, dtype=torch.int8 if bits == 3 else torch.uint8, device=x.device)
    scale_shape = (B, H, 1, D) if axis == _lib.AXIS_CHANNEL else (B, H, S, 1)
    scale = torch.empty(scale_shape, dtype=torch.float16, device=x.device)
    if x.numel() == 0:
        return packed, scale.to(x.dtype)
    import ctypes

    nb = ctypes.c_int64(0)
    _lib.check(_lib.load().fade_quant_rotated_workspace_bytes(B, H, S, D, axis, nb), op)
    ws = _lib.workspace(nb.value, x.device)
    _lib.call(
        "fade_quant_rotated", x_rot.data_ptr(), B, H, S, D, bits, axis, packed.data_ptr(),
        scale.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(x),
    )
    return packed, scale.to(x.dtype)


def rotated_quant_k(k: Tensor, R: Tensor, bits: int = 4) -> tuple[Tensor, Tensor]:
    """fade/rotated_quant.py:106-131: rotate, per-channel scale [B,H,1,D]."""
    return _quant_rotated(k, R, bits, _lib.AXIS_CHANNEL, "rotated_quant_k")


def rotated_quant_v(v: Tensor, R: Tensor, bits: int = 4) -> tuple[Tensor, Tensor]:
    """fade/rotated_quant.py:148-173: rotate, per-token scale [B,H,S,1]."""
    return _quant_rotated(v, R, bits, _lib.AXIS_TOKEN, "rotated_quant_v")


def rotated_dequant_rot(packed: Tensor, scale: Tensor, bits: int) -> Tensor:
    """fp16(code * scale) in the rotated basis (fade/rotated_quant.py:142-143)."""
    return dequant_sym(packed, scale.to(torch.float16), bits)


def _rotated_dequant(packed, scale, R, bits, dtype):
    x_rot = rotated_dequant_rot(packed, scale, bits)
    return (x_rot.float() @ R.to(x_rot.device, dtype=torch.float32)).to(dtype)


def rotated_dequant_k(packed, scale, R, bits: int = 4, dtype=torch.float16) -> Tensor:
    """fade/rotated_quant.py:134-145."""
    return _rotated_dequant(packed, scale, R, bits, dtype)


def rotated_dequant_v(packed, scale, R, bits: int = 4, dtype=torch.float16) -> Tensor:
    """fade/rotated_quant.py:176-187."""
    return _rotated_dequant(packed, scale, R, bits, dtype)


__all__ = [
    "rotated_dequant_k",
    "rotated_dequant_v",
    "rotated_quant_k",
    "rotated_quant_v",
]
