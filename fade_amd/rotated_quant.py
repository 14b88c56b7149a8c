"""Rotation-then-quantize for K/V (fade/rotated_quant.py), on MI355X kernels.

fp16 K/V with head_dim 128 go through ``fade_rotate_quant``: one fused kernel
(two for per-channel K) computes ``x_rot = x @ R.T`` on the matrix cores with
R split into fp16 hi/lo parts (fp32-GEMM accuracy) and quantizes it in place
(fp32 absmax, ``inv = reciprocal(absmax) * qmax``, round-half-even, clamp,
bit-pack); x_rot never reaches HBM.  Other shapes and dtypes take the two-step
path: an fp32 GEMM through torch, then ``fade_quant_rotated``, which is
bit-exact given ``x_rot`` (``quant_rotated_given``); bfloat16 and float32
inputs get their scale in their own dtype (one rounding of the fp32
``absmax / qmax``, as the reference's ``scale.to(k.dtype)``).  Dequantize is
``dtype(code * scale)`` in ``fade_dequant_sym`` followed by the fp32 ``@ R``
GEMM.
"""

from __future__ import annotations

import ctypes

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


def _alloc_out(shape, bits: int, axis: int, device, scale_dtype=torch.float16):
    B, H, S, D = shape
    row = D if bits == 3 else D * bits // 8
    packed = torch.empty(B, H, S, row, dtype=torch.int8 if bits == 3 else torch.uint8, device=device)
    scale_shape = (B, H, 1, D) if axis == _lib.AXIS_CHANNEL else (B, H, S, 1)
    scale = torch.empty(scale_shape, dtype=scale_dtype, device=device)
    return packed, scale


def _check(x: Tensor, bits: int, op: str) -> None:
    if bits not in _BIT_PARAMS:
        raise ValueError(f"bits must be 2, 3 or 4, got {bits}")
    if x.dim() != 4:
        raise ValueError(f"{op}: expected [B, H, S, D], got shape {tuple(x.shape)}")
    _lib.require_gpu(x, op=op)


def quant_rotated_given(
    x_rot: Tensor, bits: int, axis: int, op: str = "quant_rotated_given", scale_dtype: torch.dtype = torch.float16
):
    """Quantize an already-rotated fp32 tensor [B, H, S, D] (fade/rotated_quant.py:121-131 with
    ``axis=AXIS_CHANNEL``, 163-173 with ``AXIS_TOKEN``); bit-exact with the reference given x_rot.
    Returns (packed, scale of ``scale_dtype``: float16, bfloat16 or float32)."""
    _check(x_rot, bits, op)
    if scale_dtype not in _lib.DTYPE_CODES:
        raise ValueError(f"{op}: scale dtype must be float16, bfloat16 or float32, got {scale_dtype}")
    x_rot = x_rot.float().contiguous()
    B, H, S, D = x_rot.shape
    packed, scale = _alloc_out(x_rot.shape, bits, axis, x_rot.device, scale_dtype)
    if x_rot.numel() == 0:
        return packed, scale
    nb = ctypes.c_int64(0)
    _lib.check(_lib.load().fade_quant_rotated_workspace_bytes(B, H, S, D, axis, nb), op)
    ws = _lib.scratch(nb.value, x_rot.device)  # column partials: written in full before they are read
    if scale_dtype == torch.float16:
        _lib.call(
            "fade_quant_rotated", x_rot.data_ptr(), B, H, S, D, bits, axis, packed.data_ptr(),
            scale.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(x_rot),
        )
    else:
        _lib.call(
            "fade_quant_rotated_dtype", x_rot.data_ptr(), B, H, S, D, bits, axis, packed.data_ptr(),
            scale.data_ptr(), _lib.DTYPE_CODES[scale_dtype], ws.data_ptr(), ws.numel(), _lib.stream_of(x_rot),
        )
    return packed, scale


def _fused_ok(x: Tensor) -> bool:
    return (
        x.dtype == torch.float16
        and x.shape[-1] == 128
        and x.stride(-1) == 1
        and all(st % 8 == 0 for st in x.stride()[:3])
        and x.data_ptr() % 16 == 0
    )


def _rotate_quant_fused(x: Tensor, R: Tensor, bits: int, axis: int, op: str):
    B, H, S, D = x.shape
    packed, scale = _alloc_out(x.shape, bits, axis, x.device)
    if x.numel() == 0:
        return packed, scale
    Rd = R.to(x.device, dtype=torch.float32).contiguous()
    nb = ctypes.c_int64(0)
    _lib.check(_lib.load().fade_rotate_quant_workspace_bytes(B, H, S, D, axis, nb), op)
    ws = torch.empty(nb.value, dtype=torch.uint8, device=x.device) if nb.value else None
    sb, sh, ss, _ = x.stride()
    _lib.call(
        "fade_rotate_quant", x.data_ptr(), B, H, S, D, sb, sh, ss, Rd.data_ptr(), bits, axis,
        packed.data_ptr(), scale.data_ptr(), _lib.ptr(ws), nb.value, _lib.stream_of(x),
    )
    return packed, scale


def _quant_rotated(x: Tensor, R: Tensor, bits: int, axis: int, op: str):
    _check(x, bits, op)
    if tuple(R.shape) != (x.shape[-1], x.shape[-1]):
        raise ValueError(f"{op}: R must be [{x.shape[-1]}, {x.shape[-1]}], got {tuple(R.shape)}")
    if _fused_ok(x):
        return _rotate_quant_fused(x, R, bits, axis, op)
    sdt = x.dtype if x.dtype in _lib.DTYPE_CODES else torch.float32
    packed, scale = quant_rotated_given(_rotate(x, R), bits, axis, op, scale_dtype=sdt)
    return packed, scale.to(x.dtype)


def rotated_quant_k(k: Tensor, R: Tensor, bits: int = 4) -> tuple[Tensor, Tensor]:
    """fade/rotated_quant.py:106-131: rotate, per-channel scale [B,H,1,D]."""
    return _quant_rotated(k, R, bits, _lib.AXIS_CHANNEL, "rotated_quant_k")


def rotated_quant_v(v: Tensor, R: Tensor, bits: int = 4) -> tuple[Tensor, Tensor]:
    """fade/rotated_quant.py:148-173: rotate, per-token scale [B,H,S,1]."""
    return _quant_rotated(v, R, bits, _lib.AXIS_TOKEN, "rotated_quant_v")


def rotated_dequant_rot(packed: Tensor, scale: Tensor, bits: int, dtype: torch.dtype = torch.float16) -> Tensor:
    """``code.to(dtype) * scale.to(dtype)`` in the rotated basis (fade/rotated_quant.py:142-143)."""
    return dequant_sym(packed, scale, bits, dtype)


def _rotated_dequant(packed, scale, R, bits, dtype):
    # the rotation back runs as an fp32 GEMM for every dtype (the reference's
    # CPU path; on CUDA it multiplies bf16 in bf16)
    x_rot = rotated_dequant_rot(packed, scale, bits, dtype if dtype in _lib.DTYPE_CODES else torch.float32)
    return (x_rot.float() @ R.to(x_rot.device, dtype=torch.float32)).to(dtype)


def rotated_dequant_k(packed, scale, R, bits: int = 4, dtype=torch.float16) -> Tensor:
    """fade/rotated_quant.py:134-145."""
    return _rotated_dequant(packed, scale, R, bits, dtype)


def rotated_dequant_v(packed, scale, R, bits: int = 4, dtype=torch.float16) -> Tensor:
    """fade/rotated_quant.py:176-187."""
    return _rotated_dequant(packed, scale, R, bits, dtype)


__all__ = [
    "quant_rotated_given",
    "rotated_dequant_k",
    "rotated_dequant_v",
    "rotated_quant_k",
    "rotated_quant_v",
]
