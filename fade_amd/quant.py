"""Quantization primitives for the K/V middle tier, on MI355X kernels.

Same names, shapes, dtypes and error messages as ``fade/quant.py`` (FADE);
the arithmetic runs in ``libfade_hip.so`` and reproduces the reference's
torch rounding bit for bit (codes, packed bytes and scales).

  * K: per-channel symmetric INT4 (absmax over S), two nibbles per byte,
    high nibble = even index (fade/quant.py:26-43, 61-75).
  * V: per-token symmetric INT4 (absmax over D) (fade/quant.py:78-92).
  * INT2: symmetric, groups of ``group_size`` tokens along S with a
    per-(group, channel) scale, codes stored unpacked in int8
    (fade/quant.py:95-176).
  * ``quant_asym`` / ``dequant_asym``: per-token asymmetric groups along D
    with fp16 scale/zero -- a format this build adds (the reference has no
    zero-point quantizer).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

INT4_MIN: int = -8
INT4_MAX: int = 7
INT2_MIN: int = -2
INT2_MAX: int = 1
EPS: float = 1e-8
DEFAULT_INT2_GROUP_SIZE: int = 64


def _check_4d(x: Tensor, op: str) -> None:
    if x.dim() != 4:
        raise ValueError(f"{op}: expected [B, H, S, D], got shape {tuple(x.shape)}")


def _strides_bhs(x: Tensor) -> tuple[int, int, int]:
    if x.stride(-1) != 1:
        raise ValueError("the last (head_dim) axis must be contiguous")
    return x.stride(0), x.stride(1), x.stride(2)


def _prep_f16(x: Tensor, op: str) -> Tensor:
    _check_4d(x, op)
    _lib.require_gpu(x, op=op)
    _lib.require_f16(x, op)
    return _aligned(x)


def _prep_kv(x: Tensor, op: str) -> Tensor:
    """K/V input of the INT4 quantizers: float16, bfloat16 or float32 (the
    reference's quantizers take any float dtype and return the scale in it)."""
    _check_4d(x, op)
    _lib.require_gpu(x, op=op)
    if x.dtype not in _lib.DTYPE_CODES:
        raise ValueError(f"{op}: expected a float16, bfloat16 or float32 tensor, got {x.dtype}")
    return _aligned(x)


def _aligned(x: Tensor) -> Tensor:
    if x.stride(-1) != 1 or x.data_ptr() % 16 or any(s % 8 for s in x.stride()[:3]):
        x = x.contiguous()
    return x


def _pack_int4_last_dim(q_int8: Tensor) -> Tensor:
    """fade/quant.py:26-43: pack pairs of INT4 codes, high nibble = even index."""
    if q_int8.shape[-1] % 2 != 0:
        raise ValueError(f"last dim must be even for INT4 packing, got {q_int8.shape[-1]}")
    return _pack_codes(q_int8, 4)


def _unpack_int4_last_dim(packed: Tensor) -> Tensor:
    """fade/quant.py:46-58."""
    return _unpack_codes(packed, 4)


def _pack_codes(q: Tensor, bits: int) -> Tensor:
    _lib.require_gpu(q, op="pack")
    D = q.shape[-1]
    if D % 8 != 0:
        raise ValueError(f"fade_amd packs rows whose last dim is a multiple of 8, got {D}")
    q = q.to(torch.int8).contiguous()
    out = torch.empty(*q.shape[:-1], D * bits // 8, dtype=torch.uint8, device=q.device)
    _lib.call("fade_pack_codes", q.data_ptr(), q.numel() // D, D, bits, out.data_ptr(), _lib.stream_of(q))
    return out


def _unpack_codes(packed: Tensor, bits: int) -> Tensor:
    _lib.require_gpu(packed, op="unpack")
    D = packed.shape[-1] * 8 // bits
    if D % 8 != 0:
        raise ValueError(f"fade_amd unpacks rows whose last dim is a multiple of 8, got {D}")
    packed = packed.contiguous()
    out = torch.empty(*packed.shape[:-1], D, dtype=torch.int8, device=packed.device)
    _lib.call(
        "fade_unpack_codes", packed.data_ptr(), packed.numel() * 8 // bits // D, D, bits,
        out.data_ptr(), _lib.stream_of(packed),
    )
    return out


def quant_k_int4(k: Tensor) -> tuple[Tensor, Tensor]:
    """Per-channel symmetric INT4 for K, bit-packed (fade/quant.py:61-75).

    Returns ``(packed [B,H,S,D//2] uint8, scale [B,H,1,D] k.dtype)``; ``k`` is
    float16, bfloat16 or float32.
    """
    k = _prep_kv(k, "quant_k_int4")
    B, H, S, D = k.shape
    packed = torch.empty(B, H, S, D // 2, dtype=torch.uint8, device=k.device)
    scale = torch.empty(B, H, 1, D, dtype=k.dtype, device=k.device)
    if k.numel() == 0:
        return packed, scale
    lib = _lib.load()
    nb = ctypes_i64()
    _lib.check(lib.fade_quant_k_int4_workspace_bytes(B, H, S, D, nb), "fade_quant_k_int4_workspace_bytes")
    ws = _lib.scratch(nb.value, k.device)  # column partials: written in full before they are read
    sb, sh, ss = _strides_bhs(k)
    if k.dtype == torch.float16:
        _lib.call(
            "fade_quant_k_int4", k.data_ptr(), B, H, S, D, sb, sh, ss, packed.data_ptr(),
            scale.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(k),
        )
    else:
        _lib.call(
            "fade_quant_k_int4_dtype", k.data_ptr(), _lib.DTYPE_CODES[k.dtype], B, H, S, D, sb, sh, ss,
            packed.data_ptr(), scale.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(k),
        )
    return packed, scale


def quant_k_int4_from_colmax(k: Tensor, colmax: Tensor) -> tuple[Tensor, Tensor]:
    """``quant_k_int4`` for K whose per-channel absmax is already gathered
    (fade/quant.py:61-75, second pass only).

    ``colmax``: fp32 [B*H, parts, D] partial maxima of |K| (e.g. from
    ``fade_reassign_gather``); channel d's absmax is their max over the parts.
    Codes and scales equal ``quant_k_int4(k)``'s when the parts cover every row.
    """
    k = _prep_f16(k, "quant_k_int4_from_colmax")
    B, H, S, D = k.shape
    if colmax.dtype != torch.float32 or colmax.dim() != 3 or colmax.shape[0] != B * H or colmax.shape[2] != D:
        raise ValueError(f"colmax must be float32 [B*H={B * H}, parts, D={D}], got {tuple(colmax.shape)}")
    _lib.require_gpu(k, colmax, op="quant_k_int4_from_colmax")
    colmax = colmax.contiguous()
    packed = torch.empty(B, H, S, D // 2, dtype=torch.uint8, device=k.device)
    scale = torch.empty(B, H, 1, D, dtype=torch.float16, device=k.device)
    if k.numel() == 0:
        return packed, scale
    sb, sh, ss = _strides_bhs(k)
    _lib.call(
        "fade_quant_k_int4_from_colmax", k.data_ptr(), B, H, S, D, sb, sh, ss, colmax.data_ptr(),
        int(colmax.shape[1]), packed.data_ptr(), scale.data_ptr(), _lib.stream_of(k),
    )
    return packed, scale


def quant_v_int4(v: Tensor) -> tuple[Tensor, Tensor]:
    """Per-token symmetric INT4 for V, bit-packed (fade/quant.py:78-92).

    Returns ``(packed [B,H,S,D//2] uint8, scale [B,H,S,1] v.dtype)``; ``v`` is
    float16, bfloat16 or float32.
    """
    v = _prep_kv(v, "quant_v_int4")
    B, H, S, D = v.shape
    packed = torch.empty(B, H, S, D // 2, dtype=torch.uint8, device=v.device)
    scale = torch.empty(B, H, S, 1, dtype=v.dtype, device=v.device)
    if v.numel() == 0:
        return packed, scale
    sb, sh, ss = _strides_bhs(v)
    if v.dtype == torch.float16:
        _lib.call(
            "fade_quant_v_int4", v.data_ptr(), B, H, S, D, sb, sh, ss, packed.data_ptr(),
            scale.data_ptr(), _lib.stream_of(v),
        )
    else:
        _lib.call(
            "fade_quant_v_int4_dtype", v.data_ptr(), _lib.DTYPE_CODES[v.dtype], B, H, S, D, sb, sh, ss,
            packed.data_ptr(), scale.data_ptr(), _lib.stream_of(v),
        )
    return packed, scale


def _quant_int2_grouped(x: Tensor, group_size: int, op: str, s_actual: int | None = None):
    x = _prep_kv(x, op)
    B, H, S, D = x.shape
    s_pad = S
    if s_actual is None:
        if S % group_size != 0:
            raise ValueError(f"S={S} must be divisible by group_size={group_size}")
    else:  # fused pad_to_group: rows >= S read as zero
        s_pad = S + (-S) % group_size
    G = s_pad // group_size
    codes = torch.empty(B, H, s_pad, D, dtype=torch.int8, device=x.device)
    scale = torch.empty(B, H, G, D, dtype=x.dtype, device=x.device)
    if codes.numel() == 0:
        return codes, scale
    sb, sh, ss = _strides_bhs(x)
    if x.dtype == torch.float16:
        _lib.call(
            "fade_quant_int2_grouped", x.data_ptr(), B, H, S, s_pad, D, sb, sh, ss, group_size,
            codes.data_ptr(), scale.data_ptr(), _lib.stream_of(x),
        )
    else:
        _lib.call(
            "fade_quant_int2_grouped_dtype", x.data_ptr(), _lib.DTYPE_CODES[x.dtype], B, H, S, s_pad, D, sb, sh,
            ss, group_size, codes.data_ptr(), scale.data_ptr(), _lib.stream_of(x),
        )
    return codes, scale


def quant_k_int2(k: Tensor, group_size: int = DEFAULT_INT2_GROUP_SIZE) -> tuple[Tensor, Tensor]:
    """Per-channel INT2 for K, groups of ``group_size`` along S (fade/quant.py:95-112)."""
    return _quant_int2_grouped(k, group_size, "quant_k_int2")


def quant_v_int2(v: Tensor, group_size: int = DEFAULT_INT2_GROUP_SIZE) -> tuple[Tensor, Tensor]:
    """Grouped INT2 for V, same structure as K (fade/quant.py:130-150)."""
    return _quant_int2_grouped(v, group_size, "quant_v_int2")


def quant_int2_padded(x: Tensor, group_size: int = DEFAULT_INT2_GROUP_SIZE) -> tuple[Tensor, Tensor]:
    """``quant_v_int2(pad_to_group(x)[0])`` without materializing the padding."""
    return _quant_int2_grouped(x, group_size, "quant_int2_padded", s_actual=x.shape[-2])


def dequant(q: Tensor, scale: Tensor, dtype: torch.dtype = torch.float16) -> Tensor:
    """fade/quant.py:115-121: broadcast ``q.to(dtype) * scale.to(dtype)`` (GPU tensors only)."""
    _lib.require_gpu(q, scale, op="dequant")
    return q.to(dtype) * scale.to(dtype)


def _scale_axis(packed: Tensor, scale: Tensor) -> int:
    B, H, S = packed.shape[:3]
    if scale.shape[-2] == 1 and scale.shape[-1] != 1:
        return _lib.AXIS_CHANNEL
    if scale.shape[-1] == 1 and scale.shape[-2] == S:
        return _lib.AXIS_TOKEN
    if S == 1 and scale.shape[-1] == 1:
        return _lib.AXIS_TOKEN
    raise ValueError(f"unsupported scale shape {tuple(scale.shape)} for packed {tuple(packed.shape)}")


def dequant_sym(packed: Tensor, scale: Tensor, bits: int, dtype: torch.dtype = torch.float16) -> Tensor:
    """Unpack symmetric codes and return ``dtype(code * scale.to(dtype))``
    (float16, bfloat16 or float32, as ``q.to(dtype) * scale.to(dtype)``)."""
    _check_4d(packed, "dequant")
    _lib.require_gpu(packed, scale, op="dequant")
    if dtype not in _lib.DTYPE_CODES:
        raise ValueError(f"fade_amd dequantizes to float16, bfloat16 or float32, got {dtype}")
    axis = _scale_axis(packed, scale)
    B, H, S, nb = packed.shape
    D = nb if bits == 3 else nb * 8 // bits
    out = torch.empty(B, H, S, D, dtype=dtype, device=packed.device)
    if out.numel() == 0:
        return out
    packed = packed.contiguous()
    scale = scale.to(dtype).contiguous()
    if dtype == torch.float16:
        _lib.call(
            "fade_dequant_sym", packed.data_ptr(), scale.data_ptr(), bits, axis, B, H, S, D,
            out.data_ptr(), _lib.stream_of(packed),
        )
    else:
        _lib.call(
            "fade_dequant_sym_dtype", packed.data_ptr(), scale.data_ptr(), _lib.DTYPE_CODES[dtype], bits, axis,
            B, H, S, D, out.data_ptr(), _lib.stream_of(packed),
        )
    return out


def dequant_int4(packed: Tensor, scale: Tensor, dtype: torch.dtype = torch.float16) -> Tensor:
    """fade/quant.py:124-127: unpack and dequantize a bit-packed INT4 tensor."""
    return dequant_sym(packed, scale, 4, dtype)


def _dequant_int2(q: Tensor, scale: Tensor, group_size: int, dtype, s_out: int | None = None) -> Tensor:
    _check_4d(q, "dequant_int2")
    _lib.require_gpu(q, scale, op="dequant_int2")
    if dtype not in _lib.DTYPE_CODES:
        raise ValueError(f"fade_amd dequantizes to float16, bfloat16 or float32, got {dtype}")
    B, H, S, D = q.shape
    s_out = S if s_out is None else s_out
    out = torch.empty(B, H, s_out, D, dtype=dtype, device=q.device)
    if out.numel() == 0:
        return out
    q = q.contiguous()
    scale = scale.to(dtype).contiguous()  # q.to(dtype) * scale.to(dtype)
    if dtype == torch.float16:
        _lib.call(
            "fade_dequant_int2_grouped", q.data_ptr(), scale.data_ptr(), B, H, S, D, group_size, s_out,
            out.data_ptr(), _lib.stream_of(q),
        )
    else:
        _lib.call(
            "fade_dequant_int2_grouped_dtype", q.data_ptr(), scale.data_ptr(), _lib.DTYPE_CODES[dtype], B, H, S, D,
            group_size, s_out, out.data_ptr(), _lib.stream_of(q),
        )
    return out


def dequant_k_int2(q, scale, group_size: int = DEFAULT_INT2_GROUP_SIZE, dtype=torch.float16) -> Tensor:
    """fade/quant.py:153-163."""
    return _dequant_int2(q, scale, group_size, dtype)


def dequant_v_int2(q, scale, group_size: int = DEFAULT_INT2_GROUP_SIZE, dtype=torch.float16) -> Tensor:
    """fade/quant.py:166-176."""
    return _dequant_int2(q, scale, group_size, dtype)


def dequant_int2_trimmed(q, scale, n: int, group_size: int = DEFAULT_INT2_GROUP_SIZE) -> Tensor:
    """Dequantize and drop the ``pad_to_group`` rows in one pass (fade/cache.py:834-837, 868-872)."""
    return _dequant_int2(q, scale, group_size, scale.dtype, s_out=n)


def pad_to_group(x: Tensor, group_size: int) -> tuple[Tensor, int]:
    """fade/quant.py:179-188: zero-pad S (dim -2) to a multiple of ``group_size``."""
    S = x.shape[-2]
    if S % group_size == 0:
        return x, S
    total = S + group_size - (S % group_size)
    padded = torch.zeros(*x.shape[:-2], total, x.shape[-1], dtype=x.dtype, device=x.device)
    padded[..., :S, :] = x
    return padded, S


def quant_asym(x: Tensor, bits: int = 4, group: int = 32) -> tuple[Tensor, Tensor, Tensor]:
    """Per-token asymmetric quantization in groups of ``group`` along D.

    Returns ``(packed [B,H,S,D*bits/8] uint8, scale [B,H,S,D/group] fp16,
    zero [B,H,S,D/group] fp16)`` with ``x_hat = code * scale + zero``.
    """
    x = _prep_f16(x, "quant_asym")
    B, H, S, D = x.shape
    packed = torch.empty(B, H, S, D * bits // 8, dtype=torch.uint8, device=x.device)
    scale = torch.empty(B, H, S, D // group, dtype=torch.float16, device=x.device)
    zero = torch.empty_like(scale)
    if x.numel() == 0:
        return packed, scale, zero
    sb, sh, ss = _strides_bhs(x)
    _lib.call(
        "fade_quant_asym", x.data_ptr(), B, H, S, D, sb, sh, ss, bits, group, packed.data_ptr(),
        scale.data_ptr(), zero.data_ptr(), _lib.stream_of(x),
    )
    return packed, scale, zero


def dequant_asym(packed: Tensor, scale: Tensor, zero: Tensor, bits: int = 4, group: int = 32) -> Tensor:
    _check_4d(packed, "dequant_asym")
    _lib.require_gpu(packed, scale, zero, op="dequant_asym")
    B, H, S, nb = packed.shape
    D = nb * 8 // bits
    out = torch.empty(B, H, S, D, dtype=torch.float16, device=packed.device)
    if out.numel() == 0:
        return out
    packed, scale, zero = packed.contiguous(), scale.contiguous(), zero.contiguous()
    _lib.call(
        "fade_dequant_asym", packed.data_ptr(), scale.data_ptr(), zero.data_ptr(), bits, group,
        B, H, S, D, out.data_ptr(), _lib.stream_of(packed),
    )
    return out


def ctypes_i64():
    import ctypes

    return ctypes.c_int64(0)


__all__ = [
    "DEFAULT_INT2_GROUP_SIZE",
    "dequant",
    "dequant_asym",
    "dequant_int4",
    "dequant_k_int2",
    "dequant_v_int2",
    "pad_to_group",
    "quant_asym",
    "quant_k_int2",
    "quant_k_int4",
    "quant_k_int4_from_colmax",
    "quant_v_int2",
    "quant_v_int4",
]
