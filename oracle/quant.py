"""Numpy restatement of the reference quantizers (test infrastructure only).

Reference: ``fade/quant.py`` and ``fade/rotated_quant.py`` of FADE.  Every
fp16 (bf16) op is modelled as "compute in fp32, round to fp16 (bf16)" (torch
CPU semantics); every fp32 op as one IEEE fp32 rounding.
"""

from __future__ import annotations

import numpy as np

F16 = np.float16
F32 = np.float32

INT4_MIN, INT4_MAX = -8, 7  # fade/quant.py:18-19
INT2_MIN, INT2_MAX = -2, 1  # fade/quant.py:20-21
EPS = 1e-8  # fade/quant.py:22
DEFAULT_INT2_GROUP_SIZE = 64  # fade/quant.py:23
BIT_PARAMS = {4: (-8, 7), 3: (-4, 3), 2: (-2, 1)}  # fade/rotated_quant.py:28-32


def _f16(x):
    return np.asarray(x, dtype=F32).astype(F16)


def _rne_clamp(x32: np.ndarray, lo: int, hi: int) -> np.ndarray:
    """``.round().clamp(lo, hi).to(int8)`` with NaN -> 0 (torch CPU int cast)."""
    with np.errstate(invalid="ignore"):
        q = np.rint(x32.astype(F32))
        nan = np.isnan(q)
        q = np.clip(q, lo, hi)
        q[nan] = 0
    return q.astype(np.int8)


# --------------------------------------------------------------------------- #
# bit packing
# --------------------------------------------------------------------------- #
def pack_int4_last_dim(q: np.ndarray) -> np.ndarray:
    """fade/quant.py:26-43: byte[d] = (q[2d] & 0xF) << 4 | (q[2d+1] & 0xF)."""
    if q.shape[-1] % 2 != 0:
        raise ValueError(f"last dim must be even for INT4 packing, got {q.shape[-1]}")
    u = (q.astype(np.int16) & 0xF).astype(np.uint8)
    return ((u[..., 0::2] << 4) | u[..., 1::2]).astype(np.uint8)


def unpack_int4_last_dim(packed: np.ndarray) -> np.ndarray:
    """fade/quant.py:46-58: sign-extend each nibble; high nibble first."""
    hi = ((packed >> 4) & 0xF).astype(np.int16)
    lo = (packed & 0xF).astype(np.int16)
    hi = hi - ((hi & 8) << 1)
    lo = lo - ((lo & 8) << 1)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.int8)
    out[..., 0::2] = hi
    out[..., 1::2] = lo
    return out


def pack_int2_last_dim(q: np.ndarray) -> np.ndarray:
    """fade/rotated_quant.py:35-48: byte = c0<<6 | c1<<4 | c2<<2 | c3 (MSB first)."""
    if q.shape[-1] % 4 != 0:
        raise ValueError(f"last dim must be divisible by 4 for INT2 packing, got {q.shape[-1]}")
    u = (q.astype(np.int8) & 0x3).astype(np.uint8)
    return ((u[..., 0::4] << 6) | (u[..., 1::4] << 4) | (u[..., 2::4] << 2) | u[..., 3::4]).astype(
        np.uint8
    )


def unpack_int2_last_dim(packed: np.ndarray) -> np.ndarray:
    """fade/rotated_quant.py:51-69."""
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 4,), dtype=np.int8)
    for j, sh in enumerate((6, 4, 2, 0)):
        c = ((packed >> sh) & 0x3).astype(np.int8)
        out[..., j::4] = c - ((c & 2) << 1)
    return out


def pack_bits(q: np.ndarray, bits: int) -> np.ndarray:
    """fade/rotated_quant.py:72-79 (3-bit stays raw int8)."""
    if bits == 4:
        return pack_int4_last_dim(q)
    if bits == 2:
        return pack_int2_last_dim(q)
    return q.astype(np.int8)


def unpack_bits(packed: np.ndarray, bits: int) -> np.ndarray:
    """fade/rotated_quant.py:82-88."""
    if bits == 4:
        return unpack_int4_last_dim(packed)
    if bits == 2:
        return unpack_int2_last_dim(packed)
    return packed.astype(np.int8)


# --------------------------------------------------------------------------- #
# symmetric quantizers on fp16 input (torch fp16 per-op rounding)
# --------------------------------------------------------------------------- #
def _sym_params_f16(absmax: np.ndarray, qmax: int) -> tuple[np.ndarray, np.ndarray]:
    """``inv = qmax / absmax`` and ``scale = absmax / qmax`` on fp16 tensors.

    ``clamp(min=1e-8)`` is a no-op on fp16 (1e-8 rounds to 0; the smallest
    subnormal is 6e-8).  ``qmax / t`` is ``t.reciprocal() * qmax``
    (torch ``Tensor.__rtruediv__``), so ``inv`` is rounded twice.
    """
    a32 = absmax.astype(F32)
    with np.errstate(divide="ignore", over="ignore"):
        r = (F32(1.0) / a32).astype(F16)
        inv = (r.astype(F32) * F32(qmax)).astype(F16)
        scale = (a32 / F32(qmax)).astype(F16)
    return inv, scale


def _sym_codes_f16(x: np.ndarray, inv: np.ndarray, lo: int, hi: int) -> np.ndarray:
    with np.errstate(invalid="ignore", over="ignore"):
        prod = (x.astype(F32) * inv.astype(F32)).astype(F16)
    return _rne_clamp(prod.astype(F32), lo, hi)


def quant_k_int4(k: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fade/quant.py:61-75: per-channel (absmax over S) symmetric INT4, packed."""
    k = np.asarray(k, dtype=F16)
    absmax = np.abs(k).max(axis=-2, keepdims=True)
    inv, scale = _sym_params_f16(absmax, INT4_MAX)
    q = _sym_codes_f16(k, inv, INT4_MIN, INT4_MAX)
    return pack_int4_last_dim(q), scale


def quant_v_int4(v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fade/quant.py:78-92: per-token (absmax over D) symmetric INT4, packed."""
    v = np.asarray(v, dtype=F16)
    absmax = np.abs(v).max(axis=-1, keepdims=True)
    inv, scale = _sym_params_f16(absmax, INT4_MAX)
    q = _sym_codes_f16(v, inv, INT4_MIN, INT4_MAX)
    return pack_int4_last_dim(q), scale


def quant_int2_grouped(x: np.ndarray, group_size: int = DEFAULT_INT2_GROUP_SIZE):
    """fade/quant.py:95-112 (``quant_k_int2``) == fade/quant.py:130-150 (``quant_v_int2``).

    Both group along S with a per-(group, channel) scale; codes unpacked int8.
    """
    x = np.asarray(x, dtype=F16)
    B, H, S, D = x.shape
    if S % group_size != 0:
        raise ValueError(f"S={S} must be divisible by group_size={group_size}")
    G = S // group_size
    xg = x.reshape(B, H, G, group_size, D)
    absmax = np.abs(xg).max(axis=-2, keepdims=True)
    inv, scale = _sym_params_f16(absmax, INT2_MAX)
    q = _sym_codes_f16(xg, inv, INT2_MIN, INT2_MAX)
    return q.reshape(B, H, S, D), scale.reshape(B, H, G, D)


quant_k_int2 = quant_int2_grouped
quant_v_int2 = quant_int2_grouped


def pad_to_group(x: np.ndarray, group_size: int) -> tuple[np.ndarray, int]:
    """fade/quant.py:179-188: zero-pad the S axis (-2) to a multiple of group_size."""
    S = x.shape[-2]
    if S % group_size == 0:
        return x, S
    total = S + group_size - (S % group_size)
    out = np.zeros(x.shape[:-2] + (total, x.shape[-1]), dtype=x.dtype)
    out[..., :S, :] = x
    return out, S


def dequant(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """fade/quant.py:115-121: ``q.to(fp16) * scale.to(fp16)`` -> fp16(q*s)."""
    return (q.astype(F32) * np.asarray(scale, dtype=F16).astype(F32)).astype(F16)


def dequant_int4(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """fade/quant.py:124-127."""
    return dequant(unpack_int4_last_dim(packed), scale)


def dequant_int2_grouped(q: np.ndarray, scale: np.ndarray, group_size: int = 64) -> np.ndarray:
    """fade/quant.py:153-176 (``dequant_k_int2`` == ``dequant_v_int2``)."""
    B, H, S, D = q.shape
    G = S // group_size
    full = np.broadcast_to(scale[:, :, :, None, :], (B, H, G, group_size, D)).reshape(B, H, S, D)
    return dequant(q, full)


# --------------------------------------------------------------------------- #
# the INT4 K/V quantizers on any float dtype (fade/quant.py:61-92, 124-127):
# tests/test_quant.py:110-141 run them on bfloat16 and float32.  numpy has no
# bfloat16, so bf16 tensors are carried as their uint16 bit patterns.
# --------------------------------------------------------------------------- #
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even; every NaN -> 0x7FC0 (c10::BFloat16)."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[np.isnan(x)] = 0x7FC0
    return r


def to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    """Values of a tensor of ``dtype`` ("f16" | "bf16" | "f32") as fp32."""
    if dtype == "bf16":
        return bf16_to_f32(x)
    return np.asarray(x).astype(F32)


def from_f32(x32: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 values to ``dtype``'s storage (nearest even)."""
    if dtype == "bf16":
        return f32_to_bf16(x32)
    if dtype == "f16":
        return np.asarray(x32, dtype=F32).astype(F16)
    return np.asarray(x32, dtype=F32)


def _rnd(x32: np.ndarray, dtype: str) -> np.ndarray:
    """One torch op on ``dtype``: computed in fp32, rounded to ``dtype``."""
    return to_f32(from_f32(x32, dtype), dtype)


def _sym_params_typed(absmax32: np.ndarray, qmax: int, dtype: str):
    """``absmax.clamp(min=EPS)``, ``qmax / absmax`` (= reciprocal * qmax, two
    roundings) and ``absmax / qmax``, each op rounded to ``dtype``.  The clamp
    keeps NaN (torch.clamp propagates it); on fp16 it is a no-op."""
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        a = _rnd(np.where(np.isnan(absmax32), absmax32, np.maximum(absmax32, F32(EPS))), dtype)
        r = _rnd(F32(1.0) / a, dtype)
        inv = _rnd(r * F32(qmax), dtype)
        scale = from_f32(a / F32(qmax), dtype)
    return inv, scale


def _sym_quant_typed(x, dtype: str, axis: int):
    x32 = to_f32(x, dtype)
    absmax = np.abs(x32).max(axis=axis, keepdims=True)  # NaN-propagating, as torch's amax
    inv, scale = _sym_params_typed(absmax, INT4_MAX, dtype)
    with np.errstate(invalid="ignore", over="ignore"):
        prod = _rnd(x32 * inv, dtype)
    return pack_int4_last_dim(_rne_clamp(prod, INT4_MIN, INT4_MAX)), scale


def quant_k_int4_typed(k, dtype: str):
    """fade/quant.py:61-75 on a ``dtype`` tensor: (packed, scale [B,H,1,D] of ``dtype``)."""
    return _sym_quant_typed(k, dtype, -2)


def quant_v_int4_typed(v, dtype: str):
    """fade/quant.py:78-92 on a ``dtype`` tensor: (packed, scale [B,H,S,1] of ``dtype``)."""
    return _sym_quant_typed(v, dtype, -1)


def quant_int2_grouped_typed(x, dtype: str, group_size: int = DEFAULT_INT2_GROUP_SIZE):
    """fade/quant.py:95-112 / 130-150 on a ``dtype`` tensor: codes [B,H,S,D] int8 and
    scale [B,H,S/group,D] of ``dtype`` (each op rounded to it, the clamp live on bf16)."""
    x32 = to_f32(x, dtype)
    B, H, S, D = x32.shape
    if S % group_size != 0:
        raise ValueError(f"S={S} must be divisible by group_size={group_size}")
    G = S // group_size
    xg = x32.reshape(B, H, G, group_size, D)
    absmax = np.abs(xg).max(axis=-2, keepdims=True)
    inv, scale = _sym_params_typed(absmax, INT2_MAX, dtype)
    with np.errstate(invalid="ignore", over="ignore"):
        prod = _rnd(xg * inv, dtype)
    q = _rne_clamp(prod, INT2_MIN, INT2_MAX)
    return q.reshape(B, H, S, D), scale.reshape(B, H, G, D)


def dequant_int2_typed(q: np.ndarray, scale, dtype: str, group_size: int = DEFAULT_INT2_GROUP_SIZE) -> np.ndarray:
    """fade/quant.py:153-176 at ``dtype``: ``q.to(dtype) * scale.to(dtype)`` per group."""
    B, H, S, D = q.shape
    G = S // group_size
    s32 = to_f32(scale, dtype)
    full = np.broadcast_to(s32[:, :, :, None, :], (B, H, G, group_size, D)).reshape(B, H, S, D)
    return from_f32(q.astype(F32) * full, dtype)


def dequant_int4_typed(packed: np.ndarray, scale, dtype: str) -> np.ndarray:
    """fade/quant.py:124-127: ``q.to(dtype) * scale.to(dtype)``, in ``dtype``'s storage."""
    q = unpack_int4_last_dim(packed).astype(F32)
    return from_f32(q * to_f32(scale, dtype), dtype)


# --------------------------------------------------------------------------- #
# rotated quantizer (fp32 quant math on the rotated tensor)
# --------------------------------------------------------------------------- #
def random_orthogonal_from_gaussian(m: np.ndarray) -> np.ndarray:
    """fade/rotated_quant.py:91-96 restated: Q of the QR of a Gaussian matrix.

    The Gaussian itself comes from torch's seeded CPU generator, so the
    fixture is generated once with torch and committed
    (``tests/golden/rotation_d128_seed42.npy``).
    """
    q, _ = np.linalg.qr(m.astype(np.float64))
    return q.astype(F32)


def rotated_quant_codes(x_rot: np.ndarray, bits: int, axis: str, scale_dtype: str = "f16"):
    """fade/rotated_quant.py:121-131 (K, ``axis='channel'``) / 163-173 (V, ``axis='token'``).

    Input is the already-rotated fp32 tensor ``x.float() @ R.T``.  Returns
    (packed, scale) with the scale cast to the input's dtype ``scale_dtype``
    ("f16" | "bf16" | "f32"; ``scale.to(k.dtype)``).  ``qmax / absmax`` is
    ``reciprocal * qmax`` (two fp32 roundings); ``absmax / qmax`` is an IEEE
    fp32 division.
    """
    qmin, qmax = BIT_PARAMS[bits]
    x_rot = np.asarray(x_rot, dtype=F32)
    red = -2 if axis == "channel" else -1
    absmax = np.maximum(np.abs(x_rot).max(axis=red, keepdims=True), F32(EPS))
    inv = ((F32(1.0) / absmax).astype(F32) * F32(qmax)).astype(F32)
    scale = (absmax / F32(qmax)).astype(F32)
    q = _rne_clamp((x_rot * inv).astype(F32), qmin, qmax)
    return pack_bits(q, bits), from_f32(scale, scale_dtype)


def rotated_dequant_rot(packed: np.ndarray, scale: np.ndarray, bits: int, dtype: str = "f16") -> np.ndarray:
    """fade/rotated_quant.py:142-143 / 184-185: ``q.to(dtype) * scale.to(dtype)`` in the rotated basis."""
    if dtype == "f16":
        return dequant(unpack_bits(packed, bits), scale)
    return from_f32(unpack_bits(packed, bits).astype(F32) * to_f32(scale, dtype), dtype)


def rotated_dequant(packed, scale, R, bits):
    """fade/rotated_quant.py:134-145 / 176-187: (fp16(q*s) in fp32) @ R -> fp16."""
    xr = rotated_dequant_rot(packed, scale, bits).astype(F32)
    return (xr @ np.asarray(R, dtype=F32)).astype(F16)


# --------------------------------------------------------------------------- #
# asymmetric per-token group quantizer (build-defined format; no reference
# counterpart -- the reference has no zero-point quantizer)
# --------------------------------------------------------------------------- #
def quant_asym_group(x: np.ndarray, bits: int, group: int = 32):
    """Per-token asymmetric quantization in groups of ``group`` along D.

    Spec (shared with the HIP kernel):
      mn, mx  = min / max of the group (exact fp16)
      scale   = fp16( fp32(mx - mn) / (2^bits - 1) )
      zero    = mn
      inv     = 0 if scale == 0 else fp32( 1 / fp32(scale) )   (one reciprocal per group)
      code    = clamp(rne( fp32( fp32(x - mn) * inv ) ), 0, 2^bits-1)
      x_hat   = fp16( fp32(code * scale) + zero )
    The product with the rounded reciprocal can differ from the correctly
    rounded quotient by an ulp, so a code may differ from rne((x - mn) / scale)
    only where that quotient lies within a few ulps of a half-integer.
    Packing: 4-bit unsigned nibbles, high nibble = even index; 2-bit
    unsigned, four per byte, first element in the top bits.
    """
    x = np.asarray(x, dtype=F16)
    *lead, D = x.shape
    if D % group != 0:
        raise ValueError(f"D={D} must be divisible by group={group}")
    qmax = (1 << bits) - 1
    xg = x.reshape(*lead, D // group, group).astype(F32)
    mn = xg.min(axis=-1, keepdims=True)
    mx = xg.max(axis=-1, keepdims=True)
    scale16 = ((mx - mn).astype(F32) / F32(qmax)).astype(F16)
    s32 = scale16.astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(s32 == 0, F32(0), F32(1) / s32).astype(F32)
    t = ((xg - mn).astype(F32) * inv).astype(F32)
    q = np.clip(np.rint(t), 0, qmax).astype(np.uint8).reshape(*lead, D)
    if bits == 4:
        packed = ((q[..., 0::2] << 4) | q[..., 1::2]).astype(np.uint8)
    elif bits == 2:
        packed = ((q[..., 0::4] << 6) | (q[..., 1::4] << 4) | (q[..., 2::4] << 2) | q[..., 3::4]).astype(
            np.uint8
        )
    else:
        raise ValueError(f"bits must be 4 or 2, got {bits}")
    return packed, scale16.reshape(*lead, D // group), mn.astype(F16).reshape(*lead, D // group)


def unpack_asym_codes(packed: np.ndarray, bits: int) -> np.ndarray:
    if bits == 4:
        out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
        out[..., 0::2] = packed >> 4
        out[..., 1::2] = packed & 0xF
        return out
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 4,), dtype=np.uint8)
    for j, sh in enumerate((6, 4, 2, 0)):
        out[..., j::4] = (packed >> sh) & 0x3
    return out


def dequant_asym_group(packed, scale, zero, bits: int, group: int = 32) -> np.ndarray:
    q = unpack_asym_codes(packed, bits).astype(F32)
    *lead, D = q.shape
    qg = q.reshape(*lead, D // group, group)
    s = np.asarray(scale, dtype=F16).astype(F32)[..., None]
    z = np.asarray(zero, dtype=F16).astype(F32)[..., None]
    return ((qg * s).astype(F32) + z).astype(F16).reshape(*lead, D)
