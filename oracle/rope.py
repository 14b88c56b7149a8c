"""Numpy restatement of the eviction re-RoPE rewrite (test infrastructure only).

Reference: ``fade/cache.py:283-311`` (``_rotate_half`` / ``_apply_rope`` /
``_inverse_rope``), ``fade/cache.py:911-935`` (eviction block) and
``fade/rope.py:38-93`` (inverse frequencies and cos/sin).
"""

from __future__ import annotations

import numpy as np

F16 = np.float16
F32 = np.float32


def vanilla_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """fade/rope.py:38-46: 1 / theta ** (arange(0, D, 2) / D) in fp32.

    torch evaluates ``theta ** t`` with an fp32 ``pow`` and ``1.0 / x`` as
    ``reciprocal``; numpy's fp32 pow may differ from torch's in the last
    ulp, so tests compare these tables with a 1-ulp tolerance.
    """
    e = (np.arange(0, head_dim, 2, dtype=F32) / F32(head_dim)).astype(F32)
    p = np.power(F32(theta), e, dtype=F32)
    return (F32(1.0) / p).astype(F32)


def cos_sin_tables(positions: np.ndarray, inv_freq: np.ndarray, round_fp16: bool = True):
    """fade/rope.py:83-93: freqs = pos * inv; emb = [freqs, freqs]; cos/sin via fp16."""
    freqs = (np.asarray(positions, dtype=F32)[:, None] * inv_freq[None, :]).astype(F32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    cos = np.cos(emb.astype(np.float64)).astype(F32)
    sin = np.sin(emb.astype(np.float64)).astype(F32)
    if round_fp16:
        cos = cos.astype(F16).astype(F32)
        sin = sin.astype(F16).astype(F32)
    return cos, sin


def _rotate_half(x: np.ndarray) -> np.ndarray:
    """fade/cache.py:283-288: [-x2, x1]."""
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def apply_rope(k: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """fade/cache.py:290-299: fp32 (k*cos + rot(k)*sin), cast to k's dtype."""
    kf = np.asarray(k).astype(F32)
    a = (kf * cos).astype(F32)
    b = (_rotate_half(kf) * sin).astype(F32)
    return (a + b).astype(F32).astype(np.asarray(k).dtype)


def inverse_rope(k: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """fade/cache.py:301-311: fp32 (k*cos - rot(k)*sin), cast to k's dtype."""
    kf = np.asarray(k).astype(F32)
    a = (kf * cos).astype(F32)
    b = (_rotate_half(kf) * sin).astype(F32)
    return (a - b).astype(F32).astype(np.asarray(k).dtype)


def rerope_gather(k, v, keep_idx, cos_old, sin_old, cos_new, sin_new):
    """fade/cache.py:923-929 restricted to kept rows.

    ``k`` is [B, H, S, D] fp16 post-RoPE at the old positions; ``cos_old``
    / ``sin_old`` are [S, D]; ``cos_new`` / ``sin_new`` are [n_kept, D].
    The reference un-RoPEs every row then gathers; un-RoPE is row-wise, so
    gathering first gives identical values.
    """
    keep_idx = np.asarray(keep_idx, dtype=np.int64)
    k_kept = np.asarray(k)[:, :, keep_idx, :]
    pre = inverse_rope(k_kept, cos_old[keep_idx], sin_old[keep_idx])
    out_k = apply_rope(pre, cos_new, sin_new)
    out_v = np.asarray(v)[:, :, keep_idx, :]
    return out_k, out_v


# --------------------------------------------------------------------------- #
# the same on a bfloat16 / float32 cache: fp32 ops, each result cast to the
# cache dtype (fade/cache.py:290-311 cast to k.dtype); bf16 as uint16 bits
# --------------------------------------------------------------------------- #
def _rope_typed(k, cos, sin, dtype: str, sign: float):
    from oracle import quant as oq

    kf = oq.to_f32(k, dtype)
    a = (kf * cos).astype(F32)
    b = (_rotate_half(kf) * sin).astype(F32)
    return oq.from_f32((a + F32(sign) * b).astype(F32), dtype)


def apply_rope_typed(k, cos, sin, dtype: str):
    """fade/cache.py:290-299 on a ``dtype`` cache."""
    return _rope_typed(k, cos, sin, dtype, 1.0)


def inverse_rope_typed(k, cos, sin, dtype: str):
    """fade/cache.py:301-311 on a ``dtype`` cache."""
    return _rope_typed(k, cos, sin, dtype, -1.0)


def rerope_gather_typed(k, v, keep_idx, cos_old, sin_old, cos_new, sin_new, dtype: str):
    """``rerope_gather`` on a ``dtype`` cache (K and V in that dtype's storage)."""
    keep_idx = np.asarray(keep_idx, dtype=np.int64)
    k_kept = np.asarray(k)[:, :, keep_idx, :]
    pre = inverse_rope_typed(k_kept, cos_old[keep_idx], sin_old[keep_idx], dtype)
    out_k = apply_rope_typed(pre, cos_new, sin_new, dtype)
    return out_k, np.asarray(v)[:, :, keep_idx, :]
