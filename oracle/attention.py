"""fp32 attention over a dequantized tiered cache (test infrastructure only).

Reference structure: ``fade/kernels/int4_attention.py:179-202`` (dequantize
then ``F.scaled_dot_product_attention``), with the GQA head expansion of
``fade/kernels/fused_int4_attn.py:306-312`` (``repeat_interleave`` over
heads: query head ``h`` reads KV head ``h // (Hq // Hkv)``), the default
scale ``1/sqrt(D)`` (``fade/kernels/fused_int4_attn.py:324``) and the tier
order ``sink | middle | recent`` of ``fade/cache.py:715-808``.
"""

from __future__ import annotations

import numpy as np

from . import quant as oq

F32 = np.float32


def expand_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """``repeat_interleave(n_rep, dim=1)``."""
    return np.repeat(x, n_rep, axis=1) if n_rep > 1 else x


def sdpa_fp32(q, k, v, mask=None, scale=None):
    """Softmax attention in fp32 (float64 accumulation for the oracle).

    q: [B, Hq, Sq, D]; k, v: [B, Hkv, Sk, D]; mask: bool [Sq, Sk] (True =
    attend) or None.  Returns fp32 [B, Hq, Sq, D].
    """
    q = np.asarray(q).astype(np.float64)
    B, Hq, Sq, D = q.shape
    Hkv = k.shape[1]
    if Hq % Hkv != 0:
        raise ValueError(f"Hq={Hq} not a multiple of Hkv={Hkv}")
    k = expand_kv(np.asarray(k).astype(np.float64), Hq // Hkv)
    v = expand_kv(np.asarray(v).astype(np.float64), Hq // Hkv)
    sc = (1.0 / np.sqrt(D)) if scale is None else scale
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * sc
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v).astype(F32)


def bottom_right_causal_mask(sq: int, sk: int) -> np.ndarray:
    """Query j of a chunk appended after ``sk - sq`` cached keys sees keys < sk - sq + j + 1."""
    j = np.arange(sq)[:, None]
    t = np.arange(sk)[None, :]
    return t <= (sk - sq + j)


def _vals(x, dtype: str) -> np.ndarray:
    """Values of an fp16 / fp32 array, or of bf16 bit patterns (uint16) when ``dtype`` is "bf16"."""
    return oq.to_f32(x, "bf16") if dtype == "bf16" else np.asarray(x)


def dequant_middle(mid: dict) -> tuple[np.ndarray, np.ndarray]:
    """Dequantize a middle tier described by a dict (format key ``fmt``).

    ``mid["dtype"]`` ("f16", default, or "bf16") is the cache dtype: scales and
    fp16-layout rows are then bf16 bit patterns, and the dequantization rounds
    to bf16 as the reference does at that dtype (``q.to(dtype) *
    scale.to(dtype)``, fade/quant.py:124-127,170-176; the rotated formats'
    ``(x_rot.float() @ R).to(dtype)`` of its CPU path, fade/rotated_quant.py:142-145,184-187).
    The result is fp32 values (or fp16 for "f16").

    Formats:
      ``int4``      reference INT4: per-channel K scale, per-token V scale
                    (fade/quant.py:61-92, dequant fade/quant.py:124-127)
      ``k4v2``      reference INT4 K + literal grouped INT2 V, V trimmed
                    to ``n`` tokens (fade/cache.py:827-837)
      ``rot``       rotated symmetric codes at ``k_bits``/``v_bits`` with R
                    (fade/rotated_quant.py:134-187)
      ``asym``      build-defined per-token group-32 asymmetric format
      ``fp16``      plain fp16 middle (the flash-decode comparator)
    """
    fmt = mid["fmt"]
    dt = mid.get("dtype", "f16")
    if dt == "bf16":
        return _dequant_middle_bf16(mid)
    if fmt == "fp16":
        return np.asarray(mid["k"]), np.asarray(mid["v"])
    if fmt == "int4":
        return oq.dequant_int4(mid["kq"], mid["ks"]), oq.dequant_int4(mid["vq"], mid["vs"])
    if fmt == "k4v2":
        k = oq.dequant_int4(mid["kq"], mid["ks"])
        v = oq.dequant_int2_grouped(mid["vq"], mid["vs"], mid.get("group", 64))
        return k, v[..., : k.shape[-2], :]
    if fmt == "rot":
        R = mid["R"]
        k = oq.rotated_dequant(mid["kq"], mid["ks"], R, mid["k_bits"])
        v = oq.rotated_dequant(mid["vq"], mid["vs"], R, mid["v_bits"])
        return k, v
    if fmt == "asym":
        g = mid.get("group", 32)
        k = oq.dequant_asym_group(mid["kq"], mid["ks"], mid["kz"], mid["k_bits"], g)
        v = oq.dequant_asym_group(mid["vq"], mid["vs"], mid["vz"], mid["v_bits"], g)
        return k, v
    raise ValueError(f"unknown middle format {fmt!r}")


def _dequant_middle_bf16(mid: dict) -> tuple[np.ndarray, np.ndarray]:
    """``dequant_middle`` of a bfloat16 cache (scales and rows as bf16 bit patterns)."""
    fmt = mid["fmt"]
    b = lambda x: oq.to_f32(x, "bf16")  # noqa: E731
    if fmt == "fp16":
        return b(mid["k"]), b(mid["v"])
    if fmt == "int4":
        return b(oq.dequant_int4_typed(mid["kq"], mid["ks"], "bf16")), b(oq.dequant_int4_typed(mid["vq"], mid["vs"], "bf16"))
    if fmt == "k4v2":
        k = b(oq.dequant_int4_typed(mid["kq"], mid["ks"], "bf16"))
        v = b(oq.dequant_int2_typed(mid["vq"], mid["vs"], "bf16", mid.get("group", 64)))
        return k, v[..., : k.shape[-2], :]
    if fmt == "rot":
        R = np.asarray(mid["R"], dtype=F32)
        out = []
        for qk, sk, bits in ((mid["kq"], mid["ks"], mid["k_bits"]), (mid["vq"], mid["vs"], mid["v_bits"])):
            xr = b(oq.rotated_dequant_rot(qk, sk, bits, "bf16"))
            out.append(b(oq.from_f32((xr.astype(np.float64) @ R.astype(np.float64)).astype(F32), "bf16")))
        return out[0], out[1]
    raise ValueError(f"middle format {fmt!r} has no bfloat16 form")


def materialize(sink_k, sink_v, mid: dict | None, recent_k, recent_v, dtype: str = "f16"):
    """fade/cache.py:693-699: cat(sink, middle, recent) along S.  ``dtype`` "bf16":
    the sink / recent arrays are bf16 bit patterns (and ``mid["dtype"]`` should be "bf16")."""
    ks, vs = [], []
    if sink_k is not None and sink_k.shape[-2] > 0:
        ks.append(_vals(sink_k, dtype))
        vs.append(_vals(sink_v, dtype))
    if mid is not None:
        mk, mv = dequant_middle(mid)
        if mk.shape[-2] > 0:
            ks.append(mk)
            vs.append(mv)
    if recent_k is not None and recent_k.shape[-2] > 0:
        ks.append(_vals(recent_k, dtype))
        vs.append(_vals(recent_v, dtype))
    if dtype == "bf16":
        ks = [np.asarray(x, dtype=F32) for x in ks]
        vs = [np.asarray(x, dtype=F32) for x in vs]
    return np.concatenate(ks, axis=-2), np.concatenate(vs, axis=-2)


def tiered_decode(q, sink_k, sink_v, mid, recent_k, recent_v, dtype: str = "f16"):
    """Single-token decode over the tiered cache: fp32 SDPA of the materialized K/V.
    ``dtype`` "bf16": q, sink and recent are bf16 bit patterns (the cache's dtype)."""
    k, v = materialize(sink_k, sink_v, mid, recent_k, recent_v, dtype)
    return sdpa_fp32(_vals(q, dtype), k, v)


def ragged_prefill(q_chunks, k_full_list, v_full_list):
    """Per-sequence bottom-right causal attention of a query chunk over its cache.

    ``q_chunks[b]`` is [Hq, Sq, D]; ``k_full_list[b]`` is [Hkv, L_b + Sq, D]
    (cache followed by the chunk's own keys).
    """
    outs = []
    for qb, kb, vb in zip(q_chunks, k_full_list, v_full_list):
        sq, sk = qb.shape[-2], kb.shape[-2]
        mask = bottom_right_causal_mask(sq, sk)
        outs.append(sdpa_fp32(qb[None], kb[None], vb[None], mask=mask)[0])
    return outs
