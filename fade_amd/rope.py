"""RoPE schemes: inverse frequencies and cos/sin tables for the re-RoPE pass.

The re-RoPE kernel (``fade_rerope_gather``) consumes cos/sin tables; this
module builds them on the host CPU with torch, in the order the reference
uses (fade/rope.py:38-93): ``freqs = pos * inv_freq`` in fp32,
``emb = [freqs, freqs]``, ``cos/sin`` in fp32, rounded through the model
dtype (fp16) unless that dtype is bf16.  Building them on the host keeps
them independent of the device's libm and identical to the CPU oracle.

Scheme names, fields and the auto-detection rules follow fade/rope.py:101-474
so that ``create_tiered_cache`` resolves the same scheme from an HF config.
"""

from __future__ import annotations

import math
import warnings
from dataclasses import dataclass, field

import torch
from torch import Tensor

DEFAULT_ROPE_THETA: float = 10000.0
DEFAULT_FACTOR: float = 1.0
DEFAULT_LOW_FREQ_FACTOR: float = 1.0
DEFAULT_HIGH_FREQ_FACTOR: float = 4.0
DEFAULT_ORIGINAL_MAX_POS: int = 8192
DEFAULT_YARN_BETA_FAST: float = 32.0
DEFAULT_YARN_BETA_SLOW: float = 1.0

_HOST = torch.device("cpu")


def _vanilla_inv_freq(head_dim: int, theta: float, device=_HOST) -> Tensor:
    """fade/rope.py:38-46: ``1 / theta ** (arange(0, D, 2) / D)`` in fp32."""
    exps = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim
    return 1.0 / (theta**exps)


@dataclass
class RopeScheme:
    """Base scheme (vanilla inverse frequencies)."""

    theta: float = DEFAULT_ROPE_THETA
    head_dim: int = 64
    _inv_cache: Tensor | None = field(default=None, init=False, repr=False, compare=False)

    def _compute_inv_freq(self) -> Tensor:
        return _vanilla_inv_freq(self.head_dim, self.theta)

    def inv_freq(self, device: torch.device | None = None) -> Tensor:
        """``[head_dim // 2]`` fp32 inverse frequencies (computed once, on the host)."""
        if self._inv_cache is None:
            self._inv_cache = self._compute_inv_freq()
        return self._inv_cache if device is None else self._inv_cache.to(device)

    def _positions(self, positions: Tensor) -> Tensor:
        return positions.to(_HOST).float()

    def _emb(self, positions: Tensor) -> Tensor:
        freqs = self._positions(positions).unsqueeze(-1) * self.inv_freq().unsqueeze(0)
        return torch.cat((freqs, freqs), dim=-1)

    def host_cos_sin(self, positions: Tensor, model_dtype: torch.dtype = torch.float16):
        """``(cos, sin)`` as fp32 ``[S, head_dim]`` host tensors."""
        emb = self._emb(positions)
        cos, sin = emb.cos(), emb.sin()
        if model_dtype != torch.bfloat16:
            cos = cos.to(model_dtype).float()
            sin = sin.to(model_dtype).float()
        return cos, sin

    def compute_cos_sin(self, positions: Tensor, device, model_dtype: torch.dtype = torch.float16):
        """fade/rope.py:72-93: ``(cos, sin)`` broadcastable to ``[1, 1, S, head_dim]``."""
        cos, sin = self.host_cos_sin(positions, model_dtype)
        return cos.to(device)[None, None], sin.to(device)[None, None]

    @property
    def is_rope(self) -> bool:
        return True


@dataclass
class Vanilla(RopeScheme):
    """Standard RoPE (Qwen2, Mistral, Phi-3, Gemma-2, ...)."""


@dataclass
class LinearScaled(RopeScheme):
    """Positions divided by ``factor`` (fade/rope.py:106-124)."""

    factor: float = DEFAULT_FACTOR

    def _positions(self, positions: Tensor) -> Tensor:
        return positions.to(_HOST).float() / self.factor

    def host_cos_sin(self, positions, model_dtype=torch.float16):
        # The reference always rounds through model_dtype for this scheme.
        emb = self._emb(positions)
        return emb.cos().to(model_dtype).float(), emb.sin().to(model_dtype).float()


@dataclass
class Llama3(RopeScheme):
    """Llama-3.1 band-wise interpolation of the inverse frequencies (fade/rope.py:127-157)."""

    factor: float = DEFAULT_FACTOR
    low_freq_factor: float = DEFAULT_LOW_FREQ_FACTOR
    high_freq_factor: float = DEFAULT_HIGH_FREQ_FACTOR
    original_max_position_embeddings: int = DEFAULT_ORIGINAL_MAX_POS

    def _compute_inv_freq(self) -> Tensor:
        base = _vanilla_inv_freq(self.head_dim, self.theta)
        ctx = float(self.original_max_position_embeddings)
        wavelen = 2.0 * math.pi / base
        t = (ctx / wavelen - self.low_freq_factor) / (self.high_freq_factor - self.low_freq_factor)
        mixed = base * (1 - t) / self.factor + base * t
        low_band = wavelen > ctx / self.low_freq_factor
        high_band = wavelen < ctx / self.high_freq_factor
        return torch.where(high_band, base, torch.where(low_band, base / self.factor, mixed))


@dataclass
class NtkAware(RopeScheme):
    """theta scaled by ``factor`` before computing inverse frequencies (fade/rope.py:160-168)."""

    factor: float = DEFAULT_FACTOR

    def _compute_inv_freq(self) -> Tensor:
        return _vanilla_inv_freq(self.head_dim, self.theta * self.factor)


@dataclass
class Yarn(RopeScheme):
    """YaRN ramp between interpolated and NTK frequencies (fade/rope.py:171-193)."""

    factor: float = DEFAULT_FACTOR
    beta_fast: float = DEFAULT_YARN_BETA_FAST
    beta_slow: float = DEFAULT_YARN_BETA_SLOW
    original_max_position_embeddings: int = DEFAULT_ORIGINAL_MAX_POS

    def _compute_inv_freq(self) -> Tensor:
        base = _vanilla_inv_freq(self.head_dim, self.theta)
        ntk = _vanilla_inv_freq(self.head_dim, self.theta * self.factor)
        idx = torch.arange(base.shape[0], dtype=torch.float32)
        span = 2 * math.pi * self.original_max_position_embeddings
        lo = self.beta_fast * self.head_dim / span
        hi = self.beta_slow * self.head_dim / span
        ramp = ((idx - lo) / (hi - lo)).clamp(0.0, 1.0)
        return (1.0 - ramp) * base / self.factor + ramp * ntk


@dataclass
class Proportional(RopeScheme):
    """Gemma-4 partial rotation: head_dim denominator, zero frequencies past the rotary dims."""

    partial_rotary_factor: float = 1.0

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    def _compute_inv_freq(self) -> Tensor:
        n_rot = self.rotary_dim // 2
        exps = torch.arange(0, 2 * n_rot, 2, dtype=torch.float32) / self.head_dim
        inv = 1.0 / (self.theta**exps)
        n_pass = self.head_dim // 2 - n_rot
        if n_pass > 0:
            inv = torch.cat([inv, torch.zeros(n_pass, dtype=torch.float32)])
        return inv


@dataclass
class MRope(RopeScheme):
    """Qwen 3.5/3.6 multi-axis RoPE; text-only positions reduce to vanilla (fade/rope.py:228-272)."""

    partial_rotary_factor: float = 1.0
    mrope_section: list[int] | None = None

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    def _compute_inv_freq(self) -> Tensor:
        return _vanilla_inv_freq(self.rotary_dim, self.theta)

    def host_cos_sin(self, positions, model_dtype=torch.float16):
        emb = self._emb(positions)
        if self.rotary_dim < self.head_dim:
            emb = torch.cat([emb, torch.zeros(emb.shape[0], self.head_dim - self.rotary_dim)], dim=-1)
        return emb.cos().to(model_dtype).float(), emb.sin().to(model_dtype).float()


@dataclass
class NoRope(RopeScheme):
    """Non-RoPE models: cos = 1, sin = 0 so re-RoPE is the identity (fade/rope.py:275-298)."""

    def host_cos_sin(self, positions, model_dtype=torch.float16):
        n = int(positions.shape[0])
        return torch.ones(n, self.head_dim), torch.zeros(n, self.head_dim)

    @property
    def is_rope(self) -> bool:
        return False


def _scheme_from_params(rp: dict, head_dim: int, fallback_theta: float) -> RopeScheme:
    theta = float(rp.get("rope_theta", fallback_theta))
    kind = str(rp.get("rope_type", rp.get("type", "default"))).lower()
    prf = float(rp.get("partial_rotary_factor", 1.0))
    if kind == "proportional" or (kind in ("", "default") and prf < 1.0):
        return Proportional(theta=theta, head_dim=head_dim, partial_rotary_factor=prf)
    if kind in ("", "default"):
        return Vanilla(theta=theta, head_dim=head_dim)
    import types

    extra = {k: v for k, v in rp.items() if k not in ("rope_theta", "rope_type", "type")}
    cfg = types.SimpleNamespace(
        rope_theta=theta, rope_scaling={"type": kind, **extra}, hidden_size=head_dim, num_attention_heads=1
    )
    return extract_rope_scheme(cfg, head_dim=head_dim)


def _resolve_head_dim(cfg, head_dim):
    if head_dim is not None:
        return head_dim
    hd = getattr(cfg, "head_dim", None)
    if hd is None:
        hd = getattr(cfg, "hidden_size", 64) // getattr(cfg, "num_attention_heads", 1)
    return hd


def extract_rope_schemes_per_layer(cfg, head_dim: int | None = None) -> dict[str, RopeScheme] | None:
    """Per-layer-type schemes from a nested ``rope_parameters`` dict (fade/rope.py:331-358)."""
    rp = getattr(cfg, "rope_parameters", None)
    if not isinstance(rp, dict) or not isinstance(next(iter(rp.values()), None), dict):
        return None
    hd = _resolve_head_dim(cfg, head_dim)
    theta = float(getattr(cfg, "rope_theta", DEFAULT_ROPE_THETA) or DEFAULT_ROPE_THETA)
    return {name: _scheme_from_params(p, hd, theta) for name, p in rp.items() if isinstance(p, dict)}


def extract_rope_scheme(cfg, head_dim: int | None = None) -> RopeScheme:
    """Detect the RoPE scheme of an HF config (fade/rope.py:361-474)."""
    per_layer = extract_rope_schemes_per_layer(cfg, head_dim)
    if per_layer is not None:
        return per_layer.get("full_attention", next(iter(per_layer.values())))
    rp = getattr(cfg, "rope_parameters", None)
    theta = getattr(cfg, "rope_theta", None)
    if theta is None and isinstance(rp, dict):
        theta = rp.get("rope_theta")
    theta = float(DEFAULT_ROPE_THETA if theta is None else theta)
    hd = _resolve_head_dim(cfg, head_dim)

    if getattr(cfg, "alibi", False) or getattr(cfg, "model_type", "") in ("bloom", "mpt"):
        return NoRope(theta=theta, head_dim=hd)

    mrope = rp.get("mrope_section") if isinstance(rp, dict) else None
    if mrope is None:
        mrope = getattr(cfg, "mrope_section", None)
    if mrope is not None:
        prf = float(rp.get("partial_rotary_factor", 1.0)) if isinstance(rp, dict) else 1.0
        return MRope(theta=theta, head_dim=hd, partial_rotary_factor=prf, mrope_section=list(mrope))

    rs = getattr(cfg, "rope_scaling", None)
    if not isinstance(rs, dict):
        return Vanilla(theta=theta, head_dim=hd)
    kind = str(rs.get("type", rs.get("rope_type", ""))).lower()
    prf = float(rs.get("partial_rotary_factor", 1.0))
    if kind == "proportional" or (kind in ("", "default") and prf < 1.0):
        return Proportional(theta=theta, head_dim=hd, partial_rotary_factor=prf)
    if kind in ("", "default"):
        return Vanilla(theta=theta, head_dim=hd)
    factor = float(rs.get("factor", 1.0))
    orig = int(
        rs.get(
            "original_max_position_embeddings",
            getattr(cfg, "original_max_position_embeddings", DEFAULT_ORIGINAL_MAX_POS),
        )
    )
    if kind == "linear":
        return LinearScaled(theta=theta, head_dim=hd, factor=factor)
    if kind in ("llama3", "longrope"):
        return Llama3(
            theta=theta,
            head_dim=hd,
            factor=factor,
            low_freq_factor=float(rs.get("low_freq_factor", DEFAULT_LOW_FREQ_FACTOR)),
            high_freq_factor=float(rs.get("high_freq_factor", DEFAULT_HIGH_FREQ_FACTOR)),
            original_max_position_embeddings=orig,
        )
    if kind in ("ntk", "dynamic"):
        return NtkAware(theta=theta, head_dim=hd, factor=factor)
    if kind == "yarn":
        return Yarn(
            theta=theta,
            head_dim=hd,
            factor=factor,
            beta_fast=float(rs.get("beta_fast", DEFAULT_YARN_BETA_FAST)),
            beta_slow=float(rs.get("beta_slow", DEFAULT_YARN_BETA_SLOW)),
            original_max_position_embeddings=orig,
        )
    warnings.warn(
        f"Unknown rope_scaling type {kind!r}; falling back to vanilla RoPE.", RuntimeWarning, stacklevel=2
    )
    return Vanilla(theta=theta, head_dim=hd)


def rerope_gather(
    k: Tensor,
    v: Tensor | None,
    keep_idx: Tensor,
    cos_old: Tensor,
    sin_old: Tensor,
    cos_new: Tensor,
    sin_new: Tensor,
) -> tuple[Tensor, Tensor | None]:
    """Fused eviction re-RoPE of the kept rows (fade/cache.py:911-935).

    ``k``/``v``: [B, H, S, D] fp16, bf16 or fp32 on the GPU (K post-RoPE at its old
    positions); ``keep_idx``: ascending int64 indices of kept rows;
    ``cos_old``/``sin_old``: [S, D] fp32 tables of the old positions;
    ``cos_new``/``sin_new``: [n_kept, D] tables of the new positions.
    Returns K re-RoPE'd at the new positions and the gathered V, both
    [B, H, n_kept, D] in K's dtype (the rounding between the two rotations
    is to that dtype, as the reference's casts to k.dtype).
    """
    from . import _lib

    _lib.require_gpu(k, v, keep_idx, op="rerope_gather")
    if k.dim() != 4:
        raise ValueError(f"key_states must be [B, H, S, D]; got shape {tuple(k.shape)}")
    if v is not None and v.shape != k.shape:
        raise ValueError(f"K/V shape mismatch: {tuple(k.shape)} vs {tuple(v.shape)}")
    if k.dtype not in _lib.DTYPE_CODES:
        raise ValueError(f"rerope_gather: expected a float16, bfloat16 or float32 tensor, got {k.dtype}")
    if v is not None and v.dtype != k.dtype:
        raise ValueError(f"rerope_gather: K and V dtypes differ ({k.dtype}, {v.dtype})")
    B, H, S, D = k.shape
    n = int(keep_idx.shape[0])
    dev = k.device
    keep_idx = keep_idx.to(device=dev, dtype=torch.int64).contiguous()
    tabs = [t.to(device=dev, dtype=torch.float32).reshape(-1, D).contiguous() for t in (cos_old, sin_old, cos_new, sin_new)]
    if tabs[0].shape[0] != S or tabs[2].shape[0] != n:
        raise ValueError("cos/sin tables must cover the S old positions and the n_kept new positions")
    if k.stride(-1) != 1:
        k = k.contiguous()
    k_out = torch.empty(B, H, n, D, dtype=k.dtype, device=dev)
    v_out = None
    vs = (0, 0, 0)
    if v is not None:
        if v.stride(-1) != 1:
            v = v.contiguous()
        v_out = torch.empty(B, H, n, D, dtype=v.dtype, device=dev)
        vs = (v.stride(0), v.stride(1), v.stride(2))
    if k.dtype == torch.float16:
        _lib.call(
            "fade_rerope_gather", k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            _lib.ptr(v), *vs, B, H, S, D, keep_idx.data_ptr(), n,
            tabs[0].data_ptr(), tabs[1].data_ptr(), tabs[2].data_ptr(), tabs[3].data_ptr(),
            k_out.data_ptr(), _lib.ptr(v_out), _lib.stream_of(k),
        )
    else:
        _lib.call(
            "fade_rerope_gather_dtype", k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            _lib.ptr(v), *vs, B, H, S, D, keep_idx.data_ptr(), n,
            tabs[0].data_ptr(), tabs[1].data_ptr(), tabs[2].data_ptr(), tabs[3].data_ptr(),
            k_out.data_ptr(), _lib.ptr(v_out), _lib.DTYPE_CODES[k.dtype], _lib.stream_of(k),
        )
    return k_out, v_out


__all__ = [
    "LinearScaled",
    "Llama3",
    "MRope",
    "NoRope",
    "NtkAware",
    "Proportional",
    "RopeScheme",
    "Vanilla",
    "Yarn",
    "extract_rope_scheme",
    "extract_rope_schemes_per_layer",
    "rerope_gather",
]
