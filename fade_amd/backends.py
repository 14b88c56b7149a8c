"""Pluggable quantization backends (the ``quant_backend`` API of fade/backends.py).

Same protocol (``compress_k/v`` -> dict, ``decompress_k/v``, ``name``),
names and registry keys as the reference (fade/backends.py:35-268), plus
``int4_asym_g32`` / ``asym``: per-token asymmetric group-32 INT4 with fp16
scale/zero, the format the benchmark configurations describe.  Every
backend runs on the MI355X kernels; there is no CPU path.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Protocol, runtime_checkable

import torch
from torch import Tensor

from .quant import dequant_asym, dequant_int4, quant_asym, quant_k_int4, quant_v_int4


@runtime_checkable
class QuantBackend(Protocol):
    """fade/backends.py:35-58."""

    def compress_k(self, k: Tensor) -> dict[str, Tensor]: ...

    def decompress_k(self, compressed: dict[str, Tensor], dtype: torch.dtype) -> Tensor: ...

    def compress_v(self, v: Tensor) -> dict[str, Tensor]: ...

    def decompress_v(self, compressed: dict[str, Tensor], dtype: torch.dtype) -> Tensor: ...

    @property
    def name(self) -> str: ...


@dataclass
class SymmetricINT4Backend:
    """Per-channel K / per-token V symmetric INT4, bit-packed (fade/backends.py:62-86)."""

    @property
    def name(self) -> str:
        return "symmetric_int4"

    def compress_k(self, k: Tensor) -> dict[str, Tensor]:
        packed, scale = quant_k_int4(k)
        return {"packed": packed, "scale": scale}

    def decompress_k(self, compressed: dict[str, Tensor], dtype: torch.dtype = torch.float16) -> Tensor:
        return dequant_int4(compressed["packed"], compressed["scale"], dtype=dtype)

    def compress_v(self, v: Tensor) -> dict[str, Tensor]:
        packed, scale = quant_v_int4(v)
        return {"packed": packed, "scale": scale}

    def decompress_v(self, compressed: dict[str, Tensor], dtype: torch.dtype = torch.float16) -> Tensor:
        return dequant_int4(compressed["packed"], compressed["scale"], dtype=dtype)


@dataclass
class RotatedINT4Backend:
    """Seeded random rotation before symmetric quantization (fade/backends.py:90-159)."""

    head_dim: int = 64
    bits: int = 4
    seed: int = 42
    _R_per_device: dict = field(default_factory=dict, repr=False)

    @property
    def name(self) -> str:
        return f"rotated_int{self.bits}"

    def _get_R(self, device: torch.device | None = None) -> Tensor:
        device = torch.device(device or "cpu")
        R = self._R_per_device.get(device)
        if R is None:
            from .rotated_quant import _random_orthogonal

            R = _random_orthogonal(self.head_dim, self.seed).to(device)
            self._R_per_device[device] = R
        return R

    def compress_k(self, k: Tensor) -> dict[str, Tensor]:
        from .rotated_quant import rotated_quant_k

        packed, scale = rotated_quant_k(k, self._get_R(k.device), bits=self.bits)
        return {"packed": packed, "scale": scale}

    def decompress_k(self, compressed: dict[str, Tensor], dtype: torch.dtype = torch.float16) -> Tensor:
        from .rotated_quant import rotated_dequant_k

        p = compressed["packed"]
        return rotated_dequant_k(p, compressed["scale"], self._get_R(p.device), bits=self.bits, dtype=dtype)

    def compress_v(self, v: Tensor) -> dict[str, Tensor]:
        from .rotated_quant import rotated_quant_v

        packed, scale = rotated_quant_v(v, self._get_R(v.device), bits=self.bits)
        return {"packed": packed, "scale": scale}

    def decompress_v(self, compressed: dict[str, Tensor], dtype: torch.dtype = torch.float16) -> Tensor:
        from .rotated_quant import rotated_dequant_v

        p = compressed["packed"]
        return rotated_dequant_v(p, compressed["scale"], self._get_R(p.device), bits=self.bits, dtype=dtype)


@dataclass
class AsymGroupBackend:
    """Per-token asymmetric groups along head_dim with fp16 scale/zero (build format).

    ``bits`` is the K code width; ``v_bits`` (default: ``bits``) the V code
    width, so the K 4-bit / V 2-bit tier of the benchmark's long-context
    configuration is one backend."""

    head_dim: int = 128
    bits: int = 4
    group: int = 32
    v_bits: int | None = None

    @property
    def k_bits(self) -> int:
        return self.bits

    @property
    def value_bits(self) -> int:
        return self.bits if self.v_bits is None else self.v_bits

    @property
    def name(self) -> str:
        if self.value_bits == self.bits:
            return f"int{self.bits}_asym_g{self.group}"
        return f"k{self.bits}v{self.value_bits}_asym_g{self.group}"

    def compress_k(self, k: Tensor) -> dict[str, Tensor]:
        packed, scale, zero = quant_asym(k, self.bits, self.group)
        return {"packed": packed, "scale": scale, "zero": zero}

    def decompress_k(self, compressed: dict[str, Tensor], dtype: torch.dtype = torch.float16) -> Tensor:
        c = compressed
        return dequant_asym(c["packed"], c["scale"], c["zero"], self.bits, self.group).to(dtype)

    def compress_v(self, v: Tensor) -> dict[str, Tensor]:
        packed, scale, zero = quant_asym(v, self.value_bits, self.group)
        return {"packed": packed, "scale": scale, "zero": zero}

    def decompress_v(self, compressed: dict[str, Tensor], dtype: torch.dtype = torch.float16) -> Tensor:
        c = compressed
        return dequant_asym(c["packed"], c["scale"], c["zero"], self.value_bits, self.group).to(dtype)


@dataclass
class TurboQuantBackend:
    """Wrapper of the third-party ``turboquant-kv`` package (fade/backends.py:163-240).

    That package is not part of this build; constructing its quantizer
    raises ``ImportError`` exactly as the reference does without it.
    """

    head_dim: int = 128
    bits: float = 4
    device: str | None = None
    _tq: Any = None

    @property
    def name(self) -> str:
        return f"turboquant_{self.bits}bit"

    def _ensure_tq(self, device=None):
        if self._tq is None:
            try:
                from turboquant import TurboQuantProd  # type: ignore[import-not-found]
            except ImportError as e:
                raise ImportError(
                    "TurboQuantBackend requires turboquant-kv. Install with: pip install fade-kv[turbo]"
                ) from e
            self._tq = TurboQuantProd(head_dim=self.head_dim, bits=self.bits, device=self.device or str(device))
        return self._tq

    def compress_k(self, k: Tensor) -> dict[str, Tensor]:
        self._ensure_tq(k.device)
        raise NotImplementedError("turboquant-kv is not supported by fade_amd")

    compress_v = compress_k

    def decompress_k(self, compressed, dtype=torch.float16) -> Tensor:
        self._ensure_tq()
        raise NotImplementedError("turboquant-kv is not supported by fade_amd")

    decompress_v = decompress_k


_BACKENDS: dict[str, type] = {
    "symmetric_int4": SymmetricINT4Backend,
    "int4": SymmetricINT4Backend,
    "rotated_int4": RotatedINT4Backend,
    "rotated": RotatedINT4Backend,
    "int4_asym_g32": AsymGroupBackend,
    "asym": AsymGroupBackend,
    "turbo": TurboQuantBackend,
    "turboquant": TurboQuantBackend,
}


def get_backend(name: str = "int4", **kwargs) -> QuantBackend:
    """fade/backends.py:254-268: construct a backend by registry name."""
    cls = _BACKENDS.get(name.lower())
    if cls is None:
        raise ValueError(f"Unknown quant backend {name!r}. Available: {list(_BACKENDS.keys())}")
    if cls is SymmetricINT4Backend:
        return cls()
    fields = getattr(cls, "__dataclass_fields__", {})
    return cls(**{k: v for k, v in kwargs.items() if k in fields and not k.startswith("_")})


__all__ = [
    "AsymGroupBackend",
    "QuantBackend",
    "RotatedINT4Backend",
    "SymmetricINT4Backend",
    "TurboQuantBackend",
    "get_backend",
]
