"""Seeded synthetic workloads of the benchmark configurations.

Inputs are drawn on the CPU with ``torch.Generator`` (seed ``1000 + config
index`` by default) in fp32, cast to fp16, and copied bit-identically to
the device, so tests, the benchmark and the CPU baseline see the same
bits:  K = N(0,1) * c with per-(kv head, channel) c ~ LogNormal(0, 0.5),
V = N(0,1), Q = N(0,1).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    B: int
    Hq: int
    Hkv: int
    S: int
    D: int = 128
    n_sink: int = 4
    recent: int = 64
    v_bits: int = 4

    @property
    def mid(self) -> int:
        return self.S - self.n_sink - self.recent


CONFIGS = {
    0: DecodeConfig("c0_cpu_plumbing", B=1, Hq=32, Hkv=8, S=2048),
    1: DecodeConfig("c1_llama3_8b_decode_b16_s8192", B=16, Hq=32, Hkv=8, S=8192),
    2: DecodeConfig("c2_long_context_b4_s32768_k4v2", B=4, Hq=32, Hkv=8, S=32768, recent=256, v_bits=2),
}


@dataclass(frozen=True)
class ReropeConfig:
    B: int = 8
    Hq: int = 28
    Hkv: int = 4
    S: int = 4096
    D: int = 128
    theta: float = 1e6
    n_sink: int = 4
    recent: int = 64
    int4_budget: int = 400


def kv_tensors(B: int, Hkv: int, S: int, D: int, seed: int, Hq: int | None = None, Sq: int = 1):
    """Return CPU fp16 (q, k, v); q is None when ``Hq`` is None."""
    gen = torch.Generator().manual_seed(seed)
    chan = torch.empty(Hkv, D).log_normal_(0.0, 0.5, generator=gen)
    k = (torch.randn(B, Hkv, S, D, generator=gen) * chan[None, :, None, :]).to(torch.float16)
    v = torch.randn(B, Hkv, S, D, generator=gen).to(torch.float16)
    q = None
    if Hq is not None:
        q = torch.randn(B, Hq, Sq, D, generator=gen).to(torch.float16)
    return q, k, v


def exp_scores(S: int, seed: int) -> torch.Tensor:
    """Importance scores ~ Exponential(1) via -log(U), shared across batch and heads."""
    gen = torch.Generator().manual_seed(seed)
    u = torch.rand(S, generator=gen, dtype=torch.float64).clamp_min(1e-300)
    return (-torch.log(u)).to(torch.float32)


__all__ = ["CONFIGS", "DecodeConfig", "ReropeConfig", "exp_scores", "kv_tensors"]
