"""Tiered KV cache on MI355X kernels (drop-in for fade/cache.py's ``TieredKVCache``).

Per layer the cache holds fp16 sinks, a packed middle tier and an fp16
recent window (plus an optional INT2 tier), with the same state fields,
HF ``Cache`` protocol and tier API as the reference (fade/cache.py:52-1230).
What changes is where the work runs:

  * quantize + pack, dequantize, grouped INT2: ``libfade_hip.so`` kernels;
  * eviction re-RoPE: one fused gather/un-RoPE/re-RoPE pass over the kept
    rows only (``fade_rerope_gather``) instead of fp32 passes over all S;
  * ``decode_attention(q, layer_idx)``: attention straight from the tiers
    (``fade_tiered_decode_attn``) without the dequantize + ``torch.cat``
    materialization that ``update()`` performs for HF's attention modules.
"""

from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch
from torch import Tensor
from transformers.cache_utils import DynamicCache

from . import _lib
from .backends import AsymGroupBackend, QuantBackend, RotatedINT4Backend, SymmetricINT4Backend, get_backend
from .quant import (
    DEFAULT_INT2_GROUP_SIZE,
    dequant_int2_trimmed,
    dequant_int4,
    quant_int2_padded,
    quant_k_int4,
    quant_k_int4_from_colmax,
    quant_v_int4,
)
from .pages import PAGE_TOKENS
from .rope import RopeScheme, Vanilla, rerope_gather

DEFAULT_N_SINK: int = 4
DEFAULT_RECENT_WINDOW: int = 128
DEFAULT_INT4_BUDGET: int | None = None
DEFAULT_INT2_BUDGET: int = 0
DEFAULT_ROPE_THETA: float = 10000.0
DEFAULT_FP16_PREALLOC: int = 128
# partial column maxima the device reassignment's gather leaves for the K quantizer
_COLMAX_PARTS: int = 16
DEFAULT_MAX_DEQUANT_AGE: int | None = None

TIER_FP16: int = 0
TIER_INT4: int = 1
TIER_INT2: int = 2
TIER_EVICT: int = 3
TIER_PQ: int = 4


@dataclass
class LayerState:
    """Per-layer tier state (fade/cache.py:52-133).  ``*_pos`` hold absolute positions.

    Invariant: the position-ordered cache is ``sink | middle | fp16 recent``.
    """

    sink_k: Tensor | None = None
    sink_v: Tensor | None = None
    sink_pos: Tensor | None = None
    fp16_k: Tensor | None = None
    fp16_v: Tensor | None = None
    fp16_pos: Tensor | None = None
    int4_kq: Tensor | None = None
    int4_ks: Tensor | None = None
    int4_vq: Tensor | None = None
    int4_vs: Tensor | None = None
    int4_pos: Tensor | None = None
    int2_kq: Tensor | None = None
    int2_ks: Tensor | None = None
    int2_vq: Tensor | None = None
    int2_vs: Tensor | None = None
    int2_pos: Tensor | None = None
    int2_actual_count: int = 0
    int2_group_size: int = DEFAULT_INT2_GROUP_SIZE
    sink_count: int = 0
    next_position: int = 0
    int4_k_deq: Tensor | None = None
    int4_v_deq: Tensor | None = None
    int2_k_deq: Tensor | None = None
    int2_v_deq: Tensor | None = None
    _fp16_buf_k: Tensor | None = None
    _fp16_buf_v: Tensor | None = None
    _fp16_buf_pos: Tensor | None = None
    _fp16_len: int = 0
    _dequant_age: int = 0
    backend_k: dict | None = None
    backend_v: dict | None = None
    backend_pos: Tensor | None = None
    _compressed_bytes: int = 0
    # ragged layout (TieredKVCache.ragged_layout): per-row tier lengths, device
    # int32 [B, 3] (sink, middle, recent) and its host mirror; the tier tensors
    # are padded capacities and row b's token j (position order) sits at position j
    lens: Tensor | None = None
    lens_host: list | None = None
    # paged middle tier (TieredKVCache.page_pool, ragged layout only): the INT4 codes and
    # V scales live in 64-token pages of ``mid_pool``; ``mid_table`` is the block table
    # (int32 [B, pages per row]), ``mid_pages`` each row's page ids; int4_ks stays per row
    mid_table: Tensor | None = None
    mid_pages: list | None = None
    mid_pool: object | None = None
    mid_page_bytes: int = 0
    # rows zero-padded by the reference's per-sequence assignment (row 0's positions,
    # the earlier sink split kept): later per-sequence calls take the host path
    _padded_rows: bool = False
    # fused attention's ephemeral fp16 forms (never checkpointed): the sink followed by
    # the dequantized INT2 tier, and the dequantized middle tier of formats the prefill
    # kernel does not read in place; each with the tensors it was built from
    _front_cache: tuple | None = None
    _mid_f16_cache: tuple | None = None
    _decode_plan: tuple | None = None  # (key, TieredDecodePlan) reused while the tiers are the same objects

    def total_seq_length(self) -> int:
        if self.lens_host is not None:
            return max((sum(r) for r in self.lens_host), default=0)
        return sum(
            int(p.shape[0])
            for p in (self.sink_pos, self.fp16_pos, self.int4_pos, self.int2_pos, self.backend_pos)
            if p is not None
        )


# device RoPE tables of the device-side reassignment: (scheme, dtype, device) -> (cos, sin)
_ROPE_TABLES: dict = {}


def _sel(x: Tensor, idx: Tensor) -> Tensor:
    return x.index_select(-2, idx).contiguous()


class TieredKVCache(DynamicCache):
    """Tiered KV cache with attention-aware compression (fade/cache.py:136-225).

    Shared-tier mode (``tiers`` is ``[S]`` for all rows and heads) and
    per-sequence mode (``apply_tier_assignment_per_sequence``) as in the
    reference.  ``dtype`` float16, bfloat16 or float32, as the reference's:
    every tier, scale and dequantized copy is of it.  The fused attention
    kernels (``fused`` mode) read float16 and bfloat16 caches; the device
    reassignment and the ragged layout read float16 caches, the others use
    the host reassignment (the HIP quantizers and re-RoPE kernel at their
    dtype).
    """

    def __init__(
        self,
        n_sink: int = DEFAULT_N_SINK,
        recent_window: int = DEFAULT_RECENT_WINDOW,
        int4_budget: int | None = DEFAULT_INT4_BUDGET,
        int2_budget: int = DEFAULT_INT2_BUDGET,
        dtype: torch.dtype = torch.float16,
        cache_dequant: bool = True,
        rope_theta: float = DEFAULT_ROPE_THETA,
        head_dim: int | None = None,
        batch_size: int | None = None,
        rope_scheme: RopeScheme | None = None,
        middle_k_bits: int = 4,
        middle_v_bits: int = 4,
        quant_backend: str | QuantBackend = "int4",
    ) -> None:
        super().__init__()
        if dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError(f"fade_amd TieredKVCache supports float16, bfloat16 and float32, got {dtype}")
        self.n_sink = n_sink
        self.recent_window = recent_window
        self.int4_budget = int4_budget
        self.int2_budget = int2_budget
        self.dtype = dtype
        self.cache_dequant = cache_dequant
        self.rope_theta = rope_theta
        self.head_dim = head_dim
        self.batch_size = batch_size
        self.max_dequant_age = DEFAULT_MAX_DEQUANT_AGE
        self.middle_k_bits = middle_k_bits
        self.middle_v_bits = middle_v_bits
        if isinstance(quant_backend, str):
            self._quant_backend: QuantBackend = get_backend(quant_backend, head_dim=head_dim or 64)
        else:
            self._quant_backend = quant_backend
        self._rope_scheme = rope_scheme
        self._skip_layers: set[int] = set()
        self._layers: list[LayerState] = []
        # fused mode (attn_implementation="fade"): update() appends only and the
        # layer's attention reads the tiers in place (fade_amd/hf_attention.py)
        self.fused = False
        # apply_tier_assignment on the device for the reference INT4 layout
        self.device_reassign = True
        # apply_tier_assignment_per_sequence keeps each row's own tokens (per-row
        # tier lengths, attention over them only) instead of the reference's
        # zero-padded rows (fade/cache.py:1145-1159)
        self.ragged_layout = False
        # roadmap P4 (FADE v1.0 Release + Future Roadmap.md:30-34): at a reassignment,
        # per-token codes of tokens that stay in the middle tier are kept as they are
        # and only tokens entering it are quantized (no requantization of dequantized
        # values); per-channel K scales still span the whole tier and are recomputed
        self.incremental_quant = False
        # ragged layout: a fade_amd.pages.MiddlePagePool to keep the middle tier in
        # 64-token pages (per-row memory instead of padding to the longest row)
        self.page_pool = None
        # The device reassignment's gather reports tokens it had to drop in a status
        # word (a position outside the RoPE tables, a slot past a tier's capacity, a
        # token a row does not have: a plan the cache did not make).  Reading it costs
        # a host synchronization, so by default it is not read; True reads it after
        # every device reassignment and raises RuntimeError when a bit is set.
        self.check_reassign_status = False
        # split count of the fused decode kernel (0: the kernel's planner fills the GPU)
        self.decode_splits = 0
        self._last_reassign_counts = None

    # transformers 5.x defines a read-only ``Cache.batch_size``; the tiered cache
    # pins the batch size on the first update (fade/cache.py:367-373).
    @property
    def batch_size(self) -> int | None:
        return self.__dict__.get("_pinned_batch_size")

    @batch_size.setter
    def batch_size(self, value: int | None) -> None:
        self.__dict__["_pinned_batch_size"] = value

    # ------------------------------------------------------------ bookkeeping
    def set_skip_layers(self, layer_indices) -> None:
        self._skip_layers = set(layer_indices)

    @property
    def managed_layers(self) -> set[int]:
        return {i for i in range(len(self._layers)) if i not in self._skip_layers}

    def is_managed(self, layer_idx: int) -> bool:
        return layer_idx not in self._skip_layers

    def _ensure_rope_scheme(self) -> RopeScheme:
        if self._rope_scheme is None:
            self._rope_scheme = Vanilla(theta=self.rope_theta, head_dim=self.head_dim or 64)
        return self._rope_scheme

    @property
    def rope_scheme(self) -> RopeScheme:
        return self._ensure_rope_scheme()

    # --------------------------------------------------------------- HF API
    def update(self, key_states: Tensor, value_states: Tensor, layer_idx: int, cache_kwargs: dict | None = None):
        """Append new K/V to the fp16 tier and return the full cache in position order."""
        if key_states.dim() != 4:
            raise ValueError(f"key_states must be [B, H, S, D]; got shape {tuple(key_states.shape)}")
        if key_states.shape != value_states.shape:
            raise ValueError(f"K/V shape mismatch: {tuple(key_states.shape)} vs {tuple(value_states.shape)}")
        if self.fused and self.dtype not in _FUSED_DTYPES:  # refused before any state changes
            raise NotImplementedError(
                f"fused attention reads float16 and bfloat16 caches; this one is {self.dtype} "
                "(use the model's own attention)"
            )
        batch = int(key_states.shape[0])
        if self.batch_size is None:
            self.batch_size = batch
        elif self.batch_size != batch:
            raise ValueError(f"batch size mismatch: cache pinned to B={self.batch_size} but got B={batch}")
        if self.head_dim is None:
            self.head_dim = int(key_states.shape[-1])
        self._ensure_layer(layer_idx)
        self._append_fp16(key_states, value_states, layer_idx)
        if self.fused:
            from .hf_attention import set_active_cache

            set_active_cache(self)
            return key_states, value_states
        return self._materialize(layer_idx)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if layer_idx >= len(self._layers):
            return 0
        return self._layers[layer_idx].total_seq_length()

    def get_mask_sizes(self, cache_position, layer_idx: int = 0) -> tuple[int, int]:
        q = cache_position if isinstance(cache_position, int) else int(cache_position.shape[0])
        return self.get_seq_length(layer_idx) + q, 0

    def __len__(self) -> int:
        return len(self._layers)

    # ---------------------------------------------------------------- bytes
    def storage_bytes(self) -> int:
        keys = (
            "fp16_k", "fp16_v", "int4_kq", "int4_vq", "int4_ks", "int4_vs", "int4_k_deq", "int4_v_deq",
            "int2_kq", "int2_vq", "int2_ks", "int2_vs", "int2_k_deq", "int2_v_deq",
        )
        return sum(
            int(t.element_size() * t.numel()) for s in self._layers for t in (getattr(s, k) for k in keys) if t is not None
        ) + sum(s.mid_page_bytes for s in self._layers)

    @staticmethod
    def _layer_compressed_bytes(state: LayerState) -> int:
        keys = (
            "sink_k", "sink_v", "fp16_k", "fp16_v", "int4_kq", "int4_vq", "int4_ks", "int4_vs",
            "int2_kq", "int2_vq", "int2_ks", "int2_vs",
        )
        total = sum(int(t.element_size() * t.numel()) for t in (getattr(state, k) for k in keys) if t is not None)
        total += state.mid_page_bytes
        for d in (state.backend_k, state.backend_v):
            if isinstance(d, dict):
                total += sum(int(v.element_size() * v.numel()) for v in d.values() if isinstance(v, Tensor))
        return total

    def compressed_storage_bytes(self) -> int:
        if self._layers and any(s._compressed_bytes > 0 for s in self._layers):
            return sum(s._compressed_bytes for s in self._layers)
        return sum(self._layer_compressed_bytes(s) for s in self._layers)

    # ----------------------------------------------------------- checkpoint
    _LAYER_TENSOR_KEYS = (
        "sink_k", "sink_v", "sink_pos", "fp16_k", "fp16_v", "fp16_pos", "int4_kq", "int4_ks", "int4_vq",
        "int4_vs", "int4_pos", "int2_kq", "int2_ks", "int2_vq", "int2_vs", "int2_pos",
    )
    _LAYER_SCALAR_KEYS = ("int2_actual_count", "int2_group_size", "sink_count", "next_position")

    def cache_state_dict(self) -> dict:
        """Essential compressed form, on the CPU, same keys as fade/cache.py:510-534.

        Layers the reference has no form for add keys its loader ignores: a
        backend-compressed middle tier (``layer.{i}.backend_k.<field>``,
        ``backend_v.<field>``, ``backend_pos``) and the ragged layout
        (``layer.{i}.lens``, int32 [B, 3] per-row sink / middle / recent
        lengths; the tier tensors are then padded capacities, a paged middle
        tier gathered back into them)."""
        sd: dict = {
            "n_layers": len(self._layers),
            "n_sink": self.n_sink,
            "recent_window": self.recent_window,
            "int4_budget": self.int4_budget,
            "int2_budget": self.int2_budget,
            "batch_size": self.batch_size,
            "head_dim": self.head_dim,
            "dtype": str(self.dtype),
        }
        for i, st in enumerate(self._layers):
            vals = {k: getattr(st, k) for k in self._LAYER_TENSOR_KEYS}
            if st.mid_table is not None:  # paged: the padded tensors the pool stands for
                vals["int4_kq"], vals["int4_ks"], vals["int4_vq"], vals["int4_vs"] = self._mid_padded(st)
            for k, v in vals.items():
                if v is not None:
                    sd[f"layer.{i}.{k}"] = v.cpu()
            for k in self._LAYER_SCALAR_KEYS:
                sd[f"layer.{i}.{k}"] = getattr(st, k)
            for name in ("backend_k", "backend_v"):
                d = getattr(st, name)
                if d is not None:
                    for f, t in d.items():
                        sd[f"layer.{i}.{name}.{f}"] = t.cpu()
            if st.backend_pos is not None:
                sd[f"layer.{i}.backend_pos"] = st.backend_pos.cpu()
            if st.lens is not None:
                sd[f"layer.{i}.lens"] = torch.tensor(st.lens_host, dtype=torch.int32)
        return sd

    def load_cache_state_dict(self, sd: dict, device: torch.device | str | None = None) -> None:
        """Restore from ``cache_state_dict`` output (fade/cache.py:536-559), including
        the build's extra keys (backend-compressed middle tier, ragged layout)."""
        mv = (lambda t: t.to(device)) if device is not None else (lambda t: t)
        self._layers = []
        for i in range(sd["n_layers"]):
            st = LayerState()
            for k in self._LAYER_TENSOR_KEYS:
                v = sd.get(f"layer.{i}.{k}")
                if v is not None:
                    setattr(st, k, mv(v))
            for k in self._LAYER_SCALAR_KEYS:
                v = sd.get(f"layer.{i}.{k}")
                if v is not None:
                    setattr(st, k, v)
            for name in ("backend_k", "backend_v"):
                pre = f"layer.{i}.{name}."
                d = {key[len(pre):]: mv(t) for key, t in sd.items() if key.startswith(pre)}
                if d:
                    setattr(st, name, d)
            if sd.get(f"layer.{i}.backend_pos") is not None:
                st.backend_pos = mv(sd[f"layer.{i}.backend_pos"])
            lens = sd.get(f"layer.{i}.lens")
            if lens is not None:
                st.lens_host = [[int(x) for x in r] for r in lens.tolist()]
                ref = next((t for t in (st.sink_k, st.fp16_k, st.int4_kq) if t is not None), None)
                st.lens = lens.to(torch.int32).to(ref.device if ref is not None else (device or "cpu"))
            st._compressed_bytes = self._layer_compressed_bytes(st)
            self._layers.append(st)
        if sd.get("batch_size") is not None:
            self.batch_size = sd["batch_size"]
        if sd.get("head_dim") is not None:
            self.head_dim = sd["head_dim"]

    def dump_debug(self, path: str | Path) -> None:
        layers = []
        for i, st in enumerate(self._layers):
            d = {
                "layer_idx": i,
                "sink_count": st.sink_count,
                "next_position": st.next_position,
                "fp16_count": 0 if st.fp16_pos is None else int(st.fp16_pos.shape[0]),
                "int4_count": 0 if st.int4_pos is None else int(st.int4_pos.shape[0]),
                "int2_count": 0 if st.int2_pos is None else int(st.int2_pos.shape[0]),
                "int2_actual_count": st.int2_actual_count,
                "total_seq_length": st.total_seq_length(),
            }
            for name in ("sink", "fp16", "int4", "int2"):
                pos = getattr(st, f"{name}_pos")
                if pos is not None:
                    d[f"{name}_positions"] = pos.tolist()
            layers.append(d)
        snap = {
            "n_layers": len(self._layers), "n_sink": self.n_sink, "recent_window": self.recent_window,
            "int4_budget": self.int4_budget, "int2_budget": self.int2_budget, "batch_size": self.batch_size,
            "head_dim": self.head_dim, "layers": layers,
        }
        Path(path).write_text(json.dumps(snap, indent=2), encoding="utf-8")

    # ------------------------------------------------------------ internals
    def _ensure_layer(self, layer_idx: int) -> None:
        while len(self._layers) <= layer_idx:
            self._layers.append(LayerState())

    def _append_fp16_ragged(self, st: LayerState, k: Tensor, v: Tensor) -> None:
        """Ragged layout: row b's new tokens go to its own recent slots lens[b, 2].. ."""
        n = int(k.shape[-2])
        B, H, _, D = k.shape
        have = max(r[2] for r in st.lens_host)
        if st._fp16_buf_k is None and st.fp16_k is not None:  # restored from a checkpoint
            st._fp16_buf_k, st._fp16_buf_v = st.fp16_k.contiguous(), st.fp16_v.contiguous()
        cap = 0 if st._fp16_buf_k is None else int(st._fp16_buf_k.shape[-2])
        if have + n > cap:
            cap2 = max(2 * cap, have + n, DEFAULT_FP16_PREALLOC)
            bk = torch.zeros(B, H, cap2, D, dtype=k.dtype, device=k.device)
            bv = torch.zeros(B, H, cap2, D, dtype=v.dtype, device=v.device)
            if cap:
                bk[:, :, :cap] = st._fp16_buf_k
                bv[:, :, :cap] = st._fp16_buf_v
            st._fp16_buf_k, st._fp16_buf_v = bk, bv
        # one scatter per tensor: element [b, i] of the index pair is row b's slot lens[b, 2] + i
        rows = torch.arange(B, device=k.device)[:, None]
        slots = st.lens[:, 2].long()[:, None] + torch.arange(n, device=k.device)[None, :]
        st._fp16_buf_k[rows, :, slots] = k.permute(0, 2, 1, 3)
        st._fp16_buf_v[rows, :, slots] = v.permute(0, 2, 1, 3)
        st.lens[:, 2] += n
        for r in st.lens_host:
            r[2] += n
        top = max(r[2] for r in st.lens_host)
        st._fp16_len = top
        st.fp16_k, st.fp16_v = st._fp16_buf_k[:, :, :top], st._fp16_buf_v[:, :, :top]
        st.next_position = max(st.next_position, st.total_seq_length())
        st._dequant_age += 1

    def _append_fp16(self, k: Tensor, v: Tensor, layer_idx: int) -> None:
        """Append to the doubling fp16 buffer (fade/cache.py:608-670)."""
        st = self._layers[layer_idx]
        if st.lens is not None:
            self._append_fp16_ragged(st, k, v)
            return
        n = int(k.shape[-2])
        new_pos = torch.arange(st.next_position, st.next_position + n, device=k.device)
        st.next_position += n
        if st._fp16_buf_k is None:
            have = 0 if st.fp16_k is None else int(st.fp16_k.shape[-2])
            need = have + n
            cap = max(DEFAULT_FP16_PREALLOC, need)
            B, H, _, D = k.shape
            st._fp16_buf_k = torch.empty(B, H, cap, D, dtype=k.dtype, device=k.device)
            st._fp16_buf_v = torch.empty(B, H, cap, D, dtype=v.dtype, device=v.device)
            st._fp16_buf_pos = torch.empty(cap, dtype=torch.long, device=k.device)
            if have:
                st._fp16_buf_k[:, :, :have] = st.fp16_k
                st._fp16_buf_v[:, :, :have] = st.fp16_v
                st._fp16_buf_pos[:have] = st.fp16_pos
            st._fp16_buf_k[:, :, have:need] = k
            st._fp16_buf_v[:, :, have:need] = v
            st._fp16_buf_pos[have:need] = new_pos
            st._fp16_len = need
        else:
            old, new = st._fp16_len, st._fp16_len + n
            cap = st._fp16_buf_k.shape[-2]
            if new > cap:
                cap2 = max(cap * 2, new)
                B, H, _, D = st._fp16_buf_k.shape
                bk = torch.empty(B, H, cap2, D, dtype=k.dtype, device=k.device)
                bv = torch.empty(B, H, cap2, D, dtype=v.dtype, device=v.device)
                bp = torch.empty(cap2, dtype=torch.long, device=k.device)
                bk[:, :, :old] = st._fp16_buf_k[:, :, :old]
                bv[:, :, :old] = st._fp16_buf_v[:, :, :old]
                bp[:old] = st._fp16_buf_pos[:old]
                st._fp16_buf_k, st._fp16_buf_v, st._fp16_buf_pos = bk, bv, bp
            st._fp16_buf_k[:, :, old:new] = k
            st._fp16_buf_v[:, :, old:new] = v
            st._fp16_buf_pos[old:new] = new_pos
            st._fp16_len = new
        ln = st._fp16_len
        st.fp16_k = st._fp16_buf_k[:, :, :ln]
        st.fp16_v = st._fp16_buf_v[:, :, :ln]
        st.fp16_pos = st._fp16_buf_pos[:ln]
        st._dequant_age += 1

    def _materialize_ragged(self, st: LayerState) -> tuple[Tensor, Tensor]:
        """Ragged layout: row b = its sink | middle | recent tokens, zero-padded at the end
        to the longest row."""
        ref = st.fp16_k if st.fp16_k is not None else (st.sink_k if st.sink_k is not None else None)
        if st.int4_kq is not None or st.mid_table is not None:
            mk, mv = self._get_int4_dequant(st)
            ref = mk if ref is None else ref
        B, H, _, D = ref.shape
        top = st.total_seq_length()
        ko = torch.zeros(B, H, top, D, dtype=self.dtype, device=ref.device)
        vo = torch.zeros_like(ko)
        for b, (ls, lm, lr) in enumerate(st.lens_host):
            parts = []
            if ls:
                parts.append((st.sink_k[b, :, :ls], st.sink_v[b, :, :ls]))
            if lm:
                parts.append((mk[b, :, :lm], mv[b, :, :lm]))
            if lr:
                parts.append((st.fp16_k[b, :, :lr], st.fp16_v[b, :, :lr]))
            if parts:
                n = ls + lm + lr
                ko[b, :, :n] = torch.cat([p[0] for p in parts], dim=-2)
                vo[b, :, :n] = torch.cat([p[1] for p in parts], dim=-2)
        return ko, vo

    def _materialize(self, layer_idx: int) -> tuple[Tensor, Tensor]:
        if self._layers[layer_idx].lens is not None:
            return self._materialize_ragged(self._layers[layer_idx])
        ks, vs = self._assemble_parts(self._layers[layer_idx], want_positions=False)
        if not ks:
            raise RuntimeError(f"No cache state for layer {layer_idx}")
        return torch.cat(ks, dim=-2), torch.cat(vs, dim=-2)

    def _all_in_position_order(self, layer_idx: int) -> tuple[Tensor, Tensor, Tensor]:
        ks, vs, ps = self._assemble_parts(self._layers[layer_idx], want_positions=True)
        if not ks:
            raise RuntimeError(f"No cache state for layer {layer_idx}")
        return torch.cat(ks, dim=-2), torch.cat(vs, dim=-2), torch.cat(ps, dim=0)

    def _assemble_parts(self, st: LayerState, want_positions: bool):
        """sink | middle (INT4 + backend + INT2 merged by position) | recent (fade/cache.py:715-808)."""
        ks, vs, ps = [], [], []
        nsk = st.sink_count
        if st.sink_k is not None:
            ks.append(st.sink_k)
            vs.append(st.sink_v)
            ps.append(st.sink_pos)
        elif st.fp16_k is not None and nsk > 0:
            ks.append(st.fp16_k[..., :nsk, :])
            vs.append(st.fp16_v[..., :nsk, :])
            ps.append(st.fp16_pos[:nsk])
        mk, mv, mp = [], [], []
        if st.int4_kq is not None:
            k4, v4 = self._get_int4_dequant(st)
            mk.append(k4)
            mv.append(v4)
            mp.append(st.int4_pos)
        if st.backend_k is not None:
            mk.append(self._quant_backend.decompress_k(st.backend_k, dtype=self.dtype))
            mv.append(self._quant_backend.decompress_v(st.backend_v, dtype=self.dtype))
            mp.append(st.backend_pos)
        if st.int2_kq is not None:
            k2, v2 = self._get_int2_dequant(st)
            mk.append(k2)
            mv.append(v2)
            mp.append(st.int2_pos)
        if len(mk) == 1:
            ks.append(mk[0])
            vs.append(mv[0])
            ps.append(mp[0])
        elif mk:
            order = torch.cat(mp).argsort()
            ks.append(torch.cat(mk, dim=-2).index_select(-2, order))
            vs.append(torch.cat(mv, dim=-2).index_select(-2, order))
            ps.append(torch.cat(mp)[order])
        if st.fp16_k is not None:
            start = 0 if st.sink_k is not None else nsk
            if start < int(st.fp16_k.shape[-2]):
                ks.append(st.fp16_k[..., start:, :])
                vs.append(st.fp16_v[..., start:, :])
                ps.append(st.fp16_pos[start:])
        return (ks, vs, ps) if want_positions else (ks, vs)

    def _get_int4_dequant(self, st: LayerState) -> tuple[Tensor, Tensor]:
        """fade/cache.py:810-842 (cached fp16 copy when ``cache_dequant``)."""
        if self.max_dequant_age is not None and st._dequant_age > self.max_dequant_age and st.int4_k_deq is not None:
            st.int4_k_deq = st.int4_v_deq = None
        if self.cache_dequant and st.int4_k_deq is not None:
            return st.int4_k_deq, st.int4_v_deq
        kq, ks, vq, vs = self._mid_padded(st)
        k = dequant_int4(kq, ks, dtype=self.dtype)
        if self.middle_v_bits == 4:
            v = dequant_int4(vq, vs, dtype=self.dtype)
        else:
            n = int(st.int4_pos.shape[0])
            v = dequant_int2_trimmed(st.int4_vq, st.int4_vs, n, DEFAULT_INT2_GROUP_SIZE)
        if self.cache_dequant:
            st.int4_k_deq, st.int4_v_deq = k, v
            st._dequant_age = 0
        return k, v

    @staticmethod
    def _mid_padded(st: LayerState):
        """(K codes, K scale, V codes, V scale) of the INT4 middle tier as padded
        [B, Hkv, S, ...] tensors: the stored ones, or for a paged layer gathered from its
        pool (bit-identical to what the unpaged layout stores); None without a middle."""
        if st.mid_table is not None:
            kq, vq, vs = st.mid_pool.gather(st.mid_table, max(r[1] for r in st.lens_host))
            return kq, st.int4_ks, vq, vs
        if st.int4_kq is None:
            return None
        return st.int4_kq, st.int4_ks, st.int4_vq, st.int4_vs

    def _release_layer_pages(self, st: LayerState) -> None:
        if st.mid_pages is not None:
            st.mid_pool.free([i for row in st.mid_pages for i in row])
        st.mid_table = st.mid_pages = st.mid_pool = None
        st.mid_page_bytes = 0

    def release_pages(self) -> None:
        """Return every page this cache's layers hold to their pool and drop those
        layers' middle tiers (for a finished sequence batch whose pool serves others)."""
        for st in self._layers:
            if st.mid_table is not None:
                self._release_layer_pages(st)
                st.int4_ks = st.int4_k_deq = st.int4_v_deq = None
                st.lens_host = [[ls, 0, lr] for ls, _, lr in st.lens_host]
                st.lens = torch.tensor(st.lens_host, dtype=torch.int32, device=st.lens.device)
                st._compressed_bytes = self._layer_compressed_bytes(st)

    def _get_int2_dequant(self, st: LayerState) -> tuple[Tensor, Tensor]:
        """fade/cache.py:861-876."""
        if self.cache_dequant and st.int2_k_deq is not None:
            return st.int2_k_deq, st.int2_v_deq
        n, g = st.int2_actual_count, st.int2_group_size
        k = dequant_int2_trimmed(st.int2_kq, st.int2_ks, n, g)
        v = dequant_int2_trimmed(st.int2_vq, st.int2_vs, n, g)
        if self.cache_dequant:
            st.int2_k_deq, st.int2_v_deq = k, v
        return k, v

    # ------------------------------------------------------- tier movement
    def _rerope_kept(self, k_full, v_full, pos_full, keep_idx, n_kept):
        """Un-RoPE kept rows at their old positions and re-RoPE them at 0..n_kept-1."""
        scheme = self._ensure_rope_scheme()
        new_pos = torch.arange(n_kept, dtype=torch.long)
        cos_o, sin_o = scheme.host_cos_sin(pos_full.cpu(), self.dtype)
        cos_n, sin_n = scheme.host_cos_sin(new_pos, self.dtype)
        k_kept, v_kept = rerope_gather(k_full, v_full, keep_idx, cos_o, sin_o, cos_n, sin_n)
        return k_kept, v_kept, new_pos.to(pos_full.device)

    def _store_middle(self, st: LayerState, k_sub: Tensor, v_sub: Tensor, pos: Tensor) -> None:
        if isinstance(self._quant_backend, SymmetricINT4Backend):
            st.int4_kq, st.int4_ks = quant_k_int4(k_sub)
            if self.middle_v_bits == 4:
                st.int4_vq, st.int4_vs = quant_v_int4(v_sub)
            else:
                st.int4_vq, st.int4_vs = quant_int2_padded(v_sub, DEFAULT_INT2_GROUP_SIZE)
            st.int4_pos = pos
            st.backend_k = st.backend_v = st.backend_pos = None
        else:
            st.backend_k = self._quant_backend.compress_k(k_sub)
            st.backend_v = self._quant_backend.compress_v(v_sub)
            st.backend_pos = pos
            st.int4_kq = st.int4_vq = st.int4_ks = st.int4_vs = st.int4_pos = None

    def _reseed_fp16_buffer(self, st: LayerState) -> None:
        n = 0 if st.fp16_k is None else int(st.fp16_k.shape[-2])
        if n > 0 and st._fp16_buf_k is not None and n <= st._fp16_buf_k.shape[-2]:
            st._fp16_buf_k[:, :, :n] = st.fp16_k
            st._fp16_buf_v[:, :, :n] = st.fp16_v
            st._fp16_buf_pos[:n] = st.fp16_pos
            st._fp16_len = n
            st.fp16_k = st._fp16_buf_k[:, :, :n]
            st.fp16_v = st._fp16_buf_v[:, :, :n]
            st.fp16_pos = st._fp16_buf_pos[:n]
        else:
            st._fp16_buf_k = st._fp16_buf_v = st._fp16_buf_pos = None
            st._fp16_len = 0

    def _rope_tables(self, rows: int, device) -> tuple[Tensor, Tensor]:
        """cos/sin fp32 ``[R, D]`` (R >= rows) for positions ``0..R-1`` on ``device``.

        A row depends only on its position, so one table serves every layer and
        every later round until positions outgrow it: R is ``rows`` rounded up to
        a power of two (at least 4096), and the last table per (scheme, dtype,
        device) is kept at module level."""
        scheme = self._ensure_rope_scheme()
        key = (repr(scheme), str(self.dtype), str(device))
        tab = _ROPE_TABLES.get(key)
        if tab is None or int(tab[0].shape[0]) < rows:
            cap = max(4096, 1 << max(0, rows - 1).bit_length())
            cos, sin = scheme.host_cos_sin(torch.arange(cap, dtype=torch.long), self.dtype)
            # pinned + non_blocking: an upload that does not wait for the device
            tab = tuple(t.contiguous().pin_memory().to(device, non_blocking=True) for t in (cos, sin))
            _ROPE_TABLES[key] = tab
        return tab

    def _device_reassign_ok(self, st: LayerState) -> bool:
        k = st.sink_k if st.sink_k is not None else st.fp16_k
        if k is None and st.int4_kq is None:
            return False
        dev = (k if k is not None else st.int4_kq).device
        return (
            self.device_reassign
            and self.dtype == torch.float16  # the device gather writes fp16 tiers
            and dev.type == "cuda"
            and isinstance(self._quant_backend, SymmetricINT4Backend)
            and self.middle_k_bits == 4
            and self.middle_v_bits == 4
            and st.int2_kq is None
            and st.backend_k is None
        )

    @staticmethod
    def _middle_sources(tiers: Tensor, ns_old: int, nm_old: int, keep_idx: Tensor | None = None):
        """For the middle tier an assignment builds: (slots, old rows) of the tokens that were
        already middle tokens, and the slots of the others.  ``tiers`` is the host
        assignment over the kept tokens; ``keep_idx`` maps them back to the position
        order before eviction."""
        t = tiers.cpu()
        mids = (t == TIER_INT4).nonzero(as_tuple=False).squeeze(-1)
        src = mids if keep_idx is None else keep_idx.cpu()[mids]
        was_mid = (src >= ns_old) & (src < ns_old + nm_old)
        slots = torch.arange(int(mids.numel()))
        return slots[was_mid], (src[was_mid] - ns_old), slots[~was_mid]

    @staticmethod
    def _host_tier_counts(tiers: Tensor) -> tuple[int, int, int] | None:
        """(n_fp16, n_int4, n_int2) of a host tiers tensor, or None if it holds other values."""
        # one histogram (numpy: a few µs on the host tensor, against ~8 µs per torch op):
        # bucket 0 = values below TIER_FP16, 1..4 = tiers 0..3, 5 = above TIER_EVICT
        c = np.bincount(np.clip(tiers.numpy().astype(np.int64) + 1, 0, 5), minlength=6).tolist()
        if c[0] or c[5]:
            return None
        return c[1 + TIER_FP16], c[1 + TIER_INT4], c[1 + TIER_INT2]

    def _incremental_v(self, tiers: Tensor, ns_old: int, nm_old: int, old_v, v_new_f16: Tensor):
        """Per-token INT4 V of the new middle tier: old middle tokens keep their codes and
        scales, the others are quantized from their fp16 values (``quant_v_int4``)."""
        slots, rows, fresh = self._middle_sources(tiers, ns_old, nm_old)
        B, H, n, D = v_new_f16.shape
        dev = v_new_f16.device
        vq = torch.empty(B, H, n, D // 2, dtype=torch.uint8, device=dev)
        vs = torch.empty(B, H, n, 1, dtype=v_new_f16.dtype, device=dev)
        if slots.numel():
            si, ri = slots.to(dev), rows.to(dev)
            vq.index_copy_(2, si, old_v[0].index_select(2, ri))
            vs.index_copy_(2, si, old_v[1].index_select(2, ri))
        if fresh.numel():
            fi = fresh.to(dev)
            q, sc = quant_v_int4(v_new_f16.index_select(2, fi).contiguous())
            vq.index_copy_(2, fi, q)
            vs.index_copy_(2, fi, sc)
        return vq, vs

    @staticmethod
    def _merge_compressed(old: dict, fresh: dict | None, slots: Tensor, rows: Tensor, fresh_slots: Tensor, n: int):
        """Per-token compressed dict of n tokens: rows of ``old`` at ``slots``, rows of
        ``fresh`` at ``fresh_slots`` (every tensor is [B, H, tokens, ...])."""
        out = {}
        for key, t in old.items():
            dev = t.device
            o = torch.empty(t.shape[0], t.shape[1], n, *t.shape[3:], dtype=t.dtype, device=dev)
            if slots.numel():
                o.index_copy_(2, slots.to(dev), t.index_select(2, rows.to(dev)))
            if fresh is not None and fresh_slots.numel():
                o.index_copy_(2, fresh_slots.to(dev), fresh[key])
            out[key] = o
        return out

    _STATUS_BITS = {1: "INT2 tokens in the plan", 2: "an unknown tier value",
                    4: "a position outside the RoPE tables", 8: "a slot past a tier's capacity",
                    16: "a token the row does not have"}

    def _check_status(self, cnt: Tensor, rows: int) -> None:
        """With ``check_reassign_status``: raise if the gather dropped a token (see __init__)."""
        if not self.check_reassign_status:
            return
        words = cnt.view(-1, 4)[:rows, 3].cpu().tolist()
        bad = [(r, w) for r, w in enumerate(words) if w]
        if bad:
            r, w = bad[0]
            what = ", ".join(t for b, t in self._STATUS_BITS.items() if w & b) or f"status {w:#x}"
            raise RuntimeError(f"device reassignment dropped tokens (row {r}): {what}")

    def _apply_tier_assignment_device(self, layer_idx: int, tiers: Tensor, counts) -> bool:
        """``apply_tier_assignment`` on the device for the reference INT4 layout.

        ``fade_reassign_plan`` ranks every token of the position-ordered layer,
        ``fade_reassign_gather`` moves the kept ones (dequantizing middle rows and
        re-RoPE-ing K in registers) straight into the new sink, recent buffer and
        an fp16 middle staging tensor, which the INT4 quantizers encode.  No
        host sync when the tier counts are known on the host (a host ``tiers``
        tensor, or ``counts``); otherwise one 16-byte read of the device counts.
        Returns False (nothing changed) when the assignment holds INT2 tokens.
        """
        st = self._layers[layer_idx]
        old_v = (st.int4_vq, st.int4_vs)
        if st.sink_k is not None:
            sink = (st.sink_k, st.sink_v)
            rec_start = 0
        else:
            nsk = st.sink_count if st.fp16_k is not None else 0
            sink = (st.fp16_k[..., :nsk, :], st.fp16_v[..., :nsk, :]) if nsk > 0 else None
            rec_start = nsk
        rec = None
        if st.fp16_k is not None and rec_start < int(st.fp16_k.shape[-2]):
            rec = (st.fp16_k[..., rec_start:, :], st.fp16_v[..., rec_start:, :])
        ref = sink[0] if sink is not None else (rec[0] if rec is not None else None)
        if ref is None:
            B, H, _, half = st.int4_kq.shape
            D = 2 * half
        else:
            B, H, _, D = ref.shape
        dev = st.int4_kq.device if ref is None else ref.device
        ns_old = 0 if sink is None else int(sink[0].shape[-2])
        nm_old = 0 if st.int4_kq is None else int(st.int4_kq.shape[-2])
        nr_old = 0 if rec is None else int(rec[0].shape[-2])
        S = ns_old + nm_old + nr_old
        if int(tiers.shape[0]) != S:
            raise ValueError(f"tiers length {int(tiers.shape[0])} != cache length {S} for layer {layer_idx}")
        if counts is None and tiers.device.type == "cpu":
            counts = self._host_tier_counts(tiers)
            if counts is None:
                return False
        if counts is not None and counts[2] > 0:
            return False
        pos_parts = [p for p in (
            None if sink is None else (st.sink_pos if st.sink_k is not None else st.fp16_pos[:ns_old]),
            st.int4_pos,
            None if rec is None else st.fp16_pos[rec_start:],
        ) if p is not None]
        pos_old = torch.cat(pos_parts).to(device=dev, dtype=torch.long).contiguous()
        tiers_d = tiers.to(dtype=torch.long).contiguous()
        if tiers_d.device != dev:
            tiers_d = (tiers_d.pin_memory() if tiers_d.device.type == "cpu" else tiers_d).to(dev, non_blocking=True)
        # plan outputs in two allocations: dst | newpos | src_of | counts, and the new positions
        S1 = max(S, 1)
        i32 = torch.empty(3 * S1 + 4, dtype=torch.int32, device=dev)
        dst, newpos, src_of, cnt = i32[:S1], i32[S1 : 2 * S1], i32[2 * S1 : 3 * S1], i32[3 * S1 :]
        pos_new = torch.empty(3, S1, dtype=torch.long, device=dev)
        stream = _lib.stream_of(tiers_d)
        _lib.call("fade_reassign_plan", tiers_d.data_ptr(), 0, 1, S, self.n_sink, pos_old.data_ptr(), 0,
                  dst.data_ptr(), newpos.data_ptr(), src_of.data_ptr(), pos_new[0].data_ptr(),
                  pos_new[1].data_ptr(), pos_new[2].data_ptr(), cnt.data_ptr(), stream)
        if counts is None:
            c = cnt.cpu().tolist()  # the one host sync: tiers were on the device
            if c[3] != 0:
                return False
            n_fp16, n_int4 = c[0], c[1]
        else:
            n_fp16, n_int4 = int(counts[0]), int(counts[1])
        n_kept = n_fp16 + n_int4
        n_sink_new = min(self.n_sink, n_fp16)
        n_rec_new = n_fp16 - n_sink_new
        kd = dict(dtype=torch.float16, device=dev)
        out_sink = (torch.empty(B, H, n_sink_new, D, **kd), torch.empty(B, H, n_sink_new, D, **kd)) if n_sink_new else None
        old_cap = 0 if st._fp16_buf_k is None else int(st._fp16_buf_k.shape[-2])
        cap = max(DEFAULT_FP16_PREALLOC, n_rec_new, old_cap)
        buf = (torch.empty(B, H, cap, D, **kd), torch.empty(B, H, cap, D, **kd)) if n_rec_new else None
        mid = None
        if n_int4:  # fp16 staging of the new middle tier (read by the quantizers, then dropped)
            m2 = torch.empty(2, B, H, n_int4, D, **kd)
            mid = (m2[0], m2[1])
        tab = self._rope_tables(st.next_position, dev) if n_kept < S else None

        def cf(t):  # K and V of a tier share strides in the kernel
            return t if t[0].stride() == t[1].stride() else (t[0].contiguous(), t[1].contiguous())

        sink = None if sink is None else cf(sink)
        rec = None if rec is None else cf(rec)
        a = _lib.ReassignArgs()
        a.B, a.H, a.D, a.S = B, H, D, S
        a.n_sink_old, a.n_mid_old = ns_old, nm_old
        a.plan_rows = 1
        if sink is not None:
            a.sink_k, a.sink_v = sink[0].data_ptr(), sink[1].data_ptr()
            a.sink_sb, a.sink_sh, a.sink_ss = sink[0].stride()[:3]
        if nm_old:
            mids = [t.contiguous() for t in (st.int4_kq, st.int4_ks, st.int4_vq, st.int4_vs)]
            a.mid_kq, a.mid_ks, a.mid_vq, a.mid_vs = (t.data_ptr() for t in mids)
        if rec is not None:
            a.rec_k, a.rec_v = rec[0].data_ptr(), rec[1].data_ptr()
            a.rec_sb, a.rec_sh, a.rec_ss = rec[0].stride()[:3]
        a.dst, a.newpos, a.src_of, a.rows = dst.data_ptr(), newpos.data_ptr(), src_of.data_ptr(), n_kept
        a.counts, a.pos_old = cnt.data_ptr(), pos_old.data_ptr()
        if tab is not None:
            a.cos_tab, a.sin_tab, a.table_rows = tab[0].data_ptr(), tab[1].data_ptr(), int(tab[0].shape[0])
        if out_sink is not None:
            a.out_sink_k, a.out_sink_v, a.cap_sink = out_sink[0].data_ptr(), out_sink[1].data_ptr(), n_sink_new
        if buf is not None:
            a.out_rec_k, a.out_rec_v = buf[0].data_ptr(), buf[1].data_ptr()
            a.out_rec_sb, a.out_rec_sh, a.out_rec_ss = buf[0].stride()[:3]
            a.cap_rec = n_rec_new
        colmax = None
        if mid is not None:
            a.out_mid_k, a.out_mid_v, a.cap_mid = mid[0].data_ptr(), mid[1].data_ptr(), n_int4
            # the gather also leaves the middle K's column absmax: one quantizer pass instead of two
            colmax = torch.zeros(B * H, _COLMAX_PARTS, D, dtype=torch.float32, device=dev)
            a.mid_colmax, a.colmax_parts = colmax.data_ptr(), _COLMAX_PARTS
        _lib.check(_lib.load().fade_reassign_gather(ctypes.byref(a), stream), "fade_reassign_gather")

        # new state (the same fields as the host path)
        if out_sink is not None:
            st.sink_k, st.sink_v, st.sink_pos = out_sink[0], out_sink[1], pos_new[0, :n_sink_new]
        else:
            st.sink_k = st.sink_v = st.sink_pos = None
        if buf is not None:
            bp = torch.empty(cap, dtype=torch.long, device=dev)
            bp[:n_rec_new] = pos_new[1, :n_rec_new]
            st._fp16_buf_k, st._fp16_buf_v, st._fp16_buf_pos = buf[0], buf[1], bp
            st._fp16_len = n_rec_new
            st.fp16_k, st.fp16_v, st.fp16_pos = buf[0][:, :, :n_rec_new], buf[1][:, :, :n_rec_new], bp[:n_rec_new]
        else:
            st.fp16_k = st.fp16_v = st.fp16_pos = None
            st._fp16_buf_k = st._fp16_buf_v = st._fp16_buf_pos = None
            st._fp16_len = 0
        if mid is not None:
            st.int4_kq, st.int4_ks = quant_k_int4_from_colmax(mid[0], colmax)
            if self.incremental_quant and old_v[0] is not None and tiers.device.type == "cpu":
                st.int4_vq, st.int4_vs = self._incremental_v(tiers, ns_old, nm_old, old_v, mid[1])
            else:
                st.int4_vq, st.int4_vs = quant_v_int4(mid[1])
            st.int4_pos = pos_new[2, :n_int4]
        else:
            st.int4_kq = st.int4_vq = st.int4_ks = st.int4_vs = st.int4_pos = None
        st.backend_k = st.backend_v = st.backend_pos = None
        st.int2_kq = st.int2_vq = st.int2_ks = st.int2_vs = st.int2_pos = None
        st.int2_actual_count = 0
        if n_kept < S:
            st.next_position = n_kept
        st.int4_k_deq = st.int4_v_deq = st.int2_k_deq = st.int2_v_deq = None
        st._compressed_bytes = self._layer_compressed_bytes(st)
        st.sink_count = n_sink_new
        self._last_reassign_counts = cnt
        self._check_status(cnt, 1)
        return True

    def apply_tier_assignment(
        self, layer_idx: int, tiers: Tensor, scores: Tensor | None = None, *, counts=None
    ) -> None:
        """Move tokens between tiers (fade/cache.py:881-1057).

        Evicted tokens are dropped; the survivors are re-RoPE'd from their
        old absolute positions to contiguous positions ``0..n_kept-1`` in
        one fused pass, then split into fp16 / INT4 / INT2 and requantized.

        Layers holding the reference INT4 layout on the GPU take the device
        path (``_apply_tier_assignment_device``, same results); ``counts`` =
        ``(n_fp16, n_int4, n_int2)`` of ``tiers``, when the caller knows them,
        spares the host sync a device ``tiers`` tensor would otherwise need.
        """
        del scores
        st = self._layers[layer_idx]
        if st.lens is not None:
            raise NotImplementedError("this layer holds the ragged layout: use apply_tier_assignment_per_sequence")
        if self._device_reassign_ok(st) and self._apply_tier_assignment_device(layer_idx, tiers, counts):
            return
        # per-token backend codes that an incremental reassignment may keep
        inc = None
        if self.incremental_quant and isinstance(self._quant_backend, AsymGroupBackend) \
                and st.backend_k is not None and st.int2_kq is None:
            ns_old = st.sink_pos.shape[0] if st.sink_k is not None else (st.sink_count if st.fp16_k is not None else 0)
            inc = (st.backend_k, st.backend_v, int(ns_old), int(st.backend_pos.shape[0]))
        k_full, v_full, pos_full = self._all_in_position_order(layer_idx)
        S = int(pos_full.shape[0])
        if int(tiers.shape[0]) != S:
            raise ValueError(f"tiers length {int(tiers.shape[0])} != cache length {S} for layer {layer_idx}")
        tiers_host = tiers.cpu() if inc is not None else None
        tiers = tiers.to(pos_full.device)
        keep = tiers != TIER_EVICT
        n_kept = int(keep.sum().item())
        keep_idx = None
        if n_kept < S:
            keep_idx = keep.nonzero(as_tuple=False).squeeze(-1)
            k_full, v_full, pos_full = self._rerope_kept(k_full, v_full, pos_full, keep_idx, n_kept)
            tiers = tiers[keep]
            st.next_position = n_kept

        fp16_idx = (tiers == TIER_FP16).nonzero(as_tuple=False).squeeze(-1)
        if fp16_idx.numel() > 0:
            fk, fv, fp = _sel(k_full, fp16_idx), _sel(v_full, fp16_idx), pos_full.index_select(0, fp16_idx)
            ns = min(self.n_sink, int(fp16_idx.numel()))
            if ns > 0:
                st.sink_k, st.sink_v, st.sink_pos = fk[..., :ns, :], fv[..., :ns, :], fp[:ns]
            else:
                st.sink_k = st.sink_v = st.sink_pos = None
            if ns < int(fp16_idx.numel()):
                st.fp16_k, st.fp16_v, st.fp16_pos = fk[..., ns:, :], fv[..., ns:, :], fp[ns:]
            else:
                st.fp16_k = st.fp16_v = st.fp16_pos = None
        else:
            st.fp16_k = st.fp16_v = st.fp16_pos = None
            st.sink_k = st.sink_v = st.sink_pos = None
        self._reseed_fp16_buffer(st)

        int4_idx = (tiers == TIER_INT4).nonzero(as_tuple=False).squeeze(-1)
        if int4_idx.numel() > 0 and inc is not None:
            # incremental (per-token backend): old middle tokens keep their codes (K only
            # when nothing was evicted: re-RoPE changes K), the others are compressed
            be = self._quant_backend
            kept_tiers = tiers_host if keep_idx is None else tiers_host[keep_idx.cpu()]
            slots, rows, fresh = self._middle_sources(kept_tiers, inc[2], inc[3], keep_idx)
            n = int(int4_idx.numel())
            fi = fresh.to(int4_idx.device)
            fv = be.compress_v(_sel(v_full, int4_idx.index_select(0, fi))) if fresh.numel() else None
            st.backend_v = self._merge_compressed(inc[1], fv, slots, rows, fresh, n)
            if keep_idx is None:
                fk = be.compress_k(_sel(k_full, int4_idx.index_select(0, fi))) if fresh.numel() else None
                st.backend_k = self._merge_compressed(inc[0], fk, slots, rows, fresh, n)
            else:
                st.backend_k = be.compress_k(_sel(k_full, int4_idx))
            st.backend_pos = pos_full.index_select(0, int4_idx)
            st.int4_kq = st.int4_vq = st.int4_ks = st.int4_vs = st.int4_pos = None
        elif int4_idx.numel() > 0:
            self._store_middle(st, _sel(k_full, int4_idx), _sel(v_full, int4_idx), pos_full.index_select(0, int4_idx))
        else:
            st.int4_kq = st.int4_vq = st.int4_ks = st.int4_vs = st.int4_pos = None
            st.backend_k = st.backend_v = st.backend_pos = None

        int2_idx = (tiers == TIER_INT2).nonzero(as_tuple=False).squeeze(-1)
        if int2_idx.numel() > 0:
            g = DEFAULT_INT2_GROUP_SIZE
            st.int2_kq, st.int2_ks = quant_int2_padded(_sel(k_full, int2_idx), g)
            st.int2_vq, st.int2_vs = quant_int2_padded(_sel(v_full, int2_idx), g)
            st.int2_pos = pos_full.index_select(0, int2_idx)
            st.int2_actual_count = int(int2_idx.numel())
            st.int2_group_size = g
        else:
            st.int2_kq = st.int2_vq = st.int2_ks = st.int2_vs = st.int2_pos = None
            st.int2_actual_count = 0
        if bool((tiers == TIER_PQ).any()):
            raise RuntimeError("TIER_PQ is not supported by fade_amd (no product-quantization tier)")

        st.int4_k_deq = st.int4_v_deq = st.int2_k_deq = st.int2_v_deq = None
        st._compressed_bytes = self._layer_compressed_bytes(st)
        st.sink_count = 0 if st.sink_pos is None else int(st.sink_pos.shape[0])

    def _apply_per_sequence_ragged(self, layer_idx: int, tiers_per_row: Tensor) -> None:
        """Per-row tiers ``[B, S]`` into the ragged layout: each row keeps exactly its own
        tokens (per-row tier lengths in ``LayerState.lens``), re-RoPE'd to positions
        0..n_kept-1 where it evicted.  One plan per row (``fade_reassign_plan``), one
        gather of every row's kept tokens (``fade_reassign_gather``), then the INT4
        quantizers over the zero-padded middle (per (row, head) channel scales over
        the row's own tokens)."""
        st = self._layers[layer_idx]
        if not isinstance(self._quant_backend, SymmetricINT4Backend) or self.middle_v_bits != 4 \
                or st.int2_kq is not None or st.backend_k is not None:
            raise NotImplementedError("ragged_layout: the reference INT4 middle tier only (no INT2 tier / backend)")
        if self.dtype != torch.float16:
            raise NotImplementedError(f"ragged_layout: float16 caches only, this one is {self.dtype}")
        midp = self._mid_padded(st)  # a paged middle is read back as the padded tensors
        if st.lens is None:
            if st.sink_k is not None:
                sink, rec_start = (st.sink_k, st.sink_v), 0
            else:
                nsk = st.sink_count if st.fp16_k is not None else 0
                sink = (st.fp16_k[..., :nsk, :], st.fp16_v[..., :nsk, :]) if nsk > 0 else None
                rec_start = nsk
            rec = None
            if st.fp16_k is not None and rec_start < int(st.fp16_k.shape[-2]):
                rec = (st.fp16_k[..., rec_start:, :], st.fp16_v[..., rec_start:, :])
            ns_c = 0 if sink is None else int(sink[0].shape[-2])
            nm_c = 0 if midp is None else int(midp[0].shape[-2])
            nr_c = 0 if rec is None else int(rec[0].shape[-2])
            pos_parts = [p for p in (
                None if sink is None else (st.sink_pos if st.sink_k is not None else st.fp16_pos[:ns_c]),
                st.int4_pos, None if rec is None else st.fp16_pos[rec_start:],
            ) if p is not None]
            pos_old = torch.cat(pos_parts).to(torch.long).contiguous()
            # The reference's zero-padded per-sequence layout keeps row 0's positions
            # (fade/cache.py:1161-1167), fewer than the padded rows where row 0 is not the
            # longest.  Its next reassignment indexes the concatenated tiers by position
            # index, so token j is row j of sink | middle | recent with position pos_old[j]
            # (fade/cache.py:701-713,1084,1124-1133); the gather maps j the same way.
            S = int(pos_old.shape[0])
            if S > ns_c + nm_c + nr_c:
                raise ValueError(f"layer {layer_idx}: {S} positions for {ns_c + nm_c + nr_c} rows")
            table_rows = st.next_position
            row_len = None
        else:
            sink = None if st.sink_k is None else (st.sink_k, st.sink_v)
            rec = None if st.fp16_k is None else (st.fp16_k, st.fp16_v)
            ns_c = 0 if sink is None else int(sink[0].shape[-2])
            nm_c = 0 if midp is None else int(midp[0].shape[-2])
            nr_c = 0 if rec is None else int(rec[0].shape[-2])
            row_len = [sum(r) for r in st.lens_host]
            S = max(row_len)
            table_rows = S
        mkq = None if midp is None else midp[0]
        ref = next(t for t in (None if sink is None else sink[0], None if rec is None else rec[0], mkq)
                   if t is not None)
        B, H = int(ref.shape[0]), int(ref.shape[1])
        D = 2 * int(ref.shape[-1]) if ref is mkq else int(ref.shape[-1])
        dev = ref.device
        if st.lens is not None:
            pos_old = torch.arange(max(S, 1), dtype=torch.long, device=dev)
        if tiers_per_row.dim() != 2 or tiers_per_row.shape[0] != B:
            raise ValueError(f"tiers_per_row must be [B={B}, S={S}], got {tuple(tiers_per_row.shape)}")
        if tiers_per_row.shape[1] != S:
            raise ValueError(f"tiers_per_row S dim {tiers_per_row.shape[1]} != cache length {S}")
        rows_counts = None
        if tiers_per_row.device.type == "cpu":
            t = tiers_per_row.to(torch.long)
            rows_counts = []
            for b in range(B):
                if row_len is not None and bool((t[b, row_len[b]:] != TIER_EVICT).any()):
                    raise ValueError(f"row {b} has {row_len[b]} tokens; tiers past them must be TIER_EVICT")
                c = self._host_tier_counts(t[b])
                if c is None or c[2] > 0:
                    raise NotImplementedError("ragged_layout: tiers must be FP16, INT4 or EVICT")
                rows_counts.append(c)
        tiers_d = tiers_per_row.to(dtype=torch.long).contiguous()
        if tiers_d.device != dev:
            tiers_d = (tiers_d.pin_memory() if tiers_d.device.type == "cpu" else tiers_d).to(dev, non_blocking=True)
        i32 = dict(dtype=torch.int32, device=dev)
        dst, newpos, src_of = (torch.empty(B, max(S, 1), **i32) for _ in range(3))
        pos_new = torch.empty(3, B, max(S, 1), dtype=torch.long, device=dev)
        cnt = torch.empty(B, 4, **i32)
        stream = _lib.stream_of(tiers_d)
        _lib.call("fade_reassign_plan", tiers_d.data_ptr(), S, B, S, self.n_sink, pos_old.data_ptr(), 0,
                  dst.data_ptr(), newpos.data_ptr(), src_of.data_ptr(), pos_new[0].data_ptr(),
                  pos_new[1].data_ptr(), pos_new[2].data_ptr(), cnt.data_ptr(), stream)
        if rows_counts is None:
            c = cnt.cpu().tolist()  # device tiers: one read of the per-row counts
            if any(r[3] & 3 for r in c):
                raise NotImplementedError("ragged_layout: tiers must be FP16, INT4 or EVICT")
            rows_counts = [(r[0], r[1], 0) for r in c]
        new_lens = [[min(self.n_sink, f), i4, f - min(self.n_sink, f)] for f, i4, _ in rows_counts]
        cs = max(r[0] for r in new_lens)
        cm = max(r[1] for r in new_lens)
        cr = max(r[2] for r in new_lens)
        pool = self.page_pool
        if pool is not None:  # refuse before any state changes
            if (pool.n_kv_heads, pool.head_dim) != (H, D):
                raise ValueError(f"page pool holds {pool.n_kv_heads} KV heads x {pool.head_dim}, the layer {H} x {D}")
            need = sum(-(-r[1] // PAGE_TOKENS) for r in new_lens)
            held = 0 if st.mid_pool is not pool else sum(len(r) for r in st.mid_pages)
            if need > pool.n_free + held:
                raise RuntimeError(f"page pool exhausted: layer {layer_idx} needs {need} pages, "
                                   f"{pool.n_free + held} available")
        kd = dict(dtype=torch.float16, device=dev)
        out_sink = (torch.zeros(B, H, cs, D, **kd), torch.zeros(B, H, cs, D, **kd)) if cs else None
        cap = max(DEFAULT_FP16_PREALLOC, cr)
        buf = (torch.zeros(B, H, cap, D, **kd), torch.zeros(B, H, cap, D, **kd))
        mid = (torch.zeros(B, H, cm, D, **kd), torch.zeros(B, H, cm, D, **kd)) if cm else None
        evicting = any(f + i4 < (S if row_len is None else row_len[b]) for b, (f, i4, _) in enumerate(rows_counts))
        if evicting and row_len is None and S != ns_c + nm_c + nr_c:
            # the reference un-RoPEs the padded rows with the S positions' tables, which
            # fails on the shapes (fade/cache.py:1108-1110); the host path raises as well
            raise NotImplementedError("eviction over a zero-padded layout whose positions are row 0's")
        tab = self._rope_tables(max(table_rows, S), dev) if evicting else None
        src_lens = st.lens

        def cf(tt):
            return tt if tt[0].stride() == tt[1].stride() else (tt[0].contiguous(), tt[1].contiguous())

        sink = None if sink is None else cf(sink)
        rec = None if rec is None else cf(rec)
        a = _lib.ReassignArgs()
        a.B, a.H, a.D, a.S = B, H, D, S
        a.n_sink_old, a.n_mid_old, a.n_rec_cap = ns_c, nm_c, nr_c
        a.src_lens, a.plan_rows, a.pos_old_rs = _lib.ptr(src_lens), B, 0
        if sink is not None:
            a.sink_k, a.sink_v = sink[0].data_ptr(), sink[1].data_ptr()
            a.sink_sb, a.sink_sh, a.sink_ss = sink[0].stride()[:3]
        if nm_c:
            mids = [t.contiguous() for t in midp]
            a.mid_kq, a.mid_ks, a.mid_vq, a.mid_vs = (t.data_ptr() for t in mids)
        if rec is not None:
            a.rec_k, a.rec_v = rec[0].data_ptr(), rec[1].data_ptr()
            a.rec_sb, a.rec_sh, a.rec_ss = rec[0].stride()[:3]
        a.dst, a.newpos, a.src_of, a.rows = dst.data_ptr(), newpos.data_ptr(), src_of.data_ptr(), S
        a.counts, a.pos_old = cnt.data_ptr(), pos_old.data_ptr()
        if tab is not None:
            a.cos_tab, a.sin_tab, a.table_rows = tab[0].data_ptr(), tab[1].data_ptr(), int(tab[0].shape[0])
        if out_sink is not None:
            a.out_sink_k, a.out_sink_v, a.cap_sink = out_sink[0].data_ptr(), out_sink[1].data_ptr(), cs
        a.out_rec_k, a.out_rec_v = buf[0].data_ptr(), buf[1].data_ptr()
        a.out_rec_sb, a.out_rec_sh, a.out_rec_ss = buf[0].stride()[:3]
        a.cap_rec = cap
        colmax = None
        if mid is not None:
            a.out_mid_k, a.out_mid_v, a.cap_mid = mid[0].data_ptr(), mid[1].data_ptr(), cm
            colmax = torch.zeros(B * H, _COLMAX_PARTS, D, dtype=torch.float32, device=dev)
            a.mid_colmax, a.colmax_parts = colmax.data_ptr(), _COLMAX_PARTS
        _lib.check(_lib.load().fade_reassign_gather(ctypes.byref(a), stream), "fade_reassign_gather")

        st.sink_k, st.sink_v = (out_sink[0], out_sink[1]) if out_sink is not None else (None, None)
        st._fp16_buf_k, st._fp16_buf_v, st._fp16_buf_pos = buf[0], buf[1], None
        st._fp16_len = cr
        st.fp16_k, st.fp16_v = buf[0][:, :, :cr], buf[1][:, :, :cr]
        if mid is not None:
            st.int4_kq, st.int4_ks = quant_k_int4_from_colmax(mid[0], colmax)
            st.int4_vq, st.int4_vs = quant_v_int4(mid[1])
        else:
            st.int4_kq = st.int4_vq = st.int4_ks = st.int4_vs = None
        # the old pages were read above (stream order), so they can be handed out again
        self._release_layer_pages(st)
        if pool is not None and st.int4_kq is not None:
            st.mid_table, st.mid_pages = pool.store(st.int4_kq, st.int4_vq, st.int4_vs, [r[1] for r in new_lens])
            st.mid_pool = pool
            st.mid_page_bytes = pool.page_bytes * sum(len(r) for r in st.mid_pages)
            st.int4_kq = st.int4_vq = st.int4_vs = None
        st.sink_pos = st.fp16_pos = st.int4_pos = None
        st.backend_k = st.backend_v = st.backend_pos = None
        st.int2_kq = st.int2_vq = st.int2_ks = st.int2_vs = st.int2_pos = None
        st.int2_actual_count = 0
        st.lens = torch.tensor(new_lens, dtype=torch.int32).pin_memory().to(dev, non_blocking=True)
        st.lens_host = new_lens
        st.next_position = st.total_seq_length()
        st.sink_count = cs
        st.int4_k_deq = st.int4_v_deq = st.int2_k_deq = st.int2_v_deq = None
        st._compressed_bytes = self._layer_compressed_bytes(st)
        self._last_reassign_counts = cnt
        self._check_status(cnt, B)
        return pos_new

    def _apply_per_sequence_device(self, layer_idx: int, tiers_per_row: Tensor) -> bool:
        """The reference's per-sequence mode (rows zero-padded to the longest,
        fade/cache.py:1059-1230) through the device reassignment: one plan of every row
        and one gather of their kept tokens (``_apply_per_sequence_ragged``), then the
        per-row tiers laid out as the reference pads them: FP16 tier = each row's
        FP16 tokens in position order, middle codes as quantized over the zero-padded
        rows, positions of row 0, fields the reference leaves alone left alone.
        Returns False, with the layer untouched, where it does not apply (another
        middle format or backend, an INT2 tier, tiers other than FP16 / INT4 / EVICT)."""
        st = self._layers[layer_idx]
        if (self.dtype != torch.float16 or not isinstance(self._quant_backend, SymmetricINT4Backend) or self.middle_v_bits != 4
                or st.int2_kq is not None or st.backend_k is not None or st.lens is not None
                or self.page_pool is not None):
            return False
        kept = {f: getattr(st, f) for f in ("sink_k", "sink_v", "sink_pos", "_fp16_buf_k", "_fp16_buf_v",
                                            "_fp16_buf_pos", "_fp16_len", "_compressed_bytes")}
        try:
            pos_new = self._apply_per_sequence_ragged(layer_idx, tiers_per_row)
        except NotImplementedError:
            return False
        lh = st.lens_host
        B = len(lh)
        sink = None if st.sink_k is None else (st.sink_k, st.sink_v)
        rec = (st.fp16_k, st.fp16_v)
        H, D = int(rec[0].shape[1]), int(rec[0].shape[-1])
        dev = rec[0].device
        cs = 0 if sink is None else int(sink[0].shape[-2])
        cr = int(rec[0].shape[-2])
        nf = max(ls + lr for ls, _, lr in lh)
        fk = fv = fpos = None
        if nf:
            # row b's FP16 tier: its sink tokens, then its recent ones, zero-padded
            zero = torch.zeros(B, H, 1, D, dtype=rec[0].dtype, device=dev)
            allk = torch.cat(([sink[0]] if sink else []) + [rec[0], zero], dim=2)
            allv = torch.cat(([sink[1]] if sink else []) + [rec[1], zero], dim=2)
            idx = torch.full((B, nf), cs + cr, dtype=torch.long)
            for b, (ls, _, lr) in enumerate(lh):
                idx[b, :ls] = torch.arange(ls)
                idx[b, ls : ls + lr] = cs + torch.arange(lr)
            idx = idx.pin_memory().to(dev, non_blocking=True)
            rows = torch.arange(B, device=dev)[:, None]
            fk = allk[rows, :, idx].permute(0, 2, 1, 3).contiguous()
            fv = allv[rows, :, idx].permute(0, 2, 1, 3).contiguous()
            ls0, _, lr0 = lh[0]
            fpos = torch.cat([pos_new[0, 0, :ls0], pos_new[1, 0, :lr0]])
        ls0, lm0, _ = lh[0]
        ipos = pos_new[2, 0, :lm0] if st.int4_kq is not None else None
        min_next = min(sum(r) for r in lh)
        for f, val in kept.items():
            setattr(st, f, val)
        st.lens = st.lens_host = None
        st.fp16_k, st.fp16_v, st.fp16_pos = fk, fv, fpos
        self._reseed_fp16_buffer(st)
        st.int4_pos = ipos
        st.int2_kq = st.int2_vq = st.int2_ks = st.int2_vs = st.int2_pos = None
        st.int2_actual_count = 0
        st.int4_k_deq = st.int4_v_deq = st.int2_k_deq = st.int2_v_deq = None
        st.next_position = min_next
        st.sink_count = 0 if st.fp16_pos is None else min(self.n_sink, int(st.fp16_pos.shape[0]))
        st._padded_rows = True
        return True

    def apply_tier_assignment_per_sequence(self, layer_idx: int, tiers_per_row: Tensor, scores=None) -> None:
        """Per-row tiers ``[B, S]`` with zero-padding to the longest row (fade/cache.py:1059-1230).

        With ``ragged_layout`` set, rows keep exactly their own tokens instead
        (``_apply_per_sequence_ragged``) and attention reads only those."""
        del scores
        if self.ragged_layout:
            self._apply_per_sequence_ragged(layer_idx, tiers_per_row)
            return
        st = self._layers[layer_idx]
        if st.lens is not None:
            raise NotImplementedError("this layer holds the ragged layout; set ragged_layout to reassign it")
        if self.device_reassign and self._apply_per_sequence_device(layer_idx, tiers_per_row):
            return
        k_full, v_full, pos_full = self._all_in_position_order(layer_idx)
        B, H, _, D = k_full.shape
        S = int(pos_full.shape[0])
        if tiers_per_row.dim() != 2 or tiers_per_row.shape[0] != B:
            raise ValueError(f"tiers_per_row must be [B={B}, S={S}], got {tuple(tiers_per_row.shape)}")
        if tiers_per_row.shape[1] != S:
            raise ValueError(f"tiers_per_row S dim {tiers_per_row.shape[1]} != cache length {S}")
        dev = k_full.device
        tiers_per_row = tiers_per_row.to(dev)
        rows = {"fk": [], "fv": [], "fp": [], "ik": [], "iv": [], "ip": []}
        min_next = S
        for b in range(B):
            rt = tiers_per_row[b]
            rk, rv, rp = k_full[b : b + 1], v_full[b : b + 1], pos_full
            keep = rt != TIER_EVICT
            n_kept = int(keep.sum().item())
            if n_kept < S:
                keep_idx = keep.nonzero(as_tuple=False).squeeze(-1)
                rk, rv, rp = self._rerope_kept(rk, rv, pos_full, keep_idx, n_kept)
                rt = rt[keep]
                min_next = min(min_next, n_kept)
            for tier, kk, vk, pk in ((TIER_FP16, "fk", "fv", "fp"), (TIER_INT4, "ik", "iv", "ip")):
                idx = (rt == tier).nonzero(as_tuple=False).squeeze(-1)
                rows[kk].append(rk.index_select(-2, idx))
                rows[vk].append(rv.index_select(-2, idx))
                rows[pk].append(rp[idx])

        def pad_stack(lst):
            n = max(int(r.shape[-2]) for r in lst)
            if n == 0:
                return None
            out = torch.zeros(B, H, n, D, dtype=lst[0].dtype, device=dev)
            for b, r in enumerate(lst):
                out[b : b + 1, :, : r.shape[-2]] = r
            return out

        def first_pos(lst):
            n = max(int(r.shape[0]) for r in lst)
            return None if n == 0 else lst[0][:n]

        fk = pad_stack(rows["fk"])
        if fk is not None:
            st.fp16_k, st.fp16_v, st.fp16_pos = fk, pad_stack(rows["fv"]), first_pos(rows["fp"])
        else:
            st.fp16_k = st.fp16_v = st.fp16_pos = None
        self._reseed_fp16_buffer(st)
        ik = pad_stack(rows["ik"])
        if ik is not None:
            iv = pad_stack(rows["iv"])
            st.int4_kq, st.int4_ks = quant_k_int4(ik)
            if self.middle_v_bits == 4:
                st.int4_vq, st.int4_vs = quant_v_int4(iv)
            else:
                st.int4_vq, st.int4_vs = quant_int2_padded(iv, DEFAULT_INT2_GROUP_SIZE)
            st.int4_pos = first_pos(rows["ip"])
        else:
            st.int4_kq = st.int4_vq = st.int4_ks = st.int4_vs = st.int4_pos = None
        st.int2_kq = st.int2_vq = st.int2_ks = st.int2_vs = st.int2_pos = None
        st.int2_actual_count = 0
        st.int4_k_deq = st.int4_v_deq = st.int2_k_deq = st.int2_v_deq = None
        st.next_position = min_next
        st.sink_count = 0 if st.fp16_pos is None else min(self.n_sink, int(st.fp16_pos.shape[0]))
        st._padded_rows = True

    # ----------------------------------------------------- fused attention
    def attend(self, q: Tensor, layer_idx: int, sm_scale: float | None = None) -> Tensor:
        """Attention of ``q`` [B, Hq, Sq, D] over this layer's tiers (the ``"fade"``
        attention implementation): one token per row -> ``decode_attention``; a
        chunk -> ``prefill_attention``.  Returns fp16 [B, Hq, Sq, D]."""
        if int(q.shape[2]) == 1:
            return self.decode_attention(q, layer_idx, sm_scale)
        return self.prefill_attention(q, layer_idx, sm_scale)

    def _fp16_split(self, st: LayerState):
        """(sink, rest) fp16 K/V pairs of a layer, whether or not the sink has been split off."""
        if st.sink_k is not None:
            return (st.sink_k, st.sink_v), (None if st.fp16_k is None else (st.fp16_k, st.fp16_v))
        if st.fp16_k is None:
            return None, None
        ns = st.sink_count
        sink = (st.fp16_k[..., :ns, :], st.fp16_v[..., :ns, :]) if ns > 0 else None
        return sink, (st.fp16_k[..., ns:, :], st.fp16_v[..., ns:, :])

    def _require_f16_tiers(self, op: str) -> None:
        if self.dtype not in _FUSED_DTYPES:
            raise NotImplementedError(
                f"{op}: the tiered attention kernels read float16 and bfloat16 tiers; this cache is {self.dtype} "
                "(attend over the materialized K/V instead)"
            )

    def prefill_attention(self, q: Tensor, layer_idx: int, sm_scale: float | None = None) -> Tensor:
        """Causal attention of a chunk ``q`` [B, Hq, Sq, D] whose K/V are the last Sq
        tokens of this layer's fp16 tier (just appended by ``update``), over
        ``[sink (+ INT2 tier) | middle | recent | chunk]`` with the ragged prefill kernel.
        The reference INT4 middle tier is read in place; the other middle formats
        through their fp16 dequantization, kept between chunks."""
        from .kernels.prefill import tiered_prefill_attention
        from .kernels.tiered_attn import MiddleTier

        self._require_f16_tiers("prefill_attention")
        st = self._layers[layer_idx]
        if st.lens is not None:
            return self._prefill_attention_ragged(q, st, sm_scale)
        Sq = int(q.shape[2])
        sink, rest = self._fp16_split(st)
        if rest is None or int(rest[0].shape[-2]) < Sq:
            raise RuntimeError("prefill_attention: the chunk's K/V must be the last Sq tokens of the fp16 tier")
        n_rest = int(rest[0].shape[-2]) - Sq
        recent = None if n_rest == 0 else (rest[0][..., :n_rest, :], rest[1][..., :n_rest, :])
        chunk = (rest[0][..., n_rest:, :], rest[1][..., n_rest:, :])
        sink = self._front_tier(st, sink)
        mid = None
        if st.int4_kq is not None and self.middle_v_bits == 4 and int(q.shape[-1]) % 32 == 0:
            mid = MiddleTier("int4", st.int4_kq, st.int4_vq, st.int4_ks, st.int4_vs)
        elif st.int4_kq is not None or st.backend_k is not None:  # (packed rows in place need head_dim % 32)
            mk, mv = self._mid_fp16(st)
            mid = MiddleTier("fp16", mk, mv)
        return tiered_prefill_attention(q, chunk, sink, mid, recent, sm_scale=sm_scale)

    def _prefill_attention_ragged(self, q: Tensor, st: LayerState, sm_scale: float | None) -> Tensor:
        """``prefill_attention`` on a ragged layer: row b's chunk is the last Sq tokens of
        its own recent tier (where ``update`` appended them), at a different offset in
        every row.  Those rows are gathered into the chunk tensor; the kernel reads the
        padded tiers with the row's sink / middle / recent lengths, recent minus Sq."""
        from .kernels.prefill import tiered_prefill_attention
        from .kernels.tiered_attn import MiddleTier

        Sq = int(q.shape[2])
        if st.fp16_k is None or min(r[2] for r in st.lens_host) < Sq:
            raise RuntimeError("prefill_attention: the chunk's K/V must be the last Sq tokens of every row's recent tier")
        if st.int2_kq is not None or st.backend_k is not None or (st.int4_kq is not None and self.middle_v_bits != 4):
            raise NotImplementedError(
                "prefill_attention: the fused prefill reads fp16 tiers and the reference INT4 middle tier only"
            )
        B = int(q.shape[0])
        rows = torch.arange(B, device=q.device)[:, None]
        idx = (st.lens[:, 2].long() - Sq)[:, None] + torch.arange(Sq, device=q.device)[None, :]
        chunk = (st.fp16_k[rows, :, idx].permute(0, 2, 1, 3).contiguous(),
                 st.fp16_v[rows, :, idx].permute(0, 2, 1, 3).contiguous())
        lens = st.lens.clone()
        lens[:, 2] -= Sq
        sink = None if st.sink_k is None else (st.sink_k, st.sink_v)
        if st.mid_table is not None:  # paged: the kernel reads the pool through the block table
            pool = st.mid_pool
            mid = MiddleTier("int4", pool.k_codes, pool.v_codes, st.int4_ks, pool.v_scale,
                             length=max(r[1] for r in st.lens_host), pages=st.mid_table)
        else:
            midp = self._mid_padded(st)
            mid = None if midp is None else MiddleTier("int4", midp[0], midp[2], midp[1], midp[3])
        # rows dispatched longest first, so the longest rows do not form the tail
        order = sorted(range(B), key=lambda r: -sum(st.lens_host[r]))
        order = torch.tensor(order, dtype=torch.int32).pin_memory().to(q.device, non_blocking=True)
        return tiered_prefill_attention(q, chunk, sink, mid, (st.fp16_k, st.fp16_v), lens=lens, order=order,
                                        sm_scale=sm_scale)

    def _front_tier(self, st: LayerState, sink):
        """The fp16 tier the fused kernels read first: the sink, followed by the INT2
        tier's fp16 dequantization (fade/cache.py:861-876) when the layer has one.
        Attention over the cache is a softmax over a set of keys, so where the INT2
        tokens sit among the cache tokens does not change it.  The joined tensors are
        kept until the sink or the INT2 tier changes."""
        if st.int2_kq is None:
            return sink
        k2, v2 = self._get_int2_dequant(st)
        c = st._front_cache
        sk = None if sink is None else sink[0]
        if c is not None and c[0] is sk and c[1] is k2:
            return c[2], c[3]
        if sink is None:
            fk, fv = k2.contiguous(), v2.contiguous()
        else:
            fk, fv = torch.cat([sink[0], k2], dim=-2), torch.cat([sink[1], v2], dim=-2)
        st._front_cache = (sk, k2, fk, fv)
        return fk, fv

    def _mid_fp16(self, st: LayerState):
        """The middle tier as fp16 rows for the chunk prefill of middle formats the
        prefill kernel does not read in place (K4 + literal INT2 V, backend-compressed
        tiers): the reference's own dequantization (fade/cache.py:758-763,810-842), kept
        until the middle tier changes."""
        if st.int4_kq is not None:
            k, v = self._get_int4_dequant(st)
            src = st.int4_kq
        else:
            src = st.backend_k["packed"]
            c = st._mid_f16_cache
            if c is not None and c[0] is src:
                return c[1], c[2]
            k = self._quant_backend.decompress_k(st.backend_k, dtype=self.dtype)
            v = self._quant_backend.decompress_v(st.backend_v, dtype=self.dtype)
            st._mid_f16_cache = (src, k, v)
        return k.contiguous(), v.contiguous()

    def decode_attention(self, q: Tensor, layer_idx: int, sm_scale: float | None = None) -> Tensor:
        """Single-token attention of ``q`` [B, Hq, 1, D] straight from this layer's tiers.

        Covers the layouts the fused kernel reads in place: sink + recent fp16
        with an INT4 (reference format), INT4-K/INT2-V, rotated or
        asymmetric middle tier.  An INT2 tier (``int2_budget > 0``) is read as
        its fp16 dequantization joined to the sink, kept between calls.
        """
        from .kernels.tiered_attn import MiddleTier, TieredDecodePlan, tiered_decode_attention

        self._require_f16_tiers("decode_attention")
        st = self._layers[layer_idx]
        if st.lens is not None:
            if st.mid_table is not None:  # paged: the kernel reads the pool through the block table
                pool = st.mid_pool
                mid = MiddleTier("int4", pool.k_codes, pool.v_codes, st.int4_ks, pool.v_scale,
                                 length=max(r[1] for r in st.lens_host), pages=st.mid_table)
            elif st.int4_kq is not None:
                mid = MiddleTier("int4", st.int4_kq, st.int4_vq, st.int4_ks, st.int4_vs)
            else:  # the ragged kernel needs a middle format: one zero row no row reads (lens 0)
                B, H = int(q.shape[0]), int((st.fp16_k if st.fp16_k is not None else st.sink_k).shape[1])
                D = int(q.shape[-1])
                z8 = torch.zeros(B, H, 1, D // 2, dtype=torch.uint8, device=q.device)
                mid = MiddleTier("int4", z8, z8.clone(), torch.zeros(B, H, 1, D, dtype=self.dtype, device=q.device),
                                 torch.zeros(B, H, 1, 1, dtype=self.dtype, device=q.device))
            sink = None if st.sink_k is None else (st.sink_k, st.sink_v)
            recent = None if st.fp16_k is None or st.fp16_k.shape[-2] == 0 else (st.fp16_k, st.fp16_v)
            return tiered_decode_attention(q, sink, mid, recent, sm_scale, n_splits=self.decode_splits, lens=st.lens)
        # the recent tier's current length (the one field that moves from step to step)
        n_rec = 0 if st.fp16_k is None else int(st.fp16_k.shape[-2]) - (0 if st.sink_k is not None else st.sink_count)
        stream = _lib.current_stream_handle(q.device)
        key = self._decode_key(st, q, sm_scale, n_rec > 0, stream)
        cached = st._decode_plan
        if cached is not None and _same_key(cached[0], key):
            return cached[1].rerun(q, n_rec, stream)
        if st.sink_k is not None:
            sink = (st.sink_k, st.sink_v)
            recent = None if st.fp16_k is None else (st.fp16_k, st.fp16_v)
        elif st.fp16_k is not None:
            ns = st.sink_count
            sink = (st.fp16_k[..., :ns, :], st.fp16_v[..., :ns, :]) if ns > 0 else None
            recent = (st.fp16_k[..., ns:, :], st.fp16_v[..., ns:, :])
        else:
            sink = recent = None
        sink = self._front_tier(st, sink)
        mid = None
        rotation = None
        if st.int4_kq is not None:
            if self.middle_v_bits == 4:
                mid = MiddleTier("int4", st.int4_kq, st.int4_vq, st.int4_ks, st.int4_vs)
            else:
                mid = MiddleTier(
                    "k4v2", st.int4_kq, st.int4_vq, st.int4_ks, st.int4_vs,
                    group=DEFAULT_INT2_GROUP_SIZE, length=int(st.int4_pos.shape[0]),
                )
        elif st.backend_k is not None:
            be = self._quant_backend
            bk, bv = st.backend_k, st.backend_v
            if isinstance(be, RotatedINT4Backend) and (be.bits == 3 or int(q.shape[-1]) != 128):
                # the in-kernel rotation is the INT4 kernel's (4- and 2-bit codes, head_dim 128);
                # otherwise the middle is read through its fp16 dequantization, kept between calls
                mk, mv = self._mid_fp16(st)
                mid = MiddleTier("fp16", mk, mv)
            elif isinstance(be, RotatedINT4Backend):
                # the kernel scores the middle with q R^T and un-rotates its part of the output
                rotation = be._get_R(q.device)
                mid = MiddleTier(
                    "sym", bk["packed"], bv["packed"], bk["scale"].to(self.dtype),
                    bv["scale"].to(self.dtype), k_bits=be.bits, v_bits=be.bits,
                )
            elif isinstance(be, AsymGroupBackend):
                mid = MiddleTier(
                    "asym", bk["packed"], bv["packed"], bk["scale"], bv["scale"], bk["zero"], bv["zero"],
                    k_bits=be.bits, v_bits=be.value_bits, group=be.group,
                )
            else:
                raise RuntimeError(f"decode_attention: backend {be.name} is not read by the fused kernel")
        plan = TieredDecodePlan(q, sink, mid, recent if n_rec > 0 else None, sm_scale, n_splits=self.decode_splits,
                                stream=stream, rotation=rotation)
        st._decode_plan = (key, plan)
        return plan.run(stream)

    def _decode_key(self, st: LayerState, q: Tensor, sm_scale, has_recent: bool, stream: int) -> tuple:
        """What a decode plan of this layer depends on: the tier tensors (as
        objects: a reassignment or a grown fp16 buffer replaces them), the query's
        layout and the call's settings; the recent tier's length is set per call."""
        return (st.sink_k, st.sink_v, st._fp16_buf_k, st._fp16_buf_v,
                st.fp16_k if st._fp16_buf_k is None else None, st.sink_count, has_recent,
                st.int4_kq, st.int4_vq, st.int4_ks, st.int4_vs, st.backend_k, st.backend_v,
                st.int2_kq, st.int2_vq, st.int2_ks, st.int2_vs,
                tuple(q.shape), q.stride(), q.device, q.dtype, sm_scale, self.decode_splits, self.middle_v_bits,
                self._quant_backend, torch.are_deterministic_algorithms_enabled(), stream)


# cache dtypes the fused attention kernels read
_FUSED_DTYPES = (torch.float16, torch.bfloat16)


def _same_key(a: tuple, b: tuple) -> bool:
    """Tensors, dicts and backends compare by identity; plain values by equality."""
    if len(a) != len(b):
        return False
    for x, y in zip(a, b):
        if x is y:
            continue
        if type(x) is not type(y) or type(x) not in _KEY_VALUE_TYPES or x != y:
            return False
    return True


_KEY_VALUE_TYPES = (int, float, bool, str, tuple, torch.device, torch.dtype)


__all__ = [
    "LayerState",
    "TIER_EVICT",
    "TIER_FP16",
    "TIER_INT2",
    "TIER_INT4",
    "TIER_PQ",
    "TieredKVCache",
]
