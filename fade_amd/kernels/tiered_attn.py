"""Fused decode attention over the tiered cache (sink fp16 | packed middle | recent fp16).

The reference never fuses the tiers: every decode step dequantizes the
middle tier, ``torch.cat``s sink | middle | recent into fresh fp16 K/V and
runs SDPA (fade/cache.py:683-842).  ``tiered_decode_attention`` reads the
packed middle tier in place through ``fade_tiered_decode_attn``.

``TieredDecodePlan`` binds the tensors once and re-launches with a single
C call, which is what the decode loop (and the benchmark) uses.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch
from torch import Tensor

from .. import _lib

_FMT = {
    "fp16": _lib.MID_FP16,
    "int4": _lib.MID_SYM,
    "sym": _lib.MID_SYM,
    "k4v2": _lib.MID_K4V2G,
    "asym": _lib.MID_ASYM,
}


@dataclass
class MiddleTier:
    """Packed middle tier in one of the formats of ``include/fade_hip.h``.

    fmt ``"int4"``/``"sym"``: ``k_codes``/``v_codes`` [B,Hkv,S,D*bits/8] u8,
    ``k_scale`` [B,Hkv,1,D], ``v_scale`` [B,Hkv,S,1] (fp16).
    fmt ``"k4v2"``: INT4 K as above; ``v_codes`` int8 [B,Hkv,S_pad,D] and
    ``v_scale`` [B,Hkv,S_pad/group,D] (reference INT2-V, fade/cache.py:983-988).
    fmt ``"asym"``: codes [B,Hkv,S,D*bits/8], scale/zero [B,Hkv,S,D/group].
    fmt ``"fp16"``: ``k_codes``/``v_codes`` fp16 [B,Hkv,S,D].

    Paged (``"int4"``/``"sym"``/``"asym"``): ``pages`` int32 [B, pages_per_row]
    holds the page of each 64-token tile of a row, and every per-token tensor is
    a pool [n_pages, Hkv, 64, ...] (``paginate_middle`` builds one); ``length``
    is the longest row's middle.  Decode reads every paged format; the chunk
    prefill reads a paged reference INT4 tier (separate pools, no page_stride).
    """

    fmt: str
    k_codes: Tensor
    v_codes: Tensor
    k_scale: Tensor | None = None
    v_scale: Tensor | None = None
    k_zero: Tensor | None = None
    v_zero: Tensor | None = None
    k_bits: int = 4
    v_bits: int = 4
    group: int = 64
    length: int | None = None
    pages: Tensor | None = None
    page_stride: int = 0  # bytes between (page, kv head) blocks of an interleaved pool

    @property
    def n_tokens(self) -> int:
        return int(self.k_codes.shape[2]) if self.length is None else int(self.length)

    def tensors(self):
        return [t for t in (self.k_codes, self.v_codes, self.k_scale, self.v_scale, self.k_zero, self.v_zero,
                            self.pages) if t is not None]


# dtype codes of the attention kernels (FADE_DTYPE_F16 / FADE_DTYPE_BF16): every
# 16-bit float of a call (query, output, fp16-layout tiers, the symmetric and
# literal-INT2 scales) is of the query's dtype, as the reference's cache keeps
# every tier and scale in the model's dtype (fade/cache.py:124-160).
_ATTN_DTYPES = {torch.float16: 0, torch.bfloat16: 1}


def _attn_dtype(q: Tensor, op: str) -> int:
    if q.dtype not in _ATTN_DTYPES:
        raise ValueError(f"{op}: expected a float16 or bfloat16 query, got {q.dtype}")
    return _ATTN_DTYPES[q.dtype]


def _fp16_tier(kv: tuple[Tensor, Tensor] | None, dtype: torch.dtype = torch.float16) -> _lib.Fp16Tier:
    t = _lib.Fp16Tier()
    if kv is None or kv[0] is None or kv[0].shape[2] == 0:
        return t
    k, v = kv
    if k.dtype != dtype or v.dtype != dtype:
        raise ValueError(f"sink/recent tiers must be {dtype} (the query's dtype), got {k.dtype}/{v.dtype}")
    if k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("sink/recent tiers need a contiguous head_dim axis")
    t.k, t.v, t.len = k.data_ptr(), v.data_ptr(), int(k.shape[2])
    t.k_sb, t.k_sh, t.k_ss = k.stride(0), k.stride(1), k.stride(2)
    t.v_sb, t.v_sh, t.v_ss = v.stride(0), v.stride(1), v.stride(2)
    return t


def _mid_tier(mid: MiddleTier | None, dtype: torch.dtype = torch.float16) -> _lib.MidTier:
    m = _lib.MidTier()
    if mid is None or mid.n_tokens == 0:
        m.fmt = _lib.MID_NONE
        return m
    if mid.fmt not in _FMT:
        raise ValueError(f"unknown middle format {mid.fmt!r}")
    if mid.fmt == "asym":
        if dtype != torch.float16:
            raise ValueError("the asymmetric middle format holds fp16 tensors; it pairs with float16 queries")
        want = [mid.k_scale, mid.v_scale, mid.k_zero, mid.v_zero]
    elif mid.fmt == "fp16":
        want = [mid.k_codes, mid.v_codes]
    else:
        want = [mid.k_scale, mid.v_scale]
    for t in want:
        if t is not None and t.dtype != (torch.float16 if mid.fmt == "asym" else dtype):
            raise ValueError(f"middle tier ({mid.fmt}): scales / rows must be "
                             f"{torch.float16 if mid.fmt == 'asym' else dtype}, got {t.dtype}")
    for t in mid.tensors():
        if not t.is_contiguous() and not mid.page_stride:
            raise ValueError("middle-tier tensors must be contiguous")
    m.fmt = _FMT[mid.fmt]
    m.k_bits, m.v_bits, m.group = mid.k_bits, mid.v_bits, mid.group
    m.len = mid.n_tokens
    m.v_rows = int(mid.v_codes.shape[2])
    m.k_codes, m.v_codes = mid.k_codes.data_ptr(), mid.v_codes.data_ptr()
    m.k_scale, m.v_scale = _lib.ptr(mid.k_scale), _lib.ptr(mid.v_scale)
    m.k_zero, m.v_zero = _lib.ptr(mid.k_zero), _lib.ptr(mid.v_zero)
    if mid.pages is not None:
        if mid.length is None:
            raise ValueError("a paged middle tier needs length (the longest row's middle)")
        if mid.pages.dtype != torch.int32 or mid.pages.dim() != 2:
            raise ValueError("pages must be int32 [B, pages_per_row]")
        m.pages, m.pages_per_row = mid.pages.data_ptr(), int(mid.pages.shape[1])
        m.page_stride = int(mid.page_stride)
    return m


def paginate_middle(mid: MiddleTier, lens_mid, order=None, interleave: bool = False) -> MiddleTier:
    """A padded ``"int4"``/``"sym"``/``"asym"`` middle tier ([B, Hkv, S, ...] per token)
    as a paged one: row b's ``lens_mid[b]`` tokens go to ``ceil(lens_mid[b] / 64)``
    pages of one pool shared by the rows.  ``order`` (a permutation of the page
    ids) places the pages anywhere in the pool; default: in row order.
    ``interleave`` (``"int4"``/``"sym"``): one pool whose (page, kv head) blocks
    hold [K codes | V codes | V scales] back to back, so a tile is one
    contiguous read."""
    if mid.fmt not in ("int4", "sym", "asym") or mid.pages is not None:
        raise ValueError("paginate_middle takes an unpaged int4 / sym / asym middle tier")
    lens = [int(x) for x in lens_mid]
    B, H, S = (int(d) for d in mid.k_codes.shape[:3])
    if len(lens) != B or any(x < 0 or x > S for x in lens):
        raise ValueError(f"lens_mid must give 0..{S} tokens for each of {B} rows")
    counts = [-(-x // 64) for x in lens]
    n_pages = max(1, sum(counts))
    ppr = max(1, max(counts))
    ids = torch.arange(n_pages) if order is None else torch.as_tensor(order, dtype=torch.long)
    dev = mid.k_codes.device
    table = torch.zeros(B, ppr, dtype=torch.int32)
    src_b, src_t, dst = [], [], []
    k = 0
    for b, c in enumerate(counts):
        for t in range(c):
            table[b, t] = int(ids[k])
            src_b.append(b)
            src_t.append(t)
            dst.append(int(ids[k]))
            k += 1

    def pool(x: Tensor | None) -> Tensor | None:
        if x is None:
            return x
        pad = -(-S // 64) * 64 - S
        xp = torch.nn.functional.pad(x, (0, 0, 0, pad)) if pad else x
        tiles = xp.reshape(B, H, -1, 64, x.shape[-1])  # [B, H, tiles, 64, ...]
        out = torch.zeros(n_pages, H, 64, x.shape[-1], dtype=x.dtype, device=dev)
        if dst:
            out[torch.tensor(dst, device=dev)] = tiles[torch.tensor(src_b, device=dev), :,
                                                       torch.tensor(src_t, device=dev)]
        return out

    k_scale = mid.k_scale if mid.fmt != "asym" else pool(mid.k_scale)  # SYM K scale: per row [B,Hkv,1,D]
    if interleave:
        if mid.fmt == "asym":
            raise ValueError("interleave: int4 / sym middle tiers only")
        kp, vp, sp = pool(mid.k_codes), pool(mid.v_codes), pool(mid.v_scale)
        kb, vbytes, sb = kp[0, 0].numel(), vp[0, 0].numel(), sp[0, 0].numel() * 2
        stride = -(-(kb + vbytes + sb) // 16) * 16
        blk = torch.zeros(n_pages, H, stride, dtype=torch.uint8, device=dev)
        blk[:, :, :kb] = kp.reshape(n_pages, H, kb)
        blk[:, :, kb : kb + vbytes] = vp.reshape(n_pages, H, vbytes)
        blk[:, :, kb + vbytes : kb + vbytes + sb] = sp.reshape(n_pages, H, -1).view(torch.uint8)
        flat = blk.view(-1)
        # views into the pool at each tensor's offset in a block (the kernel reads the
        # first block's address and steps by `stride`)
        kv = flat.as_strided(kp.shape, (H * stride, stride, kp.shape[-1], 1), 0)
        vv = flat.as_strided(vp.shape, (H * stride, stride, vp.shape[-1], 1), kb)
        tail = flat[kb + vbytes :]
        half = tail[: (tail.numel() // 2) * 2].view(torch.float16)
        vs = half.as_strided(sp.shape, (H * stride // 2, stride // 2, 1, 1))
        out = MiddleTier(mid.fmt, kv, vv, k_scale, vs, k_bits=mid.k_bits, v_bits=mid.v_bits, group=mid.group,
                         length=max(lens) if lens else 0, pages=table.to(dev), page_stride=stride)
        out._pool = blk  # keeps the pool alive
        return out
    return MiddleTier(mid.fmt, pool(mid.k_codes), pool(mid.v_codes), k_scale, pool(mid.v_scale),
                      pool(mid.k_zero), pool(mid.v_zero), k_bits=mid.k_bits, v_bits=mid.v_bits, group=mid.group,
                      length=max(lens) if lens else 0, pages=table.to(dev))


class TieredDecodePlan:
    """Validated launch of the tiered decode kernel for fixed tensors.

    Holds references to every tensor it points at, the output and the
    workspace; ``run()`` enqueues the kernels on the current stream.  With
    ``stream`` given, the plan uses the zero-filled workspace shared by the
    calls on that stream (``_lib.stream_workspace``) instead of its own, and
    must then run on that stream.  With ``no_alloc`` the plan allocates no
    workspace: ``run()`` calls ``fade_tiered_decode_attn_noalloc``, whose
    kernels use the library's own per-GPU scratch (shared by every such call
    on that GPU, so such calls must not overlap on one GPU).  ``rotation``
    (fp32 [128, 128] on the device, the rotated backend's R) marks the middle
    tier as codes of ``K R^T`` / ``V R^T`` while q, sink and recent stay in the
    model's basis: the kernel scores middle tokens with ``q R^T`` and returns
    the fp16 tiers' part plus the middle part times R (no torch op per call).
    """

    def __init__(
        self,
        q: Tensor,
        sink: tuple[Tensor, Tensor] | None,
        mid: MiddleTier | None,
        recent: tuple[Tensor, Tensor] | None,
        sm_scale: float | None = None,
        out: Tensor | None = None,
        n_splits: int = 0,
        kernel: int = 0,
        lens: Tensor | None = None,
        stream: int | None = None,
        deterministic: bool | None = None,
        no_alloc: bool = False,
        rotation: Tensor | None = None,
    ) -> None:
        if q.dim() != 4 or q.shape[2] != 1:
            raise ValueError(f"q must be [B, Hq, 1, D], got {tuple(q.shape)}")
        if lens is not None:
            if lens.dim() != 2 or lens.shape[1] != 3 or lens.shape[0] != q.shape[0]:
                raise ValueError(f"lens must be [B, 3] (sink, middle, recent per row), got {tuple(lens.shape)}")
            lens = lens.to(device=q.device, dtype=torch.int32).contiguous()
        tensors = [q] + ([*sink] if sink else []) + ([*recent] if recent else []) + (mid.tensors() if mid else [])
        _lib.require_gpu(*tensors, op="tiered_decode_attention")
        dtc = _attn_dtype(q, "tiered_decode_attention")
        B, Hq, _, D = q.shape
        ref = sink[0] if sink else (recent[0] if recent else mid.k_codes)
        Hkv = int(ref.shape[1])
        if q.stride(-1) != 1:
            q = q.contiguous()
        if rotation is not None:
            if mid is None or mid.fmt not in ("int4", "sym"):
                raise ValueError("a rotation applies to a symmetric ('sym') middle tier")
            if tuple(rotation.shape) != (D, D) or rotation.dtype != torch.float32 or rotation.device != q.device:
                raise ValueError(f"rotation must be float32 [{D}, {D}] on {q.device}")
            rotation = rotation.contiguous()
        if out is None:
            out = torch.empty(B, Hq, 1, D, dtype=q.dtype, device=q.device)
        if out.dtype != q.dtype:
            raise ValueError(f"out must be {q.dtype} (the query's dtype), got {out.dtype}")
        self._keep = (q, sink, mid, recent, out, lens, rotation)
        a = _lib.DecodeArgs()
        a.B, a.Hq, a.Hkv, a.D = B, Hq, Hkv, D
        a.q, a.q_sb, a.q_sh = q.data_ptr(), q.stride(0), q.stride(1)
        a.out, a.o_sb, a.o_sh = out.data_ptr(), out.stride(0), out.stride(1)
        a.sm_scale = float(1.0 / math.sqrt(D) if sm_scale is None else sm_scale)
        a.sink, a.mid, a.recent = _fp16_tier(sink, q.dtype), _mid_tier(mid, q.dtype), _fp16_tier(recent, q.dtype)
        a.dtype = dtc
        a.n_splits, a.kernel = int(n_splits), int(kernel)
        a.lens = _lib.ptr(lens)
        if deterministic is None:
            deterministic = torch.are_deterministic_algorithms_enabled()
        a.deterministic = int(bool(deterministic))
        a.rotation = _lib.ptr(rotation)
        lib = _lib.load()
        self._lib = lib
        if no_alloc:
            self.workspace = None
            a.workspace, a.workspace_bytes = None, 0
            self._fn, self._name = lib.fade_tiered_decode_attn_noalloc, "fade_tiered_decode_attn_noalloc"
        else:
            nb = ctypes.c_int64(0)
            _lib.check(lib.fade_tiered_decode_workspace_bytes(ctypes.byref(a), nb),
                       "fade_tiered_decode_workspace_bytes")
            self.workspace = (_lib.workspace(nb.value, q.device) if stream is None
                              else _lib.stream_workspace(nb.value, q.device, stream, B * Hkv * -(-(Hq // Hkv) // 4)))
            a.workspace, a.workspace_bytes = self.workspace.data_ptr(), self.workspace.numel()
            self._fn, self._name = lib.fade_tiered_decode_attn, "fade_tiered_decode_attn"
        self.args = a
        self.out = out
        self._argp = ctypes.byref(a)
        self._ws_tiles = (int(a.sink.len) + int(a.recent.len) + 15) // 16

    def run(self, stream: int | None = None) -> Tensor:
        s = torch.cuda.current_stream(self.out.device).cuda_stream if stream is None else stream
        _lib.check(self._fn(self._argp, s), self._name)
        return self.out

    def rerun(self, q: Tensor, recent_len: int, stream: int) -> Tensor:
        """Launch again for a new query of the same shape and strides, into a new
        output, with the recent tier (same tensors) now ``recent_len`` tokens long:
        the decode loop's step, without re-validating the tiers.  The workspace
        grows if the longer row needs more splits."""
        a = self.args
        if q.stride(-1) != 1:
            q = q.contiguous()
        a.q = q.data_ptr()
        out = torch.empty_like(self.out)
        a.out = out.data_ptr()
        a.recent.len = int(recent_len)
        tiles = (int(a.sink.len) + int(a.recent.len) + 15) // 16  # the split plan moves with the fp16 tile count
        if self.workspace is not None and tiles != self._ws_tiles:
            self._ws_tiles = tiles
            nb = ctypes.c_int64(0)
            _lib.check(self._lib.fade_tiered_decode_workspace_bytes(self._argp, nb), "fade_tiered_decode_workspace_bytes")
            if nb.value > self.workspace.numel():
                B, Hq, Hkv = int(a.B), int(a.Hq), int(a.Hkv)
                self.workspace = _lib.stream_workspace(nb.value, out.device, stream, B * Hkv * -(-(Hq // Hkv) // 4))
                a.workspace, a.workspace_bytes = self.workspace.data_ptr(), self.workspace.numel()
        _lib.check(self._fn(self._argp, stream), self._name)
        return out


def tiered_decode_attention(
    q: Tensor,
    sink: tuple[Tensor, Tensor] | None,
    mid: MiddleTier | None,
    recent: tuple[Tensor, Tensor] | None,
    sm_scale: float | None = None,
    n_splits: int = 0,
    kernel: int = 0,
    lens: Tensor | None = None,
    deterministic: bool | None = None,
    rotation: Tensor | None = None,
) -> Tensor:
    """Decode attention of ``q`` [B,Hq,1,D] over the tiered cache; returns [B,Hq,1,D] of q's dtype.

    ``q`` is float16 or bfloat16, and so are the sink / recent tiers and the
    symmetric formats' scales (the reference's cache keeps everything in the
    model's dtype); the asymmetric format's scale / zero are float16.

    Query head ``h`` attends to KV head ``h // (Hq // Hkv)`` (the reference's
    ``repeat_interleave`` GQA mapping, fade/kernels/fused_int4_attn.py:306-312).
    ``lens`` [B, 3] (sink, middle, recent tokens per row; device or host int)
    makes the batch ragged: row b attends to the first ``lens[b]`` rows of each
    tier, whose tensors are then padded capacities.
    ``deterministic`` (default: ``torch.are_deterministic_algorithms_enabled()``)
    makes repeated calls on the same inputs bitwise identical; otherwise the
    INT4 kernel's waves claim tiles as they finish, and results can differ in
    the last bits between calls.
    ``rotation`` (fp32 [128, 128] R): the middle tier holds rotated codes
    (fade/rotated_quant.py:134-187) while q, sink and recent are unrotated; the
    kernel rotates q for the middle tokens and un-rotates their output part.
    """
    s = torch.cuda.current_stream(q.device).cuda_stream
    plan = TieredDecodePlan(q, sink, mid, recent, sm_scale, n_splits=n_splits, kernel=kernel, lens=lens, stream=s,
                            deterministic=deterministic, rotation=rotation)
    return plan.run(s)


__all__ = ["MiddleTier", "TieredDecodePlan", "paginate_middle", "tiered_decode_attention"]
