"""Page pool for the INT4 middle tier of ragged caches.

The reference's per-sequence mode zero-pads every row to the longest one
(fade/cache.py:1145-1159); its roadmap item A1 (paged tiers, "FADE v1.0
Release + Future Roadmap.md":41-44) replaces that padding with pages.  Here one
pool of 64-token pages serves every layer of a cache (all layers share the KV
head count and head_dim).  A page holds, for every KV head, the packed K codes,
the packed V codes and the per-token V scales of 64 consecutive middle tokens
of one row: exactly one middle tile of the decode kernel, which reads pages
through a per-row block table (``fade_mid_tier.pages``).  The per-channel K
scales span a row's whole middle tier and stay per row ([B, Hkv, 1, D]),
outside the pool.

Page 0 is all zeros and is never handed out.  Block-table slots past a row's
own pages point at it, so gathering a row's pages back into a padded tensor
gives zeros past the row's tokens, which is what the quantizers write for the
zero-padded rows of the unpaged layout: ``gather(store(x))`` is ``x``.

Pages are allocated and freed on the host (a free list); the copies into and
out of the pool run on the current stream, so a page freed by one
reassignment and reused by the next is overwritten only after every earlier
read of it in stream order.
"""

from __future__ import annotations

import torch
from torch import Tensor

PAGE_TOKENS = 64


class MiddlePagePool:
    """``n_pages`` pages of ``PAGE_TOKENS`` middle tokens for ``n_kv_heads`` heads of
    ``head_dim`` channels (reference INT4 layout: two codes a byte, fp16 V scale per
    token).  Storage: ``k_codes``/``v_codes`` uint8 [n_pages + 1, Hkv, 64, D/2] and
    ``v_scale`` fp16 [n_pages + 1, Hkv, 64, 1]; index 0 is the zero page."""

    def __init__(self, n_pages: int, n_kv_heads: int, head_dim: int, device="cuda") -> None:
        if n_pages < 1 or n_kv_heads < 1 or head_dim < 2 or head_dim % 2:
            raise ValueError(
                f"MiddlePagePool needs n_pages >= 1, n_kv_heads >= 1 and an even head_dim, "
                f"got {n_pages}, {n_kv_heads}, {head_dim}"
            )
        self.n_pages = int(n_pages)
        self.n_kv_heads = int(n_kv_heads)
        self.head_dim = int(head_dim)
        dev = torch.device(device)
        shape = (self.n_pages + 1, self.n_kv_heads, PAGE_TOKENS, self.head_dim // 2)
        self.k_codes = torch.zeros(shape, dtype=torch.uint8, device=dev)
        self.v_codes = torch.zeros(shape, dtype=torch.uint8, device=dev)
        self.v_scale = torch.zeros(shape[:3] + (1,), dtype=torch.float16, device=dev)
        self._free = list(range(self.n_pages, 0, -1))  # pop() hands out the lowest id first
        self._used = bytearray(self.n_pages + 1)

    @property
    def device(self) -> torch.device:
        return self.k_codes.device

    @property
    def n_free(self) -> int:
        return len(self._free)

    @property
    def page_bytes(self) -> int:
        """Bytes one page holds (K codes + V codes + V scales, every KV head)."""
        return self.n_kv_heads * PAGE_TOKENS * (self.head_dim + 2)

    def alloc(self, n: int) -> list[int]:
        if n < 0:
            raise ValueError(f"cannot allocate {n} pages")
        if n > len(self._free):
            raise RuntimeError(f"page pool exhausted: {n} pages requested, {len(self._free)} free of {self.n_pages}")
        ids = [self._free.pop() for _ in range(n)]
        for i in ids:
            self._used[i] = 1
        return ids

    def free(self, ids) -> None:
        ids = [int(i) for i in ids]
        for i in ids:
            if not 1 <= i <= self.n_pages:
                raise ValueError(f"page {i} is not a page of this pool (1..{self.n_pages})")
            if not self._used[i]:
                raise ValueError(f"page {i} is not allocated")
        for i in ids:
            self._used[i] = 0
        self._free.extend(reversed(ids))

    def _check(self, kq: Tensor, vq: Tensor, vs: Tensor) -> None:
        B, H, S = (int(d) for d in kq.shape[:3])
        want = {"k_codes": (kq, (B, H, S, self.head_dim // 2), torch.uint8),
                "v_codes": (vq, (B, H, S, self.head_dim // 2), torch.uint8),
                "v_scale": (vs, (B, H, S, 1), torch.float16)}
        if H != self.n_kv_heads:
            raise ValueError(f"the pool holds {self.n_kv_heads} KV heads, the tier has {H}")
        for name, (t, shape, dt) in want.items():
            if tuple(t.shape) != shape or t.dtype != dt:
                raise ValueError(f"{name}: expected {dt} {shape}, got {t.dtype} {tuple(t.shape)}")
            if t.device != self.device:
                raise ValueError(f"{name} is on {t.device}, the pool on {self.device}")

    def store(self, kq: Tensor, vq: Tensor, vs: Tensor, lens_mid) -> tuple[Tensor, list[list[int]]]:
        """Copy a padded middle tier (``kq``/``vq`` uint8 [B, Hkv, S, D/2], ``vs`` fp16
        [B, Hkv, S, 1]) into newly allocated pages: row b's first ``lens_mid[b]`` tokens
        go to ``ceil(lens_mid[b] / 64)`` pages, the last one zero-filled past them if the
        padded tensors are.  Returns the block table (int32 [B, pages per row] on the
        pool's device, the zero page in unused slots) and each row's page ids."""
        self._check(kq, vq, vs)
        B, _, S = (int(d) for d in kq.shape[:3])
        lens = [int(x) for x in lens_mid]
        if len(lens) != B or any(x < 0 or x > S for x in lens):
            raise ValueError(f"lens_mid must give 0..{S} tokens for each of {B} rows")
        counts = [-(-x // PAGE_TOKENS) for x in lens]
        ids = self.alloc(sum(counts))
        table = torch.zeros(B, max(1, max(counts, default=0)), dtype=torch.int32)
        rows, src_b, src_t, k = [], [], [], 0
        for b, c in enumerate(counts):
            row = ids[k : k + c]
            k += c
            rows.append(row)
            if c:
                table[b, :c] = torch.tensor(row, dtype=torch.int32)
            src_b += [b] * c
            src_t += range(c)
        if ids:
            idx = torch.tensor([ids, src_b, src_t], dtype=torch.long)
            if self.device.type != "cpu":
                idx = idx.pin_memory().to(self.device, non_blocking=True)
            dst, sb, stile = idx[0], idx[1], idx[2]
            pad = -(-S // PAGE_TOKENS) * PAGE_TOKENS - S
            for pool, x in ((self.k_codes, kq), (self.v_codes, vq), (self.v_scale, vs)):
                xp = torch.nn.functional.pad(x, (0, 0, 0, pad)) if pad else x
                tiles = xp.reshape(B, self.n_kv_heads, -1, PAGE_TOKENS, x.shape[-1])
                pool[dst] = tiles[sb, :, stile]  # [n, Hkv, 64, W]
        if self.device.type != "cpu":
            table = table.pin_memory().to(self.device, non_blocking=True)
        return table, rows

    def gather(self, table: Tensor, length: int) -> tuple[Tensor, Tensor, Tensor]:
        """The padded middle tier [B, Hkv, length, ...] (K codes, V codes, V scales) a
        block table describes; ``length`` <= pages per row * 64."""
        B, ppr = (int(d) for d in table.shape)
        if length > ppr * PAGE_TOKENS:
            raise ValueError(f"length {length} exceeds the table's {ppr} pages per row")
        t = table.long()

        def one(pool: Tensor) -> Tensor:
            x = pool[t]  # [B, ppr, Hkv, 64, W]
            x = x.permute(0, 2, 1, 3, 4).reshape(B, self.n_kv_heads, ppr * PAGE_TOKENS, pool.shape[-1])
            return x[:, :, :length].contiguous()

        return one(self.k_codes), one(self.v_codes), one(self.v_scale)


__all__ = ["MiddlePagePool", "PAGE_TOKENS"]
