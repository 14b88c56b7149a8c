"""The paged middle tier of ragged caches (TieredKVCache.page_pool): a cache whose
INT4 middle lives in 64-token pages of a MiddlePagePool against the same cache
without the pool, which keeps padded tensors and is checked row by row against
single-row caches on the host path (the reference's op sequence).  The stored
tiers must agree bit for bit; decode through the block table, chunked prefill and
materialize must agree too, across a second reassignment that frees and reuses pages."""

import numpy as np
import pytest
import torch

from fade_amd.cache import TIER_EVICT, TieredKVCache
from fade_amd.pages import PAGE_TOKENS, MiddlePagePool
from fade_amd.policy import _assign_one_layer

pytestmark = pytest.mark.gpu

B, H, HQ, D, N_SINK, RECENT = 3, 2, 8, 128, 4, 16


def _pair(dev, n_pages=64):
    out = []
    for paged in (False, True):
        c = TieredKVCache(n_sink=N_SINK, recent_window=RECENT, int4_budget=None, int2_budget=0, head_dim=D)
        c.ragged_layout = True
        if paged:
            c.page_pool = MiddlePagePool(n_pages, H, D, dev)
        out.append(c)
    return out


def _append(caches, n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(B, H, n, D, generator=g) * torch.exp(torch.randn(D, generator=g) * 0.5)).half().to(dev)
    v = torch.randn(B, H, n, D, generator=g).half().to(dev)
    for c in caches:
        c.update(k, v, 0)


def _reassign(caches, budgets, seed):
    S = caches[0].get_seq_length(0)
    st = caches[0]._layers[0]
    rows = [S] * B if st.lens_host is None else [sum(r) for r in st.lens_host]
    rng = np.random.default_rng(seed)
    tiers = torch.full((B, S), TIER_EVICT, dtype=torch.long)
    for b in range(B):
        tiers[b, : rows[b]] = _assign_one_layer(rows[b], torch.from_numpy(rng.exponential(size=rows[b]).astype(np.float32)),
                                                N_SINK, RECENT, budgets[b], 0)
    for c in caches:
        c.apply_tier_assignment_per_sequence(0, tiers)


def _same(plain, paged, what):
    a, p = plain._layers[0], paged._layers[0]
    assert a.lens_host == p.lens_host, what
    assert a.mid_table is None and p.int4_kq is None and p.int4_vq is None and p.int4_vs is None, what
    for f in ("sink_k", "sink_v", "fp16_k", "fp16_v", "int4_ks"):
        x, y = getattr(a, f), getattr(p, f)
        assert (x is None) == (y is None), f"{what}: {f}"
        if x is not None:
            assert torch.equal(x.cpu(), y.cpu()), f"{what}: {f} differs"
    kq, ks, vq, vs = paged._mid_padded(p)
    for name, x, y in (("int4_kq", a.int4_kq, kq), ("int4_vq", a.int4_vq, vq), ("int4_vs", a.int4_vs, vs)):
        assert x.shape == y.shape and torch.equal(x.cpu(), y.cpu()), f"{what}: {name} from the pages differs"
    pages = [len(r) for r in p.mid_pages]
    assert pages == [-(-r[1] // PAGE_TOKENS) for r in p.lens_host], what
    assert p.mid_pool.n_free == p.mid_pool.n_pages - sum(pages), what
    assert p.mid_page_bytes == sum(pages) * p.mid_pool.page_bytes
    table = p.mid_table.cpu()
    for b, row in enumerate(p.mid_pages):
        assert table[b, : len(row)].tolist() == row and not table[b, len(row):].any(), what
    ko, vo = plain._materialize(0)
    kp, vp = paged._materialize(0)
    assert torch.equal(ko.cpu(), kp.cpu()) and torch.equal(vo.cpu(), vp.cpu()), f"{what}: materialize"


def _close(x, y, tol, what):
    err = (x.float() - y.float()).abs().max().item()
    assert err <= tol, f"{what}: max |diff| {err}"


def test_paged_middle_matches_unpaged(dev):
    """Two reassignments with appends and a chunk prefill in between, eviction in some rows."""
    print("case paged middle vs padded", flush=True)
    plain, paged = _pair(dev)
    _append((plain, paged), 400, 1, dev)
    _reassign((plain, paged), [None, 150, 260], 2)
    _same(plain, paged, "first reassignment")
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, HQ, 1, D, generator=g).half().to(dev)
    _close(plain.decode_attention(q, 0), paged.decode_attention(q, 0), 1e-3, "decode")
    _append((plain, paged), 24, 4, dev)
    qc = torch.randn(B, HQ, 24, D, generator=g).half().to(dev)
    # the prefill reads the pages in place; no tile claims, so bit for bit
    assert torch.equal(plain.prefill_attention(qc, 0), paged.prefill_attention(qc, 0)), "chunk prefill"

    _reassign((plain, paged), [60, None, 130], 5)  # frees the old pages and takes new ones
    _same(plain, paged, "second reassignment")
    _close(plain.decode_attention(q, 0), paged.decode_attention(q, 0), 1e-3, "decode after the second")


def test_paged_decode_bitwise_equal_when_deterministic(dev):
    """With torch.use_deterministic_algorithms, decode through the pages equals decode of
    the padded layout bit for bit (same tiles, same fixed summation order)."""
    print("case paged decode deterministic", flush=True)
    plain, paged = _pair(dev)
    _append((plain, paged), 350, 31, dev)
    _reassign((plain, paged), [None, 90, 200], 32)
    q = torch.randn(B, HQ, 1, D, generator=torch.Generator().manual_seed(33)).half().to(dev)
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        a, b = plain.decode_attention(q, 0), paged.decode_attention(q, 0)
        assert torch.equal(a, b) and torch.equal(b, paged.decode_attention(q, 0))
    finally:
        torch.use_deterministic_algorithms(prev)


def test_paged_decode_matches_materialized_fp32(dev):
    """Decode through the block table against fp32 attention over each row's own
    materialized tokens (GQA: query head h reads KV head h // (Hq / Hkv))."""
    print("case paged decode vs fp32", flush=True)
    _, paged = _pair(dev)
    _append((paged,), 300, 7, dev)
    _reassign((paged,), [None, 40, 200], 8)
    q = torch.randn(B, HQ, 1, D, generator=torch.Generator().manual_seed(9)).half().to(dev)
    out = paged.decode_attention(q, 0)
    k, v = paged._materialize(0)
    for b, r in enumerate(paged._layers[0].lens_host):
        n = sum(r)
        kb = k[b, :, :n].float().repeat_interleave(HQ // H, dim=0)
        vb = v[b, :, :n].float().repeat_interleave(HQ // H, dim=0)
        p = torch.softmax((q[b].float() @ kb.transpose(-1, -2)) / D ** 0.5, dim=-1)
        _close(out[b], p @ vb, 2e-3, f"row {b}")


def test_page_pool_exhausted_leaves_layer_unchanged(dev):
    """A reassignment that needs more pages than the pool has raises before any change."""
    print("case page pool exhausted", flush=True)
    _, paged = _pair(dev, n_pages=4)
    _append((paged,), 200, 11, dev)
    _reassign((paged,), [60, 60, 60], 12)  # 3 rows x 1 page
    st = paged._layers[0]
    lens, table, pages = [list(r) for r in st.lens_host], st.mid_table.clone(), [list(r) for r in st.mid_pages]
    _append((paged,), 100, 13, dev)
    rows = [sum(r) for r in st.lens_host]
    S = max(rows)
    tiers = torch.full((B, S), TIER_EVICT, dtype=torch.long)
    for b in range(B):
        tiers[b, : rows[b]] = _assign_one_layer(rows[b], torch.rand(rows[b]), N_SINK, RECENT, None, 0)
    with pytest.raises(RuntimeError, match="page pool exhausted"):
        paged.apply_tier_assignment_per_sequence(0, tiers)
    assert st.mid_pages == pages and torch.equal(st.mid_table, table)
    assert [list(r) for r in st.lens_host][0][1] == lens[0][1]
    assert st.mid_pool.n_free == 1


def test_release_pages_returns_every_page(dev):
    print("case release pages", flush=True)
    _, paged = _pair(dev, n_pages=16)
    _append((paged,), 260, 21, dev)
    _reassign((paged,), [None, 100, 30], 22)
    pool = paged.page_pool
    assert pool.n_free < pool.n_pages
    paged.release_pages()
    assert pool.n_free == pool.n_pages
    st = paged._layers[0]
    assert st.mid_table is None and all(r[1] == 0 for r in st.lens_host)
    q = torch.randn(B, HQ, 1, D, generator=torch.Generator().manual_seed(23)).half().to(dev)
    assert torch.isfinite(paged.decode_attention(q, 0).float()).all()
