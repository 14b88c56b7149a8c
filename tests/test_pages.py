"""Host logic of the middle-tier page pool (fade_amd/pages.py) on CPU tensors: the
free list, and store/gather as exact inverses with zeros past each row's tokens."""

import pytest
import torch

from fade_amd.pages import PAGE_TOKENS, MiddlePagePool


def _padded(B, H, S, D, lens, seed):
    g = torch.Generator().manual_seed(seed)
    kq = torch.randint(0, 256, (B, H, S, D // 2), generator=g, dtype=torch.uint8)
    vq = torch.randint(0, 256, (B, H, S, D // 2), generator=g, dtype=torch.uint8)
    vs = torch.rand(B, H, S, 1, generator=g).half() + 0.01
    for b, n in enumerate(lens):  # the unpaged layout holds zeros past a row's tokens
        kq[b, :, n:] = 0
        vq[b, :, n:] = 0
        vs[b, :, n:] = 0
    return kq, vq, vs


@pytest.mark.parametrize("lens", [[130, 0, 64, 1], [200, 200, 200, 200], [0, 0, 0, 0]])
def test_store_gather_round_trip(lens):
    B, H, D, S = 4, 2, 16, max(max(lens), 1)
    pool = MiddlePagePool(40, H, D, "cpu")
    x = _padded(B, H, S, D, lens, 1)
    table, rows = pool.store(*x, lens)
    assert [len(r) for r in rows] == [-(-n // PAGE_TOKENS) for n in lens]
    assert pool.n_free == 40 - sum(len(r) for r in rows)
    assert sorted(i for r in rows for i in r) == list(range(1, 1 + sum(len(r) for r in rows)))
    assert table.dtype == torch.int32 and table.shape[0] == B
    for got, want in zip(pool.gather(table, S), x):
        assert torch.equal(got, want)
    assert not pool.k_codes[0].any() and not pool.v_scale[0].any()  # the zero page stays zero


def test_free_list_and_errors():
    pool = MiddlePagePool(5, 1, 8, "cpu")
    a = pool.alloc(3)
    assert a == [1, 2, 3] and pool.n_free == 2
    with pytest.raises(RuntimeError, match="page pool exhausted"):
        pool.alloc(3)
    pool.free([2])
    with pytest.raises(ValueError, match="not allocated"):
        pool.free([2])
    with pytest.raises(ValueError, match="not a page"):
        pool.free([0])
    assert pool.alloc(1) == [2]
    assert pool.page_bytes == 1 * PAGE_TOKENS * (8 + 2)
    with pytest.raises(ValueError):
        MiddlePagePool(4, 1, 7, "cpu")
    with pytest.raises(ValueError, match="KV heads"):
        pool.store(*_padded(1, 2, 10, 8, [10], 0), [10])


def test_pages_reused_after_free():
    B, H, D = 2, 1, 8
    pool = MiddlePagePool(4, H, D, "cpu")
    x1 = _padded(B, H, 128, D, [128, 100], 2)
    t1, r1 = pool.store(*x1, [128, 100])
    assert pool.n_free == 0
    pool.free([i for r in r1 for i in r])
    x2 = _padded(B, H, 70, D, [70, 5], 3)
    t2, _ = pool.store(*x2, [70, 5])
    for got, want in zip(pool.gather(t2, 70), x2):
        assert torch.equal(got, want)
