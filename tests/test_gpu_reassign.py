"""Device-side tier reassignment (fade_reassign_plan / fade_reassign_gather) against
the host path of ``apply_tier_assignment``, which follows fade/cache.py:881-1057 op
for op and is pinned to the oracle.  Every tier field must match bit for bit."""

import numpy as np
import pytest
import torch

from fade_amd.cache import TIER_EVICT, TIER_FP16, TIER_INT2, TIER_INT4, TieredKVCache
from fade_amd.policy import _assign_one_layer

pytestmark = pytest.mark.gpu

FIELDS = ("sink_k", "sink_v", "sink_pos", "fp16_k", "fp16_v", "fp16_pos", "int4_kq", "int4_ks", "int4_vq",
          "int4_vs", "int4_pos", "int2_kq")


def _pair(**kw):
    caches = []
    for dev_path in (False, True):
        c = TieredKVCache(head_dim=128, **kw)
        c.device_reassign = dev_path
        caches.append(c)
    return caches


def _append(caches, B, H, n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(B, H, n, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).half().to(dev)
    v = torch.randn(B, H, n, 128, generator=g).half().to(dev)
    for c in caches:
        c.update(k, v, 0)


def _same(a, b, what):
    for f in FIELDS:
        x, y = getattr(a._layers[0], f), getattr(b._layers[0], f)
        assert (x is None) == (y is None), f"{what}: {f} present in one path only"
        if x is not None:
            assert x.shape == y.shape, f"{what}: {f} shape {tuple(x.shape)} vs {tuple(y.shape)}"
            assert torch.equal(x.cpu(), y.cpu()), f"{what}: {f} differs"
    for f in ("next_position", "sink_count", "int2_actual_count"):
        assert getattr(a._layers[0], f) == getattr(b._layers[0], f), f"{what}: {f}"
    assert a.get_seq_length(0) == b.get_seq_length(0)


@pytest.mark.parametrize("tiers_on", ["cpu", "cuda", "cuda+counts"])
@pytest.mark.parametrize("budget", [None, 40])
def test_reassign_device_matches_host(dev, tiers_on, budget):
    """Three rounds of append + reassign (scores seeded), eviction when budget is set."""
    print(f"case reassign tiers_on={tiers_on} budget={budget}", flush=True)
    B, H = 2, 2
    host, devc = _pair(n_sink=4, recent_window=16, int4_budget=budget, int2_budget=0)
    _append((host, devc), B, H, 150, 1, dev)
    rng = np.random.default_rng(5)
    for rnd in range(3):
        S = host.get_seq_length(0)
        scores = torch.from_numpy(rng.exponential(size=S).astype(np.float32))
        tiers = _assign_one_layer(S, scores, 4, 16, budget, 0)
        counts = tuple(int((tiers == t).sum()) for t in (TIER_FP16, TIER_INT4, TIER_INT2))
        host.apply_tier_assignment(0, tiers)
        if tiers_on == "cpu":
            devc.apply_tier_assignment(0, tiers)
        elif tiers_on == "cuda":
            devc.apply_tier_assignment(0, tiers.to(dev))
        else:
            devc.apply_tier_assignment(0, tiers.to(dev), counts=counts)
        assert devc._last_reassign_counts is not None, "device path not taken"
        c = devc._last_reassign_counts.cpu().tolist()
        assert c[:3] == [counts[0], counts[1], counts[0] + counts[1]] and c[3] == 0
        _same(host, devc, f"round {rnd}")
        devc._last_reassign_counts = None
        _append((host, devc), B, H, 37 + 11 * rnd, 10 + rnd, dev)
        _same(host, devc, f"append after round {rnd}")


def test_reassign_device_decode_matches(dev):
    """Decode attention after a device reassignment equals the one after the host path."""
    print("case reassign decode", flush=True)
    host, devc = _pair(n_sink=4, recent_window=32, int4_budget=100, int2_budget=0)
    _append((host, devc), 2, 2, 400, 3, dev)
    S = host.get_seq_length(0)
    scores = torch.from_numpy(np.random.default_rng(1).exponential(size=S).astype(np.float32))
    tiers = _assign_one_layer(S, scores, 4, 32, 100, 0)
    host.apply_tier_assignment(0, tiers)
    devc.apply_tier_assignment(0, tiers)
    q = torch.randn(2, 8, 1, 128, generator=torch.Generator().manual_seed(9)).half().to(dev)
    # identical caches; the decode's tile claiming may change the fp32 sum order
    assert (host.decode_attention(q, 0).float() - devc.decode_attention(q, 0).float()).abs().max().item() <= 1e-3


def test_reassign_device_no_host_sync(dev):
    """Host tiers: plan, gather and requantization run without a host synchronization."""
    print("case reassign no sync", flush=True)
    (devc,) = _pair(n_sink=4, recent_window=16, int4_budget=30, int2_budget=0)[1:]
    _append((devc,), 1, 2, 120, 4, dev)
    S = devc.get_seq_length(0)
    tiers = _assign_one_layer(S, torch.arange(S, dtype=torch.float32), 4, 16, 30, 0)
    devc._rope_tables(devc._layers[0].next_position, dev)  # table upload done up front
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        devc.apply_tier_assignment(0, tiers)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    assert devc._last_reassign_counts is not None
    assert devc.get_seq_length(0) == 4 + 16 + 30


def test_reassign_int2_falls_back(dev):
    """An assignment with INT2 tokens takes the host path (device path declines it)."""
    print("case reassign int2 fallback", flush=True)
    host, devc = _pair(n_sink=2, recent_window=8, int4_budget=10, int2_budget=5)
    _append((host, devc), 1, 2, 60, 6, dev)
    S = host.get_seq_length(0)
    tiers = _assign_one_layer(S, torch.arange(S, dtype=torch.float32), 2, 8, 10, 5)
    assert int((tiers == TIER_INT2).sum()) == 5 and int((tiers == TIER_EVICT).sum()) > 0
    host.apply_tier_assignment(0, tiers)
    devc.apply_tier_assignment(0, tiers.to(dev))
    assert devc._last_reassign_counts is None
    _same(host, devc, "int2")
    assert devc._layers[0].int2_actual_count == 5


@pytest.mark.parametrize("tiers_on", ["cpu", "cuda"])
@pytest.mark.parametrize("budgets", [(None, None, None), (30, None, 70), (20, 45, 90)])
def test_per_sequence_device_matches_host(dev, tiers_on, budgets):
    """The reference's per-sequence mode (rows zero-padded to the longest) on the device
    path equals the host path (the reference's op sequence) field for field, bit for bit,
    with eviction in some rows or all, and after later appends."""
    print(f"case per-sequence device vs host tiers_on={tiers_on} budgets={budgets}", flush=True)
    B, H = 3, 2
    host, devc = _pair(n_sink=4, recent_window=16, int4_budget=None, int2_budget=0)
    _append((host, devc), B, H, 150, 21, dev)
    rng = np.random.default_rng(22)
    S = host.get_seq_length(0)
    tiers = torch.stack([_assign_one_layer(S, torch.from_numpy(rng.exponential(size=S).astype(np.float32)),
                                           4, 16, budgets[b], 0) for b in range(B)])
    if tiers_on == "cuda":
        tiers = tiers.to(dev)
    for c in (host, devc):
        c.apply_tier_assignment_per_sequence(0, tiers.clone())
    _same(host, devc, "reassignment")
    assert devc._layers[0]._padded_rows
    for rnd in range(2):
        _append((host, devc), B, H, 5, 23 + rnd, dev)
        _same(host, devc, f"append {rnd}")
    kh, vh = host._materialize(0)
    kd, vd = devc._materialize(0)
    assert torch.equal(kh, kd) and torch.equal(vh, vd)


@pytest.mark.parametrize("case,tiers_on", [("mismatch_keep", "cpu"), ("mismatch_keep", "cuda"),
                                           ("match_evict", "cpu"), ("match_evict", "cuda"), ("mismatch_evict", "cpu")])
def test_per_sequence_second_reassignment(dev, case, tiers_on):
    """A second per-sequence reassignment of a zero-padded layer.  The padded layout
    keeps row 0's positions (fade/cache.py:1161-1167); where row 0 is not the longest
    they are fewer than the padded rows, and the reference's next call indexes the
    concatenated tiers by position index (token j = row j of sink | middle | recent,
    fade/cache.py:701-713,1084,1124-1133).  The device path (plan + gather) must equal
    the host path bit for bit; eviction over mismatched lengths fails in the reference
    (fade/cache.py:1108-1110) and raises on both paths, the layer untouched."""
    print(f"case per-sequence second reassignment {case} tiers_on={tiers_on}", flush=True)
    B, H = 3, 2
    host, devc = _pair(n_sink=4, recent_window=16, int4_budget=None, int2_budget=0)
    _append((host, devc), B, H, 150, 31, dev)
    rng = np.random.default_rng(32)
    S = host.get_seq_length(0)
    first = (30, None, 70) if case.startswith("mismatch") else (None, None, None)
    tiers = torch.stack([_assign_one_layer(S, torch.from_numpy(rng.exponential(size=S).astype(np.float32)),
                                           4, 16, first[b], 0) for b in range(B)])
    for c in (host, devc):
        c.apply_tier_assignment_per_sequence(0, tiers.clone())
    _same(host, devc, "first reassignment")
    _append((host, devc), B, H, 7, 33, dev)
    _same(host, devc, "append")
    k_full = host._all_in_position_order(0)[0]
    S2 = int(host._all_in_position_order(0)[2].shape[0])
    assert (S2 < int(k_full.shape[-2])) == case.startswith("mismatch")
    second = (None, None, None) if case == "mismatch_keep" else (20, 45, 90)
    tiers2 = torch.stack([_assign_one_layer(S2, torch.from_numpy(rng.exponential(size=S2).astype(np.float32)),
                                            4, 16, second[b], 0) for b in range(B)])
    if tiers_on == "cuda":
        tiers2 = tiers2.to(dev)
    taken = []
    ragged = devc._apply_per_sequence_ragged

    def spy(*args):
        taken.append(1)
        return ragged(*args)

    devc._apply_per_sequence_ragged = spy
    if case == "mismatch_evict":
        for c in (host, devc):
            with pytest.raises(ValueError):
                c.apply_tier_assignment_per_sequence(0, tiers2.clone())
        _same(host, devc, "refused")
        return
    for c in (host, devc):
        c.apply_tier_assignment_per_sequence(0, tiers2.clone())
    assert taken, "device path not taken"
    _same(host, devc, "second reassignment")
    _append((host, devc), B, H, 5, 34, dev)
    _same(host, devc, "append after the second reassignment")
    kh, vh = host._materialize(0)
    kd, vd = devc._materialize(0)
    assert torch.equal(kh, kd) and torch.equal(vh, vd)


RAGGED_FIELDS = (("sink_k", 0), ("sink_v", 0), ("int4_kq", 1), ("int4_vq", 1), ("int4_vs", 1), ("fp16_k", 2),
                 ("fp16_v", 2))


def _single_row_caches(B, n_sink, recent):
    out = []
    for _ in range(B):
        c = TieredKVCache(n_sink=n_sink, recent_window=recent, int4_budget=None, int2_budget=0, head_dim=128)
        c.device_reassign = False  # the host path (the reference's op sequence)
        out.append(c)
    return out


def _check_rows(rag, singles, what):
    st = rag._layers[0]
    assert st.lens is not None
    assert st.lens.cpu().tolist() == st.lens_host
    for b, one in enumerate(singles):
        s1 = one._layers[0]
        ls, lm, lr = st.lens_host[b]
        # the single-row cache splits sink / recent the same way once reassigned
        k1 = {"sink_k": s1.sink_k, "sink_v": s1.sink_v, "fp16_k": s1.fp16_k, "fp16_v": s1.fp16_v,
              "int4_kq": s1.int4_kq, "int4_vq": s1.int4_vq, "int4_vs": s1.int4_vs}
        n = (ls, lm, lr)
        for f, tier in RAGGED_FIELDS:
            x = getattr(st, f)
            y = k1[f]
            ny = 0 if y is None else int(y.shape[-2])
            assert ny == n[tier], f"{what}: row {b} {f}: {ny} rows vs lens {n[tier]}"
            if ny:
                assert torch.equal(x[b : b + 1, :, :ny].cpu(), y.cpu()), f"{what}: row {b} {f} differs"
        if lm:
            assert torch.equal(st.int4_ks[b : b + 1].cpu(), s1.int4_ks.cpu()), f"{what}: row {b} K scale"
        assert rag.get_seq_length(0) == max(sum(r) for r in st.lens_host)
        ko, vo = rag._materialize(0)
        k1m, v1m = one._materialize(0)
        tot = ls + lm + lr
        assert torch.equal(ko[b : b + 1, :, :tot].cpu(), k1m.cpu()) and torch.equal(vo[b : b + 1, :, :tot].cpu(), v1m.cpu())
        assert not ko[b, :, tot:].any()


def test_ragged_layout_matches_single_rows(dev):
    """Ragged per-row reassignment (device) == each row alone through the host path, through
    reassignment, appends, a second reassignment and decode."""
    print("case ragged layout", flush=True)
    B, H, n_sink, recent = 3, 2, 4, 16
    rag = TieredKVCache(n_sink=n_sink, recent_window=recent, int4_budget=None, int2_budget=0, head_dim=128)
    rag.ragged_layout = True
    singles = _single_row_caches(B, n_sink, recent)
    g = torch.Generator().manual_seed(11)
    k = (torch.randn(B, H, 180, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).half().to(dev)
    v = torch.randn(B, H, 180, 128, generator=g).half().to(dev)
    rag.update(k, v, 0)
    for b, c in enumerate(singles):
        c.update(k[b : b + 1], v[b : b + 1], 0)
    rng = np.random.default_rng(3)
    budgets = [30, None, 90]

    def reassign(row_len):
        S = max(row_len)
        tiers = torch.full((B, S), TIER_EVICT, dtype=torch.long)
        for b in range(B):
            sc = torch.from_numpy(rng.exponential(size=row_len[b]).astype(np.float32))
            t = _assign_one_layer(row_len[b], sc, n_sink, recent, budgets[b], 0)
            tiers[b, : row_len[b]] = t
            singles[b].apply_tier_assignment(0, t)
        rag.apply_tier_assignment_per_sequence(0, tiers)

    reassign([180] * B)
    _check_rows(rag, singles, "first reassignment")
    for step in range(3):
        kn = torch.randn(B, H, 1, 128, generator=g).half().to(dev)
        vn = torch.randn(B, H, 1, 128, generator=g).half().to(dev)
        rag.update(kn, vn, 0)
        for b, c in enumerate(singles):
            c.update(kn[b : b + 1], vn[b : b + 1], 0)
    _check_rows(rag, singles, "appends")
    reassign([sum(r) for r in rag._layers[0].lens_host])
    _check_rows(rag, singles, "second reassignment")
    q = torch.randn(B, 8, 1, 128, generator=g).half().to(dev)
    out = rag.decode_attention(q, 0)
    for b, c in enumerate(singles):
        ref = c.decode_attention(q[b : b + 1], 0)
        assert (out[b : b + 1].float() - ref.float()).abs().max().item() <= 2e-3, b


def test_ragged_layout_chunk_prefill_matches_single_rows(dev):
    """A prefill chunk over the ragged layout: rows with different tier lengths after per-row
    reassignment, a multi-token chunk appended to every row, then prefill_attention over the
    ragged layer == each row alone (standard layout) within 2e-3; a later decode agrees too."""
    print("case ragged chunk prefill", flush=True)
    B, H, Hq, n_sink, recent, Sq = 3, 2, 8, 4, 16, 40
    rag = TieredKVCache(n_sink=n_sink, recent_window=recent, int4_budget=None, int2_budget=0, head_dim=128)
    rag.ragged_layout = True
    singles = _single_row_caches(B, n_sink, recent)
    g = torch.Generator().manual_seed(12)
    k = (torch.randn(B, H, 200, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).half().to(dev)
    v = torch.randn(B, H, 200, 128, generator=g).half().to(dev)
    rag.update(k, v, 0)
    for b, c in enumerate(singles):
        c.update(k[b : b + 1], v[b : b + 1], 0)
    rng = np.random.default_rng(4)
    budgets = [25, None, 70]
    tiers = torch.full((B, 200), TIER_EVICT, dtype=torch.long)
    for b in range(B):
        t = _assign_one_layer(200, torch.from_numpy(rng.exponential(size=200).astype(np.float32)), n_sink, recent,
                              budgets[b], 0)
        tiers[b] = t
        singles[b].apply_tier_assignment(0, t)
    rag.apply_tier_assignment_per_sequence(0, tiers)
    assert len({sum(r) for r in rag._layers[0].lens_host}) == B  # three different row lengths
    kc = torch.randn(B, H, Sq, 128, generator=g).half().to(dev)
    vc = torch.randn(B, H, Sq, 128, generator=g).half().to(dev)
    rag.update(kc, vc, 0)
    for b, c in enumerate(singles):
        c.update(kc[b : b + 1], vc[b : b + 1], 0)
    _check_rows(rag, singles, "chunk append")
    q = torch.randn(B, Hq, Sq, 128, generator=g).half().to(dev)
    out = rag.prefill_attention(q, 0)
    for b, c in enumerate(singles):
        ref = c.prefill_attention(q[b : b + 1], 0)
        assert (out[b : b + 1].float() - ref.float()).abs().max().item() <= 2e-3, f"row {b}"
    qd = torch.randn(B, Hq, 1, 128, generator=g).half().to(dev)
    outd = rag.decode_attention(qd, 0)
    for b, c in enumerate(singles):
        assert (outd[b : b + 1].float() - c.decode_attention(qd[b : b + 1], 0).float()).abs().max().item() <= 2e-3


def test_ragged_layout_rejects_shared_calls(dev):
    """A ragged layer refuses the shared-tier entry point; its checkpoint carries the
    per-row lengths (layer.{i}.lens, a key the reference's loader ignores)."""
    rag = TieredKVCache(n_sink=2, recent_window=4, int4_budget=None, int2_budget=0, head_dim=128)
    rag.ragged_layout = True
    kv = torch.randn(2, 2, 20, 128).half().to(dev)
    rag.update(kv, kv, 0)
    tiers = _assign_one_layer(20, torch.zeros(20), 2, 4, None, 0)
    rag.apply_tier_assignment_per_sequence(0, tiers.unsqueeze(0).expand(2, -1).contiguous())
    with pytest.raises(NotImplementedError):
        rag.apply_tier_assignment(0, tiers)
    sd = rag.cache_state_dict()
    assert sd["layer.0.lens"].tolist() == rag._layers[0].lens_host


@pytest.mark.parametrize("budget", [None, 50])
def test_incremental_quant_int4_v(dev, budget):
    """Reference INT4, device path, incremental_quant: K as without it (per-channel scales
    span the tier); V of tokens already in the middle keeps its codes and scales; V of
    tokens entering it equals the whole-tier requantization's."""
    print(f"case incremental int4 budget={budget}", flush=True)
    inc = TieredKVCache(n_sink=4, recent_window=16, int4_budget=budget, int2_budget=0, head_dim=128)
    ref = TieredKVCache(n_sink=4, recent_window=16, int4_budget=budget, int2_budget=0, head_dim=128)
    inc.incremental_quant = True
    _append((inc, ref), 2, 2, 140, 21, dev)
    rng = np.random.default_rng(21)
    for rnd in range(3):
        S = inc.get_seq_length(0)
        tiers = _assign_one_layer(S, torch.from_numpy(rng.exponential(size=S).astype(np.float32)), 4, 16, budget, 0)
        s0 = inc._layers[0]
        if s0.sink_k is not None:
            ns_old = int(s0.sink_k.shape[-2])
        else:
            ns_old = s0.sink_count if s0.fp16_k is not None else 0
        nm_old = 0 if s0.int4_kq is None else int(s0.int4_kq.shape[-2])
        old_vq, old_vs = s0.int4_vq, s0.int4_vs
        inc.apply_tier_assignment(0, tiers)
        ref.apply_tier_assignment(0, tiers)
        a, b = inc._layers[0], ref._layers[0]
        assert torch.equal(a.int4_kq, b.int4_kq) and torch.equal(a.int4_ks, b.int4_ks)
        slots, rows, fresh = TieredKVCache._middle_sources(tiers, ns_old, nm_old)
        if old_vq is not None and slots.numel():
            assert torch.equal(a.int4_vq[:, :, slots.to(dev)], old_vq[:, :, rows.to(dev)])
            assert torch.equal(a.int4_vs[:, :, slots.to(dev)], old_vs[:, :, rows.to(dev)])
        if fresh.numel():
            assert torch.equal(a.int4_vq[:, :, fresh.to(dev)], b.int4_vq[:, :, fresh.to(dev)])
            assert torch.equal(a.int4_vs[:, :, fresh.to(dev)], b.int4_vs[:, :, fresh.to(dev)])
        _append((inc, ref), 2, 2, 23, 121 + rnd, dev)
    q = torch.randn(2, 8, 1, 128, generator=torch.Generator().manual_seed(4)).half().to(dev)
    assert (inc.decode_attention(q, 0).float() - ref.decode_attention(q, 0).float()).abs().max().item() <= 2e-3


@pytest.mark.parametrize("budget", [None, 50])
def test_incremental_quant_asym_backend(dev, budget):
    """Asym group-32 backend (per-token K and V), incremental_quant: tokens already in the
    middle keep their codes (K only when nothing was evicted: re-RoPE changes K), tokens
    entering it are compressed from their fp16 values, as the whole-tier path does."""
    print(f"case incremental asym budget={budget}", flush=True)
    kw = dict(n_sink=4, recent_window=16, int4_budget=budget, int2_budget=0, head_dim=128,
              quant_backend="int4_asym_g32")
    inc, ref = TieredKVCache(**kw), TieredKVCache(**kw)
    inc.incremental_quant = True
    _append((inc, ref), 2, 2, 140, 22, dev)
    rng = np.random.default_rng(22)
    for rnd in range(3):
        S = inc.get_seq_length(0)
        tiers = _assign_one_layer(S, torch.from_numpy(rng.exponential(size=S).astype(np.float32)), 4, 16, budget, 0)
        s0 = inc._layers[0]
        old = None
        if s0.backend_k is not None:
            ns_old = int(s0.sink_pos.shape[0]) if s0.sink_k is not None else (s0.sink_count if s0.fp16_k is not None else 0)
            old = (s0.backend_k, s0.backend_v, ns_old, int(s0.backend_pos.shape[0]))
        evicts = bool((tiers == TIER_EVICT).any())
        inc.apply_tier_assignment(0, tiers)
        ref.apply_tier_assignment(0, tiers)
        a, b = inc._layers[0], ref._layers[0]
        if old is None:
            for key in a.backend_k:
                assert torch.equal(a.backend_k[key], b.backend_k[key]) and torch.equal(a.backend_v[key], b.backend_v[key])
        else:
            keep_idx = (tiers != TIER_EVICT).nonzero().squeeze(-1) if evicts else None
            kept = tiers if keep_idx is None else tiers[keep_idx]
            slots, rows, fresh = TieredKVCache._middle_sources(kept, old[2], old[3], keep_idx)
            for key in a.backend_v:
                if slots.numel():
                    assert torch.equal(a.backend_v[key][:, :, slots.to(dev)], old[1][key][:, :, rows.to(dev)])
                    if not evicts:
                        assert torch.equal(a.backend_k[key][:, :, slots.to(dev)], old[0][key][:, :, rows.to(dev)])
                if fresh.numel():
                    assert torch.equal(a.backend_v[key][:, :, fresh.to(dev)], b.backend_v[key][:, :, fresh.to(dev)])
                    assert torch.equal(a.backend_k[key][:, :, fresh.to(dev)], b.backend_k[key][:, :, fresh.to(dev)])
                if evicts:
                    assert torch.equal(a.backend_k[key], b.backend_k[key])
        _append((inc, ref), 2, 2, 23, 122 + rnd, dev)
    q = torch.randn(2, 8, 1, 128, generator=torch.Generator().manual_seed(4)).half().to(dev)
    assert (inc.decode_attention(q, 0).float() - ref.decode_attention(q, 0).float()).abs().max().item() <= 2e-3
