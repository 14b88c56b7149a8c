"""GPU parity of the ragged tiered prefill attention against the oracle.

Each batch row has its own sink / INT4 middle / recent lengths (tiers padded
to a common capacity) and appends a chunk of Sq tokens; the oracle
materializes the row's cache (fade/cache.py:683-842) plus the chunk and runs
fp32 attention with the bottom-right causal mask.  Tolerance: max-abs 2e-3.
"""

import numpy as np
import pytest
import torch

from fade_amd.kernels import MiddleTier, tiered_prefill_attention
from fade_amd.synthetic import kv_tensors
from oracle import attention as oatt
from oracle import quant as oq

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def _ragged(dev, B, Hq, Hkv, Sq, rows, seed, with_mid=True):
    """rows: per-row (n_sink, n_mid, n_recent).  Returns kernel inputs and oracle outputs."""
    D = 128
    caps = [max(r[i] for r in rows) for i in range(3)]
    caps[1] = caps[1] if with_mid else 0
    sink_k = np.zeros((B, Hkv, caps[0], D), np.float16)
    sink_v = np.zeros_like(sink_k)
    rec_k = np.zeros((B, Hkv, caps[2], D), np.float16)
    rec_v = np.zeros_like(rec_k)
    kq = np.zeros((B, Hkv, caps[1], D // 2), np.uint8)
    vq = np.zeros_like(kq)
    ks = np.ones((B, Hkv, 1, D), np.float16)
    vs = np.ones((B, Hkv, caps[1], 1), np.float16)
    chunk_k = np.zeros((B, Hkv, Sq, D), np.float16)
    chunk_v = np.zeros_like(chunk_k)
    qs = np.zeros((B, Hq, Sq, D), np.float16)
    q_list, k_list, v_list = [], [], []
    for b, (ns, nm, nr) in enumerate(rows):
        nm = nm if with_mid else 0
        L = ns + nm + nr
        q, k, v = kv_tensors(1, Hkv, L + Sq, D, seed=seed + b, Hq=Hq, Sq=Sq)
        q, k, v = q.numpy(), k.numpy(), v.numpy()
        qs[b] = q[0]
        sink_k[b, :, :ns], sink_v[b, :, :ns] = k[0, :, :ns], v[0, :, :ns]
        parts_k, parts_v = [k[0, :, :ns]], [v[0, :, :ns]]
        if nm:
            kq_b, ks_b = oq.quant_k_int4(k[:, :, ns : ns + nm])
            vq_b, vs_b = oq.quant_v_int4(v[:, :, ns : ns + nm])
            kq[b, :, :nm], ks[b], vq[b, :, :nm], vs[b, :, :nm] = kq_b[0], ks_b[0], vq_b[0], vs_b[0]
            parts_k.append(oq.dequant_int4(kq_b, ks_b)[0])
            parts_v.append(oq.dequant_int4(vq_b, vs_b)[0])
        rec_k[b, :, :nr], rec_v[b, :, :nr] = k[0, :, ns + nm : L], v[0, :, ns + nm : L]
        parts_k.append(k[0, :, ns + nm : L])
        parts_v.append(v[0, :, ns + nm : L])
        chunk_k[b], chunk_v[b] = k[0, :, L:], v[0, :, L:]
        parts_k.append(k[0, :, L:])
        parts_v.append(v[0, :, L:])
        q_list.append(q[0])
        k_list.append(np.concatenate(parts_k, axis=-2))
        v_list.append(np.concatenate(parts_v, axis=-2))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(sink_k), t(sink_v)) if caps[0] else None
    rec = (t(rec_k), t(rec_v)) if caps[2] else None
    mid = MiddleTier("int4", t(kq), t(vq), t(ks), t(vs)) if caps[1] else None
    lens = torch.tensor([[r[0], r[1] if with_mid else 0, r[2]] for r in rows], dtype=torch.int32)
    ref = np.stack(oatt.ragged_prefill(q_list, k_list, v_list))
    return t(qs), (t(chunk_k), t(chunk_v)), sink, mid, rec, lens, ref


@pytest.mark.parametrize(
    "B,Hq,Hkv,Sq,rows",
    [
        (3, 32, 8, 128, [(4, 700, 64), (4, 300, 64), (2, 1500, 30)]),  # config-4 shape, ragged
        (2, 8, 2, 40, [(4, 100, 64), (0, 0, 5)]),  # Sq not a multiple of 32; a row without middle
        (2, 8, 4, 17, [(1, 63, 1), (4, 64, 64)]),  # G=2, tile-boundary lengths
        (1, 4, 4, 64, [(0, 1, 0)]),  # MHA, one middle token
        (2, 28, 4, 70, [(4, 500, 64), (2, 130, 20)]),  # G=7 (Qwen2.5-7B heads): two head passes
        (1, 40, 8, 33, [(4, 200, 10)]),  # G=5: a second pass of one head
        (1, 16, 2, 96, [(4, 300, 64)]),  # G=8
        (2, 8, 4, 128, [(4, 600, 64), (2, 70, 10)]),  # G=2: each group of 4 waves covers 2 query blocks
        (1, 4, 4, 200, [(4, 333, 64)]),  # MHA: 4 query blocks per group, two groups, a partial last block
        (2, 6, 2, 100, [(3, 250, 64), (4, 64, 1)]),  # G=3: 4-head groups with one idle wave
    ],
)
def test_tiered_prefill_ragged(dev, B, Hq, Hkv, Sq, rows):
    print(f"case prefill B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} rows={rows}", flush=True)
    q, chunk, sink, mid, rec, lens, ref = _ragged(dev, B, Hq, Hkv, Sq, rows, seed=4000 + Sq)
    out = tiered_prefill_attention(q, chunk, sink, mid, rec, lens=lens)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL


@pytest.mark.parametrize("heads", [(32, 8), (28, 4), (20, 4)])
def test_tiered_prefill_paged_middle(dev, heads):
    """A paged middle tier (64-token pages of one pool, shuffled, per-row block table):
    the kernel reads the pages in place and gives the padded layout's output bit for bit;
    at 4 query heads per kv head (one head pass) and at 7 and 5 (two head passes)."""
    from fade_amd.kernels.tiered_attn import paginate_middle

    print(f"case prefill paged middle heads={heads}", flush=True)
    rows = [(4, 700, 64), (4, 130, 20), (2, 0, 64), (1, 64, 5)]
    q, chunk, sink, mid, rec, lens, ref = _ragged(dev, 4, heads[0], heads[1], 96, rows, seed=4500)
    n_pages = sum(-(-r[1] // 64) for r in rows)
    paged = paginate_middle(mid, [r[1] for r in rows], order=np.random.default_rng(3).permutation(n_pages))
    out_r = tiered_prefill_attention(q, chunk, sink, mid, rec, lens=lens)
    out_p = tiered_prefill_attention(q, chunk, sink, paged, rec, lens=lens)
    assert torch.equal(out_r, out_p)
    assert np.abs(out_p.float().cpu().numpy() - ref).max() <= ATOL


def test_tiered_prefill_order_and_fp16_only(dev):
    """Dispatch order does not change results; a cache with no middle tier works."""
    print("case prefill order / fp16-only", flush=True)
    rows = [(4, 0, 64), (4, 0, 20), (2, 0, 64)]
    q, chunk, sink, mid, rec, lens, ref = _ragged(dev, 3, 16, 4, 50, rows, seed=77, with_mid=False)
    assert mid is None
    out1 = tiered_prefill_attention(q, chunk, sink, None, rec, lens=lens)
    out2 = tiered_prefill_attention(q, chunk, sink, None, rec, lens=lens, order=torch.tensor([2, 0, 1]))
    assert torch.equal(out1, out2)
    assert np.abs(out1.float().cpu().numpy() - ref).max() <= ATOL


def test_tiered_prefill_lengths_clamped_to_capacity(dev):
    """Per-row lengths beyond the padded capacity are clamped (no read past a tier)."""
    print("case prefill clamp", flush=True)
    rows = [(4, 200, 64), (4, 200, 64)]
    q, chunk, sink, mid, rec, lens, ref = _ragged(dev, 2, 8, 2, 32, rows, seed=91)
    big = torch.tensor([[99, 10_000, 999], [4, 200, 64]], dtype=torch.int32)
    out = tiered_prefill_attention(q, chunk, sink, mid, rec, lens=big)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL
