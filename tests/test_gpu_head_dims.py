"""Head dims other than 128 on the fused attention path, against the oracle.

The reference's quantizers and kernels take any even head_dim
(fade/quant.py:36-37; its fused-kernel tests run D = 64,
tests/test_fused_blackwell.py:50-109, its INT4 SDPA tests D = 32,
tests/test_perf.py:17, its model tests D = 16, tests/test_models.py:43-49).
Here every multiple of 8 up to 256 is taken: decode at D != 128 runs the
portable kernel (every middle format; instances of capacity 32/64/128/256,
channels past D idle), the MFMA prefill kernel takes D up to 256 (a packed
middle tier in place at multiples of 32, its fp16 dequantization otherwise;
D > 128 on the capacity-256 instance, one wave per SIMD).  Tolerance: max-abs 2e-3 against fp32 attention over the oracle's
dequantized tiers, as for D = 128.
"""

import numpy as np
import pytest
import torch

from fade_amd import quant as fq
from fade_amd.kernels import MiddleTier, fused_int4_sdpa, int4_sdpa, tiered_decode_attention, tiered_prefill_attention
from fade_amd.synthetic import kv_tensors
from oracle import attention as oatt
from oracle import quant as oq

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def _t(dev, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _mid(dev, fmt, km, vm):
    """A middle tier of format ``fmt`` from fp16 K/V (numpy), for the kernel and the oracle."""
    if fmt == "fp16":
        return MiddleTier("fp16", _t(dev, km), _t(dev, vm)), {"fmt": "fp16", "k": km, "v": vm}
    kq, ks = fq.quant_k_int4(_t(dev, km))
    okq, oks = oq.quant_k_int4(km)
    if fmt == "int4":
        vq, vs = fq.quant_v_int4(_t(dev, vm))
        ovq, ovs = oq.quant_v_int4(vm)
        return MiddleTier("int4", kq, vq, ks, vs), {"fmt": "int4", "kq": okq, "ks": oks, "vq": ovq, "vs": ovs}
    if fmt == "k4v2":
        n = km.shape[2]
        vq, vs = fq.quant_int2_padded(_t(dev, vm), 64)
        ovq, ovs = oq.quant_int2_grouped(oq.pad_to_group(vm, 64)[0], 64)
        return (MiddleTier("k4v2", kq, vq, ks, vs, group=64, length=n),
                {"fmt": "k4v2", "kq": okq, "ks": oks, "vq": ovq, "vs": ovs, "group": 64})
    # asym, K 4-bit / V 2-bit, groups of 32 (16 at D = 32 would be the same layout rule)
    kp, ksc, kz = fq.quant_asym(_t(dev, km), 4, 32)
    vp, vsc, vz = fq.quant_asym(_t(dev, vm), 2, 32)
    okp, oks2, okz = oq.quant_asym_group(km, 4, 32)
    ovp, ovs2, ovz = oq.quant_asym_group(vm, 2, 32)
    return (MiddleTier("asym", kp, vp, ksc, vsc, kz, vz, k_bits=4, v_bits=2, group=32),
            {"fmt": "asym", "kq": okp, "ks": oks2, "kz": okz, "vq": ovp, "vs": ovs2, "vz": ovz,
             "k_bits": 4, "v_bits": 2, "group": 32})


@pytest.mark.parametrize("D", [32, 64, 256, 16, 80, 96, 160])
@pytest.mark.parametrize("fmt", ["int4", "fp16", "k4v2", "asym"])
@pytest.mark.parametrize("B,Hq,Hkv,S,ns,nr", [(2, 8, 2, 700, 4, 64), (1, 16, 2, 130, 0, 7), (3, 4, 4, 70, 2, 0)])
def test_decode_head_dims(dev, D, fmt, B, Hq, Hkv, S, ns, nr):
    if fmt == "asym" and D % 32:
        pytest.skip("the asymmetric format's 32-channel groups need D % 32 == 0")
    print(f"case decode D={D} {fmt} B={B} Hq={Hq} Hkv={Hkv} S={S} ns={ns} nr={nr}", flush=True)
    q, k, v = (x.numpy() for x in kv_tensors(B, Hkv, S, D, seed=300 + D + S, Hq=Hq))
    mid, omid = _mid(dev, fmt, k[:, :, ns : S - nr], v[:, :, ns : S - nr])
    sink = (_t(dev, k[:, :, :ns]), _t(dev, v[:, :, :ns])) if ns else None
    rec = (_t(dev, k[:, :, S - nr :]), _t(dev, v[:, :, S - nr :])) if nr else None
    ref = oatt.tiered_decode(q, k[:, :, :ns], v[:, :, :ns], omid, k[:, :, S - nr :], v[:, :, S - nr :])
    for n_splits in (0, 1, 3):  # 1: the portable kernel writes the output itself
        out = tiered_decode_attention(_t(dev, q), sink, mid, rec, n_splits=n_splits)
        assert out.shape == (B, Hq, 1, D)
        assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL, n_splits


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("fmt", ["int4", "fp16", None])
@pytest.mark.parametrize("B,Hq,Hkv,S,ns,nr", [(2, 14, 2, 900, 4, 64), (3, 8, 8, 333, 2, 17), (1, 32, 8, 4100, 4, 128)])
def test_decode_head_dim_64_256_matrix_core(dev, D, fmt, B, Hq, Hkv, S, ns, nr):
    """head_dims 64 and 256 on the general matrix-core kernel (kernel=3, the automatic choice
    at these head_dims for the reference INT4, fp16 and empty middle tiers): Qwen2.5-0.5B's
    14/2 heads, MHA, a partial last tile; against the oracle and the portable kernel (kernel=1)."""
    print(f"case decode D={D} matrix-core {fmt} B={B} Hq={Hq} Hkv={Hkv} S={S}", flush=True)
    q, k, v = (x.numpy() for x in kv_tensors(B, Hkv, S, D, seed=640 + S + D, Hq=Hq))
    if fmt is None:
        mid, omid = None, None
        ref = oatt.sdpa_fp32(q, k, v)
        sink, rec = (_t(dev, k), _t(dev, v)), None
    else:
        mid, omid = _mid(dev, fmt, k[:, :, ns : S - nr], v[:, :, ns : S - nr])
        ref = oatt.tiered_decode(q, k[:, :, :ns], v[:, :, :ns], omid, k[:, :, S - nr :], v[:, :, S - nr :])
        sink = (_t(dev, k[:, :, :ns]), _t(dev, v[:, :, :ns])) if ns else None
        rec = (_t(dev, k[:, :, S - nr :]), _t(dev, v[:, :, S - nr :])) if nr else None
    qd = _t(dev, q)
    outs = {}
    for kern in (3, 0, 1):
        for n_splits in (0, 1, 5):
            out = tiered_decode_attention(qd, sink, mid, rec, n_splits=n_splits, kernel=kern)
            assert out.shape == (B, Hq, 1, D)
            err = np.abs(out.float().cpu().numpy() - ref).max()
            assert err <= ATOL, (kern, n_splits, err)
            outs[(kern, n_splits)] = out
    assert (outs[(3, 0)].float() - outs[(1, 0)].float()).abs().max().item() <= ATOL


def _ragged(dev, D, B, Hq, Hkv, Sq, rows, seed, fmt="int4"):
    """rows: per-row (n_sink, n_mid, n_recent), tiers padded to common capacities."""
    caps = [max(r[i] for r in rows) for i in range(3)]
    sink_k = np.zeros((B, Hkv, caps[0], D), np.float16)
    sink_v = np.zeros_like(sink_k)
    rec_k = np.zeros((B, Hkv, caps[2], D), np.float16)
    rec_v = np.zeros_like(rec_k)
    kq = np.zeros((B, Hkv, caps[1], D // 2), np.uint8)
    vq = np.zeros_like(kq)
    ks = np.ones((B, Hkv, 1, D), np.float16)
    vs = np.ones((B, Hkv, caps[1], 1), np.float16)
    mk16 = np.zeros((B, Hkv, caps[1], D), np.float16)
    mv16 = np.zeros_like(mk16)
    chunk_k = np.zeros((B, Hkv, Sq, D), np.float16)
    chunk_v = np.zeros_like(chunk_k)
    qs = np.zeros((B, Hq, Sq, D), np.float16)
    q_list, k_list, v_list = [], [], []
    for b, (ns, nm, nr) in enumerate(rows):
        L = ns + nm + nr
        q, k, v = (x.numpy() for x in kv_tensors(1, Hkv, L + Sq, D, seed=seed + b, Hq=Hq, Sq=Sq))
        qs[b] = q[0]
        sink_k[b, :, :ns], sink_v[b, :, :ns] = k[0, :, :ns], v[0, :, :ns]
        parts_k, parts_v = [k[0, :, :ns]], [v[0, :, :ns]]
        if nm:
            km, vm = k[:, :, ns : ns + nm], v[:, :, ns : ns + nm]
            if fmt == "int4":
                kq_b, ks_b = oq.quant_k_int4(km)
                vq_b, vs_b = oq.quant_v_int4(vm)
                kq[b, :, :nm], ks[b], vq[b, :, :nm], vs[b, :, :nm] = kq_b[0], ks_b[0], vq_b[0], vs_b[0]
                parts_k.append(oq.dequant_int4(kq_b, ks_b)[0])
                parts_v.append(oq.dequant_int4(vq_b, vs_b)[0])
            else:
                mk16[b, :, :nm], mv16[b, :, :nm] = km[0], vm[0]
                parts_k.append(km[0])
                parts_v.append(vm[0])
        rec_k[b, :, :nr], rec_v[b, :, :nr] = k[0, :, ns + nm : L], v[0, :, ns + nm : L]
        parts_k.append(k[0, :, ns + nm : L])
        parts_v.append(v[0, :, ns + nm : L])
        chunk_k[b], chunk_v[b] = k[0, :, L:], v[0, :, L:]
        parts_k.append(k[0, :, L:])
        parts_v.append(v[0, :, L:])
        q_list.append(q[0])
        k_list.append(np.concatenate(parts_k, axis=-2))
        v_list.append(np.concatenate(parts_v, axis=-2))
    sink = (_t(dev, sink_k), _t(dev, sink_v)) if caps[0] else None
    rec = (_t(dev, rec_k), _t(dev, rec_v)) if caps[2] else None
    mid = None
    if caps[1]:
        mid = (MiddleTier("int4", _t(dev, kq), _t(dev, vq), _t(dev, ks), _t(dev, vs)) if fmt == "int4"
               else MiddleTier("fp16", _t(dev, mk16), _t(dev, mv16)))
    lens = torch.tensor([list(r) for r in rows], dtype=torch.int32)
    ref = np.stack(oatt.ragged_prefill(q_list, k_list, v_list))
    return _t(dev, qs), (_t(dev, chunk_k), _t(dev, chunk_v)), sink, mid, rec, lens, ref


@pytest.mark.parametrize("D", [32, 64, 16, 48, 80, 96, 256, 160, 200, 136])
@pytest.mark.parametrize("fmt", ["int4", "fp16"])
@pytest.mark.parametrize(
    "B,Hq,Hkv,Sq,rows",
    [
        (3, 8, 2, 128, [(4, 700, 64), (4, 300, 64), (2, 1500, 30)]),  # ragged rows, G=4
        (2, 8, 4, 17, [(1, 63, 1), (4, 64, 64)]),  # G=2, tile-boundary lengths
        (1, 14, 2, 70, [(4, 500, 64)]),  # G=7: two head passes
        (1, 4, 4, 33, [(0, 1, 0)]),  # MHA, one middle token
    ],
)
def test_prefill_head_dims(dev, D, fmt, B, Hq, Hkv, Sq, rows):
    print(f"case prefill D={D} {fmt} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} rows={rows}", flush=True)
    q, chunk, sink, mid, rec, lens, ref = _ragged(dev, D, B, Hq, Hkv, Sq, rows, seed=500 + D, fmt=fmt)
    out = tiered_prefill_attention(q, chunk, sink, mid, rec, lens=lens)
    assert out.shape == (B, Hq, Sq, D)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL


@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("Sq,causal", [(1, False), (5, False), (40, True), (1, True)])
def test_fused_int4_sdpa_head_dims(dev, D, Sq, causal):
    """fused_int4_sdpa (decode for one query row, the prefill kernel otherwise) with GQA."""
    print(f"case fused_int4_sdpa D={D} Sq={Sq} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(D + Sq)
    q = torch.randn(2, 8, Sq, D, generator=g).half()
    k = torch.randn(2, 2, 90, D, generator=g).half()
    v = torch.randn(2, 2, 90, D, generator=g).half()
    kq, ks = oq.quant_k_int4(k.numpy())
    vq, vs = oq.quant_v_int4(v.numpy())
    kd = np.repeat(oq.dequant_int4(kq, ks), 4, axis=1)
    vd = np.repeat(oq.dequant_int4(vq, vs), 4, axis=1)
    mask = None
    if causal:  # top-left: query i sees keys 0..i
        mask = np.arange(90)[None, :] <= np.arange(Sq)[:, None]
    ref = oatt.sdpa_fp32(q.numpy(), kd, vd, mask=mask)
    out = fused_int4_sdpa(q.to(dev), _t(dev, kq), _t(dev, ks), _t(dev, vq), _t(dev, vs), is_causal=causal)
    assert out.shape == (2, 8, Sq, D)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL


# ------------------------------------------- tests/test_fused_blackwell.py (D = 64)
def test_fused_int4_sdpa_parity_reference_shape(dev):  # :45-69
    g = torch.Generator().manual_seed(45)
    q = torch.randn(1, 4, 1, 64, generator=g).half().to(dev)
    k_fp = torch.randn(1, 4, 128, 64, generator=g).half().to(dev)
    v_fp = torch.randn(1, 4, 128, 64, generator=g).half().to(dev)
    kp, ks = fq.quant_k_int4(k_fp)
    vp, vs = fq.quant_v_int4(v_fp)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.float(), fq.dequant_int4(kp, ks).float(), fq.dequant_int4(vp, vs).float())
    fused = fused_int4_sdpa(q, kp, ks, vp, vs)
    assert fused.shape == ref.shape
    assert (fused.float() - ref).abs().max().item() < 0.05


def test_fused_int4_sdpa_causal_reference_shape(dev):  # :72-89
    g = torch.Generator().manual_seed(72)
    q = torch.randn(1, 4, 32, 64, generator=g).half().to(dev)
    k_fp = torch.randn(1, 4, 32, 64, generator=g).half().to(dev)
    v_fp = torch.randn(1, 4, 32, 64, generator=g).half().to(dev)
    kp, ks = fq.quant_k_int4(k_fp)
    vp, vs = fq.quant_v_int4(v_fp)
    out = fused_int4_sdpa(q, kp, ks, vp, vs, is_causal=True)
    assert out.shape == (1, 4, 32, 64)
    assert not torch.isnan(out).any()


def test_fused_gqa_broadcast_reference_shape(dev):  # :92-109
    g = torch.Generator().manual_seed(92)
    q = torch.randn(1, 8, 1, 64, generator=g).half().to(dev)
    k_fp = torch.randn(1, 2, 64, 64, generator=g).half().to(dev)
    v_fp = torch.randn(1, 2, 64, 64, generator=g).half().to(dev)
    kp, ks = fq.quant_k_int4(k_fp)
    vp, vs = fq.quant_v_int4(v_fp)
    out = fused_int4_sdpa(q, kp, ks, vp, vs)
    assert out.shape == (1, 8, 1, 64)
    assert not torch.isnan(out).any()


# ------------------------------------------------ tests/test_perf.py (B, H, D = 1, 2, 32)
def test_int4_sdpa_fallback_produces_valid_output(dev):  # :147-160 (float32 tensors, as the reference)
    g = torch.Generator().manual_seed(147)
    q = torch.randn(1, 2, 4, 32, generator=g).to(dev)
    k_fp = torch.randn(1, 2, 16, 32, generator=g).to(dev)
    v_fp = torch.randn(1, 2, 16, 32, generator=g).to(dev)
    kp, ks = fq.quant_k_int4(k_fp)
    vp, vs = fq.quant_v_int4(v_fp)
    out = int4_sdpa(q, kp, ks, vp, vs, dtype=torch.float32)
    assert out.shape == (1, 2, 4, 32)
    assert torch.isfinite(out).all()


def test_int4_sdpa_matches_fp16_attention_approximately(dev):  # :163-180
    g = torch.Generator().manual_seed(163)
    q = torch.randn(1, 2, 1, 32, generator=g).to(dev)
    k_fp = torch.randn(1, 2, 32, 32, generator=g).to(dev)
    v_fp = torch.randn(1, 2, 32, 32, generator=g).to(dev)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k_fp, v_fp)
    kp, ks = fq.quant_k_int4(k_fp)
    vp, vs = fq.quant_v_int4(v_fp)
    out = int4_sdpa(q, kp, ks, vp, vs, dtype=torch.float32)
    rel_err = ((out - ref).abs().mean() / ref.abs().mean()).item()
    assert rel_err < 0.3


@pytest.mark.parametrize("D", [64, 32])
def test_decode_head_dims_ragged_lens(dev, D):
    """Per-row tier lengths on the portable kernel: row b attends to the first lens[b]
    rows of each padded tier, checked against the oracle over its own tokens."""
    print(f"case decode ragged D={D}", flush=True)
    ns_c, mc, nr_c, B = 4, 600, 64, 5
    S = ns_c + mc + nr_c
    q, k, v = (x.numpy() for x in kv_tensors(B, 4, S, D, seed=77, Hq=16))
    km, vm = k[:, :, ns_c : S - nr_c], v[:, :, ns_c : S - nr_c]
    mid, omid = _mid(dev, "int4", km, vm)
    lens = np.array([[4, 600, 64], [2, 130, 17], [4, 1, 0], [0, 333, 64], [1, 0, 5]], dtype=np.int32)
    sink = (_t(dev, k[:, :, :ns_c]), _t(dev, v[:, :, :ns_c]))
    rec = (_t(dev, k[:, :, S - nr_c :]), _t(dev, v[:, :, S - nr_c :]))
    for n_splits in (0, 1, 7):
        out = tiered_decode_attention(_t(dev, q), sink, mid, rec, lens=_t(dev, lens), n_splits=n_splits)
        out = out.float().cpu().numpy()
        for b, (ls, lm, lr) in enumerate(lens):
            # the row's own middle tokens; per-channel K scales stay the whole tier's
            om = {"fmt": "int4", "kq": omid["kq"][b : b + 1, :, :lm], "ks": omid["ks"][b : b + 1],
                  "vq": omid["vq"][b : b + 1, :, :lm], "vs": omid["vs"][b : b + 1, :, :lm]}
            ref = oatt.tiered_decode(q[b : b + 1], k[b : b + 1, :, :ls], v[b : b + 1, :, :ls], om,
                                     k[b : b + 1, :, S - nr_c : S - nr_c + lr], v[b : b + 1, :, S - nr_c : S - nr_c + lr])
            assert np.abs(out[b : b + 1] - ref).max() <= ATOL, (n_splits, b)


# ------------------------------------------------------- the cache at head_dim 64
@pytest.mark.parametrize("backend,v_bits", [("int4", 4), ("int4", 2), ("rotated", 4), ("rotated3", 4),
                                            ("int4_asym_g32", 4)])
def test_cache_decode_and_prefill_head_dim_64(dev, backend, v_bits):
    """TieredKVCache at head_dim 64 (Qwen2.5-0.5B's): decode and chunk prefill over
    sink / middle / recent against fp32 attention over the cache's own materialized K/V."""
    from fade_amd import FadeConfig, TieredKVCache
    from fade_amd.backends import get_backend
    from fade_amd.policy import reassign_tiers_by_position

    print(f"case cache D=64 {backend} v_bits={v_bits}", flush=True)
    D = 64
    _, k, v = kv_tensors(1, 2, 600, D, seed=6)
    if backend == "rotated3":
        c = TieredKVCache(head_dim=D, n_sink=4, recent_window=64, int4_budget=None,
                          quant_backend=get_backend("rotated", head_dim=D, bits=3))
    else:
        kw = FadeConfig(quant_backend=backend).to_cache_kwargs()
        kw.update(head_dim=D, n_sink=4, recent_window=64, middle_v_bits=v_bits)
        c = TieredKVCache(**kw)
    c.update(k.to(dev), v.to(dev), 0)
    reassign_tiers_by_position(c, 1)
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 14, 1, D, generator=g).to(torch.float16)
    K, V = c._materialize(0)
    fused = c.decode_attention(q.to(dev), 0).float().cpu().numpy()
    ref = oatt.sdpa_fp32(q.numpy(), K.cpu().numpy(), V.cpu().numpy())
    assert np.abs(fused - ref).max() <= ATOL
    # a chunk of 40 tokens appended, then attended causally over the whole cache
    _, kc, vc = kv_tensors(1, 2, 40, D, seed=8)
    c.update(kc.to(dev), vc.to(dev), 0)
    qc = torch.randn(1, 14, 40, D, generator=g).to(torch.float16)
    K, V = c._materialize(0)
    out = c.prefill_attention(qc.to(dev), 0).float().cpu().numpy()
    ref = oatt.sdpa_fp32(qc.numpy(), K.cpu().numpy(), V.cpu().numpy(),
                         mask=oatt.bottom_right_causal_mask(40, int(K.shape[-2])))
    assert np.abs(out - ref).max() <= ATOL


def test_cache_per_sequence_head_dim_64(dev):
    """Per-sequence assignment (ragged rows) at head_dim 64: each row's tiers equal a
    single-row cache of that row, and both decode it within the parity bar."""
    from fade_amd import TieredKVCache
    from fade_amd.policy import _assign_one_layer

    print("case cache D=64 per-sequence", flush=True)
    D = 64
    _, k, v = kv_tensors(2, 2, 300, D, seed=8)
    g = torch.Generator().manual_seed(9)
    t = torch.stack([_assign_one_layer(300, torch.rand(300, generator=g), 4, 32, 100, 0) for _ in range(2)])
    c = TieredKVCache(head_dim=D, n_sink=4, recent_window=32, int4_budget=100)
    c.ragged_layout = True  # each row keeps its own tokens (per-row tier lengths)
    c.update(k.to(dev), v.to(dev), 0)
    c.apply_tier_assignment_per_sequence(0, t)
    q = torch.randn(2, 8, 1, D, generator=g).to(torch.float16).to(dev)
    out = c.decode_attention(q, 0)
    for b in range(2):
        cb = TieredKVCache(head_dim=D, n_sink=4, recent_window=32, int4_budget=100)
        cb.update(k[b : b + 1].to(dev), v[b : b + 1].to(dev), 0)
        cb.apply_tier_assignment(0, t[b].to(dev))
        ob = cb.decode_attention(q[b : b + 1], 0)
        # The ragged layout decodes with per-row lengths (portable kernel), the single-row
        # cache on the matrix-core kernel: both against fp32 attention over the single-row
        # cache's materialized tiers, at the parity bar.
        km, vm = cb._materialize(0)
        ref = torch.nn.functional.scaled_dot_product_attention(
            q[b : b + 1].float(), km.float().repeat_interleave(4, 1), vm.float().repeat_interleave(4, 1))
        e = max((out[b : b + 1].float() - ref).abs().max().item(), (ob.float() - ref).abs().max().item())
        if e > ATOL:  # say which tier differs and whether the decodes repeat
            st, sb = c._layers[0], cb._layers[0]
            ls, lm, lr = st.lens_host[b]
            tiers = {
                "sink": torch.equal(st.sink_k[b : b + 1, :, :ls], sb.sink_k),
                "int4_kq": torch.equal(st.int4_kq[b : b + 1, :, :lm], sb.int4_kq),
                "int4_ks": torch.equal(st.int4_ks[b : b + 1], sb.int4_ks),
                "int4_vq": torch.equal(st.int4_vq[b : b + 1, :, :lm], sb.int4_vq),
                "int4_vs": torch.equal(st.int4_vs[b : b + 1, :, :lm], sb.int4_vs),
                "recent": torch.equal(st.fp16_k[b : b + 1, :, :lr], sb.fp16_k),
            }
            again = (c.decode_attention(q, 0)[b : b + 1].float() - cb.decode_attention(q[b : b + 1], 0).float())
            pytest.fail(f"row {b}: error {e:.3g}; tiers equal {tiers}; re-run error {again.abs().max().item():.3g}")
