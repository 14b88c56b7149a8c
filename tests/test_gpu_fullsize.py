"""Parity at the configurations' full sizes (configs 1-4).

The oracle is too slow for a whole configuration, so each test combines
- properties that hold at any size: code range, the largest element of every
  quantization group mapping to +-7, the dequantization error bound, split
  invariance, host path == device path;
- exact checks on slices the oracle finishes in seconds. Outputs are
  independent per batch row, and K scales are per (row, head), so the oracle
  run on one or two rows is exact for those rows of the full-size GPU run.
"""

import numpy as np
import pytest
import torch

from fade_amd import quant as fq
from fade_amd.cache import TieredKVCache
from fade_amd.kernels import MiddleTier, tiered_decode_attention
from fade_amd.kernels.prefill import tiered_prefill_attention
from fade_amd.policy import _assign_one_layer
from fade_amd.synthetic import exp_scores, kv_tensors
from oracle import attention as oatt
from oracle import quant as oq

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def _codes(packed: torch.Tensor) -> torch.Tensor:
    """Two's-complement nibbles (high nibble = even channel) -> int8 codes."""
    hi = (packed >> 4).to(torch.int8)
    lo = (packed & 15).to(torch.int8)
    c = torch.stack((hi, lo), dim=-1).flatten(-2)
    return (c ^ 8) - 8


def _quant_properties(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, group_dim: int):
    """Symmetric INT4 invariants at full size; group_dim = the reduced axis (2: per channel, 3: per token)."""
    c = _codes(packed)
    assert int(c.min()) >= -7 and int(c.max()) <= 7, "codes outside [-7, 7]"
    xa = x.float().abs()
    amax = xa.amax(dim=group_dim, keepdim=True)
    at_max = (xa == amax) & (amax > 0)
    assert bool((c.abs()[at_max] == 7).all()), "a group's largest element does not map to +-7"
    deq = (c.half() * scale).float()
    err = (x.float() - deq).abs()
    bound = 0.52 * scale.float().expand_as(err)
    assert bool((err <= bound + 1e-7).all()), f"dequantization error above 0.52 scale: {float((err - bound).max())}"


def _mid_dict(kq, ks, vq, vs):
    return {"fmt": "int4", "kq": kq, "ks": ks, "vq": vq, "vs": vs}


def _nonzero_counters():
    """(buffer key, nonzero split counters) of every shared decode workspace; the
    counters of B*Hkv*passes slots sit at the front of each buffer and are zero between calls."""
    from fade_amd import _lib

    torch.cuda.synchronize()
    bad = []
    for key, ws in _lib._STREAM_WS.items():
        n = int((ws[: 4 * key[2]].view(torch.int32) != 0).sum())
        if n:
            bad.append((key, n))
    return bad


def _decode_case(dev, B, Hkv, S, ns, nr, seed, rows, check_quant=True):
    print(f"case full-size decode B={B} Hkv={Hkv} S={S} rows={rows}", flush=True)
    q, k, v = kv_tensors(B, Hkv, S, 128, seed=seed, Hq=32)
    km, vm = k[:, :, ns : S - nr], v[:, :, ns : S - nr]
    kmg, vmg = km.to(dev), vm.to(dev)
    kq, ks = fq.quant_k_int4(kmg)
    vq, vs = fq.quant_v_int4(vmg)
    if check_quant:
        _quant_properties(kmg, kq, ks, group_dim=2)
        _quant_properties(vmg, vq, vs, group_dim=3)
    del kmg, vmg
    t = lambda a: a.contiguous().to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns]), t(v[:, :, :ns]))
    rec = (t(k[:, :, S - nr :]), t(v[:, :, S - nr :]))
    mid = MiddleTier("int4", kq, vq, ks, vs)
    qg = q.to(dev)
    before = _nonzero_counters()
    out = tiered_decode_attention(qg, sink, mid, rec)
    one = tiered_decode_attention(qg, sink, mid, rec, n_splits=1)
    torch.cuda.synchronize()
    after = _nonzero_counters()
    qn, kn, vn = q.numpy(), k.numpy(), v.numpy()
    problems = []
    for b in rows:
        okq, oks = oq.quant_k_int4(kn[b : b + 1, :, ns : S - nr])
        ovq, ovs = oq.quant_v_int4(vn[b : b + 1, :, ns : S - nr])
        assert np.array_equal(kq[b : b + 1].cpu().numpy(), okq), f"row {b}: K codes differ from the oracle"
        assert np.array_equal(ks[b : b + 1].cpu().numpy().view(np.uint16), oks.view(np.uint16)), f"row {b}: K scales"
        assert np.array_equal(vq[b : b + 1].cpu().numpy(), ovq), f"row {b}: V codes differ from the oracle"
        assert np.array_equal(vs[b : b + 1].cpu().numpy().view(np.uint16), ovs.view(np.uint16)), f"row {b}: V scales"
        ref = oatt.tiered_decode(qn[b : b + 1], kn[b : b + 1, :, :ns], vn[b : b + 1, :, :ns],
                                 _mid_dict(okq, oks, ovq, ovs), kn[b : b + 1, :, S - nr :], vn[b : b + 1, :, S - nr :])
        # both calls against the oracle first, so that a failure names the wrong one
        for name, o in (("default splits", out), ("one split", one)):
            e = np.abs(o[b : b + 1].float().cpu().numpy() - ref).max(axis=(0, 2, 3))  # per query head
            if e.max() > ATOL:
                heads = [(int(h), round(float(e[h]), 4)) for h in np.nonzero(e > ATOL)[0]]
                problems.append(f"{name}, row {b}: (head, max-abs error vs the oracle) {heads[:8]}")
    diff = (out.float() - one.float()).abs().amax(dim=(2, 3))  # [B, Hq]
    slots = [(int(b), int(h), round(float(diff[b, h]), 4)) for b, h in torch.nonzero(diff > ATOL).tolist()]
    if slots:
        problems.append(f"default vs one split differ at {len(slots)} (row, head) slots, first {slots[:8]}")
    if before or after:
        problems.append(f"split counters not zero: before the calls {before}, after {after}")
    assert not problems, "; ".join(problems)


def test_config1_full_quant_and_decode(dev):
    """Config 1 (B=16, Hkv=8, S=8192, sink 4, recent 64): quantizer invariants over the whole tier,
    codes and scales of rows 0 and 15 bit-exact with the oracle, their decode within 2e-3."""
    _decode_case(dev, 16, 8, 8192, 4, 64, seed=1001, rows=(0, 15))


def test_config2_full_decode(dev):
    """Config 2 (B=4, S=32768, sink 4, recent 256): row 3 against the oracle."""
    _decode_case(dev, 4, 8, 32768, 4, 256, seed=1002, rows=(3,), check_quant=False)


FIELDS = ("sink_k", "sink_v", "sink_pos", "fp16_k", "fp16_v", "fp16_pos", "int4_kq", "int4_ks", "int4_vq",
          "int4_vs", "int4_pos")


def test_config3_full_reassignment_device_equals_host(dev):
    """Config 3 (B=8, Hkv=4, S=4096, balanced windows 4 / 64 / 400): the device reassignment leaves
    every tier bit-identical to the host path, through both steps (fill the middle, then evict)."""
    print("case full-size reassignment config 3", flush=True)
    B, H, S, D = 8, 4, 4096, 128
    _, k, v = kv_tensors(B, H, S, D, seed=1003, Hq=28)
    kd, vd = k.to(dev), v.to(dev)
    caches = []
    for dev_path in (False, True):
        c = TieredKVCache(n_sink=4, recent_window=64, int4_budget=400, int2_budget=0, head_dim=D, rope_theta=1e6)
        c.device_reassign = dev_path
        caches.append(c)
    first = S - 64
    tiers0 = _assign_one_layer(first, torch.zeros(first), 4, 64, None, 0)
    tiers1 = _assign_one_layer(S, exp_scores(S, 1003), 4, 64, 400, 0)
    for c in caches:
        c.update(kd[:, :, :first], vd[:, :, :first], 0)
        c.apply_tier_assignment(0, tiers0)
        c.update(kd[:, :, first:], vd[:, :, first:], 0)
    for what, tiers in (("after the tier fill", None), ("after eviction", tiers1)):
        if tiers is not None:
            for c in caches:
                c.apply_tier_assignment(0, tiers)
        host, devc = (cc._layers[0] for cc in caches)
        for f in FIELDS:
            x, y = getattr(host, f), getattr(devc, f)
            assert (x is None) == (y is None), f"{what}: {f} present in one path only"
            if x is not None:
                assert x.shape == y.shape and torch.equal(x.cpu(), y.cpu()), f"{what}: {f} differs"
        assert host.next_position == devc.next_position and host.sink_count == devc.sink_count
    assert caches[1].get_seq_length(0) == 4 + 400 + 64


def test_config4_full_prefill_extreme_rows(dev):
    """Config 4 (32 rows, L ~ U[512, 16384], chunk 128): the full ragged batch in one launch; its
    longest and shortest rows against a float32 reference on the GPU."""
    print("case full-size prefill config 4", flush=True)
    B, Hq, Hkv, D, Sq, ns, nr = 32, 32, 8, 128, 128, 4, 64
    gen = torch.Generator().manual_seed(1004)
    L = torch.randint(512, 16385, (B,), generator=gen)
    nm = L - ns - nr
    cap = int(nm.max())
    g = torch.Generator(device=dev).manual_seed(1004)
    rnd = lambda *shape: torch.randn(*shape, generator=g, device=dev).to(torch.float16)  # noqa: E731
    kq = torch.randint(0, 256, (B, Hkv, cap, D // 2), generator=g, device=dev, dtype=torch.uint8)
    vq = torch.randint(0, 256, (B, Hkv, cap, D // 2), generator=g, device=dev, dtype=torch.uint8)
    ks = rnd(B, Hkv, 1, D).abs() * 0.3 + 0.05
    vs = rnd(B, Hkv, cap, 1).abs() * 0.3 + 0.05
    q = rnd(B, Hq, Sq, D)
    chunk = (rnd(B, Hkv, Sq, D), rnd(B, Hkv, Sq, D))
    sink = (rnd(B, Hkv, ns, D), rnd(B, Hkv, ns, D))
    rec = (rnd(B, Hkv, nr, D), rnd(B, Hkv, nr, D))
    lens = torch.stack([torch.full((B,), ns), nm, torch.full((B,), nr)], dim=1).to(torch.int32)
    order = torch.argsort(L, descending=True).to(torch.int32)
    out = tiered_prefill_attention(q, chunk, sink, MiddleTier("int4", kq, vq, ks, vs), rec, lens=lens, order=order)
    torch.cuda.synchronize()
    for b in (int(order[0]), int(order[-1])):
        m = int(nm[b])
        kmid = (_codes(kq[b, :, :m]).half() * ks[b]).float()
        vmid = (_codes(vq[b, :, :m]).half() * vs[b, :, :m]).float()
        kk = torch.cat([sink[0][b].float(), kmid, rec[0][b].float(), chunk[0][b].float()], dim=1)
        vv = torch.cat([sink[1][b].float(), vmid, rec[1][b].float(), chunk[1][b].float()], dim=1)
        kk = kk.repeat_interleave(Hq // Hkv, dim=0)
        vv = vv.repeat_interleave(Hq // Hkv, dim=0)
        sc = torch.matmul(q[b].float(), kk.transpose(-1, -2).contiguous()) / np.sqrt(D)
        tot = int(L[b]) + Sq
        # bottom-right causal: query j sees cache keys and chunk keys 0..j
        keep = torch.arange(tot, device=dev)[None, :] <= (int(L[b]) + torch.arange(Sq, device=dev))[:, None]
        sc = sc.masked_fill(~keep[None], float("-inf"))
        ref = torch.matmul(torch.softmax(sc, dim=-1), vv)
        err = (out[b].float() - ref).abs().max().item()
        assert err <= ATOL, f"row {b} (L={int(L[b])}): prefill max-abs error {err}"


def _asym_codes(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """Unsigned codes: 4-bit high nibble first; 2-bit four per byte, first code in the top bits."""
    shifts = (4, 0) if bits == 4 else (6, 4, 2, 0)
    mask = (1 << bits) - 1
    return torch.stack([(packed >> s) & mask for s in shifts], dim=-1).flatten(-2)


def test_config2_full_asym_quant(dev):
    """Config 2 in BASELINE's format (asymmetric group-32; K 4-bit, V 2-bit) over the whole middle
    tier: codes in range, every group's min -> 0 and max -> 2^bits - 1, dequantization error within
    half a step plus fp16 rounding; batch row 2 bit-exact with the oracle."""
    print("case full-size asym quant config 2", flush=True)
    _, k, v = kv_tensors(4, 8, 32768, 128, seed=1002, Hq=32)
    ns, nr = 4, 256
    for x, bits in ((k[:, :, ns:-nr], 4), (v[:, :, ns:-nr], 2)):
        xg = x.contiguous().to(dev)
        p, s, z = fq.quant_asym(xg, bits, 32)
        qmax = (1 << bits) - 1
        c = _asym_codes(p, bits).view(*xg.shape[:3], 4, 32)
        xr = xg.view(*xg.shape[:3], 4, 32)
        live = (s > 0).unsqueeze(-1)
        mn = xr.amin(dim=-1, keepdim=True)
        mx = xr.amax(dim=-1, keepdim=True)
        assert int(c.max()) <= qmax
        assert bool((c[(xr == mn) & live] == 0).all()), "a group's minimum does not map to code 0"
        assert bool((c[(xr == mx) & live] == qmax).all()), f"a group's maximum does not map to {qmax}"
        d = fq.dequant_asym(p, s, z, bits, 32).float()
        err = (xg.float() - d).abs().view(*xg.shape[:3], 4, 32)
        bound = 0.51 * s.float().unsqueeze(-1) + d.abs().view_as(err) * 2.0**-10 + 1e-6
        assert bool((err <= bound).all()), f"dequantization error above bound: {float((err - bound).max())}"
        op, os_, oz = oq.quant_asym_group(x[2:3].numpy(), bits, 32)
        assert np.array_equal(p[2:3].cpu().numpy(), op)
        assert np.array_equal(s[2:3].cpu().numpy().view(np.uint16), os_.view(np.uint16))
        assert np.array_equal(z[2:3].cpu().numpy().view(np.uint16), oz.view(np.uint16))


def test_config2_full_rotated_quant(dev):
    """Config 2 through the rotated backend's fused rotate + quantize (2-bit K per channel, V per
    token) over the whole middle tier: no code hits -2; one (row, head) slice against the
    oracle's quantizer on an fp64 rotation (tie-aware, as the small-size tests)."""
    from fade_amd import rotated_quant as frq
    from test_gpu_quant import _check_fused_rotated

    print("case full-size rotated quant config 2", flush=True)
    _, k, _ = kv_tensors(4, 8, 32768, 128, seed=1002, Hq=32)
    x = k[:, :, 4:-256].contiguous()
    R = np.load(__file__.rsplit("/", 1)[0] + "/golden/rotation_d128_seed42.npy")
    Rd = torch.from_numpy(R).to(dev)
    xg = x.to(dev)
    kp, ks = frq.rotated_quant_k(xg, Rd, 2)
    vp, vs = frq.rotated_quant_v(xg, Rd, 2)
    for packed in (kp, vp):
        fields = torch.stack([(packed >> sh) & 3 for sh in (6, 4, 2, 0)])
        assert not bool((fields == 2).any()), "a 2-bit code is -2"
    b, h = 1, 5
    xs = x[b : b + 1, h : h + 1].numpy()
    _check_fused_rotated(xs, R, 2, "channel", kp[b : b + 1, h : h + 1].cpu().numpy(), ks[b : b + 1, h : h + 1].cpu().numpy())
    _check_fused_rotated(xs, R, 2, "token", vp[b : b + 1, h : h + 1].cpu().numpy(), vs[b : b + 1, h : h + 1].cpu().numpy())


# ---- config 2's own middle formats at full size, through the cache's decode ----
C2 = dict(B=4, Hkv=8, Hq=32, S=32768, ns=4, nr=256, seed=1002, row=3)


def _c2_cache(dev, k, v, **kw):
    """Config 2's cache: every token between the 4 sinks and the 256 recent ones in the middle tier."""
    S = int(k.shape[2])
    c = TieredKVCache(n_sink=C2["ns"], recent_window=C2["nr"], int4_budget=None, head_dim=128, **kw)
    c.update(k.to(dev), v.to(dev), 0)
    c.apply_tier_assignment(0, _assign_one_layer(S, torch.zeros(S), C2["ns"], C2["nr"], None, 0))
    return c


def _c2_decode_checks(dev, c, q, kn, vn, mid_ref, what):
    """Decode of the whole batch through the cache: every row split-invariant (one split vs
    the planner's), row C2['row'] within 2e-3 of the oracle's dequant + fp32 SDPA."""
    qd = q.to(dev)
    out = c.decode_attention(qd, 0)
    c.decode_splits = 1
    one = c.decode_attention(qd, 0)
    c.decode_splits = 0
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all()), f"{what}: non-finite output"
    d = (out.float() - one.float()).abs().amax(dim=(1, 2, 3))
    assert float(d.max()) <= ATOL, f"{what}: one split differs from the default splits by {d.tolist()}"
    b, ns, nr = C2["row"], C2["ns"], C2["nr"]
    ref = oatt.tiered_decode(q.numpy()[b : b + 1], kn[b : b + 1, :, :ns], vn[b : b + 1, :, :ns], mid_ref,
                             kn[b : b + 1, :, -nr:], vn[b : b + 1, :, -nr:])
    err = float(np.abs(out[b : b + 1].float().cpu().numpy() - ref).max())
    assert err <= ATOL, f"{what}: row {b} decode max-abs error {err}"


def test_config2_full_k4_literal_v2_decode(dev):
    """Config 2 in the reference's INT4-K / INT2-V layout (fade/cache.py:983-988: V grouped 64
    along S, int8 codes): row 3's codes and scales bit-exact with the oracle, decode within 2e-3."""
    print("case full-size config 2 K4 + literal V2 decode", flush=True)
    q, k, v = kv_tensors(C2["B"], C2["Hkv"], C2["S"], 128, seed=C2["seed"], Hq=C2["Hq"])
    c = _c2_cache(dev, k, v, middle_v_bits=2)
    st = c._layers[0]
    b, ns, nr = C2["row"], C2["ns"], C2["nr"]
    kn, vn = k.numpy(), v.numpy()
    okq, oks = oq.quant_k_int4(kn[b : b + 1, :, ns:-nr])
    vpad, _ = oq.pad_to_group(vn[b : b + 1, :, ns:-nr], 64)
    ovq, ovs = oq.quant_int2_grouped(vpad, 64)
    assert np.array_equal(st.int4_kq[b : b + 1].cpu().numpy(), okq), "K codes differ from the oracle"
    assert np.array_equal(st.int4_ks[b : b + 1].cpu().numpy().view(np.uint16), oks.view(np.uint16)), "K scales"
    assert np.array_equal(st.int4_vq[b : b + 1].cpu().numpy(), ovq), "INT2 V codes differ from the oracle"
    assert np.array_equal(st.int4_vs[b : b + 1].cpu().numpy().view(np.uint16), ovs.view(np.uint16)), "INT2 V scales"
    mid = {"fmt": "k4v2", "kq": okq, "ks": oks, "vq": ovq, "vs": ovs, "group": 64}
    _c2_decode_checks(dev, c, q, kn, vn, mid, "K4 + literal V2")


def test_config2_full_asym_k4v2_decode(dev):
    """Config 2 in BASELINE's format (asymmetric group-32, K 4-bit / V 2-bit) through the cache:
    row 3's codes, scales and zeros bit-exact with the oracle, decode within 2e-3."""
    from fade_amd.backends import AsymGroupBackend

    print("case full-size config 2 asym K4/V2 decode", flush=True)
    q, k, v = kv_tensors(C2["B"], C2["Hkv"], C2["S"], 128, seed=C2["seed"], Hq=C2["Hq"])
    c = _c2_cache(dev, k, v, quant_backend=AsymGroupBackend(head_dim=128, bits=4, group=32, v_bits=2))
    st = c._layers[0]
    b, ns, nr = C2["row"], C2["ns"], C2["nr"]
    kn, vn = k.numpy(), v.numpy()
    mid = {"fmt": "asym", "k_bits": 4, "v_bits": 2, "group": 32}
    for name, x, comp, bits in (("K", kn, st.backend_k, 4), ("V", vn, st.backend_v, 2)):
        op, os_, oz = oq.quant_asym_group(x[b : b + 1, :, ns:-nr], bits, 32)
        assert np.array_equal(comp["packed"][b : b + 1].cpu().numpy(), op), f"{name} codes differ from the oracle"
        assert np.array_equal(comp["scale"][b : b + 1].cpu().numpy().view(np.uint16), os_.view(np.uint16)), name
        assert np.array_equal(comp["zero"][b : b + 1].cpu().numpy().view(np.uint16), oz.view(np.uint16)), name
        p = name.lower()
        mid.update({f"{p}q": op, f"{p}s": os_, f"{p}z": oz})
    _c2_decode_checks(dev, c, q, kn, vn, mid, "asym K4/V2")


def test_config2_full_rotated_k2v2_decode(dev):
    """Config 2's rotated-2bit variant (seed-42 rotation, K and V 2-bit) through the cache: decode of
    the cache's own codes within 2e-3 of the oracle's rotated dequant (fade/rotated_quant.py:134-187)
    + fp32 SDPA.  The codes themselves are pinned by test_config2_full_rotated_quant."""
    from fade_amd.backends import RotatedINT4Backend

    print("case full-size config 2 rotated K2/V2 decode", flush=True)
    q, k, v = kv_tensors(C2["B"], C2["Hkv"], C2["S"], 128, seed=C2["seed"], Hq=C2["Hq"])
    c = _c2_cache(dev, k, v, quant_backend=RotatedINT4Backend(head_dim=128, bits=2))
    st = c._layers[0]
    b = C2["row"]
    R = np.load(__file__.rsplit("/", 1)[0] + "/golden/rotation_d128_seed42.npy")
    bk, bv = st.backend_k, st.backend_v
    mid = {"fmt": "rot", "R": R, "k_bits": 2, "v_bits": 2,
           "kq": bk["packed"][b : b + 1].cpu().numpy(), "ks": bk["scale"][b : b + 1].half().cpu().numpy(),
           "vq": bv["packed"][b : b + 1].cpu().numpy(), "vs": bv["scale"][b : b + 1].half().cpu().numpy()}
    _c2_decode_checks(dev, c, q, k.numpy(), v.numpy(), mid, "rotated K2/V2")
