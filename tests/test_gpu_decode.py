"""GPU parity of the fused tiered decode attention against the oracle.

Tolerance: max-abs 2e-3 on the fp16 output against fp32 attention over the
oracle's dequantized tiers (the bar BASELINE.json states for attention).
"""

import numpy as np
import pytest
import torch

from fade_amd import quant as fq
from fade_amd import rotated_quant as frq
from fade_amd.kernels import MiddleTier, check_fused_parity, fused_int4_sdpa, tiered_decode_attention
from fade_amd.synthetic import kv_tensors
from oracle import attention as oatt
from oracle import quant as oq

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def _case(B, Hq, Hkv, S, ns, nr, seed):
    q, k, v = kv_tensors(B, Hkv, S, 128, seed=seed, Hq=Hq)
    return q.numpy(), k.numpy(), v.numpy(), ns, nr


class _Err(float):
    """A max-abs error that carries a diagnosis for the assertion message."""

    def __new__(cls, value, note=""):
        o = super().__new__(cls, value)
        o.note = note
        return o

    def __repr__(self):
        return f"{float(self)!r} ({self.note})" if self.note else repr(float(self))


def _stored_partials_err(qt, sink, mid_gpu, rec, kernel, n_splits, ref):
    """Max-abs error against ``ref`` of the split partials that the last call
    left in the workspace shared by the calls on the current stream, merged
    on the CPU; None when that call had one split.

    The packed INT4 kernel stores partial (m, l, acc) of split j, kv pair bkv
    and group head h at index ((P bkv + h // 4) n + j) 4 + h % 4 (P head
    passes, n splits), (m, l) after the counters and acc after those, and
    its last workgroup merges them.  After a wrong output, a small error here
    says that every split's partial was right and the merge read something
    else; a large one says that a split computed a wrong partial."""
    import ctypes

    from fade_amd import _lib
    from fade_amd.kernels.tiered_attn import TieredDecodePlan

    s = torch.cuda.current_stream(qt.device).cuda_stream
    plan = TieredDecodePlan(qt, sink, mid_gpu, rec, n_splits=n_splits, kernel=kernel, stream=s)
    nb = ctypes.c_int64(0)
    _lib.check(plan._lib.fade_tiered_decode_workspace_bytes(plan._argp, nb), "fade_tiered_decode_workspace_bytes")
    B, Hq, _, D = qt.shape
    Hkv = int(plan.args.Hkv)
    G = Hq // Hkv
    P = -(-G // 4)
    rows = B * max(Hq, Hkv * 4 * P)
    r256 = lambda x: (x + 255) // 256 * 256  # noqa: E731
    ml_off = r256(4 * B * Hkv * P)
    n = next((n for n in range(1, 1 << 16) if ml_off + r256(rows * n * 8) + rows * n * D * 4 == nb.value), None)
    if n is None or n == 1:
        return None
    ws = plan.workspace.cpu().numpy()
    acc_off = ml_off + r256(rows * n * 8)
    ml = ws[ml_off : ml_off + rows * n * 8].view(np.float32)
    acc = ws[acc_off : acc_off + rows * n * D * 4].view(np.float32)
    out = np.zeros((B, Hq, D), np.float64)
    for b in range(B):
        for kvh in range(Hkv):
            for h in range(G):
                pis = [((P * (b * Hkv + kvh) + h // 4) * n + j) * 4 + h % 4 for j in range(n)]
                m = np.array([ml[2 * pi] for pi in pis], np.float64)
                w = np.exp2(m - m.max())
                L = sum(w[j] * ml[2 * pi + 1] for j, pi in enumerate(pis))
                o = sum(w[j] * acc[pi * D : pi * D + D].astype(np.float64) for j, pi in enumerate(pis))
                out[b, kvh * G + h] = o / L
    return float(np.abs(out - ref.reshape(B, Hq, D)).max())


def _run(dev, q, k, v, ns, nr, mid_gpu, mid_oracle, kernel=0, n_splits=0):
    S = k.shape[2]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns]), t(v[:, :, :ns])) if ns else None
    rec = (t(k[:, :, S - nr :]), t(v[:, :, S - nr :])) if nr else None
    out = tiered_decode_attention(t(q), sink, mid_gpu, rec, kernel=kernel, n_splits=n_splits)
    ref = oatt.tiered_decode(q, k[:, :, :ns], v[:, :, :ns], mid_oracle, k[:, :, S - nr :], v[:, :, S - nr :])
    err = np.abs(out.float().cpu().numpy() - ref).max()
    if err <= ATOL:
        return err
    # a failure says whether the split partials the call stored were right
    # (read before anything else runs on the shared workspace), whether the
    # same call, run again, agrees, and whether the GPU-quantized middle tier
    # equals the oracle's codes and scales
    part = _stored_partials_err(t(q), sink, mid_gpu, rec, kernel, n_splits, ref) if kernel == 2 else None
    again = tiered_decode_attention(t(q), sink, mid_gpu, rec, kernel=kernel, n_splits=n_splits)
    err2 = np.abs(again.float().cpu().numpy() - ref).max()
    same_mid = None
    if mid_oracle.get("fmt") == "int4" and mid_gpu.fmt == "int4":
        same_mid = all(
            np.array_equal(getattr(mid_gpu, a).cpu().numpy().view(np.uint8), np.asarray(mid_oracle[b]).view(np.uint8))
            for a, b in (("k_codes", "kq"), ("v_codes", "vq"), ("k_scale", "ks"), ("v_scale", "vs"))
        )
    stored = "n/a" if part is None else f"{part:.3g}"
    return _Err(err, f"stored split partials merged on the CPU: error {stored}, re-run error {err2:.3g}, "
                     f"middle tier equal to the oracle's: {same_mid}")


def _int4_mid(dev, k, v, ns, nr):
    S = k.shape[2]
    km, vm = k[:, :, ns : S - nr], v[:, :, ns : S - nr]
    kq, ks = fq.quant_k_int4(torch.from_numpy(np.ascontiguousarray(km)).to(dev))
    vq, vs = fq.quant_v_int4(torch.from_numpy(np.ascontiguousarray(vm)).to(dev))
    okq, oks = oq.quant_k_int4(km)
    ovq, ovs = oq.quant_v_int4(vm)
    return MiddleTier("int4", kq, vq, ks, vs), {"fmt": "int4", "kq": okq, "ks": oks, "vq": ovq, "vs": ovs}


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,ns,nr",
    [
        (1, 32, 8, 2048, 4, 64),  # config 0
        (2, 28, 4, 700, 4, 64),  # GQA 7 (Qwen2.5-7B heads)
        (1, 8, 8, 130, 0, 0),  # MHA, middle only, ragged tile
        (3, 16, 4, 5, 2, 2),  # tiny: one middle token
        (1, 32, 8, 333, 4, 256),  # config 2 windows
    ],
)
@pytest.mark.parametrize("kernel", [0, 1, 3])
def test_tiered_decode_int4(dev, B, Hq, Hkv, S, ns, nr, kernel):
    print(f"case decode int4 B={B} Hq={Hq} Hkv={Hkv} S={S} ns={ns} nr={nr} kernel={kernel}", flush=True)
    q, k, v, ns, nr = _case(B, Hq, Hkv, S, ns, nr, seed=1000 + S)
    mid, omid = _int4_mid(dev, k, v, ns, nr)
    err = _run(dev, q, k, v, ns, nr, mid, omid, kernel=kernel)
    assert err <= ATOL, err


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,ns,nr",
    [
        (2, 8, 4, 777, 4, 64),  # G=2: padded head columns
        (1, 12, 4, 1000, 0, 0),  # G=3, no fp16 tiers
        (2, 8, 8, 600, 1, 0),  # G=1, sink only
        (1, 4, 1, 300, 0, 37),  # one kv head, ragged recent window
        (2, 32, 8, 4096, 4, 64),  # config-1 shape, shorter
    ],
)
def test_tiered_decode_int4_fast_path_shapes(dev, B, Hq, Hkv, S, ns, nr):
    """GQA groups of 1..4 heads take the INT4 kernel with the fused split merge."""
    print(f"case decode int4 fast B={B} Hq={Hq} Hkv={Hkv} S={S} ns={ns} nr={nr}", flush=True)
    q, k, v, ns, nr = _case(B, Hq, Hkv, S, ns, nr, seed=2000 + S)
    mid, omid = _int4_mid(dev, k, v, ns, nr)
    for n_splits in (0, 1, 5):
        assert _run(dev, q, k, v, ns, nr, mid, omid, kernel=2, n_splits=n_splits) <= ATOL, n_splits


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,ns,nr,n_splits",
    [
        (1, 4, 1, 300, 0, 37, 0),  # eight one-tile splits
        (2, 8, 4, 777, 4, 64, 3),  # G=2
        (2, 28, 4, 700, 4, 64, 5),  # G=7: heads 4..6 in the second pass's slot
        (1, 32, 8, 2048, 4, 64, 0),  # config 0
    ],
)
def test_stored_split_partials_merge_to_the_output(dev, B, Hq, Hkv, S, ns, nr, n_splits):
    """The split partials a packed-kernel call leaves in the shared workspace,
    merged on the CPU, match the oracle: the layout the failure diagnosis
    decodes is the kernel's."""
    print(f"case stored partials B={B} Hq={Hq} Hkv={Hkv} S={S} n_splits={n_splits}", flush=True)
    q, k, v, ns, nr = _case(B, Hq, Hkv, S, ns, nr, seed=3000 + S)
    mid, omid = _int4_mid(dev, k, v, ns, nr)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns]), t(v[:, :, :ns])) if ns else None
    rec = (t(k[:, :, S - nr :]), t(v[:, :, S - nr :])) if nr else None
    out = tiered_decode_attention(t(q), sink, mid, rec, kernel=2, n_splits=n_splits)
    ref = oatt.tiered_decode(q, k[:, :, :ns], v[:, :, :ns], omid, k[:, :, S - nr :], v[:, :, S - nr :])
    part = _stored_partials_err(t(q), sink, mid, rec, 2, n_splits, ref)
    assert part is not None, "the call ran one split"
    assert part <= ATOL, part
    assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL


def test_tiered_decode_int4_plan_replays(dev):
    """Repeated launches of one plan reuse the workspace: the split counters reset every call."""
    from fade_amd.kernels.tiered_attn import TieredDecodePlan

    print("case decode int4 plan replays", flush=True)
    q, k, v, ns, nr = _case(2, 32, 8, 3000, 4, 64, seed=11)
    S = k.shape[2]
    mid, omid = _int4_mid(dev, k, v, ns, nr)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    plan = TieredDecodePlan(t(q), (t(k[:, :, :ns]), t(v[:, :, :ns])), mid, (t(k[:, :, S - nr :]), t(v[:, :, S - nr :])))
    outs = [plan.run().clone() for _ in range(4)]
    torch.cuda.synchronize()
    ref = oatt.tiered_decode(q, k[:, :, :ns], v[:, :, :ns], omid, k[:, :, S - nr :], v[:, :, S - nr :])
    # waves claim tiles in the order they free a stage, so the fp32 sums may
    # differ between runs in their last bits: every run against the oracle
    for o in outs:
        assert (o.float() - outs[0].float()).abs().max().item() <= 1e-3
        assert np.abs(o.float().cpu().numpy() - ref).max() <= ATOL
    counters = plan.workspace[: 2 * 8 * 4].view(torch.int32)
    assert int(counters.abs().sum()) == 0


def test_tiered_decode_shared_stream_workspace(dev):
    """tiered_decode_attention shares one zero-filled workspace per (device, stream, B*Hkv):
    calls of several shapes in turn (same B*Hkv with different split layouts, a longer row
    that outgrows its buffer, other B*Hkv), then on a second stream, all match the oracle
    and leave every buffer's counters at zero."""
    from fade_amd import _lib

    print("case decode shared stream workspace", flush=True)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    cases = []
    for seed, (B, S) in enumerate([(2, 3000), (1, 700), (2, 9000), (2, 3000), (3, 1500), (10, 600), (2, 1200)]):
        q, k, v, ns, nr = _case(B, 32, 8, S, 4, 64, seed=40 + seed)
        mid, omid = _int4_mid(dev, k, v, ns, nr)
        ref = oatt.tiered_decode(q, k[:, :, :ns], v[:, :, :ns], omid, k[:, :, S - nr :], v[:, :, S - nr :])
        args = (t(q), (t(k[:, :, :ns]), t(v[:, :, :ns])), mid, (t(k[:, :, S - nr :]), t(v[:, :, S - nr :])))
        cases.append((args, ref))
    side = torch.cuda.Stream(dev)
    for rnd in range(2):
        for args, ref in cases:
            if rnd == 0:
                out = tiered_decode_attention(*args)
            else:
                side.wait_stream(torch.cuda.current_stream(dev))
                with torch.cuda.stream(side):
                    out = tiered_decode_attention(*args)
                torch.cuda.current_stream(dev).wait_stream(side)
            torch.cuda.synchronize()
            assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL
    shared = {key: ws for key, ws in _lib._STREAM_WS.items() if key[0] == torch.device(dev).index or key[0] == 0}
    assert {key[2] for key in shared} >= {8, 16, 24, 80}
    for key, ws in shared.items():  # the counters of B*Hkv pairs sit at the front of the buffer
        assert int(ws[: 4 * key[2]].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("n_splits", [1, 3, 64])
def test_tiered_decode_split_counts(dev, n_splits):
    print(f"case decode splits={n_splits}", flush=True)
    q, k, v, ns, nr = _case(1, 32, 8, 1500, 4, 64, seed=5)
    mid, omid = _int4_mid(dev, k, v, ns, nr)
    assert _run(dev, q, k, v, ns, nr, mid, omid, n_splits=n_splits) <= ATOL


def test_tiered_decode_fp16_middle_flash_decode(dev):
    print("case decode fp16 comparator", flush=True)
    q, k, v, ns, nr = _case(2, 32, 8, 1024, 4, 64, seed=6)
    S = k.shape[2]
    km, vm = k[:, :, ns : S - nr], v[:, :, ns : S - nr]
    mid = MiddleTier("fp16", torch.from_numpy(np.ascontiguousarray(km)).to(dev),
                     torch.from_numpy(np.ascontiguousarray(vm)).to(dev))
    assert _run(dev, q, k, v, ns, nr, mid, {"fmt": "fp16", "k": km, "v": vm}) <= ATOL


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,ns,nr,n_splits,kernel",
    [
        (1, 32, 8, 1200, 4, 256, 0, 0),  # config-2 windows, auto kernel choice
        (1, 32, 8, 1200, 4, 256, 0, 1),  # portable kernel
        (2, 8, 4, 777, 4, 64, 3, 2),  # G=2, ragged last group of 64
        (1, 4, 1, 301, 0, 37, 1, 2),  # one kv head, one split
        (2, 12, 4, 2000, 4, 64, 0, 2),  # G=3
        (3, 16, 4, 5, 2, 2, 0, 2),  # one middle token (one padded group)
    ],
)
def test_tiered_decode_k4_v2_literal(dev, B, Hq, Hkv, S, ns, nr, n_splits, kernel):
    """Config-2 parity format: INT4 K + reference grouped INT2 V (int8 codes, [G, D] scales)."""
    print(f"case decode k4v2 B={B} Hq={Hq} Hkv={Hkv} S={S} ns={ns} nr={nr} splits={n_splits} kernel={kernel}",
          flush=True)
    q, k, v, ns, nr = _case(B, Hq, Hkv, S, ns, nr, seed=7 + S)
    S = k.shape[2]
    km, vm = k[:, :, ns : S - nr], v[:, :, ns : S - nr]
    n = km.shape[2]
    kq, ks = fq.quant_k_int4(torch.from_numpy(np.ascontiguousarray(km)).to(dev))
    vq, vs = fq.quant_int2_padded(torch.from_numpy(np.ascontiguousarray(vm)).to(dev), 64)
    okq, oks = oq.quant_k_int4(km)
    ovq, ovs = oq.quant_int2_grouped(oq.pad_to_group(vm, 64)[0], 64)
    mid = MiddleTier("k4v2", kq, vq, ks, vs, group=64, length=n)
    omid = {"fmt": "k4v2", "kq": okq, "ks": oks, "vq": ovq, "vs": ovs, "group": 64}
    assert _run(dev, q, k, v, ns, nr, mid, omid, kernel=kernel, n_splits=n_splits) <= ATOL


@pytest.mark.parametrize("bits", [2, 4])
def test_tiered_decode_rotated(dev, bits):
    """Rotated K/V codes: attend in the rotated basis (q R^T, o R) -- the reference rounds
    k_hat through fp16 after rotating back, which the 2e-3 bar absorbs."""
    print(f"case decode rotated bits={bits}", flush=True)
    R = torch.from_numpy(np.load(__file__.rsplit("/", 1)[0] + "/golden/rotation_d128_seed42.npy")).to(dev)
    q, k, v, ns, nr = _case(1, 32, 8, 900, 0, 0, seed=8)
    kt, vt = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    kp, ks = frq.rotated_quant_k(kt, R, bits)
    vp, vs = frq.rotated_quant_v(vt, R, bits)
    mid = MiddleTier("sym", kp, vp, ks, vs, k_bits=bits, v_bits=bits)
    qt = torch.from_numpy(q).to(dev)
    q_rot = (qt.float() @ R.T).to(torch.float16)
    out = (tiered_decode_attention(q_rot, None, mid, None).float() @ R).cpu().numpy()
    omid = {"fmt": "rot", "kq": kp.cpu().numpy(), "ks": ks.cpu().numpy(), "vq": vp.cpu().numpy(),
            "vs": vs.cpu().numpy(), "R": R.cpu().numpy(), "k_bits": bits, "v_bits": bits}
    ref = oatt.tiered_decode(q, k[:, :, :0], v[:, :, :0], omid, k[:, :, :0], v[:, :, :0])
    assert np.abs(out - ref).max() <= ATOL


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,ns,nr,n_splits,bits,det",
    [
        (1, 32, 8, 1500, 4, 64, 0, 2, False),
        (2, 8, 4, 777, 4, 64, 3, 2, False),  # G=2
        (1, 4, 1, 300, 0, 37, 1, 2, False),  # one kv head, no sink; one split asked for: fp16 split + one middle split
        (2, 12, 4, 2000, 4, 256, 0, 2, True),  # G=3, config-2 windows, deterministic order
        (1, 28, 4, 1000, 4, 64, 0, 2, False),  # G=7: two head passes
        (1, 32, 8, 600, 0, 0, 0, 2, False),  # no fp16 tokens: the fp16 split is empty
        (2, 32, 8, 1300, 4, 64, 0, 4, False),  # rotated 4-bit
        (1, 20, 4, 900, 4, 100, 5, 4, False),  # 4-bit, G=5
    ],
)
def test_tiered_decode_rotation_in_kernel(dev, B, Hq, Hkv, S, ns, nr, n_splits, bits, det):
    """Rotated middle tier with q, sink and recent in the model's basis (what the cache
    holds): the kernel scores the middle with q R^T and un-rotates its output part.
    Oracle: the reference's rotated dequant (codes -> x_rot_hat -> @ R, rounded to fp16,
    fade/rotated_quant.py:134-187) concatenated with the fp16 tiers, then fp32 SDPA."""
    print(f"case decode rotation in kernel B={B} Hq={Hq} Hkv={Hkv} S={S} ns={ns} nr={nr} splits={n_splits} "
          f"bits={bits} det={det}", flush=True)
    R = torch.from_numpy(np.load(__file__.rsplit("/", 1)[0] + "/golden/rotation_d128_seed42.npy")).to(dev)
    q, k, v, ns, nr = _case(B, Hq, Hkv, S, ns, nr, seed=4100 + S + bits)
    S = k.shape[2]
    km = torch.from_numpy(np.ascontiguousarray(k[:, :, ns : S - nr])).to(dev)
    vm = torch.from_numpy(np.ascontiguousarray(v[:, :, ns : S - nr])).to(dev)
    kp, ks = frq.rotated_quant_k(km, R, bits)
    vp, vs = frq.rotated_quant_v(vm, R, bits)
    mid = MiddleTier("sym", kp, vp, ks.half(), vs.half(), k_bits=bits, v_bits=bits)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns]), t(v[:, :, :ns])) if ns else None
    rec = (t(k[:, :, S - nr :]), t(v[:, :, S - nr :])) if nr else None
    out = tiered_decode_attention(t(q), sink, mid, rec, n_splits=n_splits, deterministic=det,
                                  rotation=R).float().cpu().numpy()
    omid = {"fmt": "rot", "kq": kp.cpu().numpy(), "ks": ks.half().cpu().numpy(), "vq": vp.cpu().numpy(),
            "vs": vs.half().cpu().numpy(), "R": R.cpu().numpy(), "k_bits": bits, "v_bits": bits}
    ref = oatt.tiered_decode(q, k[:, :, :ns], v[:, :, :ns], omid, k[:, :, S - nr :], v[:, :, S - nr :])
    assert np.isfinite(out).all()
    assert np.abs(out - ref).max() <= ATOL
    if det:
        again = tiered_decode_attention(t(q), sink, mid, rec, n_splits=n_splits, deterministic=True,
                                        rotation=R).float().cpu().numpy()
        assert np.array_equal(out, again)


def test_tiered_decode_rotation_rejects(dev):
    """A rotation needs the matrix-core INT4 kernel and a symmetric middle tier."""
    R = torch.eye(128, dtype=torch.float32, device=dev)
    q, k, v, ns, nr = _case(1, 8, 2, 300, 4, 16, seed=5)
    km = torch.from_numpy(np.ascontiguousarray(k[:, :, 4:-16])).to(dev)
    kp, ks = fq.quant_k_int4(km)
    vp, vs = fq.quant_v_int4(torch.from_numpy(np.ascontiguousarray(v[:, :, 4:-16])).to(dev))
    mid = MiddleTier("int4", kp, vp, ks, vs)
    qt = torch.from_numpy(q).to(dev)
    with pytest.raises(ValueError, match="rotated middle tier needs the matrix-core INT4 kernel"):
        tiered_decode_attention(qt, None, mid, None, kernel=1, rotation=R)
    with pytest.raises(ValueError, match="float32"):
        tiered_decode_attention(qt, None, mid, None, rotation=R.half())


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,ns,nr,n_splits",
    [
        (1, 32, 8, 1500, 4, 64, 0),
        (2, 8, 4, 777, 4, 64, 3),  # G=2
        (1, 4, 1, 300, 0, 37, 1),  # one kv head, ragged recent window
        (2, 12, 4, 2000, 4, 256, 0),  # G=3, config-2 windows
        (1, 16, 2, 900, 4, 64, 0),  # G=8: eight heads in one pass
        (2, 24, 4, 700, 4, 64, 3),  # G=6
        # short fp16 windows: a partial tile, half a tile, one tile and a token, sink only;
        # several tiles in one split and one tile per split
        (2, 8, 2, 400, 0, 5, 0),
        (1, 8, 2, 400, 0, 8, 4),
        (2, 16, 4, 500, 1, 8, 1),
        (1, 8, 2, 400, 3, 0, 0),
        (1, 32, 8, 700, 4, 9, 0),
    ],
)
def test_tiered_decode_sym2_fast_path(dev, B, Hq, Hkv, S, ns, nr, n_splits):
    """Rotated 2-bit middle tier (K per channel, V per token) on the matrix-core kernel.

    Attention runs in the rotated basis: q, sink and recent are rotated (fp32 x @ R^T,
    rounded to fp16) and the oracle dequantizes the codes with R = I, so the check is
    the kernel's attention over exactly the tiers it was given."""
    print(f"case decode sym2 B={B} Hq={Hq} Hkv={Hkv} S={S} ns={ns} nr={nr} splits={n_splits}", flush=True)
    R = torch.from_numpy(np.load(__file__.rsplit("/", 1)[0] + "/golden/rotation_d128_seed42.npy")).to(dev)
    q, k, v, ns, nr = _case(B, Hq, Hkv, S, ns, nr, seed=3000 + S)
    rot = lambda a: (torch.from_numpy(np.ascontiguousarray(a)).to(dev).float() @ R.T).to(torch.float16)  # noqa: E731
    qr, kr, vr = rot(q), rot(k), rot(v)
    km = torch.from_numpy(np.ascontiguousarray(k[:, :, ns : S - nr])).to(dev)
    vm = torch.from_numpy(np.ascontiguousarray(v[:, :, ns : S - nr])).to(dev)
    kp, ks = frq.rotated_quant_k(km, R, 2)
    vp, vs = frq.rotated_quant_v(vm, R, 2)
    mid = MiddleTier("sym", kp, vp, ks, vs, k_bits=2, v_bits=2)
    sink = (kr[:, :, :ns].contiguous(), vr[:, :, :ns].contiguous()) if ns else None
    rec = (kr[:, :, S - nr :].contiguous(), vr[:, :, S - nr :].contiguous()) if nr else None
    out = tiered_decode_attention(qr, sink, mid, rec, kernel=2, n_splits=n_splits).float().cpu().numpy()
    eye = np.eye(128, dtype=np.float32)
    omid = {"fmt": "rot", "kq": kp.cpu().numpy(), "ks": ks.cpu().numpy(), "vq": vp.cpu().numpy(),
            "vs": vs.cpu().numpy(), "R": eye, "k_bits": 2, "v_bits": 2}
    krn, vrn, qrn = kr.cpu().numpy(), vr.cpu().numpy(), qr.cpu().numpy()
    ref = oatt.tiered_decode(qrn, krn[:, :, :ns], vrn[:, :, :ns], omid, krn[:, :, S - nr :], vrn[:, :, S - nr :])
    assert np.abs(out - ref).max() <= ATOL


@pytest.mark.parametrize("n_splits", [0, 1, 7])
def test_tiered_decode_sym2_ragged_lens(dev, n_splits):
    """Per-row tier lengths on the symmetric 2-bit instance (fp16 tiles counted per row in
    the kernel): each row against the oracle over its own tokens, in the rotated basis as
    in the fast-path test."""
    print(f"case decode sym2 ragged n_splits={n_splits}", flush=True)
    R = torch.from_numpy(np.load(__file__.rsplit("/", 1)[0] + "/golden/rotation_d128_seed42.npy")).to(dev)
    ns_c, mc, nr_c, B = 4, 600, 64, 5
    S = ns_c + mc + nr_c
    q, k, v, _, _ = _case(B, 16, 4, S, ns_c, nr_c, seed=79)
    rot = lambda a: (torch.from_numpy(np.ascontiguousarray(a)).to(dev).float() @ R.T).to(torch.float16)  # noqa: E731
    qr, kr, vr = rot(q), rot(k), rot(v)
    kp, ks = frq.rotated_quant_k(torch.from_numpy(np.ascontiguousarray(k[:, :, ns_c : S - nr_c])).to(dev), R, 2)
    vp, vs = frq.rotated_quant_v(torch.from_numpy(np.ascontiguousarray(v[:, :, ns_c : S - nr_c])).to(dev), R, 2)
    mid = MiddleTier("sym", kp, vp, ks, vs, k_bits=2, v_bits=2)
    omid = {"fmt": "rot", "kq": kp.cpu().numpy(), "ks": ks.cpu().numpy(), "vq": vp.cpu().numpy(),
            "vs": vs.cpu().numpy(), "R": np.eye(128, dtype=np.float32), "k_bits": 2, "v_bits": 2}
    lens = np.array([[4, 600, 64], [2, 130, 9], [4, 1, 0], [0, 333, 8], [1, 0, 5]], dtype=np.int32)
    sink = (kr[:, :, :ns_c].contiguous(), vr[:, :, :ns_c].contiguous())
    rec = (kr[:, :, S - nr_c :].contiguous(), vr[:, :, S - nr_c :].contiguous())
    out = tiered_decode_attention(qr, sink, mid, rec, lens=torch.from_numpy(lens).to(dev), n_splits=n_splits,
                                  kernel=2).float().cpu().numpy()
    krn, vrn, qrn = kr.cpu().numpy(), vr.cpu().numpy(), qr.cpu().numpy()
    for b, (ls, lm, lr) in enumerate(lens):
        ref = oatt.tiered_decode(
            qrn[b : b + 1], krn[b : b + 1, :, :ls], vrn[b : b + 1, :, :ls], _row_slice_mid(omid, b, lm),
            krn[b : b + 1, :, S - nr_c : S - nr_c + lr], vrn[b : b + 1, :, S - nr_c : S - nr_c + lr],
        )
        err = np.abs(out[b : b + 1] - ref).max()
        assert err <= ATOL, (b, err)


def _asym_mid(dev, k, v, ns, nr, k_bits, v_bits):
    S = k.shape[2]
    km, vm = k[:, :, ns : S - nr], v[:, :, ns : S - nr]
    kp, ksc, kz = fq.quant_asym(torch.from_numpy(np.ascontiguousarray(km)).to(dev), k_bits, 32)
    vp, vsc, vz = fq.quant_asym(torch.from_numpy(np.ascontiguousarray(vm)).to(dev), v_bits, 32)
    mid = MiddleTier("asym", kp, vp, ksc, vsc, kz, vz, k_bits=k_bits, v_bits=v_bits, group=32)
    okp, oks, okz = oq.quant_asym_group(km, k_bits, 32)
    ovp, ovs, ovz = oq.quant_asym_group(vm, v_bits, 32)
    omid = {"fmt": "asym", "kq": okp, "ks": oks, "kz": okz, "vq": ovp, "vs": ovs, "vz": ovz,
            "k_bits": k_bits, "v_bits": v_bits, "group": 32}
    return mid, omid


@pytest.mark.parametrize("k_bits,v_bits", [(4, 4), (4, 2), (2, 2), (2, 4)])
@pytest.mark.parametrize("kernel", [0, 1])
def test_tiered_decode_asym(dev, k_bits, v_bits, kernel):
    """Asymmetric group-32 middle tier (build format): matrix-core path (0) and portable kernel (1)."""
    print(f"case decode asym K{k_bits}V{v_bits} kernel={kernel}", flush=True)
    q, k, v, ns, nr = _case(2, 32, 8, 800, 4, 64, seed=9)
    mid, omid = _asym_mid(dev, k, v, ns, nr, k_bits, v_bits)
    assert _run(dev, q, k, v, ns, nr, mid, omid, kernel=kernel) <= ATOL


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,ns,nr,n_splits,k_bits,v_bits",
    [
        (1, 32, 8, 2048, 4, 64, 0, 4, 4),  # config 0 as BASELINE states it
        (2, 8, 4, 777, 4, 64, 3, 4, 2),  # G=2, ragged last tile
        (1, 4, 1, 301, 0, 37, 1, 4, 2),  # one kv head, odd middle length, one split
        (2, 12, 4, 2000, 4, 256, 0, 4, 2),  # G=3, config-2 windows
        (1, 8, 8, 65, 0, 0, 0, 2, 2),  # MHA, middle only, one token past a tile
        (3, 16, 4, 5, 2, 2, 0, 4, 4),  # one middle token
        (1, 32, 8, 1200, 4, 256, 5, 2, 4),
    ],
)
def test_tiered_decode_asym_fast_path(dev, B, Hq, Hkv, S, ns, nr, n_splits, k_bits, v_bits):
    """The matrix-core kernel is required (kernel=2) for the group-32 asymmetric formats."""
    print(f"case decode asym fast B={B} Hq={Hq} Hkv={Hkv} S={S} ns={ns} nr={nr} splits={n_splits} "
          f"K{k_bits}V{v_bits}", flush=True)
    q, k, v, ns, nr = _case(B, Hq, Hkv, S, ns, nr, seed=5000 + S)
    mid, omid = _asym_mid(dev, k, v, ns, nr, k_bits, v_bits)
    assert _run(dev, q, k, v, ns, nr, mid, omid, kernel=2, n_splits=n_splits) <= ATOL


def test_fused_int4_sdpa_api_and_parity_helper(dev):
    print("case fused_int4_sdpa", flush=True)
    res = check_fused_parity()
    assert res["passed"], res
    q, k, v, _, _ = _case(2, 8, 2, 300, 0, 0, seed=10)
    kq, ks = oq.quant_k_int4(k)
    vq, vs = oq.quant_v_int4(v)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    out = fused_int4_sdpa(t(q), t(kq), t(ks), t(vq), t(vs))
    ref = oatt.tiered_decode(q, None, None, {"fmt": "int4", "kq": kq, "ks": ks, "vq": vq, "vs": vs}, None, None)
    assert out.shape == (2, 8, 1, 128) and out.dtype == torch.float16
    assert np.abs(out.float().cpu().numpy() - ref).max() <= ATOL


def test_decode_errors(dev):
    print("case decode errors", flush=True)
    q = torch.zeros(1, 6, 1, 128, dtype=torch.float16, device=dev)
    k = torch.zeros(1, 4, 10, 128, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="not a multiple"):
        tiered_decode_attention(q, (k, k), None, None)
    q = torch.zeros(1, 4, 1, 128, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="empty"):
        tiered_decode_attention(q, (k[:, :, :0], k[:, :, :0]), None, None)


def _row_slice_mid(omid, b, lm):
    """The oracle middle tier of batch row b restricted to its first lm tokens."""
    out = {}
    for key, val in omid.items():
        if not isinstance(val, np.ndarray) or key == "R":
            out[key] = val
        elif key == "ks" and omid["fmt"] in ("int4", "rot"):
            out[key] = val[b : b + 1]  # per-channel K scale [B,H,1,D]
        else:
            out[key] = val[b : b + 1, :, :lm]
    return out


@pytest.mark.parametrize("Hq,Hkv,fmt", [(28, 4, "int4"), (20, 4, "int4"), (16, 2, "asym"), (56, 8, "int4")])
def test_tiered_decode_ragged_paged_gqa_5_to_8(dev, Hq, Hkv, fmt):
    """GQA groups of 5-8 query heads (Qwen2.5-7B's 28/4, 20/4, 16/2, 56/8) with per-row
    lengths and a paged middle tier: the INT4 kernel serves all heads of a kv head in
    one pass (reference INT4 format) or in two head passes (asymmetric format).
    Each row against the oracle over its own tokens; paged == padded bit for bit in
    deterministic mode; repeated plans on one stream share a workspace."""
    from fade_amd.kernels.tiered_attn import paginate_middle

    print(f"case decode ragged/paged GQA {Hq}/{Hkv} {fmt}", flush=True)
    ns_c, mc, nr_c, B = 4, 700, 64, 3
    S = ns_c + mc + nr_c
    q, k, v, _, _ = _case(B, Hq, Hkv, S, ns_c, nr_c, seed=95 + Hq)
    mid, omid = _int4_mid(dev, k, v, ns_c, nr_c) if fmt == "int4" else _asym_mid(dev, k, v, ns_c, nr_c, 4, 4)
    lens = np.array([[4, 700, 64], [1, 129, 7], [4, 0, 33]], dtype=np.int32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns_c]), t(v[:, :, :ns_c]))
    rec = (t(k[:, :, S - nr_c :]), t(v[:, :, S - nr_c :]))
    n_pages = int(sum(-(-int(x) // 64) for x in lens[:, 1]))
    paged = paginate_middle(mid, lens[:, 1], order=np.random.default_rng(2).permutation(n_pages))
    # kernel 4 (int4): all heads of a kv head in one pass whatever the size
    for kernel in ((0, 4) if fmt == "int4" else (0,)):
        out_r = tiered_decode_attention(t(q), sink, mid, rec, lens=t(lens), deterministic=True, kernel=kernel)
        out_p = tiered_decode_attention(t(q), sink, paged, rec, lens=t(lens), deterministic=True, kernel=kernel)
        assert torch.equal(out_r, out_p)
        out = out_r.float().cpu().numpy()
        for b, (ls, lm, lr) in enumerate(lens):
            ref = oatt.tiered_decode(
                q[b : b + 1], k[b : b + 1, :, :ls], v[b : b + 1, :, :ls], _row_slice_mid(omid, b, lm),
                k[b : b + 1, :, S - nr_c : S - nr_c + lr], v[b : b + 1, :, S - nr_c : S - nr_c + lr],
            )
            assert np.abs(out[b : b + 1] - ref).max() <= ATOL, (kernel, b)
        for n_splits in (1, 5):  # other split counts, claims on: still within the oracle's tolerance
            o = tiered_decode_attention(t(q), sink, paged, rec, lens=t(lens), n_splits=n_splits, kernel=kernel)
            assert (o.float() - out_r.float()).abs().max().item() <= 1e-3


@pytest.mark.parametrize(
    "B,Hq,Hkv,S,ns,nr,n_splits",
    [
        (2, 20, 4, 900, 4, 64, 0),  # G=5
        (1, 24, 4, 333, 4, 0, 3),  # G=6, no recent tier, a ragged last tile
        (2, 64, 8, 1200, 4, 64, 0),  # G=8 (Llama-3-70B heads)
        (1, 8, 1, 70, 2, 5, 1),  # G=8, one split, a short middle tier
        (3, 56, 8, 2100, 4, 256, 7),  # G=7
    ],
)
@pytest.mark.parametrize("det", [False, True])
def test_tiered_decode_int4_eight_heads_one_pass(dev, B, Hq, Hkv, S, ns, nr, n_splits, det):
    """GQA 5-8 on the reference INT4 format: every query head of a kv head in one
    pass of the matrix-core kernel (eight heads x two sub-tiles in the QK^T
    columns), each kv tile read once; against the oracle, and bitwise repeatable
    in deterministic mode."""
    print(f"case decode int4 eight heads B={B} Hq={Hq} Hkv={Hkv} S={S} splits={n_splits} det={det}", flush=True)
    q, k, v, ns, nr = _case(B, Hq, Hkv, S, ns, nr, seed=5000 + S + Hq)
    mid, omid = _int4_mid(dev, k, v, ns, nr)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns]), t(v[:, :, :ns])) if ns else None
    rec = (t(k[:, :, S - nr :]), t(v[:, :, S - nr :])) if nr else None
    ref = oatt.tiered_decode(q, k[:, :, :ns], v[:, :, :ns], omid, k[:, :, S - nr :], v[:, :, S - nr :])
    # kernel 4: the eight-head instance whatever the size; 0: the automatic choice
    # (two head passes at these sizes)
    for kernel in (4, 0):
        out = tiered_decode_attention(t(q), sink, mid, rec, n_splits=n_splits, deterministic=det, kernel=kernel)
        err = np.abs(out.float().cpu().numpy() - ref)
        assert err.max() <= ATOL, (kernel, [(int(b), int(h)) for b, h in zip(*np.nonzero(err.max(axis=(2, 3)) > ATOL))][:8])
        if det:
            again = tiered_decode_attention(t(q), sink, mid, rec, n_splits=n_splits, deterministic=True, kernel=kernel)
            assert torch.equal(out, again)


@pytest.mark.parametrize("fmt", ["int4", "asym42"])
@pytest.mark.parametrize("n_splits", [0, 1, 7])
@pytest.mark.parametrize("kernel", [0, 1])
def test_tiered_decode_ragged_lens(dev, fmt, n_splits, kernel):
    """Per-row tier lengths (ragged batch): row b attends to the first lens[b] rows of
    each padded tier; each row is checked against the oracle over its own tokens.
    Matrix-core INT4 kernel (0) and portable kernel (1)."""
    print(f"case decode ragged {fmt} n_splits={n_splits} kernel={kernel}", flush=True)
    ns_c, mc, nr_c = 4, 600, 64
    S = ns_c + mc + nr_c
    B = 5
    q, k, v, _, _ = _case(B, 16, 4, S, ns_c, nr_c, seed=77)
    if fmt == "int4":
        mid, omid = _int4_mid(dev, k, v, ns_c, nr_c)
    else:
        mid, omid = _asym_mid(dev, k, v, ns_c, nr_c, 4, 2)
    lens = np.array([[4, 600, 64], [2, 130, 17], [4, 1, 0], [0, 333, 64], [1, 0, 5]], dtype=np.int32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns_c]), t(v[:, :, :ns_c]))
    rec = (t(k[:, :, S - nr_c :]), t(v[:, :, S - nr_c :]))
    out = tiered_decode_attention(t(q), sink, mid, rec, lens=t(lens), n_splits=n_splits,
                                  kernel=kernel).float().cpu().numpy()
    for b, (ls, lm, lr) in enumerate(lens):
        ref = oatt.tiered_decode(
            q[b : b + 1], k[b : b + 1, :, :ls], v[b : b + 1, :, :ls], _row_slice_mid(omid, b, lm),
            k[b : b + 1, :, S - nr_c : S - nr_c + lr], v[b : b + 1, :, S - nr_c : S - nr_c + lr],
        )
        err = np.abs(out[b : b + 1] - ref).max()
        assert err <= ATOL, (b, err)


@pytest.mark.parametrize("D", [128, 64, 256])
@pytest.mark.parametrize("n_splits", [0, 1, 7])
def test_tiered_decode_ragged_lens_general_kernel(dev, D, n_splits):
    """Per-row tier lengths on the general matrix-core kernel (kernel=3; the automatic
    choice at head dims 64 and 256): each row against the oracle over its own tokens,
    rows with no sink, no middle or no recent tokens included."""
    print(f"case decode ragged general kernel D={D} n_splits={n_splits}", flush=True)
    ns_c, mc, nr_c = 4, 600, 64
    S = ns_c + mc + nr_c
    B = 5
    q, k, v = (x.numpy() for x in kv_tensors(B, 4, S, D, seed=78 + D, Hq=16))
    mid, omid = _int4_mid(dev, k, v, ns_c, nr_c)
    lens = np.array([[4, 600, 64], [2, 130, 17], [4, 1, 0], [0, 333, 64], [1, 0, 5]], dtype=np.int32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns_c]), t(v[:, :, :ns_c]))
    rec = (t(k[:, :, S - nr_c :]), t(v[:, :, S - nr_c :]))
    for kernel in (3, 0):
        out = tiered_decode_attention(t(q), sink, mid, rec, lens=t(lens), n_splits=n_splits,
                                      kernel=kernel).float().cpu().numpy()
        for b, (ls, lm, lr) in enumerate(lens):
            ref = oatt.tiered_decode(
                q[b : b + 1], k[b : b + 1, :, :ls], v[b : b + 1, :, :ls], _row_slice_mid(omid, b, lm),
                k[b : b + 1, :, S - nr_c : S - nr_c + lr], v[b : b + 1, :, S - nr_c : S - nr_c + lr],
            )
            err = np.abs(out[b : b + 1] - ref).max()
            assert err <= ATOL, (kernel, b, err)


@pytest.mark.parametrize("fmt", ["int4", "asym42"])
def test_tiered_decode_paged_middle(dev, fmt):
    """Paged middle tier: rows' 64-token tiles scattered over a shared pool in a
    shuffled order (separate pools, and for INT4 one interleaved pool); the result
    matches the padded ragged layout and the oracle over each row's own tokens
    (waves claim tiles dynamically, so the summation order may differ)."""
    from fade_amd.kernels.tiered_attn import paginate_middle

    print(f"case decode paged {fmt}", flush=True)
    ns_c, mc, nr_c = 4, 600, 64
    S = ns_c + mc + nr_c
    B = 5
    q, k, v, _, _ = _case(B, 16, 4, S, ns_c, nr_c, seed=78)
    if fmt == "int4":
        mid, omid = _int4_mid(dev, k, v, ns_c, nr_c)
    else:
        mid, omid = _asym_mid(dev, k, v, ns_c, nr_c, 4, 2)
    lens = np.array([[4, 600, 64], [2, 130, 17], [4, 1, 0], [0, 333, 64], [1, 0, 5]], dtype=np.int32)
    n_pages = sum(-(-int(x) // 64) for x in lens[:, 1])
    order = np.random.default_rng(0).permutation(n_pages)
    paged = paginate_middle(mid, lens[:, 1], order=order)
    assert paged.k_codes.shape[0] == n_pages  # the pool holds exactly the rows' pages
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns_c]), t(v[:, :, :ns_c]))
    rec = (t(k[:, :, S - nr_c :]), t(v[:, :, S - nr_c :]))
    out_p = tiered_decode_attention(t(q), sink, paged, rec, lens=t(lens), n_splits=3)
    out_r = tiered_decode_attention(t(q), sink, mid, rec, lens=t(lens), n_splits=3)
    assert (out_p.float() - out_r.float()).abs().max().item() <= ATOL
    if fmt == "int4":  # one pool of [K | V | V scales] blocks
        inter = paginate_middle(mid, lens[:, 1], order=order, interleave=True)
        assert inter.page_stride == 8320
        out_i = tiered_decode_attention(t(q), sink, inter, rec, lens=t(lens), n_splits=3)
        assert (out_i.float() - out_r.float()).abs().max().item() <= ATOL
    out = out_p.float().cpu().numpy()
    for b, (ls, lm, lr) in enumerate(lens):
        ref = oatt.tiered_decode(
            q[b : b + 1], k[b : b + 1, :, :ls], v[b : b + 1, :, :ls], _row_slice_mid(omid, b, lm),
            k[b : b + 1, :, S - nr_c : S - nr_c + lr], v[b : b + 1, :, S - nr_c : S - nr_c + lr],
        )
        assert np.abs(out[b : b + 1] - ref).max() <= ATOL, b


@pytest.mark.parametrize("fmt", ["int4", "asym"])
def test_tiered_decode_deterministic_repeats(dev, fmt):
    """deterministic=True (or torch.use_deterministic_algorithms): repeated calls give
    bitwise-identical outputs, still within the oracle's tolerance, and the paged and
    padded ragged layouts of the same tokens give bitwise-identical outputs too."""
    from fade_amd.kernels.tiered_attn import paginate_middle

    print(f"case decode deterministic {fmt}", flush=True)
    ns_c, mc, nr_c, B = 4, 1500, 64, 3
    S = ns_c + mc + nr_c
    q, k, v, _, _ = _case(B, 32, 8, S, ns_c, nr_c, seed=91)
    mid, omid = _int4_mid(dev, k, v, ns_c, nr_c) if fmt == "int4" else _asym_mid(dev, k, v, ns_c, nr_c, 4, 4)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    sink = (t(k[:, :, :ns_c]), t(v[:, :, :ns_c]))
    rec = (t(k[:, :, S - nr_c :]), t(v[:, :, S - nr_c :]))
    qd = t(q)
    outs = [tiered_decode_attention(qd, sink, mid, rec, n_splits=2, deterministic=True).clone() for _ in range(6)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ref = oatt.tiered_decode(q, k[:, :, :ns_c], v[:, :, :ns_c], omid, k[:, :, S - nr_c :], v[:, :, S - nr_c :])
    assert np.abs(outs[0].float().cpu().numpy() - ref).max() <= ATOL
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        assert torch.equal(tiered_decode_attention(qd, sink, mid, rec, n_splits=2), outs[0])
    finally:
        torch.use_deterministic_algorithms(prev)
    lens = np.array([[4, 1500, 64], [2, 700, 30], [4, 65, 1]], dtype=np.int32)
    paged = paginate_middle(mid, lens[:, 1], order=np.random.default_rng(1).permutation(int(sum(-(-x // 64) for x in lens[:, 1]))))
    out_p = [tiered_decode_attention(qd, sink, paged, rec, lens=t(lens), n_splits=2, deterministic=True) for _ in range(3)]
    out_r = tiered_decode_attention(qd, sink, mid, rec, lens=t(lens), n_splits=2, deterministic=True)
    for o in out_p:
        assert torch.equal(o, out_r)


def test_tiered_decode_hip_graph_replays(dev):
    """Decode captured in a HIP graph: every replay, with eager work and synchronizations in
    between (a new query written in place), matches the eager call on the same inputs (to the
    attention bar: waves claim tiles dynamically, so the summation order may differ)."""
    from fade_amd.kernels import TieredDecodePlan

    print("case decode graph replays", flush=True)
    q, k, v, ns, nr = _case(2, 32, 8, 900, 4, 64, seed=31)
    mid, _ = _int4_mid(dev, k, v, ns, nr)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    S = k.shape[2]
    qd = t(q)
    plan = TieredDecodePlan(qd, (t(k[:, :, :ns]), t(v[:, :, :ns])), mid, (t(k[:, :, S - nr :]), t(v[:, :, S - nr :])))
    plan.run()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        plan.run(s.cuda_stream)
    gen = torch.Generator().manual_seed(5)
    for rep in range(4):
        qd.copy_(torch.randn(qd.shape, generator=gen).half().to(dev))
        eager = plan.run().clone()
        torch.cuda.synchronize()
        plan.out.zero_()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert (plan.out.float() - eager.float()).abs().max().item() <= ATOL, rep
        assert plan.out.abs().sum().item() > 0, rep
