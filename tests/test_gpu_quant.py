"""GPU parity of the quantize / pack / dequantize kernels against the CPU oracle (bit-exact)."""

import numpy as np
import pytest
import torch

from fade_amd import _lib
from fade_amd import quant as fq
from fade_amd import rotated_quant as frq
from fade_amd.synthetic import kv_tensors
from oracle import quant as oq

pytestmark = pytest.mark.gpu
# head dims 128 / 64 / 256 and others that are multiples of 8 (the reference takes any even D)
SHAPES = [(1, 8, 1980, 128), (2, 3, 67, 128), (1, 2, 5, 64), (1, 1, 300, 256), (2, 3, 67, 96),
          (1, 2, 40, 80), (1, 3, 33, 16), (1, 1, 50, 160), (1, 2, 21, 48)]
F16 = np.float16


def _u16(x):
    return x.view(np.uint16)


def _edge_tensor(shape, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(shape) * rng.lognormal(0, 0.5, size=shape[-1])).astype(F16)
    x.reshape(-1)[::89] = F16(0.5)
    x.reshape(-1)[1::101] = F16(-2.5)
    x[..., 0, :] = 0
    x[..., 3] = 0
    x[..., 5] = F16(6e-8)
    x[..., 7] = F16(-3e-5)
    return x


@pytest.mark.parametrize("shape", SHAPES)
def test_quant_k_int4_bit_exact(dev, shape):
    print(f"case quant_k_int4 {shape}", flush=True)
    x = _edge_tensor(shape, 0)
    packed, scale = fq.quant_k_int4(torch.from_numpy(x).to(dev))
    op, osc = oq.quant_k_int4(x)
    assert np.array_equal(packed.cpu().numpy(), op)
    assert np.array_equal(_u16(scale.cpu().numpy()), _u16(osc))


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("parts", [1, 16])
def test_quant_k_int4_from_colmax_bit_exact(dev, shape, parts):
    """The second pass alone, on column maxima spread over `parts` partials (rows
    dealt round-robin, as the gather's workgroups fold into them): equal to the
    oracle's quant_k_int4, bit for bit."""
    print(f"case quant_k_int4_from_colmax {shape} parts={parts}", flush=True)
    x = _edge_tensor(shape, 2)
    B, H, S, D = shape
    a = np.abs(x.astype(np.float32)).reshape(B * H, S, D)
    colmax = np.zeros((B * H, parts, D), dtype=np.float32)
    for p in range(parts):
        if p < S:
            colmax[:, p] = a[:, p::parts].max(axis=1)
    packed, scale = fq.quant_k_int4_from_colmax(torch.from_numpy(x).to(dev), torch.from_numpy(colmax).to(dev))
    op, osc = oq.quant_k_int4(x)
    assert np.array_equal(packed.cpu().numpy(), op)
    assert np.array_equal(_u16(scale.cpu().numpy()), _u16(osc))


@pytest.mark.parametrize("shape", SHAPES)
def test_quant_v_int4_bit_exact(dev, shape):
    print(f"case quant_v_int4 {shape}", flush=True)
    x = _edge_tensor(shape, 1)
    packed, scale = fq.quant_v_int4(torch.from_numpy(x).to(dev))
    op, osc = oq.quant_v_int4(x)
    assert np.array_equal(packed.cpu().numpy(), op)
    assert np.array_equal(_u16(scale.cpu().numpy()), _u16(osc))


def test_quant_config0_seeded_inputs_bit_exact(dev):
    """Config 0 (1 x 8 kv heads x 2048, middle tier 4..1984) on the benchmark generator's inputs."""
    print("case config0 quant", flush=True)
    _, k, v = kv_tensors(1, 8, 2048, 128, seed=1000, Hq=32)
    km, vm = k[:, :, 4:1984], v[:, :, 4:1984]
    kp, ks = fq.quant_k_int4(km.to(dev))
    vp, vs = fq.quant_v_int4(vm.to(dev))
    okp, oks = oq.quant_k_int4(km.numpy())
    ovp, ovs = oq.quant_v_int4(vm.numpy())
    assert np.array_equal(kp.cpu().numpy(), okp) and np.array_equal(_u16(ks.cpu().numpy()), _u16(oks))
    assert np.array_equal(vp.cpu().numpy(), ovp) and np.array_equal(_u16(vs.cpu().numpy()), _u16(ovs))


def test_quant_strided_views(dev):
    """A view into a larger buffer (the recent-window layout) quantizes like its copy."""
    print("case quant strided", flush=True)
    x = _edge_tensor((2, 4, 96, 128), 2)
    big = torch.from_numpy(x).to(dev)
    view = big[:, :, 10:74]
    assert not view.is_contiguous()
    a = fq.quant_k_int4(view)
    b = fq.quant_k_int4(view.contiguous())
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    c = fq.quant_v_int4(view)
    d = fq.quant_v_int4(view.contiguous())
    assert torch.equal(c[0], d[0]) and torch.equal(c[1], d[1])


@pytest.mark.parametrize("shape", SHAPES)
def test_quant_int4_nan_inf_bit_exact(dev, shape):
    """fp16 K and V (and grouped INT2) with a NaN, a +inf and a -inf: the rows
    and channels they touch take the quantizers' scalar path (NaN scales and codes 0, inf scales
    with codes 0: finite x * 0, inf * 0 -> NaN -> 0), the rest the packed fp16
    path; both bit-exact against the oracle."""
    print(f"case quant_int4 nan/inf {shape}", flush=True)
    x = _edge_tensor(shape, 5)
    x[0, 0, 2, 9] = np.nan
    x[0, -1, 3, 10] = np.inf
    x[-1, 0, x.shape[2] - 1, 11] = -np.inf
    for quant, oquant in ((fq.quant_k_int4, oq.quant_k_int4), (fq.quant_v_int4, oq.quant_v_int4)):
        packed, scale = quant(torch.from_numpy(x).to(dev))
        op, osc = oquant(x)
        assert np.array_equal(packed.cpu().numpy(), op)
        _same(scale.cpu().numpy(), osc, "f16")
    # the reference literal grouped INT2 (64-token groups) on the same input
    q, sc = fq.quant_int2_padded(torch.from_numpy(x).to(dev), 64)
    oqv, osc = oq.quant_int2_grouped(oq.pad_to_group(x, 64)[0], 64)
    assert np.array_equal(q.cpu().numpy(), oqv)
    _same(sc.cpu().numpy(), osc, "f16")


@pytest.mark.parametrize("D", [128, 96, 16])
def test_dequant_int4_bit_exact(dev, D):
    print(f"case dequant_int4 D={D}", flush=True)
    x = _edge_tensor((2, 2, 40, D), 3)
    op, osc = oq.quant_k_int4(x)
    out = fq.dequant_int4(torch.from_numpy(op).to(dev), torch.from_numpy(osc).to(dev))
    assert np.array_equal(_u16(out.cpu().numpy()), _u16(oq.dequant_int4(op, osc)))
    op, osc = oq.quant_v_int4(x)
    out = fq.dequant_int4(torch.from_numpy(op).to(dev), torch.from_numpy(osc).to(dev))
    assert np.array_equal(_u16(out.cpu().numpy()), _u16(oq.dequant_int4(op, osc)))


def test_dequant_int4_unaligned_channel_scale(dev):
    """A per-channel scale tensor at a 2-byte offset (a contiguous view into a
    larger buffer) takes the dequantizer's scalar loop; still bit-exact."""
    print("case dequant_int4 unaligned scale", flush=True)
    x = _edge_tensor((2, 2, 40, 128), 6)
    op, osc = oq.quant_k_int4(x)
    buf = torch.empty(osc.size + 1, dtype=torch.float16, device=dev)
    buf[1:] = torch.from_numpy(osc.reshape(-1)).to(dev)
    sc = buf[1:].view(osc.shape)
    assert sc.data_ptr() % 16 != 0
    out = fq.dequant_int4(torch.from_numpy(op).to(dev), sc)
    assert np.array_equal(_u16(out.cpu().numpy()), _u16(oq.dequant_int4(op, osc)))


# -------------------------------------------- bfloat16 / float32 K/V input
_TDT = {"bf16": torch.bfloat16, "f32": torch.float32, "f16": torch.float16}


def _typed_edge(shape, seed, dtype):
    """``_edge_tensor``'s cases in ``dtype`` storage (bf16 as uint16 bits), plus
    a channel under the 1e-8 clamp and one NaN (its channel's and token's
    scales go NaN, their codes 0, as torch's amax/clamp/int8 cast give)."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(shape) * rng.lognormal(0, 0.5, size=shape[-1])).astype(np.float32)
    x.reshape(-1)[::89] = 0.5
    x.reshape(-1)[1::101] = -2.5
    x[..., 0, :] = 0
    x[..., 3] = 0
    x[..., 5] = 3e-9
    x[..., 7] = -3e-5
    x[0, 0, 2, 9] = np.nan
    return oq.from_f32(x, dtype)


def _dev_typed(x, dtype, dev):
    if dtype == "bf16":
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _host_typed(t, dtype):
    t = t.cpu().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16) if dtype == "bf16" else t.numpy()


def _same(got, ref, dtype):
    """Bit-exact, except that a NaN matches any NaN pattern."""
    g, r = oq.to_f32(got, dtype), oq.to_f32(ref, dtype)
    nan = np.isnan(r)
    assert np.array_equal(np.isnan(g), nan)
    assert np.array_equal(g[~nan].view(np.uint32), r[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("shape", SHAPES)
def test_quant_int4_typed_bit_exact(dev, dtype, shape):
    print(f"case quant_int4 {dtype} {shape}", flush=True)
    x = _typed_edge(shape, 4, dtype)
    xd = _dev_typed(x, dtype, dev)
    for quant, oquant in ((fq.quant_k_int4, oq.quant_k_int4_typed), (fq.quant_v_int4, oq.quant_v_int4_typed)):
        packed, scale = quant(xd)
        assert scale.dtype == _TDT[dtype]
        op, osc = oquant(x, dtype)
        assert np.array_equal(packed.cpu().numpy(), op)
        _same(_host_typed(scale, dtype), osc, dtype)
        assert np.isnan(oq.to_f32(osc, dtype)).sum() == 1


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_dequant_int4_typed_bit_exact(dev, dtype):
    print(f"case dequant_int4 {dtype}", flush=True)
    x = _typed_edge((2, 2, 40, 128), 5, dtype)
    for oquant in (oq.quant_k_int4_typed, oq.quant_v_int4_typed):
        op, osc = oquant(x, dtype)
        out = fq.dequant_int4(torch.from_numpy(op).to(dev), _dev_typed(osc, dtype, dev), dtype=_TDT[dtype])
        assert out.dtype == _TDT[dtype]
        _same(_host_typed(out, dtype), oq.dequant_int4_typed(op, osc, dtype), dtype)


def test_dequant_int4_fp16_scale_to_bf16(dev):
    """``dequant_int4(packed, fp16 scale, dtype=bf16)``: the scale is cast to
    bf16 first (``scale.to(dtype)``), then the product rounds to bf16."""
    x = _edge_tensor((1, 2, 33, 64), 6)
    op, osc = oq.quant_v_int4(x)
    out = fq.dequant_int4(torch.from_numpy(op).to(dev), torch.from_numpy(osc).to(dev), dtype=torch.bfloat16)
    ref = oq.dequant_int4_typed(op, oq.from_f32(osc.astype(np.float32), "bf16"), "bf16")
    _same(_host_typed(out, "bf16"), ref, "bf16")


@pytest.mark.parametrize("bits", [4, 2])
def test_pack_unpack_roundtrip_exhaustive(dev, bits):
    print(f"case pack bits={bits}", flush=True)
    lo, hi = (-8, 8) if bits == 4 else (-2, 2)
    rng = np.random.default_rng(4)
    q = rng.integers(lo, hi, size=(3, 5, 128)).astype(np.int8)
    packed = fq._pack_codes(torch.from_numpy(q).to(dev), bits).cpu().numpy()
    assert np.array_equal(packed, oq.pack_bits(q, bits))
    back = fq._unpack_codes(torch.from_numpy(packed).to(dev), bits).cpu().numpy()
    assert np.array_equal(back, q)


@pytest.mark.parametrize("S", [128, 100, 1])
def test_quant_int2_grouped_bit_exact(dev, S):
    print(f"case int2 grouped S={S}", flush=True)
    x = _edge_tensor((2, 3, max(S, 8), 128), 5)[:, :, :S]
    xp, _ = oq.pad_to_group(x, 64)
    oqv, osc = oq.quant_int2_grouped(xp, 64)
    q, sc = fq.quant_int2_padded(torch.from_numpy(np.ascontiguousarray(x)).to(dev), 64)
    assert np.array_equal(q.cpu().numpy(), oqv)
    assert np.array_equal(_u16(sc.cpu().numpy()), _u16(osc))
    deq = fq.dequant_int2_trimmed(q, sc, S, 64).cpu().numpy()
    assert np.array_equal(_u16(deq), _u16(oq.dequant_int2_grouped(oqv, osc, 64)[:, :, :S]))
    if S % 64 == 0:
        q2, sc2 = fq.quant_v_int2(torch.from_numpy(x).to(dev))
        assert torch.equal(q2, q) and torch.equal(sc2, sc)
    else:
        with pytest.raises(ValueError, match="divisible by group_size"):
            fq.quant_k_int2(torch.from_numpy(np.ascontiguousarray(x)).to(dev))


@pytest.mark.parametrize("group,D,S", [(32, 128, 100), (128, 128, 300), (256, 128, 300), (128, 256, 200), (16, 48, 70)])
def test_quant_int2_grouped_group_sizes(dev, group, D, S):
    """Other group sizes, on a strided view: the single-pass kernel keeps up to
    8 rows per lane in registers (group <= 8 * 256 / (D / 8) rows); beyond that
    (group 256 at D=128, 128 at D=256) the per-channel loop kernel runs.  Both
    bit-exact against the oracle."""
    print(f"case int2 grouped group={group} D={D} S={S}", flush=True)
    full = _edge_tensor((2, 3, S + 9, D), 11)
    x = full[:, :, 4 : 4 + S]  # rows strided inside a larger tensor
    xp, _ = oq.pad_to_group(np.ascontiguousarray(x), group)
    oqv, osc = oq.quant_int2_grouped(xp, group)
    xd = torch.from_numpy(full).to(dev)[:, :, 4 : 4 + S]
    q, sc = fq.quant_int2_padded(xd, group)
    assert np.array_equal(q.cpu().numpy(), oqv)
    assert np.array_equal(_u16(sc.cpu().numpy()), _u16(osc))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("S,D", [(128, 128), (100, 128), (1, 128), (70, 64), (64, 256), (65, 32), (90, 96), (64, 16)])
def test_quant_int2_grouped_typed_bit_exact(dev, dtype, S, D):
    print(f"case int2 grouped {dtype} S={S} D={D}", flush=True)
    x = _typed_edge((2, 3, 128, D), 8, dtype)[:, :, :S]
    xp, _ = oq.pad_to_group(x, 64)
    oqv, osc = oq.quant_int2_grouped_typed(xp, dtype, 64)
    q, sc = fq.quant_int2_padded(_dev_typed(x, dtype, dev), 64)
    assert sc.dtype == _TDT[dtype]
    assert np.array_equal(q.cpu().numpy(), oqv)
    _same(_host_typed(sc, dtype), osc, dtype)
    deq = fq.dequant_int2_trimmed(q, sc, S, 64)
    assert deq.dtype == _TDT[dtype]
    _same(_host_typed(deq, dtype), oq.dequant_int2_typed(oqv, osc, dtype, 64)[:, :, :S], dtype)
    if S % 64 == 0:
        q2, sc2 = fq.quant_k_int2(_dev_typed(x, dtype, dev))
        assert torch.equal(q2, q) and torch.equal(sc2.nan_to_num(), sc.nan_to_num())
        # the reference's default: dequantize to float16 (scale.to(fp16) first)
        d16 = fq.dequant_k_int2(q2, sc2, 64).cpu().numpy()
        s16 = oq.to_f32(osc, dtype).astype(np.float16)
        _same(d16, oq.dequant_int2_grouped(oqv, s16, 64), "f16")


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_rotated_quant_bit_exact_given_rotation(dev, bits):
    """Codes and scales are bit-exact given x_rot; x_rot itself is an fp32 GEMM (tolerance)."""
    print(f"case rotated bits={bits}", flush=True)
    R = torch.from_numpy(np.load(__file__.rsplit("/", 1)[0] + "/golden/rotation_d128_seed42.npy"))
    x = torch.from_numpy(_edge_tensor((2, 2, 70, 128), 6)).to(dev)
    x_rot = (x.float() @ R.to(dev).T).contiguous()
    xr = x_rot.cpu().numpy()
    ref_rot = x.cpu().float().numpy() @ R.numpy().T
    assert np.abs(xr - ref_rot).max() < 1e-4
    kp, ks = frq.quant_rotated_given(x_rot, bits, _lib.AXIS_CHANNEL)
    vp, vs = frq.quant_rotated_given(x_rot, bits, _lib.AXIS_TOKEN)
    okp, oks = oq.rotated_quant_codes(xr, bits, "channel")
    ovp, ovs = oq.rotated_quant_codes(xr, bits, "token")
    assert np.array_equal(kp.cpu().numpy().view(np.uint8), okp.view(np.uint8))
    assert np.array_equal(_u16(ks.cpu().numpy()), _u16(oks))
    assert np.array_equal(vp.cpu().numpy().view(np.uint8), ovp.view(np.uint8))
    assert np.array_equal(_u16(vs.cpu().numpy()), _u16(ovs))
    deq = frq.rotated_dequant_rot(kp, ks, bits).cpu().numpy()
    assert np.array_equal(_u16(deq), _u16(oq.rotated_dequant_rot(okp, oks, bits)))
    # bfloat16 / float32 K/V: scales emitted in their dtype, dequantized in it
    for dt in ("bf16", "f32"):
        for axis, ax in ((_lib.AXIS_CHANNEL, "channel"), (_lib.AXIS_TOKEN, "token")):
            p_, s_ = frq.quant_rotated_given(x_rot, bits, axis, scale_dtype=_TDT[dt])
            op_, os_ = oq.rotated_quant_codes(xr, bits, ax, dt)
            assert s_.dtype == _TDT[dt]
            assert np.array_equal(p_.cpu().numpy().view(np.uint8), op_.view(np.uint8))
            _same(_host_typed(s_, dt), os_, dt)
            d_ = frq.rotated_dequant_rot(p_, s_, bits, _TDT[dt])
            _same(_host_typed(d_, dt), oq.rotated_dequant_rot(op_, os_, bits, dt), dt)


def _check_fused_rotated(x16, R, bits, axis, packed, scale):
    """Fused rotate+quant against the oracle's quantizer on an fp64 rotation.

    The kernel's x_rot is an fp32-accurate GEMM (x exact, R split into fp16 hi/lo),
    so it differs from the fp64 product by ~1e-6 relative.  The fp16 scales must agree
    to one fp16 ulp (exactly, except where absmax / qmax rounds at a tie), and a code
    may differ only by one, and only where the fp64 value of x_rot * inv lies within
    1e-3 of a rounding boundary (a wrong channel, row or scale moves codes by whole
    units far from any boundary)."""
    xr64 = x16.astype(np.float64) @ R.astype(np.float64).T
    ocodes_p, oscale = oq.rotated_quant_codes(xr64.astype(np.float32), bits, axis)
    s_got = scale.astype(np.float32)
    s_ref = oscale.astype(np.float32)
    assert s_got.shape == s_ref.shape
    ulp = np.abs(np.spacing(oscale)).astype(np.float32)
    assert np.all(np.abs(s_got - s_ref) <= ulp), "scale off by more than one fp16 ulp"
    qmax = {4: 7, 3: 3, 2: 1}[bits]
    red = -2 if axis == "channel" else -1
    absmax = np.maximum(np.abs(xr64.astype(np.float32)).max(axis=red, keepdims=True), np.float32(1e-8))
    # a differing scale: absmax / qmax (fp64) sits at the fp16 rounding midpoint of the two
    s64 = np.maximum(np.abs(xr64).max(axis=red, keepdims=True), 1e-8) / qmax
    mid = (s_got.astype(np.float64) + s_ref.astype(np.float64)) / 2
    sbad = s_got != s_ref
    assert np.all(np.abs(s64 - mid)[sbad] <= 1e-5 * s64[sbad]), "scale differs away from an fp16 tie"
    got = oq.unpack_bits(packed, bits).astype(np.int32)
    ref = oq.unpack_bits(ocodes_p, bits).astype(np.int32)
    t = xr64 * (np.float64(qmax) / absmax.astype(np.float64))
    near = np.abs(np.abs(t - np.floor(t)) - 0.5) < 1e-3
    bad = got != ref
    assert np.all(np.abs(got - ref)[bad] == 1)
    assert np.all(near[bad]), f"{int((bad & ~near).sum())} codes differ away from a rounding boundary"
    assert bad.mean() < 1e-3


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("shape", [(2, 3, 70, 128), (1, 8, 2000, 128), (1, 1, 5, 128)])
def test_rotate_quant_fused(dev, bits, shape):
    """fade_rotate_quant (fused MFMA rotation + quantize), K per-channel and V per-token,
    on a contiguous tensor and on the strided middle slice the cache quantizes."""
    print(f"case rotate_quant_fused bits={bits} shape={shape}", flush=True)
    R = np.load(__file__.rsplit("/", 1)[0] + "/golden/rotation_d128_seed42.npy")
    Rd = torch.from_numpy(R).to(dev)
    x16 = _edge_tensor(shape, 7)
    xt = torch.from_numpy(x16).to(dev)
    assert frq._fused_ok(xt)
    kp, ks = frq.rotated_quant_k(xt, Rd, bits)
    vp, vs = frq.rotated_quant_v(xt, Rd, bits)
    _check_fused_rotated(x16, R, bits, "channel", kp.cpu().numpy(), ks.cpu().numpy())
    _check_fused_rotated(x16, R, bits, "token", vp.cpu().numpy(), vs.cpu().numpy())
    # strided view: rows 3 .. S-2 of a bigger tensor (the cache's middle tier)
    S = shape[2]
    if S > 8:
        big = torch.from_numpy(_edge_tensor((shape[0], shape[1], S + 5, 128), 8)).to(dev)
        view = big[:, :, 3 : S - 2]
        assert not view.is_contiguous() and frq._fused_ok(view)
        xv = view.cpu().numpy()
        kp, ks = frq.rotated_quant_k(view, Rd, bits)
        vp, vs = frq.rotated_quant_v(view, Rd, bits)
        _check_fused_rotated(xv, R, bits, "channel", kp.cpu().numpy(), ks.cpu().numpy())
        _check_fused_rotated(xv, R, bits, "token", vp.cpu().numpy(), vs.cpu().numpy())


def test_rotate_quant_fused_rejects(dev):
    """Argument checks of the C-ABI entry (no launch)."""
    import ctypes

    lib = _lib.load()
    nb = ctypes.c_int64(0)
    assert lib.fade_rotate_quant_workspace_bytes(1, 1, 10, 64, _lib.AXIS_TOKEN, nb) != 0
    assert lib.fade_rotate_quant_workspace_bytes(1, 1, 10, 128, 7, nb) != 0
    assert lib.fade_rotate_quant_workspace_bytes(1, 2, 1000, 128, _lib.AXIS_CHANNEL, nb) == 0 and nb.value > 0
    x = torch.zeros(1, 2, 1000, 128, dtype=torch.float16, device=dev)
    R = torch.eye(128, device=dev)
    pk = torch.empty(1, 2, 1000, 64, dtype=torch.uint8, device=dev)
    sc = torch.empty(1, 2, 1, 128, dtype=torch.float16, device=dev)
    rc = lib.fade_rotate_quant(x.data_ptr(), 1, 2, 1000, 128, 2000 * 128, 1000 * 128, 128, R.data_ptr(), 4,
                               _lib.AXIS_CHANNEL, pk.data_ptr(), sc.data_ptr(), None, 0, None)
    assert rc != 0 and "workspace" in lib.fade_hip_last_error().decode()


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("group", [32, 16])
@pytest.mark.parametrize("D", [128, 96])
def test_asym_group_quant_bit_exact(dev, bits, group, D):
    print(f"case asym bits={bits} group={group} D={D}", flush=True)
    x = _edge_tensor((2, 3, 50, D), 7)
    x[0, 0, 1, :32] = F16(1.25)
    p, s, z = fq.quant_asym(torch.from_numpy(x).to(dev), bits, group)
    op, os_, oz = oq.quant_asym_group(x, bits, group)
    assert np.array_equal(p.cpu().numpy(), op)
    assert np.array_equal(_u16(s.cpu().numpy()), _u16(os_))
    assert np.array_equal(_u16(z.cpu().numpy()), _u16(oz))
    d = fq.dequant_asym(p, s, z, bits, group).cpu().numpy()
    assert np.array_equal(_u16(d), _u16(oq.dequant_asym_group(op, os_, oz, bits, group)))


def test_empty_and_error_inputs(dev):
    print("case empty/errors", flush=True)
    e = torch.zeros(1, 2, 0, 128, dtype=torch.float16, device=dev)
    p, s = fq.quant_v_int4(e)
    assert p.shape == (1, 2, 0, 64) and s.shape == (1, 2, 0, 1)
    with pytest.raises(ValueError, match="float16, bfloat16 or float32"):
        fq.quant_k_int4(torch.zeros(1, 1, 4, 128, dtype=torch.float64, device=dev))
    with pytest.raises(ValueError, match="head_dim must be"):  # even, but not a multiple of 8
        fq.quant_v_int4(torch.zeros(1, 1, 4, 100, dtype=torch.float16, device=dev))
    with pytest.raises(ValueError, match="head_dim must be"):
        fq.quant_v_int4(torch.zeros(1, 1, 4, 264, dtype=torch.float16, device=dev))
