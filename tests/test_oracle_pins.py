"""Pins of the CPU oracle (no GPU): every oracle function is checked against
something independent of its own formula -- brute force, torch's own fp16/fp32
op semantics (the library the reference runs on), closed forms, invariants,
and the reference's known-answer test.
"""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import policy as opol
from oracle import quant as oq
from oracle import rope as orope

F16 = np.float16


# ----------------------------------------------------------------- packing
def test_pack_int4_brute_force_all_pairs():
    """fade/quant.py:33-34 docstring: byte = (high nibble = q[2d], low nibble = q[2d+1])."""
    pairs = np.array(list(itertools.product(range(-8, 8), repeat=2)), dtype=np.int8)
    packed = oq.pack_int4_last_dim(pairs)[:, 0]
    for (a, b), byte in zip(pairs, packed):
        assert int(byte) == (((int(a) + 16) % 16) << 4) | ((int(b) + 16) % 16)
    assert np.array_equal(oq.unpack_int4_last_dim(packed[:, None]), pairs)
    assert len(set(packed.tolist())) == 256


def test_pack_int2_brute_force_all_quads():
    """fade/rotated_quant.py:39: byte = (v0 << 6) | (v1 << 4) | (v2 << 2) | v3."""
    quads = np.array(list(itertools.product(range(-2, 2), repeat=4)), dtype=np.int8)
    packed = oq.pack_int2_last_dim(quads)[:, 0]
    for q, byte in zip(quads, packed):
        u = [(int(x) + 4) % 4 for x in q]
        assert int(byte) == (u[0] << 6) | (u[1] << 4) | (u[2] << 2) | u[3]
    assert np.array_equal(oq.unpack_int2_last_dim(packed[:, None]), quads)


def test_pack_rejects_bad_last_dim():
    with pytest.raises(ValueError, match="even"):
        oq.pack_int4_last_dim(np.zeros((2, 3), np.int8))
    with pytest.raises(ValueError, match="divisible by 4"):
        oq.pack_int2_last_dim(np.zeros((2, 6), np.int8))


# ------------------------------------------------- rounding model vs torch
ALL_POS_F16 = np.arange(1, 0x7C00, dtype=np.uint16).view(F16)


@pytest.mark.parametrize("qmax", [7, 1])
def test_sym_params_match_torch_fp16_for_every_positive_fp16(qmax):
    """``qmax / absmax`` and ``absmax / qmax`` on fp16 tensors, exhaustively."""
    t = torch.from_numpy(ALL_POS_F16.copy())
    inv, scale = oq._sym_params_f16(ALL_POS_F16, qmax)
    assert np.array_equal(inv.view(np.uint16), (qmax / t).numpy().view(np.uint16))
    assert np.array_equal(scale.view(np.uint16), (t / qmax).numpy().view(np.uint16))


def test_single_rounding_of_inv_would_be_wrong():
    """The double rounding matters: a one-rounding model disagrees with torch."""
    single = (np.float32(7) / ALL_POS_F16.astype(np.float32)).astype(F16)
    inv, _ = oq._sym_params_f16(ALL_POS_F16, 7)
    assert np.sum(single.view(np.uint16) != inv.view(np.uint16)) > 1000


def _torch_quant_k(k):  # torch ops in the order of fade/quant.py:71-74
    absmax = k.abs().amax(dim=-2, keepdim=True).clamp(min=1e-8)
    q = (k * (7 / absmax)).round().clamp(-8, 7).to(torch.int8)
    return q, absmax / 7


def _torch_quant_v(v):  # fade/quant.py:88-91
    absmax = v.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    q = (v * (7 / absmax)).round().clamp(-8, 7).to(torch.int8)
    return q, absmax / 7


def _hard_fp16(shape, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(shape) * rng.lognormal(0, 0.5, size=shape[-1])).astype(F16)
    # ties: values that land exactly on .5 code boundaries after scaling
    x.reshape(-1)[::97] = F16(0.5)
    x[..., 0, :] = 0  # a zero token row
    x[..., 3] = 0  # a zero channel
    x[..., 5] = F16(6e-8)  # subnormal channel
    return x


def test_quant_int4_matches_torch_ops_codes_and_scales():
    k = _hard_fp16((2, 3, 67, 64), 0)
    qt, st = _torch_quant_k(torch.from_numpy(k))
    packed, scale = oq.quant_k_int4(k)
    assert np.array_equal(oq.unpack_int4_last_dim(packed), qt.numpy())
    assert np.array_equal(scale.view(np.uint16), st.numpy().view(np.uint16))
    qt, st = _torch_quant_v(torch.from_numpy(k))
    packed, scale = oq.quant_v_int4(k)
    assert np.array_equal(oq.unpack_int4_last_dim(packed), qt.numpy())
    assert np.array_equal(scale.view(np.uint16), st.numpy().view(np.uint16))


def test_quant_int4_invariants():
    rng = np.random.default_rng(1)
    k = (rng.standard_normal((2, 2, 50, 32)) * 3).astype(F16)
    packed, scale = oq.quant_k_int4(k)
    q = oq.unpack_int4_last_dim(packed)
    assert q.min() >= -7 and q.max() <= 7  # -8 never produced for finite nonzero data
    am = np.abs(k).argmax(axis=-2)
    top = np.take_along_axis(q, am[:, :, None, :], axis=-2)
    assert np.all(np.abs(top) == 7)
    deq = oq.dequant_int4(packed, scale).astype(np.float32)
    s = scale.astype(np.float32)
    assert np.all(np.abs(deq - k.astype(np.float32)) <= 0.5 * s * 1.01 + 2e-3)
    z = np.zeros((1, 1, 4, 16), F16)
    pz, sz = oq.quant_k_int4(z)
    assert np.all(pz == 0) and np.all(sz == 0)


def test_quant_int2_grouped_matches_torch_ops():
    x = _hard_fp16((2, 2, 128, 32), 2)
    t = torch.from_numpy(x).view(2, 2, 2, 64, 32)
    absmax = t.abs().amax(dim=-2, keepdim=True).clamp(min=1e-8)
    qt = (t * (1 / absmax)).round().clamp(-2, 1).to(torch.int8).view(2, 2, 128, 32)
    q, s = oq.quant_int2_grouped(x, 64)
    assert np.array_equal(q, qt.numpy())
    assert np.array_equal(s.view(np.uint16), (absmax / 1).squeeze(-2).numpy().view(np.uint16))
    assert set(np.unique(q)) <= {-1, 0, 1}
    with pytest.raises(ValueError, match="divisible by group_size"):
        oq.quant_int2_grouped(x[:, :, :100], 64)


# ---------------------------------------- bfloat16 / float32 INT4 quantizers
ALL_POS_BF16 = np.arange(1, 0x7F80, dtype=np.uint16)  # every positive finite bf16


def _t_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _bits_bf16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_bf16_conversion_matches_torch():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(20000) * np.exp(rng.uniform(-40, 40, 20000))).astype(np.float32)
    u = x.view(np.uint32)
    u[:2000] = (u[:2000] & 0xFFFF0000) | 0x8000  # exact ties, both parities
    x[2000:2004] = [np.inf, -np.inf, np.nan, -np.nan]
    x[2004:2010] = [1e-40, -1e-42, 3.3895314e38, 3.4028235e38, 0.0, -0.0]  # subnormal, overflow to inf
    ref = _bits_bf16(torch.from_numpy(x).to(torch.bfloat16))
    got = oq.f32_to_bf16(x)
    # NaN: any NaN pattern (torch's scalar conversion gives 0x7FC0, its
    # vectorized CPU one 0xFFFF); every other value bit-exact
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all(np.isnan(oq.bf16_to_f32(got[nan]))) and np.all(np.isnan(oq.bf16_to_f32(ref[nan])))
    assert np.array_equal(oq.bf16_to_f32(ref[~nan]), torch.from_numpy(x[~nan]).to(torch.bfloat16).float().numpy())


@pytest.mark.parametrize("qmax", [7, 1])
def test_sym_params_match_torch_bf16_for_every_positive_bf16(qmax):
    """``absmax.clamp(min=1e-8)``, ``qmax / absmax``, ``absmax / qmax`` on bf16
    tensors, exhaustively -- the clamp is live on bf16 (1e-8 is representable)."""
    t = _t_bf16(np.concatenate([[0], ALL_POS_BF16]).astype(np.uint16)).clamp(min=1e-8)
    inv, scale = oq._sym_params_typed(oq.bf16_to_f32(np.concatenate([[0], ALL_POS_BF16])), qmax, "bf16")
    assert np.array_equal(oq.f32_to_bf16(inv), _bits_bf16(qmax / t))
    assert np.array_equal(scale, _bits_bf16(t / qmax))


def _hard_typed(shape, seed, dtype):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(shape) * rng.lognormal(0, 0.5, size=shape[-1])).astype(np.float32)
    x.reshape(-1)[::97] = 0.5  # lands on .5 code boundaries after scaling
    x[..., 0, :] = 0  # a zero token row
    x[..., 3] = 0  # a zero channel
    x[..., 5] = 3e-9  # a channel below the 1e-8 clamp (bf16/fp32 hold it)
    x[..., 6] = rng.standard_normal(shape[:-1]) * 1e-9
    x[0, 1, 7, 9] = np.nan  # a NaN: its channel's and token's scale go NaN, their codes 0
    return oq.from_f32(x, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f32", "f16"])
def test_quant_int4_typed_matches_torch_ops(dtype):
    x = _hard_typed((2, 3, 67, 64), 7, dtype)
    t = _t_bf16(x) if dtype == "bf16" else torch.from_numpy(x)
    bits = _bits_bf16 if dtype == "bf16" else (lambda a: a.numpy().view(np.uint16 if dtype == "f16" else np.uint32))
    raw = (lambda a: a) if dtype == "bf16" else (lambda a: a.view(np.uint16 if dtype == "f16" else np.uint32))
    for quant, tq in ((oq.quant_k_int4_typed, _torch_quant_k), (oq.quant_v_int4_typed, _torch_quant_v)):
        qt, st = tq(t)
        packed, scale = quant(x, dtype)
        assert np.array_equal(oq.unpack_int4_last_dim(packed), qt.numpy())
        nan = np.isnan(oq.to_f32(scale, dtype))
        assert nan.sum() == 1 and np.array_equal(nan, torch.isnan(st).numpy())
        assert np.array_equal(raw(scale)[~nan], bits(st)[~nan])
    if dtype == "f16":  # the fp16 path is the same function
        assert np.array_equal(oq.quant_k_int4_typed(x, "f16")[0], oq.quant_k_int4(x)[0])
        assert np.array_equal(oq.quant_v_int4_typed(x, "f16")[1].view(np.uint16), oq.quant_v_int4(x)[1].view(np.uint16))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_dequant_int4_typed_matches_torch(dtype):
    rng = np.random.default_rng(11)
    q = rng.integers(-8, 8, size=(2, 2, 9, 16)).astype(np.int8)
    s = oq.from_f32(rng.standard_normal((2, 2, 1, 16)).astype(np.float32), dtype)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    st = _t_bf16(s) if dtype == "bf16" else torch.from_numpy(s)
    ref = torch.from_numpy(q).to(tdt) * st
    got = oq.dequant_int4_typed(oq.pack_int4_last_dim(q), s, dtype)
    assert np.array_equal(got, _bits_bf16(ref) if dtype == "bf16" else ref.numpy())


@pytest.mark.parametrize("dtype", ["bf16", "f32", "f16"])
def test_quant_int2_typed_matches_torch_ops(dtype):
    """fade/quant.py:95-112 run by torch on a bf16 / fp32 / fp16 tensor."""
    x = _hard_typed((2, 2, 128, 32), 11, dtype)
    t = (_t_bf16(x) if dtype == "bf16" else torch.from_numpy(x)).view(2, 2, 2, 64, 32)
    absmax = t.abs().amax(dim=-2, keepdim=True).clamp(min=1e-8)
    qt = (t * (1 / absmax)).round().clamp(-2, 1).to(torch.int8).view(2, 2, 128, 32)
    st = (absmax / 1).squeeze(-2)
    q, s = oq.quant_int2_grouped_typed(x, dtype, 64)
    assert np.array_equal(q, qt.numpy())
    if dtype == "bf16":
        same = np.isnan(oq.bf16_to_f32(s)) == torch.isnan(st.float()).numpy()
        fin = ~np.isnan(oq.bf16_to_f32(s))
        assert same.all() and np.array_equal(s[fin], _bits_bf16(st)[fin])
    else:
        assert np.array_equal(s, st.numpy(), equal_nan=True)
    if dtype == "f16":
        qf, sf = oq.quant_int2_grouped(x, 64)
        assert np.array_equal(q, qf) and np.array_equal(s.view(np.uint16), sf.view(np.uint16))
    # dequant: q.to(dtype) * scale.to(dtype), the scale repeated over the group
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32, "f16": torch.float16}[dtype]
    sfull = st.unsqueeze(-2).expand(2, 2, 2, 64, 32).reshape(2, 2, 128, 32)
    ref = qt.to(tdt) * sfull.to(tdt)
    got = oq.dequant_int2_typed(q, s, dtype, 64)
    rb = _bits_bf16(ref) if dtype == "bf16" else ref.numpy()
    nan = np.isnan(oq.to_f32(got, dtype))
    assert np.array_equal(nan, torch.isnan(ref.float()).numpy())
    assert np.array_equal(got[~nan], rb[~nan])


def test_typed_quant_would_fail_without_the_bf16_clamp():
    """A model without the clamp (fp16's no-op) disagrees with torch on bf16."""
    x = _hard_typed((1, 2, 16, 16), 3, "bf16")
    qt, _ = _torch_quant_k(_t_bf16(x))
    x32 = oq.bf16_to_f32(x)
    absmax = np.abs(x32).max(axis=-2, keepdims=True)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        inv = oq._rnd(oq._rnd(np.float32(1) / absmax, "bf16") * np.float32(7), "bf16")
        wrong = oq._rne_clamp(oq._rnd(x32 * inv, "bf16"), -8, 7)
    assert not np.array_equal(wrong, qt.numpy())


def test_dequant_matches_torch():
    rng = np.random.default_rng(3)
    q = rng.integers(-8, 8, size=(2, 2, 9, 16)).astype(np.int8)
    s = rng.standard_normal((2, 2, 1, 16)).astype(F16)
    ref = torch.from_numpy(q).to(torch.float16) * torch.from_numpy(s)
    assert np.array_equal(oq.dequant(q, s).view(np.uint16), ref.numpy().view(np.uint16))


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("axis", ["channel", "token"])
def test_rotated_quantizer_matches_torch_fp32_ops(bits, axis):
    """fade/rotated_quant.py:127-131 / 169-173 on an fp32 rotated tensor."""
    rng = np.random.default_rng(4)
    xr = rng.standard_normal((2, 2, 33, 32)).astype(np.float32)
    xr[0, 0, :, 1] = 0  # zero channel -> EPS clamp path
    qmin, qmax = oq.BIT_PARAMS[bits]
    t = torch.from_numpy(xr)
    dim = -2 if axis == "channel" else -1
    absmax = t.abs().amax(dim=dim, keepdim=True).clamp(min=1e-8)
    qt = (t * (qmax / absmax)).round().clamp(qmin, qmax).to(torch.int8)
    packed, scale = oq.rotated_quant_codes(xr, bits, axis)
    assert np.array_equal(oq.unpack_bits(packed, bits), qt.numpy())
    assert np.array_equal(scale.view(np.uint16), (absmax / qmax).to(torch.float16).numpy().view(np.uint16))
    # bfloat16 / float32 K and V: the same fp32 scale cast to their dtype
    _, sb = oq.rotated_quant_codes(xr, bits, axis, "bf16")
    assert np.array_equal(sb, _bits_bf16((absmax / qmax).to(torch.bfloat16)))
    _, sf = oq.rotated_quant_codes(xr, bits, axis, "f32")
    assert np.array_equal(sf.view(np.uint32), (absmax / qmax).numpy().view(np.uint32))
    for dt, tdt in (("bf16", torch.bfloat16), ("f32", torch.float32)):
        s_dt = sb if dt == "bf16" else sf
        st = _t_bf16(s_dt) if dt == "bf16" else torch.from_numpy(s_dt)
        ref = qt.to(tdt) * st
        got = oq.rotated_dequant_rot(packed, s_dt, bits, dt)
        assert np.array_equal(got, _bits_bf16(ref) if dt == "bf16" else ref.numpy())


def test_rotation_fixture_is_orthogonal_and_matches_torch_qr():
    R = np.load(f"{__import__('os').path.dirname(__file__)}/golden/rotation_d128_seed42.npy")
    assert R.shape == (128, 128) and R.dtype == np.float32
    assert np.abs(R @ R.T - np.eye(128)).max() < 1e-5
    gen = torch.Generator().manual_seed(42)
    q, _ = torch.linalg.qr(torch.randn(128, 128, generator=gen))
    assert np.array_equal(q.numpy(), R)


@pytest.mark.parametrize("bits", [4, 2])
def test_asym_group_invariants(bits):
    """Build-defined format: self-consistency only (the reference has no such format)."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((2, 2, 20, 64)) * 2).astype(F16)
    x[0, 0, 0, :32] = F16(1.5)  # constant group -> scale 0, codes 0
    packed, scale, zero = oq.quant_asym_group(x, bits, 32)
    codes = oq.unpack_asym_codes(packed, bits).reshape(2, 2, 20, 2, 32)
    qmax = (1 << bits) - 1
    assert codes.min() >= 0 and codes.max() <= qmax
    assert scale[0, 0, 0, 0] == 0 and np.all(codes[0, 0, 0, 0] == 0)
    xg = x.reshape(2, 2, 20, 2, 32)
    assert np.array_equal(zero, xg.min(axis=-1))
    nz = scale.astype(np.float32) > 0
    assert np.all(codes.min(axis=-1)[nz] == 0)
    deq = oq.dequant_asym_group(packed, scale, zero, bits, 32).astype(np.float32).reshape(xg.shape)
    err = np.abs(deq - xg.astype(np.float32))
    bound = 0.5 * scale.astype(np.float32)[..., None] * 1.01 + 8e-3
    assert np.all(err <= bound)
    # codes are the nearest integers to the exact quotient (x - min) / scale,
    # clamped, wherever that quotient is not within 1e-5 of a half-integer
    s64 = scale.astype(np.float64)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        exact = (xg.astype(np.float64) - zero.astype(np.float64)[..., None]) / s64
    want = np.clip(np.floor(exact + 0.5), 0, qmax)
    clear = (s64 > 0) & (np.abs(exact - np.floor(exact) - 0.5) > 1e-5)
    clear = np.broadcast_to(clear, codes.shape)
    assert clear.mean() > 0.99
    assert np.array_equal(codes[clear], want[clear].astype(codes.dtype))
    # the group maximum lands on the top code or one below it (the fp16 scale rounds either way)
    top = codes.max(axis=-1)[nz]
    assert np.all(top >= qmax - 1)


# ------------------------------------------------------------------- RoPE
def test_inv_freq_and_tables_match_torch():
    """fade/rope.py:44-46, 83-92 evaluated by torch on the host."""
    D, theta = 128, 1e6
    inv_t = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    inv_o = orope.vanilla_inv_freq(D, theta)
    exact = 1.0 / theta ** (np.arange(0, D, 2) / D)  # closed form in float64
    ulp = np.spacing(np.abs(inv_t.numpy()))
    assert np.all(np.abs(inv_o - exact) <= 2 * ulp)
    assert np.all(np.abs(inv_t.numpy() - exact) <= 2 * ulp)
    pos = torch.arange(4096)
    emb = pos.float()[:, None] * inv_t[None]
    emb = torch.cat([emb, emb], -1)
    cos_t = emb.cos().to(torch.float16).float().numpy()
    cos_o, _ = orope.cos_sin_tables(pos.numpy(), inv_t.numpy())
    assert np.mean(cos_o == cos_t) > 0.999
    assert np.abs(cos_o - cos_t).max() <= 2 ** -11


def test_rope_is_a_plane_rotation():
    """apply(k) rotates each (k[i], k[i+D/2]) pair by angle pos*inv_freq[i]."""
    rng = np.random.default_rng(6)
    D = 16
    k = rng.standard_normal((1, 1, 5, D)).astype(np.float32)
    ang = rng.uniform(-4, 4, size=(5, D // 2))
    cos = np.cos(np.concatenate([ang, ang], -1)).astype(np.float32)
    sin = np.sin(np.concatenate([ang, ang], -1)).astype(np.float32)
    out = orope.apply_rope(k, cos, sin)
    x, y = k[..., : D // 2].astype(np.float64), k[..., D // 2 :].astype(np.float64)
    ex = x * np.cos(ang) - y * np.sin(ang)
    ey = y * np.cos(ang) + x * np.sin(ang)
    assert np.allclose(out, np.concatenate([ex, ey], -1), atol=1e-5)
    back = orope.inverse_rope(out, cos, sin)
    assert np.allclose(back, k, atol=1e-5)  # tests/test_cache.py:187-196 bar


def test_rerope_identity_when_positions_do_not_move():
    rng = np.random.default_rng(7)
    k = (rng.standard_normal((1, 2, 10, 32)) * 3).astype(F16)
    v = rng.standard_normal((1, 2, 10, 32)).astype(F16)
    inv = orope.vanilla_inv_freq(32, 1e4)
    cos, sin = orope.cos_sin_tables(np.arange(10), inv)
    keep = np.array([0, 1, 2, 3])
    ko, vo = orope.rerope_gather(k, v, keep, cos, sin, cos[:4], sin[:4])
    assert np.array_equal(vo, v[:, :, :4])
    k4 = k[:, :, :4].astype(np.float32)
    d = np.abs(ko.astype(np.float32) - k4)
    # fp16-rounded cos/sin make cos^2 + sin^2 = 1 only to ~2^-11, relative to
    # the rotated pair's magnitude, plus two fp16 roundings of the result.
    pair = np.abs(k4) + np.abs(np.concatenate([k4[..., 16:], k4[..., :16]], -1))
    assert np.all(d <= pair * 2.0 ** -9 + 2 * np.spacing(np.abs(k[:, :, :4])).astype(np.float32))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_rerope_typed_matches_torch_ops(dtype):
    """fade/cache.py:290-311 on a bf16 / fp32 cache, evaluated by torch: fp32
    math, each of un-RoPE and re-RoPE cast to the cache dtype."""
    rng = np.random.default_rng(12)
    D, S = 64, 40
    k = oq.from_f32((rng.standard_normal((2, 3, S, D)) * 4).astype(np.float32), dtype)
    v = oq.from_f32(rng.standard_normal((2, 3, S, D)).astype(np.float32), dtype)
    inv = orope.vanilla_inv_freq(D, 1e4)
    cos_o, sin_o = orope.cos_sin_tables(np.arange(S) + 100, inv, round_fp16=False)
    keep = np.array([0, 3, 4, 9, 17, 30, 39])
    cos_n, sin_n = orope.cos_sin_tables(np.arange(len(keep)), inv, round_fp16=False)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    kt = (_t_bf16(k) if dtype == "bf16" else torch.from_numpy(k))[:, :, keep]

    def rot(x):
        return torch.cat((-x[..., D // 2:], x[..., : D // 2]), -1)

    co, so = torch.from_numpy(cos_o[keep]), torch.from_numpy(sin_o[keep])
    pre = (kt.float() * co - rot(kt.float()) * so).to(tdt)
    post = (pre.float() * torch.from_numpy(cos_n) + rot(pre.float()) * torch.from_numpy(sin_n)).to(tdt)
    ko, vo = orope.rerope_gather_typed(k, v, keep, cos_o, sin_o, cos_n, sin_n, dtype)
    assert np.array_equal(ko, _bits_bf16(post) if dtype == "bf16" else post.numpy())
    assert np.array_equal(vo, v[:, :, keep])
    # a single rounding (no cast between un-RoPE and re-RoPE) differs on bf16
    if dtype == "bf16":
        once = (kt.float() * co - rot(kt.float()) * so)
        once = (once * torch.from_numpy(cos_n) + rot(once) * torch.from_numpy(sin_n)).to(tdt)
        assert not np.array_equal(ko, _bits_bf16(once))


# ----------------------------------------------------------------- policy
def test_assign_one_layer_reference_kat():
    """tests/test_cache_batched.py:275-292 of the reference."""
    scores = np.array([0.1, 0.2, 5.0, 4.0, 3.0, 0.5, 0.4, 0.3])
    tiers = opol.assign_one_layer(8, scores, 1, 1, 2, 0)
    assert tiers[0] == opol.TIER_FP16 and tiers[-1] == opol.TIER_FP16
    assert set(np.nonzero(tiers == opol.TIER_INT4)[0]) == {2, 3}


def test_assign_one_layer_brute_force():
    rng = np.random.default_rng(8)
    for S in (1, 3, 9, 40):
        for ns, nr, b4, b2 in ((2, 3, 5, 4), (0, 0, 1, 0), (4, 64, None, 0), (1, 1, 100, 0)):
            sc = rng.standard_normal(S)
            t = opol.assign_one_layer(S, sc, ns, nr, b4, b2)
            fp = set(range(min(ns, S))) | set(range(max(min(ns, S), S - nr), S))
            assert set(np.nonzero(t == 0)[0]) == fp
            mid = [i for i in range(S) if i not in fp]
            ranked = sorted(mid, key=lambda i: -sc[i])
            if b4 is None or b4 >= len(mid):
                assert set(np.nonzero(t == 1)[0]) == set(mid)
            else:
                assert set(np.nonzero(t == 1)[0]) == set(ranked[:b4])
                assert set(np.nonzero(t == 2)[0]) == set(ranked[b4 : b4 + b2])


# -------------------------------------------------------------- attention
def test_sdpa_brute_force_loops_with_gqa():
    rng = np.random.default_rng(9)
    B, Hq, Hkv, Sq, Sk, D = 1, 4, 2, 2, 5, 3
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, Sq, D), (B, Hkv, Sk, D), (B, Hkv, Sk, D)))
    out = oatt.sdpa_fp32(q, k, v)
    for h in range(Hq):
        kv = h // (Hq // Hkv)
        for i in range(Sq):
            s = [sum(q[0, h, i, d] * k[0, kv, j, d] for d in range(D)) / math.sqrt(D) for j in range(Sk)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            for d in range(D):
                ref = sum(w[j] * v[0, kv, j, d] for j in range(Sk)) / sum(w)
                assert abs(out[0, h, i, d] - ref) < 1e-5


def test_sdpa_uniform_keys_average_values_and_causal_mask():
    rng = np.random.default_rng(10)
    k = np.ones((1, 1, 6, 4))
    v = rng.standard_normal((1, 1, 6, 4))
    q = rng.standard_normal((1, 2, 1, 4))
    assert np.allclose(oatt.sdpa_fp32(q, k, v)[0, :, 0], v[0, 0].mean(0), atol=1e-6)
    m = oatt.bottom_right_causal_mask(2, 6)
    assert m.tolist() == [[1, 1, 1, 1, 1, 0], [1, 1, 1, 1, 1, 1]]
    q2 = rng.standard_normal((1, 1, 2, 4))
    out = oatt.sdpa_fp32(q2, k, v, mask=m)
    assert np.allclose(out[0, 0, 0], v[0, 0, :5].mean(0), atol=1e-6)


@pytest.mark.parametrize("bits", [4, 2])
def test_bf16_rotated_middle_matches_torch_cpu_sequence(bits):
    """The oracle's bfloat16 rotated middle tier against torch running the
    reference's CPU sequence on bf16 tensors (fade/rotated_quant.py:134-145):
    ``(q.to(bf16) * scale.to(bf16)).to(float32) @ R.float()``, then ``.to(bf16)``.
    The fp32 product's summation order is torch's own, so results agree to one
    bf16 rounding step: equal bits, or neighbours where the fp32 value sits on
    a rounding boundary."""
    rng = np.random.default_rng(21 + bits)
    B, H, S, D = 2, 2, 9, 128
    qmin, qmax = oq.BIT_PARAMS[bits]
    q = rng.integers(qmin, qmax + 1, size=(B, H, S, D)).astype(np.int8)
    s = oq.f32_to_bf16(rng.uniform(0.05, 2.0, (B, H, S, 1)).astype(np.float32))
    R = np.load(f"{__import__('os').path.dirname(__file__)}/golden/rotation_d128_seed42.npy")
    packed = oq.pack_bits(q, bits)
    mid = {"fmt": "rot", "dtype": "bf16", "R": R, "k_bits": bits, "v_bits": bits,
           "kq": packed, "ks": s, "vq": packed, "vs": s}
    k, v = oatt.dequant_middle(mid)
    ref = ((torch.from_numpy(q).to(torch.bfloat16) * _t_bf16(s)).to(torch.float32) @ torch.from_numpy(R)).to(torch.bfloat16)
    rb = _bits_bf16(ref).astype(np.int32)
    gb = oq.f32_to_bf16(k).astype(np.int32)
    assert np.array_equal(k, v)
    assert np.abs(rb - gb).max() <= 1 and (rb != gb).mean() < 0.01


def test_bf16_tiered_decode_matches_torch_materialized_sdpa():
    """oatt.tiered_decode with dtype "bf16" (q, sink, recent and the INT4 middle's
    scales as bf16 bits) against torch: the reference INT4 dequantization on bf16
    tensors, torch.cat of the tiers, GQA repeat_interleave and float64 softmax
    attention (fade/cache.py:693-699, fade/kernels/fused_int4_attn.py:306-312)."""
    rng = np.random.default_rng(31)
    B, Hq, Hkv, D, ns, nm, nr = 2, 8, 2, 32, 3, 40, 5
    bf = lambda *shape: oq.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))  # noqa: E731
    q, sk, sv, rk, rv = bf(B, Hq, 1, D), bf(B, Hkv, ns, D), bf(B, Hkv, ns, D), bf(B, Hkv, nr, D), bf(B, Hkv, nr, D)
    kq = rng.integers(0, 256, (B, Hkv, nm, D // 2), dtype=np.uint8)
    vq = rng.integers(0, 256, (B, Hkv, nm, D // 2), dtype=np.uint8)
    ks = oq.f32_to_bf16(rng.uniform(0.01, 1.0, (B, Hkv, 1, D)).astype(np.float32))
    vs = oq.f32_to_bf16(rng.uniform(0.01, 1.0, (B, Hkv, nm, 1)).astype(np.float32))
    mid = {"fmt": "int4", "dtype": "bf16", "kq": kq, "ks": ks, "vq": vq, "vs": vs}
    got = oatt.tiered_decode(q, sk, sv, mid, rk, rv, dtype="bf16")
    unpack = lambda p: torch.from_numpy(oq.unpack_int4_last_dim(p).astype(np.int8))  # noqa: E731
    km = unpack(kq).to(torch.bfloat16) * _t_bf16(ks)
    vm = unpack(vq).to(torch.bfloat16) * _t_bf16(vs)
    k = torch.cat([_t_bf16(sk), km, _t_bf16(rk)], dim=-2).double().repeat_interleave(Hq // Hkv, dim=1)
    v = torch.cat([_t_bf16(sv), vm, _t_bf16(rv)], dim=-2).double().repeat_interleave(Hq // Hkv, dim=1)
    p = torch.softmax(_t_bf16(q).double() @ k.transpose(-1, -2) / math.sqrt(D), dim=-1)
    assert np.abs(got - (p @ v).float().numpy()).max() < 1e-6
