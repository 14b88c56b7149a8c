"""GPU parity of the quantize / pack / dequantize kernels against the CPU oracle (bit-exact)."""

import numpy as np
import pytest
import torch

from fade_amd import quant as fq
from fade_amd import rotated_quant as frq
from fade_amd.synthetic import kv_tensors
from oracle import quant as oq

pytestmark = pytest.mark.gpu
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


@pytest.mark.parametrize("shape", [(1, 8, 1980, 128), (2, 3, 67, 128), (1, 2, 5, 64), (1, 1, 300, 256)])
def test_quant_k_int4_bit_exact(dev, shape):
    print(f"case quant_k_int4 {shape}", flush=True)
    x = _edge_tensor(shape, 0)
    packed, scale = fq.quant_k_int4(torch.from_numpy(x).to(dev))
    op, osc = oq.quant_k_int4(x)
    assert np.array_equal(packed.cpu().numpy(), op)
    assert np.array_equal(_u16(scale.cpu().numpy()), _u16(osc))


@pytest.mark.parametrize("shape", [(1, 8, 1980, 128), (2, 3, 67, 128), (1, 2, 5, 64), (1, 1, 300, 256)])
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


def test_dequant_int4_bit_exact(dev):
    print("case dequant_int4", flush=True)
    x = _edge_tensor((2, 2, 40, 128), 3)
    op, osc = oq.quant_k_int4(x)
    out = fq.dequant_int4(torch.from_numpy(op).to(dev), torch.from_numpy(osc).to(dev))
    assert np.array_equal(_u16(out.cpu().numpy()), _u16(oq.dequant_int4(op, osc)))
    op, osc = oq.quant_v_int4(x)
    out = fq.dequant_int4(torch.from_numpy(op).to(dev), torch.from_numpy(osc).to(dev))
    assert np.array_equal(_u16(out.cpu().numpy()), _u16(oq.dequant_int4(op, osc)))


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
    kp, ks = frq.rotated_quant_k(x, R.to(dev), bits)
    vp, vs = frq.rotated_quant_v(x, R.to(dev), bits)
    okp, oks = oq.rotated_quant_codes(xr, bits, "channel")
    ovp, ovs = oq.rotated_quant_codes(xr, bits, "token")
    assert np.array_equal(kp.cpu().numpy().view(np.uint8), okp.view(np.uint8))
    assert np.array_equal(_u16(ks.cpu().numpy()), _u16(oks))
    assert np.array_equal(vp.cpu().numpy().view(np.uint8), ovp.view(np.uint8))
    assert np.array_equal(_u16(vs.cpu().numpy()), _u16(ovs))
    deq = frq.rotated_dequant_rot(kp, ks, bits).cpu().numpy()
    assert np.array_equal(_u16(deq), _u16(oq.rotated_dequant_rot(okp, oks, bits)))


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("group", [32, 16])
def test_asym_group_quant_bit_exact(dev, bits, group):
    print(f"case asym bits={bits} group={group}", flush=True)
    x = _edge_tensor((2, 3, 50, 128), 7)
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
    with pytest.raises(ValueError, match="float16"):
        fq.quant_k_int4(torch.zeros(1, 1, 4, 128, device=dev))
    with pytest.raises(ValueError, match="head_dim must be"):
        fq.quant_v_int4(torch.zeros(1, 1, 4, 96, dtype=torch.float16, device=dev))
