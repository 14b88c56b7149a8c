"""The allocation-free decode entry point (fade_tiered_decode_attn_noalloc, no reference
counterpart) against fade_tiered_decode_attn on the same inputs, through the C ABI: two
calls in a row, the second with a smaller input (the library scratch keeps the first call's
contents), then an interleaving with the workspace entry point."""

import numpy as np
import pytest
import torch

from fade_amd.kernels import MiddleTier
from fade_amd.kernels.tiered_attn import TieredDecodePlan
from fade_amd.quant import quant_asym, quant_k_int4, quant_v_int4
from fade_amd.synthetic import kv_tensors
from oracle import attention as oatt
from oracle import quant as oq

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def _case(dev, B, Hq, Hkv, S, ns, nr, seed, fmt="int4"):
    q, k, v = kv_tensors(B, Hkv, S, 128, seed=seed, Hq=Hq)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    km, vm = kd[:, :, ns : S - nr].contiguous(), vd[:, :, ns : S - nr].contiguous()
    if fmt == "int4":
        kq, ks = quant_k_int4(km)
        vq, vs = quant_v_int4(vm)
        mid = MiddleTier("int4", kq, vq, ks, vs)
        okq, oks = oq.quant_k_int4(k.numpy()[:, :, ns : S - nr])
        ovq, ovs = oq.quant_v_int4(v.numpy()[:, :, ns : S - nr])
        mref = {"fmt": "int4", "kq": okq, "ks": oks, "vq": ovq, "vs": ovs}
    else:
        kq, ks, kz = quant_asym(km, 4, 32)
        vq, vs, vz = quant_asym(vm, 4, 32)
        mid = MiddleTier("asym", kq, vq, ks, vs, kz, vz, k_bits=4, v_bits=4, group=32)
        mref = {"fmt": "asym", "k_bits": 4, "v_bits": 4, "group": 32}
        for p_, x in (("k", k), ("v", v)):
            a, b, c = oq.quant_asym_group(x.numpy()[:, :, ns : S - nr], 4, 32)
            mref.update({f"{p_}q": a, f"{p_}s": b, f"{p_}z": c})
    sink = (kd[:, :, :ns], vd[:, :, :ns])
    rec = (kd[:, :, S - nr :], vd[:, :, S - nr :])
    ref = oatt.tiered_decode(q.numpy(), k.numpy()[:, :, :ns], v.numpy()[:, :, :ns], mref,
                             k.numpy()[:, :, S - nr :], v.numpy()[:, :, S - nr :])
    return (qd, sink, mid, rec), ref


def _both(args):
    a = TieredDecodePlan(*args, deterministic=True).run()
    b = TieredDecodePlan(*args, deterministic=True, no_alloc=True).run()
    torch.cuda.synchronize()
    return a.clone(), b.clone()


@pytest.mark.parametrize("fmt", ["int4", "asym"])
def test_noalloc_equals_workspace_entry_two_calls(dev, fmt):
    """Second call smaller than the first: the scratch's leftover partials and counters from
    the first call must not leak into it.  Deterministic tile order makes the two entry
    points' outputs bitwise comparable (same kernel, same splits)."""
    for case in ((4, 32, 8, 3000, 4, 64, 11), (2, 16, 4, 700, 4, 64, 12)):
        print(f"case noalloc fmt={fmt} shape={case}", flush=True)
        args, ref = _case(dev, *case, fmt=fmt)
        a, b = _both(args)
        assert torch.equal(a, b), f"{fmt} {case}: noalloc differs from the workspace entry point"
        err = float(np.abs(b.float().cpu().numpy() - ref).max())
        assert err <= ATOL, f"{fmt} {case}: max-abs error {err} vs the oracle"


def test_noalloc_gqa8_two_passes_then_gqa4(dev):
    """Two head passes (8 query heads per kv head: twice the counter slots), then a GQA-4 call."""
    for case in ((3, 32, 4, 1500, 4, 64, 13), (1, 8, 2, 400, 4, 32, 14)):
        print(f"case noalloc gqa shape={case}", flush=True)
        args, ref = _case(dev, *case)
        a, b = _both(args)
        assert torch.equal(a, b)
        assert float(np.abs(b.float().cpu().numpy() - ref).max()) <= ATOL


def test_noalloc_rejects_too_many_counters(dev):
    """More (row, kv head, head pass) slots than the scratch's counter region: a clear error."""
    q = torch.zeros(40000, 2, 1, 128, dtype=torch.float16, device=dev)
    kv = torch.zeros(40000, 2, 1, 128, dtype=torch.float16, device=dev)
    plan = TieredDecodePlan(q, (kv, kv), None, None, no_alloc=True)
    with pytest.raises(ValueError, match="split counters"):
        plan.run()
