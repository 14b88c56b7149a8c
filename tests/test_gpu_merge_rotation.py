"""The fused split merge with caches of different contents taking turns on one
shared stream workspace (the decode loop's pattern: one call per layer).

Every call leaves partials of its own cache in the workspace, so a merge that
read a partial of the previous call (or a tile stage holding a previous tile)
would return another cache's numbers.  Deterministic calls must reproduce
their cache's first output bit for bit, and every call must stay within the
bar of the one-split result, which merges nothing.  The configs' full shapes:
config 1 (B=16, S=8192) and config 2 (B=4, S=32768); and one or two kv heads
of a short row, where every split holds one tile and all the workgroups of a
(row, kv head) reach the merge together.
"""

import pytest
import torch

from fade_amd import quant as fq
from fade_amd.kernels import MiddleTier, tiered_decode_attention

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def _cache(dev, B, Hkv, S, ns, nr, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    chan = torch.empty(Hkv, 128, device=dev).log_normal_(0.0, 0.5, generator=g)
    k = (torch.randn(B, Hkv, S, 128, device=dev, generator=g) * chan[None, :, None, :]).half()
    v = torch.randn(B, Hkv, S, 128, device=dev, generator=g).half()
    q = torch.randn(B, 4 * Hkv, 1, 128, device=dev, generator=g).half()
    kq, ks = fq.quant_k_int4(k[:, :, ns : S - nr].contiguous())
    vq, vs = fq.quant_v_int4(v[:, :, ns : S - nr].contiguous())
    sink = (k[:, :, :ns].contiguous(), v[:, :, :ns].contiguous())
    rec = (k[:, :, S - nr :].contiguous(), v[:, :, S - nr :].contiguous())
    return q, sink, MiddleTier("int4", kq, vq, ks, vs), rec


@pytest.mark.parametrize("B,Hkv,S,ns,nr", [(16, 8, 8192, 4, 64), (4, 8, 32768, 4, 256), (1, 1, 300, 0, 37),
                                            (1, 2, 160, 4, 17)])
def test_split_merge_rotating_caches(dev, B, Hkv, S, ns, nr):
    print(f"case merge rotation B={B} Hkv={Hkv} S={S}", flush=True)
    cases = []
    for seed in (21, 22, 23):
        args = _cache(dev, B, Hkv, S, ns, nr, seed)
        one = tiered_decode_attention(*args, n_splits=1, deterministic=True)
        first = tiered_decode_attention(*args, deterministic=True)
        cases.append((args, one, first))
    torch.cuda.synchronize()
    for i, (_, one, first) in enumerate(cases):
        e = (first.float() - one.float()).abs().max().item()
        assert e <= ATOL, f"cache {i}: default splits vs one split {e}"
    differ = torch.zeros((), dtype=torch.int64, device=dev)
    worst = torch.zeros((), device=dev)
    for _ in range(60):
        for args, one, first in cases:
            o = tiered_decode_attention(*args, deterministic=True)
            differ += (o != first).any().long()
            o = tiered_decode_attention(*args, deterministic=False)
            worst = torch.maximum(worst, (o.float() - one.float()).abs().max())
    torch.cuda.synchronize()
    assert int(differ) == 0, f"{int(differ)} of 180 deterministic calls differ from their cache's first output"
    assert float(worst) <= ATOL, f"a claiming call is {float(worst)} from the one-split result"
