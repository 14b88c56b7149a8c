"""The CPU baseline's torch restatement (oracle/torch_cpu.py) against the numpy oracle:
nibble unpacking over all 256 bytes, dequantization bit-exact with the oracle's
fp16(code * scale), and the decode step within fp32 rounding of the oracle's SDPA."""

import numpy as np
import torch

from fade_amd.synthetic import kv_tensors
from oracle import attention as oatt
from oracle import quant as oq
from oracle import torch_cpu


def test_unpack_all_bytes():
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(1, 256)
    got = torch_cpu.unpack_int4(b).numpy()
    assert np.array_equal(got, oq.unpack_int4_last_dim(b.numpy()))
    # closed form: high nibble first, two's complement
    hi = np.array([(x >> 4) - 16 * ((x >> 4) >= 8) for x in range(256)])
    assert np.array_equal(got[0, 0::2], hi)


def test_decode_step_matches_oracle():
    q, k, v = kv_tensors(2, 4, 300, 128, seed=5, Hq=16)
    ns, nr = 4, 20
    kq, ks = oq.quant_k_int4(k.numpy()[:, :, ns:-nr])
    vq, vs = oq.quant_v_int4(v.numpy()[:, :, ns:-nr])
    t = torch.from_numpy
    deq = torch_cpu.dequant_int4(t(kq), t(ks), torch.float16).numpy()
    assert np.array_equal(deq.view(np.uint16), oq.dequant_int4(kq, ks).view(np.uint16))
    ref = oatt.tiered_decode(q.numpy(), k.numpy()[:, :, :ns], v.numpy()[:, :, :ns],
                             {"fmt": "int4", "kq": kq, "ks": ks, "vq": vq, "vs": vs},
                             k.numpy()[:, :, -nr:], v.numpy()[:, :, -nr:])
    for mode, tol in (("fp16", 1e-5), ("fp32", 2e-3)):
        out = torch_cpu.decode_step(q, (k[:, :, :ns], v[:, :, :ns]), (t(kq), t(ks), t(vq), t(vs)),
                                    (k[:, :, -nr:], v[:, :, -nr:]), mode=mode).numpy()
        assert np.abs(out - ref).max() <= tol, mode
