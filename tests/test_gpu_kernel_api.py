"""The reference's kernel-level API on the HIP kernels: ``fused_int4_sdpa`` with several query
rows and the top-left ``is_causal`` mask (fade/kernels/fused_int4_attn.py:165-169,277-342),
``int4_sdpa`` (fade/kernels/int4_attention.py:206-225), the parity helpers
(``check_parity``, fade/kernels/int4_attention.py:228-269), and the prefill kernel's
mask modes, each against the oracle's dequantize + fp32 SDPA with an explicit mask."""

import numpy as np
import pytest
import torch

from fade_amd.kernels import MiddleTier, fused_int4_sdpa
from fade_amd.kernels.int4_attention import check_parity, int4_sdpa
from fade_amd.kernels.prefill import tiered_prefill_attention
from fade_amd.quant import quant_k_int4, quant_v_int4
from fade_amd.synthetic import kv_tensors
from oracle import attention as oatt
from oracle import quant as oq

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def _top_left(sq: int, sk: int) -> np.ndarray:
    """fade/kernels/fused_int4_attn.py:168-169: query i sees key j when i >= j."""
    return np.arange(sk)[None, :] <= np.arange(sq)[:, None]


def _packed(dev, B, Hq, Hkv, Sq, Sk, seed):
    q, k, v = kv_tensors(B, Hkv, Sk, 128, seed=seed, Hq=Hq)
    q = torch.randn(B, Hq, Sq, 128, generator=torch.Generator().manual_seed(seed + 1)).to(torch.float16)
    kp, ks = quant_k_int4(k.to(dev))
    vp, vs = quant_v_int4(v.to(dev))
    okq, oks = oq.quant_k_int4(k.numpy())
    ovq, ovs = oq.quant_v_int4(v.numpy())
    assert np.array_equal(kp.cpu().numpy(), okq) and np.array_equal(vp.cpu().numpy(), ovq)
    kd, vd = oq.dequant_int4(okq, oks), oq.dequant_int4(ovq, ovs)
    return q, (kp, ks, vp, vs), kd, vd


@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 8, 2, 37, 300), (1, 4, 4, 100, 64), (1, 28, 4, 5, 1000), (3, 32, 8, 64, 64)])
def test_fused_int4_sdpa_query_rows(dev, shape, is_causal):
    """Several query rows in one launch; top-left causal including S_q > S_k (the rows past S_k
    see every key) and S_q == S_k (the reference test's square case)."""
    B, Hq, Hkv, Sq, Sk = shape
    print(f"case fused_int4_sdpa shape={shape} causal={is_causal}", flush=True)
    q, packed, kd, vd = _packed(dev, B, Hq, Hkv, Sq, Sk, seed=40 + Sq)
    out = fused_int4_sdpa(q.to(dev), *packed, is_causal=is_causal)
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, Sq, 128) and out.dtype == torch.float16
    ref = oatt.sdpa_fp32(q.numpy(), kd, vd, mask=_top_left(Sq, Sk) if is_causal else None)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    assert err <= ATOL, f"max-abs error {err}"


def test_fused_int4_sdpa_single_row_causal_sees_key_zero(dev):
    """Top-left causal with one query row: the row sees key 0 only, so the output is V's row 0."""
    print("case fused_int4_sdpa Sq=1 causal", flush=True)
    q, packed, kd, vd = _packed(dev, 2, 8, 2, 1, 200, seed=50)
    out = fused_int4_sdpa(q.to(dev), *packed, is_causal=True).float().cpu().numpy()
    ref = np.repeat(vd[:, :, :1].astype(np.float32), 4, axis=1)
    assert np.abs(out - ref).max() <= ATOL


def test_int4_sdpa_query_rows(dev):
    """int4_sdpa: single and several query rows (no mask), as the reference's torch path computes."""
    for Sq in (1, 19):
        print(f"case int4_sdpa Sq={Sq}", flush=True)
        q, packed, kd, vd = _packed(dev, 2, 4, 4, Sq, 333, seed=60 + Sq)
        out = int4_sdpa(q.to(dev), *packed)
        ref = oatt.sdpa_fp32(q.numpy(), kd, vd)
        assert float(np.abs(out.float().cpu().numpy() - ref).max()) <= ATOL


@pytest.mark.parametrize("S_q", [1, 16])
def test_check_parity_helper(dev, S_q):
    """fade/kernels/int4_attention.py:228-269: the helper's keys and its pass/fail result."""
    print(f"case check_parity S_q={S_q}", flush=True)
    res = check_parity(S_q=S_q)
    assert set(res) == {"passed", "max_abs_error", "mean_abs_error", "atol", "rtol"}
    assert res["passed"], res
    assert res["max_abs_error"] < 2e-3


@pytest.mark.parametrize("mask", ["top_left", "none"])
def test_prefill_mask_modes_over_tiers(dev, mask):
    """The prefill kernel's top-left and unmasked modes over [sink | INT4 middle | recent | chunk],
    with per-row lengths (ragged rows), against fp32 SDPA over each row's concatenated keys."""
    print(f"case prefill mask={mask}", flush=True)
    B, Hq, Hkv, Sq, ns, nr, nc = 3, 16, 4, 70, 4, 20, 30
    caps = (ns, 250, nr)
    lens = np.array([[4, 250, 20], [2, 100, 7], [4, 0, 20]], dtype=np.int32)
    g = torch.Generator().manual_seed(70)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.float16)  # noqa: E731
    sink = (r(B, Hkv, caps[0], 128), r(B, Hkv, caps[0], 128))
    rec = (r(B, Hkv, caps[2], 128), r(B, Hkv, caps[2], 128))
    chunk = (r(B, Hkv, nc, 128), r(B, Hkv, nc, 128))
    km, vm = r(B, Hkv, caps[1], 128), r(B, Hkv, caps[1], 128)
    q = r(B, Hq, Sq, 128)
    t = lambda x: x.to(dev)  # noqa: E731
    kq, ks = quant_k_int4(t(km))
    vq, vs = quant_v_int4(t(vm))
    out = tiered_prefill_attention(t(q), (t(chunk[0]), t(chunk[1])), (t(sink[0]), t(sink[1])),
                                   MiddleTier("int4", kq, vq, ks, vs), (t(rec[0]), t(rec[1])),
                                   lens=torch.from_numpy(lens), mask=mask)
    out = out.float().cpu().numpy()
    okq, oks = oq.quant_k_int4(km.numpy())
    ovq, ovs = oq.quant_v_int4(vm.numpy())
    kd, vd = oq.dequant_int4(okq, oks), oq.dequant_int4(ovq, ovs)
    for b in range(B):
        a, m, c = (int(x) for x in lens[b])
        K = np.concatenate([sink[0][b, :, :a].numpy(), kd[b, :, :m], rec[0][b, :, :c].numpy(), chunk[0][b].numpy()], 1)
        V = np.concatenate([sink[1][b, :, :a].numpy(), vd[b, :, :m], rec[1][b, :, :c].numpy(), chunk[1][b].numpy()], 1)
        msk = _top_left(Sq, K.shape[1]) if mask == "top_left" else None
        ref = oatt.sdpa_fp32(q.numpy()[b : b + 1], K[None], V[None], mask=msk)
        err = float(np.abs(out[b : b + 1] - ref).max())
        assert err <= ATOL, f"row {b}: max-abs error {err}"


def test_prefill_mask_argument_errors(dev):
    q = torch.zeros(1, 4, 8, 128, dtype=torch.float16, device=dev)
    kv = torch.zeros(1, 4, 8, 128, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="mask"):
        tiered_prefill_attention(q, (kv, kv), mask="diagonal")
    with pytest.raises(ValueError, match="chunk"):
        tiered_prefill_attention(q, None, (kv, kv))
