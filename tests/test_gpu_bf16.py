"""Fused attention over bfloat16 caches: decode and chunk prefill kernels,
the cache's fused mode and HF generate() on a bfloat16 model.

The reference keeps every tier and scale of a cache in the model's dtype and
attends over the dequantized tiers (fade/cache.py:683-842; bf16 dequantization
``q.to(bf16) * scale.to(bf16)``, fade/quant.py:124-127).  The oracle restates
that at bf16 (its bf16 rounding pinned against torch in
tests/test_oracle_pins.py) and runs float64 softmax attention.

Tolerance (bfloat16 outputs): |out - ref| <= 4e-3 + 2^-7 |ref|.  The output's
own rounding is up to 2^-9 |ref|, and the probabilities enter P V as bfloat16
(8 significant bits), as they do in the reference's bf16 SDPA; the fp16
kernels' bar (2e-3, tests/test_gpu_decode.py) stays for fp16 caches.
"""

import numpy as np
import pytest
import torch

from fade_amd import quant as fq
from fade_amd import rotated_quant as frq
from fade_amd.kernels import MiddleTier, tiered_decode_attention, tiered_prefill_attention
from fade_amd.synthetic import kv_tensors
from oracle import attention as oatt
from oracle import quant as oq

pytestmark = pytest.mark.gpu
ATOL, RTOL = 4e-3, 2.0**-7
BF = torch.bfloat16


def _bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> its uint16 bit patterns (the oracle's bf16 form)."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def _excess(out: torch.Tensor, ref: np.ndarray) -> float:
    """max(|out - ref| - RTOL |ref|): within tolerance when <= ATOL."""
    o = out.float().cpu().numpy()
    return float((np.abs(o - ref) - RTOL * np.abs(ref)).max())


def _kv(dev, B, Hq, Hkv, S, D, seed):
    q, k, v = kv_tensors(B, Hkv, S, D, seed=seed, Hq=Hq)
    return q.to(dev, BF), k.to(dev, BF), v.to(dev, BF)


def _middle(fmt, km, vm, R=None):
    """GPU middle tier of a bf16 cache and the oracle's description of it."""
    if fmt == "int4":
        kq, ks = fq.quant_k_int4(km)
        vq, vs = fq.quant_v_int4(vm)
        # codes and scales bit-exact against the oracle's bf16 quantizer (fade/quant.py:61-92 at bf16)
        okq, oks = oq.quant_k_int4_typed(_bits(km), "bf16")
        ovq, ovs = oq.quant_v_int4_typed(_bits(vm), "bf16")
        assert np.array_equal(kq.cpu().numpy(), okq) and np.array_equal(_bits(ks), oks)
        assert np.array_equal(vq.cpu().numpy(), ovq) and np.array_equal(_bits(vs), ovs)
        return MiddleTier("int4", kq, vq, ks, vs), {"fmt": "int4", "dtype": "bf16", "kq": okq, "ks": oks,
                                                    "vq": ovq, "vs": ovs}
    if fmt == "k4v2":
        kq, ks = fq.quant_k_int4(km)
        vq, vs = fq.quant_int2_padded(vm)
        mid = MiddleTier("k4v2", kq, vq, ks, vs, group=64, length=int(km.shape[2]))
        return mid, {"fmt": "k4v2", "dtype": "bf16", "kq": kq.cpu().numpy(), "ks": _bits(ks),
                     "vq": vq.cpu().numpy(), "vs": _bits(vs), "group": 64}
    bits = 4 if fmt == "rot4" else 2
    kq, ks = frq.rotated_quant_k(km, R, bits)
    vq, vs = frq.rotated_quant_v(vm, R, bits)
    assert ks.dtype == BF and vs.dtype == BF
    mid = MiddleTier("sym", kq, vq, ks, vs, k_bits=bits, v_bits=bits)
    return mid, {"fmt": "rot", "dtype": "bf16", "R": R.cpu().numpy(), "k_bits": bits, "v_bits": bits,
                 "kq": kq.cpu().numpy(), "ks": _bits(ks), "vq": vq.cpu().numpy(), "vs": _bits(vs)}


SHAPES = [
    (2, 32, 8, 700, 4, 64),  # GQA 4 (Llama-3 heads)
    (2, 28, 4, 700, 4, 64),  # GQA 7: two head passes at this size; kernel 4: eight heads per pass
    (1, 8, 8, 130, 0, 0),  # MHA, middle only, ragged tile
]


@pytest.mark.parametrize("B,Hq,Hkv,S,ns,nr", SHAPES)
@pytest.mark.parametrize("fmt,kernel", [("int4", 0), ("int4", 1), ("int4", 4), ("k4v2", 0), ("k4v2", 1), ("rot4", 0),
                                        ("rot2", 0)])
def test_decode_bf16_formats(dev, B, Hq, Hkv, S, ns, nr, fmt, kernel):
    print(f"case bf16 decode {fmt} kernel={kernel} B={B} Hq={Hq} Hkv={Hkv} S={S}", flush=True)
    q, k, v = _kv(dev, B, Hq, Hkv, S, 128, seed=700 + S + Hq)
    R = frq._random_orthogonal(128, 42).to(dev) if fmt.startswith("rot") else None
    mid, omid = _middle(fmt, k[:, :, ns : S - nr].contiguous(), v[:, :, ns : S - nr].contiguous(), R)
    sink = (k[:, :, :ns], v[:, :, :ns]) if ns else None
    rec = (k[:, :, S - nr :], v[:, :, S - nr :]) if nr else None
    out = tiered_decode_attention(q, sink, mid, rec, kernel=kernel, rotation=R)
    assert out.dtype == BF
    kb, vb = _bits(k), _bits(v)
    ref = oatt.tiered_decode(_bits(q), kb[:, :, :ns], vb[:, :, :ns], omid, kb[:, :, S - nr :], vb[:, :, S - nr :],
                             dtype="bf16")
    assert _excess(out, ref) <= ATOL


@pytest.mark.parametrize("D,kernel", [(64, 0), (64, 1), (64, 3), (80, 0), (256, 0), (256, 1), (256, 3), (128, 3)])
def test_decode_bf16_head_dims(dev, D, kernel):
    """Head dims other than 128: 64 and 256 on the general matrix-core kernel (the automatic
    choice; kernel 3), 80 on the portable one (bf16 dot products; kernel 1 everywhere)."""
    print(f"case bf16 decode head_dim={D} kernel={kernel}", flush=True)
    B, Hq, Hkv, S, ns, nr = 2, 16, 4, 300, 4, 32
    q, k, v = _kv(dev, B, Hq, Hkv, S, D, seed=800 + D)
    mid, omid = _middle("int4", k[:, :, ns : S - nr].contiguous(), v[:, :, ns : S - nr].contiguous())
    out = tiered_decode_attention(q, (k[:, :, :ns], v[:, :, :ns]), mid, (k[:, :, S - nr :], v[:, :, S - nr :]),
                                  kernel=kernel)
    kb, vb = _bits(k), _bits(v)
    ref = oatt.tiered_decode(_bits(q), kb[:, :, :ns], vb[:, :, :ns], omid, kb[:, :, S - nr :], vb[:, :, S - nr :],
                             dtype="bf16")
    assert _excess(out, ref) <= ATOL


@pytest.mark.parametrize("D", [64, 128, 256])
def test_decode_bf16_general_kernel_fp16_layout_middle(dev, D):
    """The general matrix-core kernel (kernel 3) over bf16 rows only: a plain-row middle
    tier joined to the sink and recent tiers, GQA 7 (Qwen2.5-0.5B's 14/2 heads)."""
    print(f"case bf16 decode general kernel fp16-layout middle D={D}", flush=True)
    B, Hq, Hkv, S, ns, nr = 2, 14, 2, 333, 4, 17
    q, k, v = _kv(dev, B, Hq, Hkv, S, D, seed=910 + D)
    mk, mv = k[:, :, ns : S - nr].contiguous(), v[:, :, ns : S - nr].contiguous()
    out = tiered_decode_attention(q, (k[:, :, :ns], v[:, :, :ns]), MiddleTier("fp16", mk, mv),
                                  (k[:, :, S - nr :], v[:, :, S - nr :]), kernel=3)
    kb, vb = _bits(k), _bits(v)
    omid = {"fmt": "fp16", "dtype": "bf16", "k": _bits(mk), "v": _bits(mv)}
    ref = oatt.tiered_decode(_bits(q), kb[:, :, :ns], vb[:, :, :ns], omid, kb[:, :, S - nr :], vb[:, :, S - nr :],
                             dtype="bf16")
    assert _excess(out, ref) <= ATOL


def test_decode_bf16_fp16_layout_middle(dev):
    """A middle tier of plain bf16 rows (the layout the cache uses for formats it
    reads through their dequantization) on the portable kernel."""
    print("case bf16 decode fp16-layout middle", flush=True)
    B, Hq, Hkv, S, ns, nr = 2, 32, 8, 400, 4, 64
    q, k, v = _kv(dev, B, Hq, Hkv, S, 128, seed=901)
    mk, mv = k[:, :, ns : S - nr].contiguous(), v[:, :, ns : S - nr].contiguous()
    out = tiered_decode_attention(q, (k[:, :, :ns], v[:, :, :ns]), MiddleTier("fp16", mk, mv),
                                  (k[:, :, S - nr :], v[:, :, S - nr :]))
    kb, vb = _bits(k), _bits(v)
    omid = {"fmt": "fp16", "dtype": "bf16", "k": _bits(mk), "v": _bits(mv)}
    ref = oatt.tiered_decode(_bits(q), kb[:, :, :ns], vb[:, :, :ns], omid, kb[:, :, S - nr :], vb[:, :, S - nr :],
                             dtype="bf16")
    assert _excess(out, ref) <= ATOL


def test_decode_bf16_ragged_rows_and_determinism(dev):
    """Per-row tier lengths (each row against the oracle over its own tokens), and
    deterministic calls bitwise identical."""
    print("case bf16 decode ragged + deterministic", flush=True)
    B, Hq, Hkv, S, ns, nr = 3, 32, 8, 600, 4, 64
    q, k, v = _kv(dev, B, Hq, Hkv, S, 128, seed=902)
    mid, omid = _middle("int4", k[:, :, ns : S - nr].contiguous(), v[:, :, ns : S - nr].contiguous())
    sink, rec = (k[:, :, :ns], v[:, :, :ns]), (k[:, :, S - nr :], v[:, :, S - nr :])
    lens = torch.tensor([[4, 532, 64], [2, 100, 10], [0, 1, 1]], dtype=torch.int32)
    out = tiered_decode_attention(q, sink, mid, rec, lens=lens, deterministic=True)
    again = tiered_decode_attention(q, sink, mid, rec, lens=lens, deterministic=True)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    kb, vb, qb = _bits(k), _bits(v), _bits(q)
    for b, (ls, lm, lr) in enumerate(lens.tolist()):
        # the oracle row: the row's own middle rows (its scales are per-channel over
        # the padded tier, so the middle keeps the whole tier's K scale)
        ob = {**omid, "kq": omid["kq"][b : b + 1, :, :lm], "ks": omid["ks"][b : b + 1],
              "vq": omid["vq"][b : b + 1, :, :lm], "vs": omid["vs"][b : b + 1, :, :lm]}
        ref = oatt.tiered_decode(qb[b : b + 1], kb[b : b + 1, :, :ls], vb[b : b + 1, :, :ls], ob,
                                 kb[b : b + 1, :, S - nr : S - nr + lr], vb[b : b + 1, :, S - nr : S - nr + lr],
                                 dtype="bf16")
        assert _excess(out[b : b + 1], ref) <= ATOL, b


def test_decode_bf16_refusals(dev):
    """Mixed dtypes and the asymmetric format (fp16 by definition) are refused."""
    q, k, v = _kv(dev, 1, 8, 8, 130, 128, seed=903)
    mid, _ = _middle("int4", k[:, :, 4:].contiguous(), v[:, :, 4:].contiguous())
    with pytest.raises(ValueError):
        tiered_decode_attention(q, (k[:, :, :4].half(), v[:, :, :4].half()), mid, None)
    with pytest.raises(ValueError):
        tiered_decode_attention(q.half(), (k[:, :, :4], v[:, :, :4]), None, None)
    kq, ks, kz = fq.quant_asym(k[:, :, 4:].half().contiguous(), 4, 32)
    vq, vs, vz = fq.quant_asym(v[:, :, 4:].half().contiguous(), 4, 32)
    with pytest.raises(ValueError):
        tiered_decode_attention(q, None, MiddleTier("asym", kq, vq, ks, vs, kz, vz, group=32), None)


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 32, 8), (64, 28, 4), (256, 8, 4)])
@pytest.mark.parametrize("with_mid", [True, False])
def test_prefill_bf16(dev, D, Hq, Hkv, with_mid):
    """Ragged chunk prefill on bf16 tiers: the middle tier dequantized in the kernel
    to bf16(code * scale), bf16 MFMAs; each row against the oracle's bottom-right
    causal attention over its own [sink | middle | recent | chunk]."""
    print(f"case bf16 prefill D={D} Hq={Hq} Hkv={Hkv} mid={with_mid}", flush=True)
    B, Sq = 2, 70
    rows = [(4, 500, 64), (2, 130, 20)]
    caps = [max(r[i] for r in rows) for i in range(3)]
    z = lambda *s: torch.zeros(*s, dtype=BF, device=dev)  # noqa: E731
    sink_k, sink_v, rec_k, rec_v = z(B, Hkv, caps[0], D), z(B, Hkv, caps[0], D), z(B, Hkv, caps[2], D), z(B, Hkv, caps[2], D)
    kq = torch.zeros(B, Hkv, caps[1], D // 2, dtype=torch.uint8, device=dev)
    vq = torch.zeros_like(kq)
    ks, vs = torch.ones(B, Hkv, 1, D, dtype=BF, device=dev), torch.ones(B, Hkv, caps[1], 1, dtype=BF, device=dev)
    qs, ck, cv = z(B, Hq, Sq, D), z(B, Hkv, Sq, D), z(B, Hkv, Sq, D)
    q_l, k_l, v_l = [], [], []
    for b, (ns, nm, nr) in enumerate(rows):
        nm = nm if with_mid else 0
        L = ns + nm + nr
        q, k, v = kv_tensors(1, Hkv, L + Sq, D, seed=1000 + b, Hq=Hq, Sq=Sq)
        q, k, v = q.to(dev, BF), k.to(dev, BF), v.to(dev, BF)
        qs[b], ck[b], cv[b] = q[0], k[0, :, L:], v[0, :, L:]
        sink_k[b, :, :ns], sink_v[b, :, :ns] = k[0, :, :ns], v[0, :, :ns]
        rec_k[b, :, :nr], rec_v[b, :, :nr] = k[0, :, ns + nm : L], v[0, :, ns + nm : L]
        pk, pv = [oq.to_f32(_bits(k[0, :, :ns]), "bf16")], [oq.to_f32(_bits(v[0, :, :ns]), "bf16")]
        if nm:
            kqb, ksb = fq.quant_k_int4(k[:, :, ns : ns + nm].contiguous())
            vqb, vsb = fq.quant_v_int4(v[:, :, ns : ns + nm].contiguous())
            kq[b, :, :nm], ks[b], vq[b, :, :nm], vs[b, :, :nm] = kqb[0], ksb[0], vqb[0], vsb[0]
            mk, mv = oatt.dequant_middle({"fmt": "int4", "dtype": "bf16", "kq": kqb.cpu().numpy(), "ks": _bits(ksb),
                                          "vq": vqb.cpu().numpy(), "vs": _bits(vsb)})
            pk.append(mk[0])
            pv.append(mv[0])
        pk += [oq.to_f32(_bits(k[0, :, ns + nm :]), "bf16")]
        pv += [oq.to_f32(_bits(v[0, :, ns + nm :]), "bf16")]
        q_l.append(oq.to_f32(_bits(q[0]), "bf16"))
        k_l.append(np.concatenate(pk, axis=-2))
        v_l.append(np.concatenate(pv, axis=-2))
    mid = MiddleTier("int4", kq, vq, ks, vs) if with_mid else None
    lens = torch.tensor([[r[0], r[1] if with_mid else 0, r[2]] for r in rows], dtype=torch.int32)
    out = tiered_prefill_attention(qs, (ck, cv), (sink_k, sink_v), mid, (rec_k, rec_v), lens=lens)
    assert out.dtype == BF
    ref = np.stack(oatt.ragged_prefill(q_l, k_l, v_l))
    assert _excess(out, ref) <= ATOL


def _tiny_model(dev, impl, heads=4, kv_heads=2, head_dim=128):
    from transformers import AutoConfig, AutoModelForCausalLM

    cfg = AutoConfig.for_model(
        "llama", vocab_size=128, hidden_size=head_dim * heads, intermediate_size=256, num_hidden_layers=2,
        num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=head_dim, max_position_embeddings=256,
        rope_theta=500000.0, tie_word_embeddings=True,
    )
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(cfg, attn_implementation="sdpa")
    model.to(device=dev, dtype=BF).eval()
    model.set_attn_implementation(impl)
    return model, cfg


def _steps(model, cache, ids, n, middle_after_prompt):
    from fade_amd.cache import TIER_FP16, TIER_INT4

    logits = []
    with torch.no_grad():
        out = model(ids, past_key_values=cache, use_cache=True)
        logits.append(out.logits[:, -1].float())
        if middle_after_prompt:
            for li in range(len(cache)):
                S = cache.get_seq_length(li)
                tiers = torch.full((S,), TIER_INT4, dtype=torch.long, device=ids.device)
                tiers[: cache.n_sink] = TIER_FP16
                tiers[S - 4 :] = TIER_FP16
                cache.apply_tier_assignment(li, tiers)
        tok = out.logits[:, -1:].argmax(-1)
        for _ in range(n):
            out = model(tok, past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1].float())
            tok = out.logits[:, -1:].argmax(-1)
    return logits


@pytest.mark.parametrize("middle", [False, True])
def test_bf16_llama_fused_logits_match_materialized(dev, middle):
    """A bfloat16 Llama-shaped model with attn_implementation="fade" on a bfloat16
    tiered cache: prompt through the prefill kernel, decode steps through the
    matrix-core kernel, against the same cache class returning dequantized bf16
    K/V to the model's SDPA (the reference's path)."""
    from fade_amd import create_tiered_cache

    print(f"case bf16 generate fused vs materialized middle={middle}", flush=True)
    model, cfg = _tiny_model(dev, "fade")
    kw = {"n_sink": 2, "recent_window": 8, "int4_budget": None, "int2_budget": 0}
    ids = torch.randint(0, cfg.vocab_size, (2, 40), device=dev)
    cache = create_tiered_cache(model, dtype=BF, **kw)
    assert cache.fused
    fused = _steps(model, cache, ids, 3, middle)
    assert all(st.int4_k_deq is None for st in cache._layers)  # nothing was materialized
    model.set_attn_implementation("sdpa")
    ref_cache = create_tiered_cache(model, dtype=BF, **kw)
    assert not ref_cache.fused
    ref = _steps(model, ref_cache, ids, 3, middle)
    for a, b in zip(fused, ref):
        # bf16 activations through two layers: the logits' own bf16 noise is ~1e-2
        assert (a - b).abs().max().item() <= 6e-2


def test_bf16_generate_runs_on_fused_kernels(dev):
    from fade_amd import create_tiered_cache

    print("case bf16 generate()", flush=True)
    model, cfg = _tiny_model(dev, "fade")
    ids = torch.randint(0, cfg.vocab_size, (1, 24), device=dev)
    cache = create_tiered_cache(model, dtype=BF, n_sink=2, recent_window=8, int4_budget=None, int2_budget=0)
    with torch.no_grad():
        out = model.generate(ids, past_key_values=cache, max_new_tokens=6, do_sample=False)
    assert out.shape == (1, 30)
