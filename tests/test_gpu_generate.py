"""HF generate() on the fused tiered kernels (attn_implementation="fade").

Pins from the reference's own tests, on a tiny random-init Qwen2 (no
downloads; head_dim 128, and 64 in one test, fp16 on the GPU):
  * greedy generate == a manual greedy loop (tests/test_generate.py:88-117);
  * with no eviction the first token equals a plain DynamicCache's
    (tests/test_eval_gate.py:104-138);
  * batched == unbatched (tests/test_integration.py:87-151).
Plus: the fused path's logits against the materialized path (the same cache
class returning dequantized K/V to the model's SDPA), with and without an
INT4 middle tier, and a check that the kernels actually ran.
"""

import pytest
import torch

from fade_amd import create_tiered_cache
from fade_amd.cache import TIER_FP16, TIER_INT4

pytestmark = pytest.mark.gpu


def _tiny_model(dev, impl, heads=4, kv_heads=2, head_dim=128):
    from transformers import AutoConfig, AutoModelForCausalLM

    cfg = AutoConfig.for_model(
        "qwen2", vocab_size=128, hidden_size=head_dim * heads, intermediate_size=256, num_hidden_layers=2,
        num_attention_heads=heads, num_key_value_heads=kv_heads, max_position_embeddings=256, rope_theta=10000.0,
        tie_word_embeddings=True,
    )
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(cfg, attn_implementation="sdpa")
    model.to(device=dev, dtype=torch.float16).eval()
    model.set_attn_implementation(impl)
    return model, cfg


def _cache(model, **kw):
    kw = {"n_sink": 2, "recent_window": 8, "int4_budget": None, "int2_budget": 0, **kw}
    return create_tiered_cache(model, dtype=torch.float16, **kw)


def _steps(model, cache, ids, n, middle_after_prompt=False):
    """Prompt forward + n greedy decode steps; returns the list of logits."""
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


def test_fused_cache_mode_and_kernels_run(dev, monkeypatch):
    print("case generate fused mode", flush=True)
    model, cfg = _tiny_model(dev, "fade")
    cache = _cache(model)
    assert cache.fused
    calls = {"decode": 0, "prefill": 0}
    import fade_amd.kernels.prefill as kp
    import fade_amd.kernels.tiered_attn as kt

    real_run, real_rerun, real_p = kt.TieredDecodePlan.run, kt.TieredDecodePlan.rerun, kp.tiered_prefill_attention

    def run(self, *a, **k):  # decode launches: a plan's first launch, then its relaunches
        calls["decode"] += 1
        return real_run(self, *a, **k)

    def rerun(self, *a, **k):
        calls["decode"] += 1
        return real_rerun(self, *a, **k)

    def p(*a, **k):
        calls["prefill"] += 1
        return real_p(*a, **k)

    monkeypatch.setattr(kt.TieredDecodePlan, "run", run)
    monkeypatch.setattr(kt.TieredDecodePlan, "rerun", rerun)
    monkeypatch.setattr(kp, "tiered_prefill_attention", p)
    ids = torch.randint(0, cfg.vocab_size, (1, 12), device=dev)
    _steps(model, cache, ids, 2)
    assert calls["prefill"] == cfg.num_hidden_layers and calls["decode"] == 2 * cfg.num_hidden_layers
    # nothing was materialized
    assert all(st.int4_k_deq is None for st in cache._layers)


@pytest.mark.parametrize("middle", [False, True])
def test_fused_logits_match_materialized(dev, middle):
    print(f"case generate fused vs materialized middle={middle}", flush=True)
    model, cfg = _tiny_model(dev, "fade")
    ids = torch.randint(0, cfg.vocab_size, (2, 40), device=dev)
    fused = _steps(model, _cache(model), ids, 3, middle_after_prompt=middle)
    model.set_attn_implementation("sdpa")
    ref_cache = _cache(model)
    assert not ref_cache.fused
    ref = _steps(model, ref_cache, ids, 3, middle_after_prompt=middle)
    for a, b in zip(fused, ref):
        assert (a - b).abs().max().item() <= 2e-2


@pytest.mark.parametrize("heads,kv_heads", [(7, 1), (8, 1), (5, 1)])
def test_fused_logits_match_materialized_gqa_5_to_8(dev, heads, kv_heads):
    """Query-head groups of 5-8 (Qwen2.5-7B's 7): the prompt goes through the prefill
    kernel's two head passes, the decode steps through the matrix-core kernel."""
    print(f"case generate fused vs materialized GQA {heads}/{kv_heads}", flush=True)
    model, cfg = _tiny_model(dev, "fade", heads, kv_heads)
    ids = torch.randint(0, cfg.vocab_size, (2, 40), device=dev)
    fused = _steps(model, _cache(model), ids, 3, middle_after_prompt=True)
    model.set_attn_implementation("sdpa")
    ref = _steps(model, _cache(model), ids, 3, middle_after_prompt=True)
    for a, b in zip(fused, ref):
        assert (a - b).abs().max().item() <= 2e-2


def test_fused_logits_match_materialized_head_dim_64(dev):
    """Qwen2.5-0.5B's attention shape (14 query heads / 2 kv heads, head_dim 64): the
    prompt through the prefill kernel's D = 64 instance (two head passes), the decode
    steps through the portable kernel."""
    print("case generate fused vs materialized head_dim 64", flush=True)
    model, cfg = _tiny_model(dev, "fade", 14, 2, head_dim=64)
    ids = torch.randint(0, cfg.vocab_size, (2, 40), device=dev)
    fused = _steps(model, _cache(model), ids, 3, middle_after_prompt=True)
    model.set_attn_implementation("sdpa")
    ref = _steps(model, _cache(model), ids, 3, middle_after_prompt=True)
    for a, b in zip(fused, ref):
        assert (a - b).abs().max().item() <= 2e-2


def test_generate_greedy_matches_manual_loop(dev):
    print("case generate greedy vs manual", flush=True)
    model, cfg = _tiny_model(dev, "fade")
    ids = torch.randint(0, cfg.vocab_size, (1, 8), device=dev)
    gen = model.generate(ids, past_key_values=_cache(model), max_new_tokens=4, do_sample=False)
    cache = _cache(model)
    toks = []
    with torch.no_grad():
        out = model(ids, past_key_values=cache, use_cache=True)
        tok = out.logits[:, -1:].argmax(-1)
        toks.append(tok)
        for _ in range(3):
            out = model(tok, past_key_values=cache, use_cache=True)
            tok = out.logits[:, -1:].argmax(-1)
            toks.append(tok)
    manual = torch.cat([ids, *toks], dim=-1)
    n = min(gen.shape[1], manual.shape[1])
    assert torch.equal(gen[:, :n], manual[:, :n])


def test_first_token_matches_dynamic_cache(dev):
    print("case generate first token vs DynamicCache", flush=True)
    from transformers import DynamicCache

    model, cfg = _tiny_model(dev, "fade")
    ids = torch.randint(0, cfg.vocab_size, (1, 16), device=dev)
    with torch.no_grad():
        a = model(ids, past_key_values=_cache(model), use_cache=True).logits[:, -1].float()
        model.set_attn_implementation("sdpa")
        b = model(ids, past_key_values=DynamicCache(), use_cache=True).logits[:, -1].float()
    assert a.argmax(-1).tolist() == b.argmax(-1).tolist()
    assert (a - b).abs().max().item() <= 2e-2


def test_batched_equals_unbatched(dev):
    print("case generate batched vs unbatched", flush=True)
    model, cfg = _tiny_model(dev, "fade")
    ids = torch.randint(0, cfg.vocab_size, (2, 24), device=dev)
    both = _steps(model, _cache(model), ids, 2, middle_after_prompt=True)
    for r in range(2):
        one = _steps(model, _cache(model), ids[r : r + 1], 2, middle_after_prompt=True)
        for a, b in zip(both, one):
            assert (a[r] - b[0]).abs().max().item() <= 2e-3


def test_bf16_model_on_bf16_tiered_cache(dev):
    """A bfloat16 model on TieredKVCache(dtype=bfloat16), attending over the
    materialized K/V (attn_implementation="sdpa", as the reference runs bf16
    models): before any compression its logits equal a DynamicCache's bit for
    bit; after an INT4 middle tier the tiers and scales are bf16, the decode
    steps stay close to the uncompressed cache, and generate() runs."""
    print("case generate bf16 cache", flush=True)
    from transformers import DynamicCache

    model, cfg = _tiny_model(dev, "sdpa")
    model.to(torch.bfloat16)
    ids = torch.randint(0, cfg.vocab_size, (1, 24), device=dev)
    kw = {"n_sink": 2, "recent_window": 8, "int4_budget": None, "int2_budget": 0}
    with torch.no_grad():
        a = model(ids, past_key_values=create_tiered_cache(model, dtype=torch.bfloat16, **kw), use_cache=True).logits
        b = model(ids, past_key_values=DynamicCache(), use_cache=True).logits
    assert torch.equal(a, b)
    cache = create_tiered_cache(model, dtype=torch.bfloat16, **kw)
    tiered = _steps(model, cache, ids, 3, middle_after_prompt=True)
    st = cache._layers[0]
    assert st.int4_kq is not None and st.int4_ks.dtype == torch.bfloat16 and st.fp16_k.dtype == torch.bfloat16
    plain = _steps(model, DynamicCache(), ids, 3)
    assert tiered[0].tolist() == plain[0].tolist()  # the prompt's logits precede the tiering
    assert all(torch.isfinite(t).all() for t in tiered)
    # the first decode step feeds both caches the same token
    assert (tiered[1] - plain[1]).abs().max().item() <= 0.1 * plain[1].abs().max().item()
    gen = model.generate(ids, past_key_values=create_tiered_cache(model, dtype=torch.bfloat16, **kw), max_new_tokens=4,
                         do_sample=False)
    assert gen.shape[0] == 1 and 24 < gen.shape[1] <= 28
