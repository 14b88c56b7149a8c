"""Per-architecture runs through the tiered cache, after the reference's
tests/test_models.py:38-200: a tiny random-init model of each family
(hidden 64, 4 heads: head_dim 16), a 16-token prefill, one decode step, a
tier reassignment (sink 2 + recent 4 fp16, the rest INT4, no eviction) and
one more decode step, in float32 as the reference runs them (on the GPU here:
the cache's kernels have no CPU path).  Checked as there: sequence lengths,
the tier sizes, the detected RoPE scheme, the GQA scale shapes.

Plus the fused path (attn_implementation="fade", fp16) at head dims other than
32/64/128/256: its logits against the same cache class returning materialized
K/V to the model's own SDPA.
"""

import pytest
import torch

from fade_amd import create_tiered_cache
from fade_amd.cache import TIER_FP16, TIER_INT4
from fade_amd.policy import reassign_tiers_by_position
from fade_amd.rope import Llama3, NoRope, Vanilla

pytestmark = pytest.mark.gpu


def _run_model(dev, model_type, extra_cfg=None, expect_scheme=Vanilla):
    from transformers import AutoConfig, AutoModelForCausalLM

    cfg_kwargs = dict(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, max_position_embeddings=128, tie_word_embeddings=True)
    if model_type in ("qwen2", "llama", "mistral", "phi3", "gemma2", "falcon"):
        cfg_kwargs["num_key_value_heads"] = 2
    if model_type == "mistral":
        cfg_kwargs["sliding_window"] = 64
    if model_type == "phi3":  # its padding_idx defaults to 32000
        cfg_kwargs["vocab_size"] = 32064
        cfg_kwargs["original_max_position_embeddings"] = 128
    if model_type == "gemma2":
        cfg_kwargs["head_dim"] = 16
    if model_type == "falcon":
        cfg_kwargs.pop("intermediate_size")
    cfg_kwargs.update(extra_cfg or {})
    cfg = AutoConfig.for_model(model_type, **cfg_kwargs)
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(cfg, attn_implementation="eager").to(device=dev, dtype=torch.float32)
    model.eval()
    n_layers = cfg.num_hidden_layers
    cache = create_tiered_cache(model, dtype=torch.float32, n_sink=2, recent_window=4, int4_budget=None, int2_budget=0)
    assert isinstance(cache.rope_scheme, expect_scheme), type(cache.rope_scheme).__name__
    ids = torch.randint(0, cfg.vocab_size, (1, 16), device=dev)
    with torch.no_grad():
        out = model(ids, past_key_values=cache, use_cache=True)
        assert out.logits.shape == (1, 16, cfg.vocab_size)
        assert cache.get_seq_length(0) == 16
        out2 = model(out.logits[:, -1:].argmax(-1), past_key_values=cache, use_cache=True)
        assert cache.get_seq_length(0) == 17
        reassign_tiers_by_position(cache, n_layers)
        st = cache._layers[0]
        n_sink = st.sink_k.shape[-2] if st.sink_k is not None else 0
        n_recent = st.fp16_k.shape[-2] if st.fp16_k is not None else 0
        assert n_sink + n_recent == 6
        assert st.int4_kq.shape[-2] == 17 - 6
        out3 = model(out2.logits[:, -1:].argmax(-1), past_key_values=cache, use_cache=True)
        assert out3.logits.shape == (1, 1, cfg.vocab_size)
        assert torch.isfinite(out3.logits).all()
        assert cache.get_seq_length(0) == 18
    return cache, cfg


@pytest.mark.parametrize("model_type", ["qwen2", "llama", "mistral", "phi3", "gemma2"])
def test_architecture(dev, model_type):  # tests/test_models.py:122-151
    print(f"case model {model_type} head_dim 16", flush=True)
    _run_model(dev, model_type)


def test_llama3_scaling(dev):  # tests/test_models.py:130-145
    print("case model llama3 rope scaling", flush=True)
    _run_model(dev, "llama", extra_cfg={"rope_theta": 500000.0, "rope_scaling": {
        "type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
        "original_max_position_embeddings": 128}}, expect_scheme=Llama3)


def test_falcon_alibi(dev):  # tests/test_models.py:156-168
    print("case model falcon alibi", flush=True)
    try:
        _run_model(dev, "falcon", extra_cfg={"alibi": True}, expect_scheme=NoRope)
    except ValueError as e:
        if "torch>=2.6" in str(e) or "or_mask_function" in str(e):
            pytest.skip(f"Falcon ALiBi mask needs another torch: {e}")
        raise


def test_gqa_int4_scale_shapes(dev):  # tests/test_models.py:172-186
    print("case model GQA scale shapes", flush=True)
    cache, cfg = _run_model(dev, "qwen2")
    st = cache._layers[0]
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
    assert st.int4_ks.shape[1] == cfg.num_key_value_heads and st.int4_ks.shape[-1] == head_dim
    assert st.int4_vs.shape[1] == cfg.num_key_value_heads and st.int4_vs.shape[-1] == 1


def _tiny_fp16(dev, impl, heads, kv_heads, head_dim):
    from transformers import AutoConfig, AutoModelForCausalLM

    cfg = AutoConfig.for_model(
        "qwen2", vocab_size=128, hidden_size=head_dim * heads, intermediate_size=256, num_hidden_layers=2,
        num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=head_dim, max_position_embeddings=256,
        rope_theta=10000.0, tie_word_embeddings=True,
    )
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(cfg, attn_implementation="sdpa").to(device=dev, dtype=torch.float16)
    model.eval()
    model.set_attn_implementation(impl)
    return model, cfg


def _steps(model, cache, ids, n, chunk):
    logits = []
    with torch.no_grad():
        out = model(ids, past_key_values=cache, use_cache=True)
        logits.append(out.logits[:, -1].float())
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
        # a chunk of tokens over the tiered cache (the prefill kernel)
        out = model(chunk, past_key_values=cache, use_cache=True)
        logits.append(out.logits[:, -1].float())
    return logits


@pytest.mark.parametrize("head_dim,heads,kv_heads", [(16, 4, 2), (80, 8, 2), (96, 8, 4), (48, 6, 2), (256, 8, 4)])
def test_fused_logits_match_materialized_other_head_dims(dev, head_dim, heads, kv_heads):
    """Head dims other than 128 (the reference's tiny models use 16; phi-2 80,
    phi-3 96, Gemma 256): prompt, INT4 middle, decode steps and a chunk through the fused kernels,
    against the model's SDPA over the same cache's materialized tiers."""
    print(f"case fused vs materialized head_dim {head_dim} heads {heads}/{kv_heads}", flush=True)
    model, cfg = _tiny_fp16(dev, "fade", heads, kv_heads, head_dim)
    kw = {"n_sink": 2, "recent_window": 8, "int4_budget": None, "int2_budget": 0}
    ids = torch.randint(0, cfg.vocab_size, (2, 40), device=dev)
    chunk = torch.randint(0, cfg.vocab_size, (2, 8), device=dev)
    cache = create_tiered_cache(model, dtype=torch.float16, **kw)
    assert cache.fused
    fused = _steps(model, cache, ids, 3, chunk)
    model.set_attn_implementation("sdpa")
    ref = _steps(model, create_tiered_cache(model, dtype=torch.float16, **kw), ids, 3, chunk)
    for a, b in zip(fused, ref):
        assert (a - b).abs().max().item() <= 2e-2
