"""Hugging Face `generate` on the paged cache, CPU: a locally constructed random-weight Llama
(no network) decodes the same tokens with bit-identical logits as with transformers'
DynamicCache (the reference's generate integration, kv_cache.py:226-303,
patch_models.py:235-261)."""

import pytest
import torch

transformers = pytest.importorskip("transformers")

from barqtrain import create_paged_kv_cache  # noqa: E402


def tiny_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
                      pad_token_id=0, eos_token_id=None)
    return LlamaForCausalLM(cfg).eval(), cfg


def decode(model, ids, cache, new_tokens):
    out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new_tokens,
                         do_sample=False, past_key_values=cache, return_dict_in_generate=True,
                         output_logits=True)
    return out.sequences, torch.stack(out.logits)


@pytest.mark.parametrize("page", [4, 16])
def test_generate_matches_dynamic_cache(page):
    from transformers.cache_utils import DynamicCache

    model, cfg = tiny_llama()
    ids = torch.randint(1, 512, (2, 13), generator=torch.Generator().manual_seed(1))
    new = 18
    ref_seq, ref_logits = decode(model, ids, DynamicCache(config=cfg), new)
    cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=13 + new, page_size=page)
    seq, logits = decode(model, ids, cache, new)
    assert torch.equal(seq, ref_seq)
    assert torch.equal(logits.view(torch.int32), ref_logits.view(torch.int32))
    assert cache.get_seq_length() == 13 + new - 1


def test_generate_with_paged_attention_on_host_pool():
    """The "barq_paged" attention implementation over a fused-attention cache in host memory
    (gathered K/V, fp32 attention): same tokens as DynamicCache with eager attention, logits
    within fp32 rounding; with padding (left-padded batch) the mask is honoured."""
    from transformers.cache_utils import DynamicCache

    from barqtrain_amd import attention

    model, cfg = tiny_llama()
    model.config._attn_implementation = "eager"
    ids = torch.randint(1, 512, (2, 13), generator=torch.Generator().manual_seed(1))
    new = 18
    ref_seq, ref_logits = decode(model, ids, DynamicCache(config=cfg), new)
    attention.enable_paged_attention(model)
    cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=13 + new, page_size=4)
    assert all(layer.fused_attention for layer in cache.layers)
    seq, logits = decode(model, ids, cache, new)
    assert torch.equal(seq, ref_seq)
    torch.testing.assert_close(logits, ref_logits, rtol=1e-5, atol=1e-5)

    # left padding: row 1 has 4 pad tokens; compare with the eager model on the same mask
    mask = torch.ones_like(ids)
    mask[1, :4] = 0
    model.config._attn_implementation = "eager"
    ref = model.generate(ids, attention_mask=mask, max_new_tokens=6, do_sample=False,
                         past_key_values=DynamicCache(config=cfg), return_dict_in_generate=True,
                         output_logits=True)
    attention.enable_paged_attention(model)
    cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=13 + 6, page_size=4)
    got = model.generate(ids, attention_mask=mask, max_new_tokens=6, do_sample=False,
                         past_key_values=cache, return_dict_in_generate=True, output_logits=True)
    assert torch.equal(got.sequences, ref.sequences)
    torch.testing.assert_close(torch.stack(got.logits), torch.stack(ref.logits), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("page", [4, 16])
def test_beam_search_matches_dynamic_cache(page):
    """num_beams=4: generate reorders the cache after every step (Cache.reorder_cache); the
    paged cache selects rows in place, sharing full pages between beams, and returns the same
    beams with the same scores as DynamicCache."""
    from transformers.cache_utils import DynamicCache

    model, cfg = tiny_llama()
    model.config._attn_implementation = "eager"
    ids = torch.randint(1, 512, (2, 13), generator=torch.Generator().manual_seed(4))
    new = 20
    kw = dict(attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False, num_beams=4,
              num_return_sequences=2, return_dict_in_generate=True, output_scores=True)
    ref = model.generate(ids, past_key_values=DynamicCache(config=cfg), **kw)
    cache = create_paged_kv_cache(model, max_batch_size=8, max_cache_len=13 + new, page_size=page)
    got = model.generate(ids, past_key_values=cache, **kw)
    assert torch.equal(got.sequences, ref.sequences)
    assert torch.equal(got.sequences_scores, ref.sequences_scores)
    assert all(layer.pool.shared for layer in cache.layers), "beams never shared pages"


def test_generate_on_fp8_quantised_pages_tracks_full_precision():
    """kv_quant="fp8_e4m3" with an 8-token residual window: most of each row's history is read
    back from fp8 codes; greedy tokens agree with DynamicCache on at least 90 % of steps (here:
    all) and the logits stay within 5 % relative (L2) -- quantisation is lossy by design."""
    from transformers.cache_utils import DynamicCache

    model, cfg = tiny_llama()
    model.config._attn_implementation = "eager"
    ids = torch.randint(1, 512, (2, 40), generator=torch.Generator().manual_seed(1))
    new = 30
    ref_seq, ref_logits = decode(model, ids, DynamicCache(config=cfg), new)
    cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=40 + new, page_size=4,
                                  kv_quant="fp8_e4m3", residual_window=8)
    seq, logits = decode(model, ids, cache, new)
    assert all(int(layer.pool.cold_blocks.min()) >= 14 for layer in cache.layers)
    assert (seq[:, 40:] == ref_seq[:, 40:]).float().mean() >= 0.9
    assert ((logits - ref_logits).norm() / ref_logits.norm()) < 0.05


def test_paged_route_rejects_options_it_does_not_implement():
    """Logit soft-capping, attention sinks, sliding windows and dropout raise on the paged route
    instead of being dropped (a model with them would otherwise change its logits silently)."""
    import types

    from barqtrain_amd import attention

    layer = types.SimpleNamespace(pool=None)
    q = torch.zeros(1, 4, 1, 8)
    k = torch.zeros(1, 2, 3, 8)
    k._barq_paged_layer = layer
    for kw in ({"softcap": 30.0}, {"s_aux": torch.zeros(4)}, {"sliding_window": 4096}, {"dropout": 0.1}):
        with pytest.raises(NotImplementedError):
            attention.paged_attention_forward(None, q, k, k, None, **kw)
