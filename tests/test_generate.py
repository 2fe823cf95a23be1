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


def _paged_key(layer, t):
    t._barq_paged_layer = layer
    return t


@pytest.mark.parametrize("opts", [{"softcap": 3.0}, {"sinks": True}, {"softcap": 2.0, "sinks": True}])
def test_fp32_attention_options_match_the_models_own_attention(opts):
    """Soft-capping and attention sinks in the paged route's fp32 attention against the eager
    attention of the models that define them (transformers' Gemma 2 and gpt-oss), in float64 with
    grouped heads, a prefill-shaped causal mask and a padded row; then through the route itself
    on a host layer (previously the route refused these options)."""
    import types

    from transformers.models.gemma2 import modeling_gemma2
    from transformers.models.gpt_oss import modeling_gpt_oss

    from barqtrain_amd import attention

    gen = torch.Generator().manual_seed(3)
    B, Hq, Hkv, T, S, D = 2, 4, 2, 5, 9, 8
    q = torch.randn(B, Hq, T, D, generator=gen, dtype=torch.float64) * 2
    k = torch.randn(B, Hkv, S, D, generator=gen, dtype=torch.float64) * 2
    v = torch.randn(B, Hkv, S, D, generator=gen, dtype=torch.float64)
    pos, qpos = torch.arange(S), S - T + torch.arange(T)
    visible = (pos[None, :] <= qpos[:, None]).expand(B, 1, T, S).clone()
    visible[1, :, :, :2] = False  # row 1 left-padded by two
    add_mask = torch.zeros(B, 1, T, S, dtype=torch.float64).masked_fill(~visible, torch.finfo(torch.float64).min)
    sinks = torch.randn(Hq, generator=gen, dtype=torch.float64) if opts.get("sinks") else None
    module = types.SimpleNamespace(num_key_value_groups=Hq // Hkv, training=False, head_dim=D, sinks=sinks)
    scale = D ** -0.5
    softcap = opts.get("softcap")
    if sinks is None:
        ref, _ = modeling_gemma2.eager_attention_forward(module, q, k, v, add_mask, scaling=scale, softcap=softcap)
    elif softcap is None:
        ref, _ = modeling_gpt_oss.eager_attention_forward(module, q, k, v, add_mask, scaling=scale)
    else:  # both: gpt-oss's sink softmax over Gemma 2's capped scores
        kk, vv = k.repeat_interleave(2, 1), v.repeat_interleave(2, 1)
        capped = torch.tanh(torch.matmul(q, kk.transpose(2, 3)) * scale / softcap) * softcap
        logits = torch.cat([capped + add_mask, sinks.reshape(1, -1, 1, 1).expand(B, -1, T, 1)], dim=-1)
        ref = torch.matmul(torch.softmax(logits, dim=-1)[..., :-1], vv).transpose(1, 2)
    got = attention._fp32_attention(q, k, v, visible, scale, softcap=softcap, sinks=sinks)
    torch.testing.assert_close(got, ref.to(got.dtype), rtol=1e-6, atol=1e-6)
    layer = types.SimpleNamespace(pool=types.SimpleNamespace(kv_heads=Hkv, on_gpu=False),
                                  current_tensors=lambda: (k, v))
    kw = {"softcap": softcap} if softcap is not None else {}
    if sinks is not None:
        kw["s_aux"] = sinks
    out, _ = attention.paged_attention_forward(module, q, _paged_key(layer, k.clone()), v, visible,
                                               scaling=scale, **kw)
    torch.testing.assert_close(out, got)


def test_fp32_attention_sliding_window_without_a_mask():
    """A sliding window with no mask from transformers (the route applies it): query position p
    sees keys k with p - W < k <= p, transformers' overlay; against the mask built from it."""
    from transformers.masking_utils import and_masks, causal_mask_function, sliding_window_overlay

    from barqtrain_amd import attention

    gen = torch.Generator().manual_seed(4)
    B, H, T, S, D, W = 1, 2, 3, 11, 8, 4
    q = torch.randn(B, H, T, D, generator=gen, dtype=torch.float64)
    k = torch.randn(B, H, S, D, generator=gen, dtype=torch.float64)
    v = torch.randn(B, H, S, D, generator=gen, dtype=torch.float64)
    fn = and_masks(causal_mask_function, sliding_window_overlay(W))
    t = torch.tensor
    mask = torch.tensor([[bool(fn(t(0), t(0), t(S - T + i), t(j))) for j in range(S)] for i in range(T)])
    mask = mask.reshape(1, 1, T, S)
    assert int(mask.sum()) == T * W
    ref = attention._fp32_attention(q, k, v, mask, 0.3)
    got = attention._fp32_attention(q, k, v, None, 0.3, sliding_window=W)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)


def tiny_gemma2(seed=0, dtype=torch.float32):
    from transformers import Gemma2Config, Gemma2ForCausalLM

    torch.manual_seed(seed)
    # Gemma 2's attention options: logit soft-capping on every layer and a sliding window on every
    # other layer (here 8 positions, so the decode steps run past it)
    cfg = Gemma2Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=32, max_position_embeddings=256,
                       sliding_window=8, attn_logit_softcapping=20.0, final_logit_softcapping=30.0,
                       query_pre_attn_scalar=32, pad_token_id=0, eos_token_id=None, bos_token_id=1)
    return Gemma2ForCausalLM(cfg).to(dtype).eval(), cfg


def test_generate_gemma2_softcap_and_sliding_window_on_paged_route():
    """A tiny Gemma 2 (soft-capped logits, sliding-window layers) on the "barq_paged" route over a
    host pool decodes the tokens transformers' eager attention with DynamicCache decodes, logits
    within fp32 rounding."""
    from transformers.cache_utils import DynamicCache

    from barqtrain_amd import attention

    model, cfg = tiny_gemma2()
    model.config._attn_implementation = "eager"
    ids = torch.randint(2, 512, (2, 11), generator=torch.Generator().manual_seed(2))
    new = 12
    ref_seq, ref_logits = decode(model, ids, DynamicCache(config=cfg), new)
    attention.enable_paged_attention(model)
    cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=11 + new, page_size=4)
    seq, logits = decode(model, ids, cache, new)
    assert torch.equal(seq, ref_seq)
    torch.testing.assert_close(logits, ref_logits, rtol=1e-4, atol=1e-4)
