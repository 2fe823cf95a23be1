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
