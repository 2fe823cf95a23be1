"""The reference's KV-cache tests (BarqTrain tests/test_kv_cache.py:24-130), run against this
package through the reference import path ``barqtrain``.  CPU tensors, no GPU needed."""

import types

import torch

from barqtrain.kv_cache import (
    BarqPagedKVCache,
    BarqPagedKVCacheLayer,
    create_paged_kv_cache,
    maybe_prepare_paged_kv_generate_kwargs,
)


class ThreeLayerText:
    num_hidden_layers = 3


class WrapperConfig:
    def get_text_config(self, decoder=True):
        return ThreeLayerText()


def test_layer_update_returns_concatenated_history():
    # tests/test_kv_cache.py:24-47: 3 then 2 tokens, page size 4 (second append crosses slot 4)
    layer = BarqPagedKVCacheLayer(max_batch_size=1, max_cache_len=8, page_size=4)
    first_k = torch.arange(24, dtype=torch.float32).view(1, 2, 3, 4)
    first_v = first_k + 100.0
    keys, values = layer.update(first_k, first_v)
    assert keys.shape == values.shape == (1, 2, 3, 4)
    assert torch.equal(keys, first_k) and torch.equal(values, first_v)
    assert layer.get_seq_length() == 3

    second_k = torch.arange(16, dtype=torch.float32).view(1, 2, 2, 4) + 1000.0
    second_v = second_k + 100.0
    keys, values = layer.update(second_k, second_v)
    assert keys.shape == values.shape == (1, 2, 5, 4)
    assert torch.equal(keys, torch.cat([first_k, second_k], dim=2))
    assert torch.equal(values, torch.cat([first_v, second_v], dim=2))
    assert layer.get_seq_length() == 5


def test_cache_has_one_layer_per_decoder_layer():
    # tests/test_kv_cache.py:50-62
    cache = create_paged_kv_cache(WrapperConfig(), max_batch_size=2, max_cache_len=64, page_size=16)
    assert isinstance(cache, BarqPagedKVCache)
    assert len(cache.layers) == 3
    assert (cache.barqtrain_max_batch_size, cache.barqtrain_max_cache_len, cache.page_size) == (2, 64, 16)


def _model(max_length=32):
    return types.SimpleNamespace(
        config=WrapperConfig(),
        generation_config=types.SimpleNamespace(max_new_tokens=None, max_length=max_length),
        _barqtrain_paged_kv_supported=True,
    )


def test_generate_kwargs_receive_a_cache(monkeypatch):
    # tests/test_kv_cache.py:65-86: budget = prompt 8 + 4 new tokens
    monkeypatch.setattr("barqtrain.kv_cache._get_cuda_backend", lambda: object())
    monkeypatch.setenv("BARQTRAIN_PAGED_KV_MIN_CACHE_LEN", "0")
    prompt = types.SimpleNamespace(shape=(2, 8), device=torch.device("cuda"))
    kwargs, used = maybe_prepare_paged_kv_generate_kwargs(_model(), (), {"input_ids": prompt, "max_new_tokens": 4})
    assert used is True and kwargs["use_cache"] is True
    cache = kwargs["past_key_values"]
    assert isinstance(cache, BarqPagedKVCache)
    assert (cache.barqtrain_max_batch_size, cache.barqtrain_max_cache_len) == (2, 12)


def test_generate_kwargs_skip_short_budgets(monkeypatch):
    # tests/test_kv_cache.py:89-107: 32 + 16 < 256 -> no cache
    monkeypatch.setattr("barqtrain.kv_cache._get_cuda_backend", lambda: object())
    monkeypatch.setenv("BARQTRAIN_PAGED_KV_MIN_CACHE_LEN", "256")
    prompt = types.SimpleNamespace(shape=(1, 32), device=torch.device("cuda"))
    kwargs, used = maybe_prepare_paged_kv_generate_kwargs(_model(), (), {"input_ids": prompt, "max_new_tokens": 16})
    assert used is False and "past_key_values" not in kwargs


def test_generate_wrapper_records_usage(monkeypatch):
    # tests/test_kv_cache.py:110-130
    import barqtrain.patch_models as patch_models

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = WrapperConfig()

        def generate(self, *args, **kwargs):
            return kwargs

    monkeypatch.setattr("barqtrain.kv_cache.maybe_prepare_paged_kv_generate_kwargs",
                        lambda model, args, kwargs: ({**kwargs, "sentinel": True}, True))
    monkeypatch.setattr("barqtrain.kv_cache.paged_kv_supported_for_model", lambda model: True)
    model = patch_models._patch_generate_with_paged_kv(Model(), "Dummy")
    result = model.generate(input_ids="tokens")
    assert result["sentinel"] is True
    assert model._barqtrain_last_generate_used_paged_kv is True
    assert model._barqtrain_paged_kv_supported is True


def test_generate_kwargs_gates(monkeypatch):
    """The remaining gates of kv_cache.py:243-303: explicit cache, env switch, unsupported model,
    missing backend, CPU prompt, embeds / mask as the shape source, max_length budget."""
    monkeypatch.setattr("barqtrain.kv_cache._get_cuda_backend", lambda: object())
    monkeypatch.setenv("BARQTRAIN_PAGED_KV_MIN_CACHE_LEN", "0")
    gpu = torch.device("cuda")
    prompt = types.SimpleNamespace(shape=(3, 5), device=gpu)
    assert maybe_prepare_paged_kv_generate_kwargs(_model(), (), {"input_ids": prompt, "past_key_values": 1})[1] is False
    monkeypatch.setenv("BARQTRAIN_ENABLE_PAGED_KV", "off")
    assert maybe_prepare_paged_kv_generate_kwargs(_model(), (), {"input_ids": prompt})[1] is False
    monkeypatch.delenv("BARQTRAIN_ENABLE_PAGED_KV")
    unsupported = _model()
    unsupported._barqtrain_paged_kv_supported = False
    assert maybe_prepare_paged_kv_generate_kwargs(unsupported, (), {"input_ids": prompt})[1] is False
    cpu_prompt = types.SimpleNamespace(shape=(3, 5), device=torch.device("cpu"))
    assert maybe_prepare_paged_kv_generate_kwargs(_model(), (), {"input_ids": cpu_prompt})[1] is False
    # positional prompt, generation_config max_length 32 -> budget max(32, 5)
    kw, used = maybe_prepare_paged_kv_generate_kwargs(_model(), (prompt,), {})
    assert used and kw["past_key_values"].barqtrain_max_cache_len == 32
    kw, used = maybe_prepare_paged_kv_generate_kwargs(_model(), (), {"inputs_embeds": prompt, "max_length": 40})
    assert used and kw["past_key_values"].barqtrain_max_cache_len == 40
    kw, used = maybe_prepare_paged_kv_generate_kwargs(_model(None), (), {"attention_mask": prompt})
    assert used is False  # no budget at all
    monkeypatch.setenv("BARQTRAIN_PAGED_KV_PAGE_SIZE", "32")
    kw, used = maybe_prepare_paged_kv_generate_kwargs(_model(), (), {"attention_mask": prompt, "max_new_tokens": 3})
    assert used and kw["past_key_values"].page_size == 32 and kw["past_key_values"].barqtrain_max_cache_len == 8
    monkeypatch.setattr("barqtrain.kv_cache._get_cuda_backend", lambda: None)
    assert maybe_prepare_paged_kv_generate_kwargs(_model(), (), {"input_ids": prompt})[1] is False


def test_decode_step_strides_of_hf_accepted_without_copy():
    """HF decode hands over K (after RoPE) and V (a transposed view) that differ only in the
    stride of the size-1 sequence dimension; the pool takes them as they are."""
    from barqtrain_amd.paged import PagePool

    base_k = torch.randn(3, 2, 1, 128)                    # K: [B, H, 1, D] contiguous
    base_v = torch.randn(3, 1, 2, 128).transpose(1, 2)    # V: [B, 1, H, D] viewed as [B, H, 1, D]
    assert base_k.stride() != base_v.stride()
    k, v = PagePool._compatible_pair(base_k, base_v)
    assert k.data_ptr() == base_k.data_ptr() and v.data_ptr() == base_v.data_ptr()
    prefill_k = torch.randn(3, 21, 2, 128).transpose(1, 2)
    prefill_v = torch.randn(3, 2, 21, 128)                 # genuinely different layouts: copied
    k, v = PagePool._compatible_pair(prefill_k, prefill_v)
    assert k.stride() == v.stride() and k.is_contiguous()
