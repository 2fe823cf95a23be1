"""Quantised (fp8) KV pages through the layer API on host-memory tensors, against the oracle
QuantLayerOracle bit for bit: random programs of ragged and long (chunked) appends, crops within
the residual window, row releases and resets; page accounting of the hot pool and the cold store;
the flag plumbing of create_paged_kv_cache.  CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvgen import hf_layout, to_bits
from oracle.kv_quant_oracle import QuantLayerOracle

DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def check_accounting(pool):
    """Host shadow = device state: stack tops, frontiers, and every page held exactly once."""
    P = pool.page_size
    bt = pool.block_table.numpy()
    assert int(pool.ctrl[0]) == pool.free_count and int(pool.ctrl[2]) == pool.cold_free
    hot, cold = [], []
    for r in range(pool.max_batch):
        n = -(-int(pool.high_water[r]) // P)
        row = bt[r, :n]
        c = int(pool.cold_blocks[r])
        assert (row[:c] <= -2).all() and (row[c:] >= 0).all(), (r, row, c)
        cold += (-2 - row[:c]).tolist()
        hot += row[c:].tolist()
    assert len(set(hot)) == len(hot) and len(set(cold)) == len(cold)
    assert not set(hot) & set(pool.free_pages[: pool.free_count].tolist())
    assert not set(cold) & set(pool.free_cold[: pool.cold_free].tolist())
    assert len(hot) + pool.free_count == pool.num_pages and len(cold) + pool.cold_free == pool.num_cold


@pytest.mark.parametrize("dtype,page,window,seed", [(torch.bfloat16, 4, 8, 0), (torch.float16, 16, 16, 1),
                                                    (torch.float32, 5, 0, 2), (torch.bfloat16, 8, 24, 3)])
def test_random_programs_match_the_oracle(dtype, page, window, seed):
    from barqtrain_amd.kv_cache import BarqPagedKVCacheLayer

    H, D, Bmax, cap = 2, 16, 4, 96
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    layer = BarqPagedKVCacheLayer(max_batch_size=Bmax, max_cache_len=cap, page_size=page, kv_quant="fp8_e4m3",
                                  residual_window=window)
    oracle = QuantLayerOracle(Bmax, cap, page, window, DT[dtype])
    quantised = 0
    for it in range(50):
        r = rng.random()
        if r < 0.6 or not oracle.is_initialized:
            b = int(rng.integers(1, Bmax + 1))
            t = int(rng.integers(1, 40)) if rng.random() < 0.3 else 1
            if oracle.is_initialized and int(oracle.seq_lens[:b].max()) + t > cap:
                continue
            k = hf_layout(b, H, t, D, dtype, gen) * 3
            v = hf_layout(b, H, t, D, dtype, gen)
            gk, gv = layer.update(k, v)
            ok, ov = oracle.update(to_bits(k), to_bits(v))
            assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov), it
        elif r < 0.75:
            cur = oracle.current_batch_size
            lo = int(max((oracle.cold[:cur].max() if cur else 0) * page, 0))
            m = int(rng.integers(lo, cap))
            layer.crop(m)
            oracle.crop(m)
        elif r < 0.9 and oracle.current_batch_size:
            rows = sorted(rng.choice(Bmax, size=int(rng.integers(1, 3)), replace=False).tolist())
            layer.free_rows(rows)
            oracle.release_rows(rows)
        else:
            layer.reset()
            oracle.reset()
        if layer.is_initialized:
            check_accounting(layer.pool)
            quantised += int(layer.pool.cold_blocks.sum())
        if layer.current_batch_size:
            gk, gv = layer.current_tensors()
            ok, ov = oracle.current_tensors()
            assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov), it
    assert quantised > 0


def test_stored_codes_and_scales_are_the_oracles():
    from barqtrain_amd.paged import QuantPagePool

    P, H, D, W = 4, 2, 8, 4
    pool = QuantPagePool(max_batch=2, max_blocks=8, page_size=P, kv_heads=H, head_dim=D, dtype=torch.bfloat16,
                         device="cpu", window=W)
    oracle = QuantLayerOracle(2, 32, P, W, "bf16")
    gen = torch.Generator().manual_seed(4)
    k, v = hf_layout(2, H, 19, D, torch.bfloat16, gen), hf_layout(2, H, 19, D, torch.bfloat16, gen)
    k[0, 1, 3, 5] = float("nan")
    v[1, 0, 2, :] = 0.0
    v[1, 0, 6, 2] = float("inf")
    pool.append(k, v)
    oracle.append(to_bits(k), to_bits(v))
    assert pool.cold_blocks.tolist() == [3, 3]
    for r in range(2):
        for j in range(3):
            c = -2 - int(pool.block_table[r, j])
            for key, codes, scales in ((True, pool.key_codes, pool.key_scales), (False, pool.value_codes, pool.value_scales)):
                want_codes, want_scales = oracle.quantized_page(r, j, key)
                assert np.array_equal(codes[c].numpy(), want_codes), (r, j, key)
                assert np.array_equal(scales[c].numpy(), want_scales), (r, j, key)
    gk, gv = pool.gather(2)   # NaN and infinities read back as the oracle's signed quiet NaN
    ok, ov = oracle.current_tensors()
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)


def test_long_prefill_runs_in_chunks_within_a_small_hot_pool():
    from barqtrain_amd.paged import QuantPagePool

    pool = QuantPagePool(max_batch=2, max_blocks=64, page_size=16, kv_heads=1, head_dim=8, dtype=torch.float16,
                         device="cpu", window=32, chunk=64)
    assert pool.num_pages == 2 * (6 + 2)  # ceil((32 + 64) / 16) + 2 pages per row
    gen = torch.Generator().manual_seed(5)
    k, v = hf_layout(2, 1, 1000, 8, torch.float16, gen), hf_layout(2, 1, 1000, 8, torch.float16, gen)
    gk, _ = pool.update(k, v)
    assert gk.shape == (2, 1, 1000, 8)
    assert pool.cold_blocks.tolist() == [(1000 - 32) // 16] * 2
    mem = pool.memory_bytes()
    assert mem["hot_pages"] < mem["cold_store"]


def test_crop_into_quantised_blocks_is_refused_and_changes_nothing():
    from barqtrain_amd.paged import QuantPagePool

    pool = QuantPagePool(max_batch=1, max_blocks=8, page_size=4, kv_heads=1, head_dim=4, dtype=torch.float32,
                         device="cpu", window=4)
    gen = torch.Generator().manual_seed(6)
    pool.append(hf_layout(1, 1, 14, 4, torch.float32, gen), hf_layout(1, 1, 14, 4, torch.float32, gen))
    assert pool.cold_blocks.tolist() == [2]
    with pytest.raises(ValueError):
        pool.crop(1, 7)
    assert pool.lens.tolist() == [14] and int(pool.seq_lens[0]) == 14
    pool.crop(1, 8)
    assert pool.lens.tolist() == [8]
    with pytest.raises(NotImplementedError):
        pool.select_rows([0])


def test_factory_flag_and_environment(monkeypatch):
    from barqtrain.kv_cache import create_paged_kv_cache

    class Text:
        num_hidden_layers = 2

    class Config:
        def get_text_config(self, decoder=True):
            return Text()

    cache = create_paged_kv_cache(Config(), max_batch_size=1, max_cache_len=64, kv_quant="fp8", residual_window=16)
    assert all(l.kv_quant == "fp8_e4m3" and l.residual_window == 16 for l in cache.layers)
    monkeypatch.setenv("BARQTRAIN_KV_QUANT", "fp8_e4m3")
    monkeypatch.setenv("BARQTRAIN_KV_QUANT_WINDOW", "32")
    cache = create_paged_kv_cache(Config(), max_batch_size=1, max_cache_len=64)
    assert all(l.kv_quant == "fp8_e4m3" and l.residual_window == 32 for l in cache.layers)
    cache.update(torch.randn(1, 2, 40, 8), torch.randn(1, 2, 40, 8), 0)
    assert type(cache.layers[0].pool).__name__ == "QuantPagePool"
    monkeypatch.delenv("BARQTRAIN_KV_QUANT")
    assert create_paged_kv_cache(Config(), max_batch_size=1, max_cache_len=64).layers[0].kv_quant is None
    with pytest.raises(ValueError):
        create_paged_kv_cache(Config(), max_batch_size=1, max_cache_len=64, kv_quant="int4")
