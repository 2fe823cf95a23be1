"""Host pools: an operation that raises changes nothing.

* a quantised pool's prefill longer than its chunk checks every chunk's capacity, hot pages and
  cold pages before the first chunk runs;
* a crop of a pool whose rows share pages checks room for the copies it makes before lowering
  any length;
* a selection rewrites the host length shadow in place, so views of it (a captured decode step
  keeps one per pool) see the new lengths.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvgen import hf_layout, to_bits
from oracle.kv_oracle import DenseLayerOracle


def quant_pool(**kw):
    from barqtrain_amd.paged import QuantPagePool

    args = dict(max_batch=1, max_blocks=16, page_size=16, kv_heads=2, head_dim=8, dtype=torch.float32,
                device="cpu", window=16, chunk=64)
    args.update(kw)
    return QuantPagePool(**args)


def state(pool):
    return (pool.lens.copy(), pool.hw.copy(), pool.cold_blocks.copy(), pool.free_count, pool.cold_free,
            pool.seq_lens.clone(), pool.high_water.clone(), pool.block_table.clone(), pool.ctrl[:3].clone())


def assert_same_state(a, b):
    for x, y in zip(a, b):
        if isinstance(x, torch.Tensor):
            assert torch.equal(x, y)
        elif isinstance(x, np.ndarray):
            assert np.array_equal(x, y)
        else:
            assert x == y


def test_chunked_prefill_past_max_length_changes_nothing():
    from barqtrain_amd.paged import PagedKVCapacityError

    pool = quant_pool()
    gen = torch.Generator().manual_seed(0)
    k = hf_layout(1, 2, 100, 8, torch.float32, gen)
    before = state(pool)
    with pytest.raises(PagedKVCapacityError):
        pool.append(k, k, max_length=96)
    assert_same_state(before, state(pool))
    pool.append(k[:, :, :96], k[:, :, :96], max_length=96)  # the same prefill within the limit
    assert int(pool.lens[0]) == 96


def test_chunked_prefill_that_drains_the_hot_pool_changes_nothing():
    from barqtrain_amd.paged import PagedKVPoolExhausted

    # 4 hot pages: the first 64-token chunk takes 4 and returns 3 to quantisation, the second
    # needs 4 with 3 free -- refused before the first chunk runs.
    pool = quant_pool(num_pages=4)
    gen = torch.Generator().manual_seed(1)
    k = hf_layout(1, 2, 128, 8, torch.float32, gen)
    before = state(pool)
    with pytest.raises(PagedKVPoolExhausted):
        pool.append(k, k)
    assert_same_state(before, state(pool))
    with pytest.raises(PagedKVPoolExhausted):
        pool.update(k, k)
    assert_same_state(before, state(pool))
    pool.append(k[:, :, :64], k[:, :, :64])  # one chunk fits
    assert int(pool.lens[0]) == 64 and int(pool.cold_blocks[0]) == 3


def test_chunked_prefill_that_drains_the_cold_store_changes_nothing():
    from barqtrain_amd.paged import PagedKVPoolExhausted

    pool = quant_pool(num_cold=4)  # 128 tokens quantise 7 blocks
    gen = torch.Generator().manual_seed(2)
    k = hf_layout(1, 2, 128, 8, torch.float32, gen)
    before = state(pool)
    with pytest.raises(PagedKVPoolExhausted):
        pool.append(k, k)
    assert_same_state(before, state(pool))


def test_crop_on_shared_pages_without_room_changes_nothing():
    from barqtrain_amd.kv_cache import BarqPagedKVCacheLayer
    from barqtrain_amd.paged import PagedKVPoolExhausted

    H, D, P = 1, 4, 4
    layer = BarqPagedKVCacheLayer(max_batch_size=2, max_cache_len=16, page_size=P)
    oracle = DenseLayerOracle(2, 16, P)
    gen = torch.Generator().manual_seed(3)
    k = hf_layout(1, H, 6, D, torch.float32, gen)
    layer.update(k, k)
    oracle.update(to_bits(k), to_bits(k))
    # a 4-page pool: two rows sharing block 0, each with its own partial block 1
    layer.pool = _shrunk(layer.pool, 4)
    layer.batch_select_indices(torch.tensor([0, 0]))
    oracle.batch_select_indices([0, 0])
    k = hf_layout(2, H, 1, D, torch.float32, gen)
    layer.update(k, k)
    oracle.update(to_bits(k), to_bits(k))
    pool = layer.pool
    before = (pool.lens.copy(), pool.hw.copy(), pool.seq_lens.clone(), pool.block_table.clone())
    with pytest.raises(PagedKVPoolExhausted):
        layer.crop(6)
    assert np.array_equal(before[0], pool.lens) and np.array_equal(before[1], pool.hw)
    assert torch.equal(before[2], pool.seq_lens) and torch.equal(before[3], pool.block_table)
    # the rows stay consistent: a further append to both matches the oracle
    k = hf_layout(2, H, 1, D, torch.float32, gen)
    gk, gv = layer.update(k, k)
    ok, ov = oracle.update(to_bits(k), to_bits(k))
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)


def _shrunk(pool, num_pages):
    """The same rows in a pool of `num_pages` pages (rows copied in order)."""
    return pool.copy_rows(list(range(pool.max_batch)), num_pages=num_pages)


def test_selection_updates_shadow_views_in_place():
    from barqtrain_amd.paged import PagePool

    pool = PagePool(max_batch=3, max_blocks=4, page_size=4, kv_heads=1, head_dim=4, dtype=torch.float32,
                    device="cpu")
    gen = torch.Generator().manual_seed(4)
    k = hf_layout(3, 1, 5, 4, torch.float32, gen)
    pool.append(k, k)
    k = hf_layout(1, 1, 3, 4, torch.float32, gen)
    pool.append(k, k)  # lengths 8, 5, 5
    stacked_lens, stacked_hw = pool.lens[None].copy(), pool.hw[None].copy()
    pool.lens, pool.hw = stacked_lens[0], stacked_hw[0]  # as CapturedDecodeStep holds them
    pool.select_rows([2, 0])
    assert pool.lens.base is stacked_lens and pool.hw.base is stacked_hw
    assert stacked_lens[0].tolist() == [5, 8, 0] and stacked_hw[0].tolist() == [5, 8, 0]
    assert pool.seq_lens.tolist() == [5, 8, 0]
