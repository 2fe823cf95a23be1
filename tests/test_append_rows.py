"""PagePool.append_rows on a host pool: freed rows re-prefilled (pages other rows released) while
the rest keep decoding, at high occupancy, against the oracle after every step; and the
argument and capacity errors, which change nothing."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvgen import hf_layout, to_bits
from oracle.kv_oracle import DenseLayerOracle


def host_pool(B, cap, P, H, D, num_pages=None):
    from barqtrain_amd.paged import PagePool

    return PagePool(max_batch=B, max_blocks=-(-cap // P), page_size=P, kv_heads=H, head_dim=D,
                    dtype=torch.float32, device="cpu", num_pages=num_pages)


@pytest.mark.parametrize("page,seed", [(4, 0), (5, 1)])
def test_refill_freed_rows_while_others_decode(page, seed):
    B, H, D, ctx, steps = 6, 2, 4, 20, 30
    cap = ctx + steps + 2
    live = B * -(-ctx // page)
    pool = host_pool(B, cap, page, H, D, num_pages=int(np.ceil(live / 0.9)) + B)
    oracle = DenseLayerOracle(B, cap, page)
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    k = hf_layout(B, H, ctx, D, torch.float32, gen)
    pool.append(k, k)
    oracle.append(to_bits(k), to_bits(k))
    for step in range(steps):
        rows = sorted(rng.choice(B, size=2, replace=False).tolist())
        pool.free_rows(rows)
        oracle.release_rows(rows)
        t = int(rng.integers(1, ctx + 1))
        kr = hf_layout(2, H, t, D, torch.float32, gen)
        vr = hf_layout(2, H, t, D, torch.float32, gen)
        pool.append_rows(rows, kr, vr)
        oracle.append_rows(rows, to_bits(kr), to_bits(vr))
        k = hf_layout(B, H, 1, D, torch.float32, gen)
        gk, gv = pool.update(k, k)
        ok, ov = oracle.update(to_bits(k), to_bits(k))
        assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov), step
        assert list(pool.lens) == pool.seq_lens.tolist()
        assert pool.free_count == int(pool.ctrl[0])
    assert int(pool.ctrl[1]) == 0


def test_append_rows_errors_change_nothing():
    from barqtrain_amd.paged import PagedKVCapacityError, PagedKVPoolExhausted

    pool = host_pool(3, 16, 4, 1, 4, num_pages=5)
    gen = torch.Generator().manual_seed(0)
    k = hf_layout(3, 1, 4, 4, torch.float32, gen)
    pool.append(k, k)  # 3 of 5 pages
    before = (pool.lens.copy(), pool.seq_lens.clone(), pool.block_table.clone(), pool.free_count)

    def same():
        assert np.array_equal(before[0], pool.lens) and torch.equal(before[1], pool.seq_lens)
        assert torch.equal(before[2], pool.block_table) and before[3] == pool.free_count

    two = hf_layout(2, 1, 4, 4, torch.float32, gen)
    with pytest.raises(ValueError):
        pool.append_rows([1, 1], two, two)
    with pytest.raises(IndexError):
        pool.append_rows([0, 3], two, two)
    with pytest.raises(ValueError):
        pool.append_rows([0], two, two)
    with pytest.raises(PagedKVCapacityError):
        pool.append_rows([0, 2], hf_layout(2, 1, 13, 4, torch.float32, gen), hf_layout(2, 1, 13, 4, torch.float32, gen))
    with pytest.raises(PagedKVPoolExhausted):
        pool.append_rows([0, 2], hf_layout(2, 1, 8, 4, torch.float32, gen), hf_layout(2, 1, 8, 4, torch.float32, gen))
    same()
