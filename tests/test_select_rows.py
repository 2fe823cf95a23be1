"""Copy-on-write row selection (beam ops) on a host-memory pool: random programs of ragged
appends, selections (repeats, permutations, shrinking), crops, row releases and resets through
the reference layer API (kv_cache.py:166-186), compared element for element with the oracle
after every operation, with the pool's sharing invariants checked each time."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from capi_pool import check_pool_invariants
from kvgen import hf_layout, to_bits
from oracle.kv_oracle import DenseLayerOracle


def invariants(pool):
    check_pool_invariants(pool.block_table.numpy(), pool.seq_lens.numpy(), pool.high_water.numpy(),
                          pool.free_pages.numpy(), pool.ctrl.numpy(), pool.page_shares.numpy(),
                          pool.page_size)
    top = int(pool.ctrl[0])
    assert pool.free_count <= top and (not pool.free_exact or pool.free_count == top)
    assert list(pool.lens) == pool.seq_lens.tolist() and list(pool.hw) == pool.high_water.tolist()


@pytest.mark.parametrize("page,seed", [(4, 0), (16, 1), (5, 2)])
def test_random_program_with_shared_pages(page, seed):
    from barqtrain_amd.kv_cache import BarqPagedKVCacheLayer

    H, D, Bmax, cap = 2, 8, 6, 60
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    layer = BarqPagedKVCacheLayer(max_batch_size=Bmax, max_cache_len=cap, page_size=page)
    oracle = DenseLayerOracle(Bmax, cap, page)
    shared_seen = 0
    for it in range(120):
        r = rng.random()
        if r < 0.45 or not oracle.is_initialized:
            b = int(rng.integers(1, layer.max_batch_size + 1))
            t = int(rng.integers(1, 9)) if rng.random() < 0.4 else 1
            if oracle.is_initialized and int(oracle.seq_lens[:b].max()) + t > cap:
                continue
            k = hf_layout(b, H, t, D, torch.float32, gen)
            v = hf_layout(b, H, t, D, torch.float32, gen)
            gk, gv = layer.update(k, v)
            ok, ov = oracle.update(to_bits(k), to_bits(v))
            assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov), it
        elif r < 0.70 and layer.current_batch_size:
            n = int(rng.integers(1, Bmax + 1))
            rows = rng.integers(0, layer.current_batch_size, size=n).tolist()
            layer.batch_select_indices(torch.tensor(rows))
            oracle.batch_select_indices(rows)
            shared_seen += int(layer.pool.page_shares.sum())
        elif r < 0.80:
            m = int(rng.integers(-6, cap))
            layer.crop(m)
            oracle.crop(m)
        elif r < 0.90 and layer.current_batch_size:
            rows = sorted(rng.choice(layer.max_batch_size, size=int(rng.integers(1, 3)), replace=False).tolist())
            layer.free_rows(rows)
            oracle.release_rows(rows)
        elif r < 0.93:
            layer.reset()
            oracle.reset()
        if layer.is_initialized:
            invariants(layer.pool)
        if layer.current_batch_size:
            gk, gv = layer.current_tensors()
            ok, ov = oracle.current_tensors()
            assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov), it
    assert shared_seen > 0, "the program never shared a page"


def test_selection_shares_history_instead_of_copying():
    """Eight beams of one 96-token prompt (page 16): the 6 full pages are held once, each beam
    owns only its partial last page; after more decode steps and re-selections the page count
    stays that of the distinct histories."""
    from barqtrain_amd.paged import PagePool

    H, D, P = 2, 8, 16
    pool = PagePool(max_batch=8, max_blocks=16, page_size=P, kv_heads=H, head_dim=D,
                    dtype=torch.float32, device="cpu")
    gen = torch.Generator().manual_seed(3)
    pool.append(torch.randn(1, H, 100, D, generator=gen), torch.randn(1, H, 100, D, generator=gen))
    pool.select_rows([0] * 8)
    used = pool.num_pages - int(pool.ctrl[0])
    assert used == 6 + 8, used           # 6 shared full pages + 8 private copies of page 6
    assert int(pool.page_shares.max()) == 7
    for step in range(12):
        pool.append(torch.randn(8, H, 1, D, generator=gen), torch.randn(8, H, 1, D, generator=gen))
        pool.select_rows(sorted(np.random.default_rng(step).integers(0, 8, size=8).tolist()))
    invariants(pool)
    assert pool.num_pages - int(pool.ctrl[0]) < 8 * 7, "histories were copied, not shared"
