"""Host-side append planning of PagePool (pages an append takes, longest row after it) against a
per-row restatement: row b maps blocks ceil(hw_b / P) .. min(ceil((len_b + T) / P), max_blocks)
- 1 for the first time, on random lengths, high-water marks, page sizes and token counts; and the
capacity error when a row would pass the limit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from barqtrain_amd.paged import PagedKVCapacityError, PagePool


def _reference_need(lens, hw, T, P, mb):
    need = 0
    for l, h in zip(lens.tolist(), hw.tolist()):
        first = -(-h // P)
        end = min(-(-(l + T) // P), mb)
        need += max(end - first, 0)
    return need


def test_plan_matches_per_row_restatement():
    rng = np.random.default_rng(11)
    checked = 0
    for _ in range(1500):
        P = int(rng.choice([1, 3, 16, 32]))
        mb = int(rng.integers(1, 20))
        B = int(rng.integers(1, 9))
        pool = PagePool(max_batch=B, max_blocks=mb, page_size=P, kv_heads=1, head_dim=4, dtype=torch.float32,
                        device="cpu")
        cap = mb * P
        lens = rng.integers(0, cap + 1, size=B)
        hw = np.maximum(lens, rng.integers(0, cap + 1, size=B))
        pool.lens[:] = lens
        pool.hw[:] = hw
        pool.free_count = 10**9
        T = int(rng.integers(1, 2 * P + 2))
        batch = int(rng.integers(1, B + 1))
        if lens[:batch].max() + T > cap:
            with pytest.raises(PagedKVCapacityError):
                pool.check_append(batch, T)
            continue
        need = pool.check_append(batch, T)
        assert need == _reference_need(lens[:batch], hw[:batch], T, P, mb)
        checked += 1
    assert checked > 500
