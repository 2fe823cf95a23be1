"""PagePool.append_rows: freed rows re-prefilled (pages other rows released) while the rest keep
decoding, at high occupancy, against the oracle after every step -- on a host pool and (gpu) on a
device pool, where each row's append is its own launch over the one-row metadata view sharing the
device free stack; and the argument and capacity errors, which change nothing."""

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


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,page,seed", [(torch.bfloat16, 16, 3), (torch.float16, 5, 4)])
def test_refill_freed_rows_on_gpu_pool(dtype, page, seed):
    """The GPU path of append_rows: per step two rows freed, re-prefilled with a ragged number of
    tokens, then a decode update of every row; the gathered K/V bit-exact against the oracle each
    step, and the host shadow's free count equal to the device stack top."""
    from barqtrain_amd.paged import CTRL_ERRORS, CTRL_FREE_TOP, PagePool

    assert torch.cuda.is_available(), "GPU test collected without a visible GPU"
    B, H, D, ctx, steps = 8, 8, 128, 64, 24
    cap = 2 * ctx + steps + 2
    num_pages = B * -(-cap // page)  # every row can reach the capacity
    pool = PagePool(max_batch=B, max_blocks=-(-cap // page), page_size=page, kv_heads=H, head_dim=D,
                    dtype=dtype, device="cuda", num_pages=num_pages)
    oracle = DenseLayerOracle(B, cap, page)
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    k = hf_layout(B, H, ctx, D, dtype, gen)
    v = hf_layout(B, H, ctx, D, dtype, gen)
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    for step in range(steps):
        rows = sorted(rng.choice(B, size=2, replace=False).tolist())
        pool.free_rows(rows)
        oracle.release_rows(rows)
        t = int(rng.integers(1, 2 * ctx))
        kr = hf_layout(2, H, t, D, dtype, gen)
        vr = hf_layout(2, H, t, D, dtype, gen)
        pool.append_rows(rows[::-1] if step % 2 else rows, (kr.flip(0) if step % 2 else kr).cuda(),
                         (vr.flip(0) if step % 2 else vr).cuda())
        oracle.append_rows(rows, to_bits(kr), to_bits(vr))
        k = hf_layout(B, H, 1, D, dtype, gen)
        v = hf_layout(B, H, 1, D, dtype, gen)
        gk, gv = pool.update(k.cuda(), v.cuda())
        ok, ov = oracle.update(to_bits(k), to_bits(v))
        assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov), step
        assert list(pool.lens) == pool.seq_lens.cpu().tolist()
        assert pool.free_count == int(pool.ctrl[CTRL_FREE_TOP].item()), step
    assert int(pool.ctrl[CTRL_ERRORS].item()) == 0
