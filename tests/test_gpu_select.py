"""GPU parity of barq_kv_select_rows (in-place row selection sharing full pages), called through
the C ABI, against the oracle's batch_select_indices (restating kv_cache.py:166-186).

Bit-exact: gathers are compared as raw element bits with the oracle after every operation, and
the pool's sharing invariants (page_shares = holders - 1, free stack = unheld pages, shared
blocks only below their row's length) are checked each time.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from capi_pool import CPool
from kvgen import hf_layout, to_bits
from oracle.kv_oracle import DenseLayerOracle

pytestmark = pytest.mark.gpu

ERR_POOL_EXHAUSTED, ERR_BAD_INDEX = 1, 4

SHAPES = [
    # heads, dim, page, dtype
    (2, 4, 4, torch.float32),
    (3, 80, 5, torch.bfloat16),
    (1, 3, 1, torch.float16),
    (8, 128, 16, torch.bfloat16),
]


def assert_same(pool: CPool, oracle: DenseLayerOracle, what: str):
    ok, ov = oracle.current_tensors()
    gk, gv = pool.gather(ok.shape[0], ok.shape[2])
    for g, w, name in ((gk, ok, "K"), (gv, ov, "V")):
        g = to_bits(g)
        if not np.array_equal(g, w):
            bad = np.argwhere(g != w)
            raise AssertionError(f"{what} {name}: {len(bad)} elements differ, first at {bad[0].tolist()}")


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"h{s[0]}d{s[1]}p{s[2]}{str(s[3])[6:]}")
@pytest.mark.parametrize("seed", [0, 1])
def test_random_programs_with_selection(capi, shape, seed):
    H, D, P, dtype = shape
    rng = np.random.default_rng(seed * 17 + P)
    Bmax, cap = 6, 48
    mb = -(-cap // P)
    # A selection takes the copies' pages before it releases the old ones: room for both.
    pool = CPool(max_batch=Bmax, max_blocks=mb, page_size=P, heads=H, dim=D, dtype=dtype,
                 num_pages=2 * Bmax * mb)
    oracle = DenseLayerOracle(Bmax, cap, P)
    gen = torch.Generator().manual_seed(seed)
    shared = False
    for it in range(60):
        r = rng.random()
        cur = oracle.current_batch_size
        if r < 0.45 or not cur:
            b = int(rng.integers(1, oracle.max_batch_size + 1))
            t = int(rng.integers(1, 7)) if rng.random() < 0.4 else 1
            if oracle.is_initialized and int(oracle.seq_lens[:b].max()) + t > cap:
                continue
            k, v = hf_layout(b, H, t, D, dtype, gen), hf_layout(b, H, t, D, dtype, gen)
            oracle.append(to_bits(k), to_bits(v))
            got = pool.update(k.cuda(), v.cuda(), oracle.get_seq_length())
            ok, ov = oracle.current_tensors()
            assert np.array_equal(to_bits(got[0]), ok) and np.array_equal(to_bits(got[1]), ov), f"update it{it}"
        elif r < 0.75:
            rows = rng.integers(0, cur, size=int(rng.integers(1, Bmax + 1))).tolist()
            pool.select_rows(rows)
            oracle.batch_select_indices(rows)
            shared |= bool(pool.shares.any())
            assert_same(pool, oracle, f"select {rows} it{it}")
        elif r < 0.87:
            m = int(rng.integers(0, cap))
            pool.crop(cur, m)
            pool.select_rows(list(range(Bmax)))   # re-open cropped shared blocks for writing
            oracle.crop(m)
            assert_same(pool, oracle, f"crop {m} it{it}")
        else:
            rows = sorted(rng.choice(cur, size=int(rng.integers(1, min(cur, 2) + 1)), replace=False).tolist())
            pool.free_rows(rows)
            oracle.release_rows(rows)
            assert_same(pool, oracle, f"free {rows} it{it}")
        pool.check_invariants()
    assert pool.errors() == 0
    assert shared, "the program never shared a page"


def test_beam_fanout_shares_full_pages(capi):
    """One 100-token row (page 16) fanned out to 8 beams holds 6 shared pages + 8 private
    copies of the partial one; decode steps and beam reorders keep only distinct histories."""
    H, D, P, dtype = 8, 128, 16, torch.bfloat16
    pool = CPool(max_batch=8, max_blocks=16, page_size=P, heads=H, dim=D, dtype=dtype)
    oracle = DenseLayerOracle(8, 256, P)
    gen = torch.Generator().manual_seed(5)
    k, v = hf_layout(1, H, 100, D, dtype, gen), hf_layout(1, H, 100, D, dtype, gen)
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    pool.select_rows([0] * 8)
    oracle.batch_select_indices([0] * 8)
    assert pool.num_pages - pool.free_top() == 6 + 8
    assert int(pool.shares.max()) == 7
    pool.check_invariants()
    rng = np.random.default_rng(0)
    for step in range(40):
        k, v = hf_layout(8, H, 1, D, dtype, gen), hf_layout(8, H, 1, D, dtype, gen)
        pool.append(k.cuda(), v.cuda())
        oracle.append(to_bits(k), to_bits(v))
        beams = sorted(rng.integers(0, 8, size=8).tolist())
        pool.select_rows(beams)
        oracle.batch_select_indices(beams)
        pool.check_invariants()
    assert_same(pool, oracle, "after 40 beam steps")
    assert pool.num_pages - pool.free_top() < 8 * 9, "histories were copied, not shared"
    assert pool.errors() == 0


def test_bad_source_row_is_flagged_and_leaves_an_empty_row(capi):
    H, D, P, dtype = 2, 8, 4, torch.float32
    pool = CPool(max_batch=3, max_blocks=4, page_size=P, heads=H, dim=D, dtype=dtype)
    oracle = DenseLayerOracle(3, 16, P)
    gen = torch.Generator().manual_seed(2)
    k, v = hf_layout(3, H, 6, D, dtype, gen), hf_layout(3, H, 6, D, dtype, gen)
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    pool.select_rows([2, 7, 0])
    assert pool.errors() == ERR_BAD_INDEX
    pool.check_invariants()
    assert pool.lens.tolist() == [6, 0, 6]
    oracle.batch_select_indices([2, 0, 0])
    oracle.release_rows([1])
    assert_same(pool, oracle, "bad index")


def test_exhausted_pool_is_flagged(capi):
    """Four rows of 6 tokens in pages of 4 (two blocks each, the second partial) fill 8 of 9
    pages; selecting [0, 1, 2, 3] needs 4 pages for the partial blocks while only 1 is free."""
    H, D, P, dtype = 1, 4, 4, torch.float32
    pool = CPool(max_batch=4, max_blocks=4, page_size=P, heads=H, dim=D, dtype=dtype, num_pages=9)
    gen = torch.Generator().manual_seed(3)
    k, v = hf_layout(4, H, 6, D, dtype, gen), hf_layout(4, H, 6, D, dtype, gen)
    pool.append(k.cuda(), v.cuda())
    assert pool.free_top() == 1
    pool.select_rows([0, 1, 2, 3])
    assert pool.errors() & ERR_POOL_EXHAUSTED
    pool.reset()
    pool.check_invariants()
    assert pool.errors() == 0
