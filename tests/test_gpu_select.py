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


def test_exhausted_pool_is_flagged_and_left_unchanged(capi):
    """Four rows of 6 tokens in pages of 4 (two blocks each, the second partial) fill 8 of 9
    pages.  A permutation copies nothing (each tail moves to its only taker) and succeeds even
    on a full pool; [0, 0, 0, 0] needs 3 copies with 1 page free: the selection is abandoned
    whole -- the error bit is set and the pool is exactly as before."""
    H, D, P, dtype = 1, 4, 4, torch.float32
    pool = CPool(max_batch=4, max_blocks=4, page_size=P, heads=H, dim=D, dtype=dtype, num_pages=9)
    oracle = DenseLayerOracle(4, 16, P)
    gen = torch.Generator().manual_seed(3)
    k, v = hf_layout(4, H, 6, D, dtype, gen), hf_layout(4, H, 6, D, dtype, gen)
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    k, v = hf_layout(1, H, 1, D, dtype, gen), hf_layout(1, H, 1, D, dtype, gen)
    pool.append(k.cuda(), v.cuda())          # row 0 reaches 7 tokens; the last free page stays free
    oracle.append(to_bits(k), to_bits(v))
    oracle.current_batch_size = 4
    assert pool.free_top() == 1
    pool.select_rows([3, 2, 1, 0])
    oracle.batch_select_indices([3, 2, 1, 0])
    assert pool.errors() == 0 and pool.free_top() == 1
    assert_same(pool, oracle, "permutation on a full pool")
    pool.check_invariants()
    before = [t.clone() for t in (pool.bt, pool.lens, pool.hw, pool.free, pool.shares)]
    pool.select_rows([0, 0, 0, 0])
    assert pool.errors() == ERR_POOL_EXHAUSTED
    after = (pool.bt, pool.lens, pool.hw, pool.free, pool.shares)
    assert all(torch.equal(x, y) for x, y in zip(before, after))
    assert pool.free_top() == 1
    assert_same(pool, oracle, "abandoned selection")


def select_layers(pools, rows):
    """barq_kv_select_rows_layers over CPools through the C ABI."""
    import ctypes

    from barqtrain_amd import _capi

    lib = pools[0].lib
    arr = (_capi.BarqKVPool * len(pools))(*[p.s for p in pools])
    words = lib.barq_kv_select_workspace_words(ctypes.byref(pools[0].s), len(pools), len(rows))
    assert words >= 0
    ws = torch.empty(max(words, 1), dtype=torch.int32, device="cuda")
    idx = torch.tensor(rows or [0], dtype=torch.int32, device="cuda")
    _capi.check(lib.barq_kv_select_rows_layers(arr, len(pools), idx.data_ptr(), len(rows), ws.data_ptr(),
                                               ws.numel(), _capi.current_stream()))
    torch.cuda.current_stream().synchronize()


@pytest.mark.parametrize("layers", [3, 35])
def test_layer_batched_selection_matches_per_layer_oracles(capi, layers):
    """One selection applied to every pool of a model-like stack (35 pools: two launch sets),
    each pool with its own data and page count, against one oracle per pool."""
    H, D, P, dtype = 2, 16, 4, torch.bfloat16
    Bmax, cap = 5, 32
    mb = -(-cap // P)
    pools = [CPool(max_batch=Bmax, max_blocks=mb, page_size=P, heads=H, dim=D, dtype=dtype,
                   num_pages=2 * Bmax * mb + l) for l in range(layers)]
    oracles = [DenseLayerOracle(Bmax, cap, P) for _ in range(layers)]
    rng = np.random.default_rng(layers)
    gen = torch.Generator().manual_seed(layers)

    def all_same(what):
        for l, (p, o) in enumerate(zip(pools, oracles)):
            assert_same(p, o, f"{what} layer {l}")
            p.check_invariants()

    for it in range(24):
        o0 = oracles[0]
        cur = o0.current_batch_size
        r = rng.random()
        if r < 0.45 or not cur:
            b = int(rng.integers(1, o0.max_batch_size + 1))
            t = int(rng.integers(1, 6)) if rng.random() < 0.4 else 1
            if o0.is_initialized and int(o0.seq_lens[:b].max()) + t > cap:
                continue
            for p, o in zip(pools, oracles):
                k, v = hf_layout(b, H, t, D, dtype, gen), hf_layout(b, H, t, D, dtype, gen)
                p.append(k.cuda(), v.cuda())
                o.append(to_bits(k), to_bits(v))
        elif r < 0.8:
            rows = rng.integers(0, cur, size=int(rng.integers(0, Bmax + 1))).tolist()
            select_layers(pools, rows)
            for o in oracles:
                if rows:
                    o.batch_select_indices(rows)
                else:
                    o.release_rows(range(o.max_batch_size))
                    o.current_batch_size = 0
            if rows:
                all_same(f"select {rows} it{it}")
        else:
            m = int(rng.integers(0, cap))
            for p in pools:
                p.crop(cur, m)
            select_layers(pools, list(range(Bmax)))
            for o in oracles:
                o.crop(m)
            all_same(f"crop {m} it{it}")
    for p in pools:
        p.check_invariants()
        assert p.errors() == 0


def test_beam_search_generate_on_gpu(hip):
    """generate(num_beams=4) on a GPU paged cache: every step's reorder runs as one layer-batched
    selection; beams and scores equal DynamicCache's."""
    pytest.importorskip("transformers")
    from transformers.cache_utils import DynamicCache

    from barqtrain import create_paged_kv_cache
    from barqtrain_amd import paged
    from test_gpu_layer import tiny_llama

    model, cfg = tiny_llama()
    model = model.to("cuda")
    ids = torch.randint(1, 512, (2, 19), generator=torch.Generator().manual_seed(6)).to("cuda")
    new = 24
    kw = dict(attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False, num_beams=4,
              num_return_sequences=2, return_dict_in_generate=True, output_scores=True)
    ref = model.generate(ids, past_key_values=DynamicCache(config=cfg), **kw)
    calls = []
    real = paged.select_rows_layers

    def counting(pools, rows):
        calls.append(len(list(pools)))
        return real(pools, rows)

    import barqtrain_amd.kv_cache as kv_cache

    kv_cache.select_rows_layers = counting
    try:
        cache = create_paged_kv_cache(model, max_batch_size=8, max_cache_len=19 + new, page_size=16)
        got = model.generate(ids, past_key_values=cache, **kw)
    finally:
        kv_cache.select_rows_layers = real
    assert torch.equal(got.sequences, ref.sequences)
    assert torch.equal(got.sequences_scores, ref.sequences_scores)
    assert calls and all(c == len(cache.layers) for c in calls)
    for layer in cache.layers:
        pool = layer.pool
        assert pool.on_gpu and pool.errors() == 0 and pool.shared
