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


def _fake_pools(count, *, blocks=8, batch=4, shares=True, **geom):
    """Pools with distinct, non-null, never-dereferenced addresses: every call below is
    rejected or sized on the host before any launch."""
    from barqtrain_amd import _capi

    g = dict(pages=batch * blocks, batch=batch, blocks=blocks, page=16, heads=8, dim=128, elem=2)
    g.update(geom)
    pools = []
    for i in range(count):
        base = (i + 1) << 24
        ptrs = [base + (k << 16) for k in range(8)]
        if not shares:
            ptrs[7] = 0
        pools.append(_capi.BarqKVPool(*ptrs, g["pages"], g["batch"], g["blocks"], g["page"], g["heads"],
                                      g["dim"], g["elem"]))
    return pools


def PagePool_words(fake, n):
    from barqtrain_amd.paged import PagePool

    pool = PagePool(max_batch=fake.max_batch, max_blocks=fake.max_blocks, page_size=4, kv_heads=1, head_dim=1,
                    dtype=torch.float32, device="cpu")
    return pool.select_workspace_words(n)


def test_select_workspace_words_and_rejections():
    import ctypes

    from barqtrain_amd import _capi

    lib = _capi.load_library()
    INVALID = 1
    words = lib.barq_kv_select_workspace_words
    one = _fake_pools(1)[0]
    # per pool: table [n, blocks], lengths, marks, ranks [n], first takers [max_batch], top, go
    per = lambda n: n * (8 + 3) + 4 + 2  # noqa: E731
    assert words(ctypes.byref(one), 1, 4) == per(4)
    assert words(ctypes.byref(one), 3, 4) == 3 * per(4)
    assert words(ctypes.byref(one), 40, 2) == 32 * per(2)     # 32 pools per launch set
    assert words(ctypes.byref(one), 1, 0) == per(0)
    assert words(ctypes.byref(one), 0, 4) == -1
    assert words(ctypes.byref(one), 1, 5) == -1               # more rows than the pool holds
    big = _fake_pools(1, batch=8193, pages=8193 * 8)[0]
    assert words(ctypes.byref(big), 1, 4) == -1               # beyond 8192 rows
    for n in range(5):
        assert PagePool_words(one, n) == words(ctypes.byref(one), 1, n)

    def call(pools, rows=2, ws_words=None):
        arr = (_capi.BarqKVPool * len(pools))(*pools)
        need = len(pools) * per(rows) if ws_words is None else ws_words
        return lib.barq_kv_select_rows_layers(arr, len(pools), 1 << 12, rows, 1 << 13, need, None)

    ok = _fake_pools(3)
    assert call(ok, ws_words=3 * per(2) - 1) == INVALID       # workspace one word short
    assert call(ok, rows=5) == INVALID                        # rows beyond max_batch
    assert call(ok, rows=-1) == INVALID
    assert call([ok[0], ok[1], ok[0]]) == INVALID              # a pool named twice
    assert call(ok[:2] + _fake_pools(1, blocks=9)) == INVALID  # geometry differs
    assert call(ok[:2] + _fake_pools(1, heads=4, pages=64)) == INVALID
    assert call(_fake_pools(2, shares=False)) == INVALID       # no page_shares
    arr = (_capi.BarqKVPool * 1)(*ok[:1])
    assert lib.barq_kv_select_rows_layers(arr, 0, 1 << 12, 2, 1 << 13, 20, None) == INVALID
    assert lib.barq_kv_select_rows(ctypes.byref(_fake_pools(1, shares=False)[0]), 1 << 12, 2, 1 << 13, 100,
                                   None) == INVALID
    assert lib.barq_kv_select_rows(ctypes.byref(ok[0]), 1 << 12, 2, 0, 100, None) == INVALID  # no workspace


def test_cache_reorder_matches_per_layer_oracles():
    """Cache-level batch_select_indices / reorder_cache / batch_repeat_interleave (one selection
    for every layer) against one oracle per layer, each layer holding different data."""
    from barqtrain.kv_cache import create_paged_kv_cache

    class Text:
        num_hidden_layers = 3

    class Config:
        def get_text_config(self, decoder=True):
            return Text()

    H, D, P, cap = 2, 8, 4, 40
    cache = create_paged_kv_cache(Config(), max_batch_size=8, max_cache_len=cap, page_size=P)
    oracles = [DenseLayerOracle(8, cap, P) for _ in range(3)]
    gen = torch.Generator().manual_seed(9)

    def step(b, t):
        for l, o in enumerate(oracles):
            k, v = hf_layout(b, H, t, D, torch.float32, gen), hf_layout(b, H, t, D, torch.float32, gen)
            gk, gv = cache.update(k, v, l)
            ok, ov = o.update(to_bits(k), to_bits(v))
            assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)

    def same():
        for layer, o in zip(cache.layers, oracles):
            gk, gv = layer.current_tensors()
            ok, ov = o.current_tensors()
            assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
            invariants(layer.pool)

    step(2, 7)
    cache.batch_repeat_interleave(3)
    for o in oracles:
        o.batch_repeat_interleave(3)
    same()
    step(6, 2)
    cache.reorder_cache(torch.tensor([5, 5, 0, 1, 3, 3]))
    for o in oracles:
        o.reorder_cache([5, 5, 0, 1, 3, 3])
    same()
    step(6, 1)
    cache.batch_select_indices(torch.tensor([-1, 2, 2]))
    for o in oracles:
        o.batch_select_indices([5, 2, 2])
    same()
    with pytest.raises(IndexError):
        cache.batch_select_indices(torch.tensor([3]))


def test_host_pool_moves_tails_and_abandons_what_does_not_fit():
    """Host-memory mirror of the device semantics: a permutation on a full pool copies nothing;
    a selection whose copies exceed the free stack changes nothing and sets POOL_EXHAUSTED."""
    from barqtrain_amd.paged import PagePool

    H, D, P = 1, 4, 4
    pool = PagePool(max_batch=4, max_blocks=4, page_size=P, kv_heads=H, head_dim=D, dtype=torch.float32,
                    device="cpu", num_pages=9)
    oracle = DenseLayerOracle(4, 16, P)
    gen = torch.Generator().manual_seed(3)
    k, v = hf_layout(4, H, 7, D, torch.float32, gen), hf_layout(4, H, 7, D, torch.float32, gen)
    pool.append(k, v)
    oracle.append(to_bits(k), to_bits(v))
    assert int(pool.ctrl[0]) == 1
    pool.select_rows([3, 2, 1, 0])
    oracle.batch_select_indices([3, 2, 1, 0])
    assert int(pool.ctrl[0]) == 1 and int(pool.ctrl[1]) == 0
    gk, gv = pool.gather(4)
    ok, ov = oracle.current_tensors()
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
    invariants(pool)
    with pytest.raises(Exception, match="exhausted"):
        pool.select_rows([0, 0, 0, 0])    # the host check refuses: 3 copies, 1 page free
    state = [t.clone() for t in pool.tensors[2:]]
    from barqtrain_amd.paged import _HostOps

    _HostOps.pool_select_rows_(pool.tensors, torch.tensor([0, 0, 0, 0], dtype=torch.int32))
    assert int(pool.ctrl[1]) == 1  # POOL_EXHAUSTED, nothing else changed
    pool.ctrl[1] = 0
    assert all(torch.equal(x, y) for x, y in zip(state, pool.tensors[2:]))


def test_crop_on_shared_rows_copies_only_shared_tails():
    """Two beams share 3 full pages; cropping into the shared region re-opens them for writing:
    the identity selection copies those pages for each beam (not the exclusive ones) and appends
    after the crop leave the other beam's history intact."""
    from barqtrain_amd.paged import PagePool

    H, D, P = 1, 4, 4
    pool = PagePool(max_batch=2, max_blocks=6, page_size=P, kv_heads=H, head_dim=D, dtype=torch.float32,
                    device="cpu")
    oracle = DenseLayerOracle(2, 24, P)
    gen = torch.Generator().manual_seed(8)
    k, v = hf_layout(1, H, 13, D, torch.float32, gen), hf_layout(1, H, 13, D, torch.float32, gen)
    pool.append(k, v)
    oracle.append(to_bits(k), to_bits(v))
    pool.select_rows([0, 0])
    oracle.batch_select_indices([0, 0])
    assert int(pool.page_shares.sum()) == 3
    top = int(pool.ctrl[0])
    pool.crop(2, 5)                       # blocks 1 and 2 (positions 4-11) become tails of both rows
    oracle.crop(5)
    assert int(pool.page_shares.sum()) == 1     # block 0 stays shared
    # 2 shared tail pages copied for each row (4 pages taken), the 2 originals returned; the
    # rows' own partial pages move
    assert int(pool.ctrl[0]) == top - 4 + 2
    invariants(pool)
    k, v = hf_layout(2, H, 3, D, torch.float32, gen), hf_layout(2, H, 3, D, torch.float32, gen)
    gk, gv = pool.update(k, v)
    ok, ov = oracle.update(to_bits(k), to_bits(v))
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
    invariants(pool)
