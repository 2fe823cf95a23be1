"""Quantised (fp8) KV pages through the layer API on host-memory tensors, against the oracle
QuantLayerOracle bit for bit: random programs of ragged and long (chunked) appends, crops (also
below quantised blocks, which re-opens them), beam selections (quantised blocks shared, hot
blocks moved or copied), row releases and resets; page accounting of the hot pool and the cold
store; beam search in generate(); the flag plumbing of create_paged_kv_cache.  CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvgen import hf_layout, to_bits
from oracle.kv_quant_oracle import QuantLayerOracle

DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def check_accounting(pool):
    """Host shadow against the device state: stack tops (exact, or lower bounds after a
    selection), frontiers; every hot page held once; a cold page held by k blocks has
    cold_shares k - 1; each stack holds exactly the pages no block holds."""
    P = pool.page_size
    bt = pool.block_table.numpy()
    top, ctop = int(pool.ctrl[0]), int(pool.ctrl[2])
    assert top == pool.free_count if pool.free_exact else top >= pool.free_count
    assert ctop == pool.cold_free if pool.cold_exact else ctop >= pool.cold_free
    hot, cold = [], []
    for r in range(pool.max_batch):
        n = -(-int(pool.high_water[r]) // P)
        row = bt[r, :n]
        c = int(pool.cold_blocks[r])
        assert (row[:c] <= -2).all() and (row[c:] >= 0).all(), (r, row, c)
        assert (bt[r, n:] == -1).all()
        cold += (-2 - row[:c]).tolist()
        hot += row[c:].tolist()
    held = np.bincount(np.asarray(cold, dtype=np.int64), minlength=pool.num_cold)
    assert len(set(hot)) == len(hot)
    assert (pool.cold_shares.numpy() == np.maximum(held - 1, 0)).all()
    assert not set(hot) & set(pool.free_pages[:top].tolist())
    assert not set(cold) & set(pool.free_cold[:ctop].tolist())
    assert len(hot) + top == pool.num_pages and int((held > 0).sum()) + ctop == pool.num_cold


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
            b = int(rng.integers(1, (oracle.max_batch_size if oracle.is_initialized else Bmax) + 1))
            t = int(rng.integers(1, 40)) if rng.random() < 0.3 else 1
            if oracle.is_initialized and int(oracle.seq_lens[:b].max()) + t > cap:
                continue
            k = hf_layout(b, H, t, D, dtype, gen) * 3
            v = hf_layout(b, H, t, D, dtype, gen)
            gk, gv = layer.update(k, v)
            ok, ov = oracle.update(to_bits(k), to_bits(v))
            assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov), it
        elif r < 0.7:
            m = int(rng.integers(0, cap))  # below quantised blocks too: they are re-opened
            layer.crop(m)
            oracle.crop(m)
        elif r < 0.8 and oracle.current_batch_size:
            cur = oracle.current_batch_size
            n = int(rng.integers(1, Bmax + 1))
            rows = rng.integers(0, cur, size=n).tolist()  # repeats, drops and reorders
            layer.batch_select_indices(torch.tensor(rows))
            oracle.batch_select_indices(rows)
        elif r < 0.9 and oracle.current_batch_size:
            rows = sorted(rng.choice(oracle.max_batch_size, size=min(int(rng.integers(1, 3)), oracle.max_batch_size),
                                     replace=False).tolist())
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
    assert pool.num_pages == 2 * ((6 + 2) + (2 + 1))  # ceil((32 + 64) / 16) + 2, ceil(32 / 16) + 1 per row
    gen = torch.Generator().manual_seed(5)
    k, v = hf_layout(2, 1, 1000, 8, torch.float16, gen), hf_layout(2, 1, 1000, 8, torch.float16, gen)
    gk, _ = pool.update(k, v)
    assert gk.shape == (2, 1, 1000, 8)
    assert pool.cold_blocks.tolist() == [(1000 - 32) // 16] * 2
    mem = pool.memory_bytes()
    assert mem["hot_pages"] < mem["cold_store"]


def test_crop_below_quantised_blocks_reopens_them():
    """Crop to 5 tokens of a row with blocks 0-1 quantised: block 1 (holding position 5) becomes
    a hot page holding its dequantised read -- the gather reads the same bits as before -- and
    the next append writes into it; without room for the page the crop raises, changing nothing."""
    from barqtrain_amd.paged import PagedKVPoolExhausted, QuantPagePool

    pool = QuantPagePool(max_batch=1, max_blocks=8, page_size=4, kv_heads=1, head_dim=4, dtype=torch.float32,
                         device="cpu", window=4)
    oracle = QuantLayerOracle(1, 32, 4, 4, "f32")
    gen = torch.Generator().manual_seed(6)
    k, v = hf_layout(1, 1, 14, 4, torch.float32, gen), hf_layout(1, 1, 14, 4, torch.float32, gen)
    pool.append(k, v)
    oracle.append(to_bits(k), to_bits(v))
    assert pool.cold_blocks.tolist() == [2]
    before = to_bits(pool.gather(1)[0])
    free, cold_free = pool.free_count, pool.cold_free
    pool.crop(1, 5)
    oracle.crop(5)
    assert pool.lens.tolist() == [5] and pool.cold_blocks.tolist() == [1]
    assert pool.free_count == free - 1 and pool.cold_free == cold_free + 1
    assert int(pool.block_table[0, 1]) >= 0 and int(pool.block_table[0, 0]) <= -2
    assert np.array_equal(to_bits(pool.gather(1, 14)[0]), before)
    k, v = hf_layout(1, 1, 3, 4, torch.float32, gen), hf_layout(1, 1, 3, 4, torch.float32, gen)
    gk, gv = pool.update(k, v)
    ok, ov = oracle.update(to_bits(k), to_bits(v))
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
    check_accounting(pool)

    full = QuantPagePool(max_batch=1, max_blocks=8, page_size=4, kv_heads=1, head_dim=4, dtype=torch.float32,
                         device="cpu", window=4, chunk=4, num_pages=3)
    full.append(hf_layout(1, 1, 14, 4, torch.float32, gen), hf_layout(1, 1, 14, 4, torch.float32, gen))
    assert full.free_count == 1 and full.cold_blocks.tolist() == [2]  # re-opening 2 blocks needs 2
    state = (full.lens.copy(), full.block_table.clone(), full.seq_lens.clone())
    with pytest.raises(PagedKVPoolExhausted):
        full.crop(1, 2)
    assert np.array_equal(state[0], full.lens) and torch.equal(state[1], full.block_table)
    assert torch.equal(state[2], full.seq_lens)


def test_beam_selection_shares_quantised_blocks_and_moves_hot_ones():
    """Rows [0, 0, 1]: both takers of row 0 share its quantised blocks (cold_shares 1); the first
    takes its hot pages, the second copies them; row 1's pages move.  Then a crop re-opens a
    shared block for one row only, and releasing rows returns cold pages when unshared."""
    from barqtrain_amd.paged import QuantPagePool

    P, H, D, W = 4, 2, 8, 4
    pool = QuantPagePool(max_batch=3, max_blocks=8, page_size=P, kv_heads=H, head_dim=D, dtype=torch.bfloat16,
                         device="cpu", window=W)
    oracle = QuantLayerOracle(3, 32, P, W, "bf16")
    gen = torch.Generator().manual_seed(7)
    k, v = hf_layout(2, H, 18, D, torch.bfloat16, gen), hf_layout(2, H, 18, D, torch.bfloat16, gen)
    pool.append(k, v)
    oracle.append(to_bits(k), to_bits(v))
    hot0 = pool.block_table[0, 3:5].clone()
    pool.select_rows([0, 0, 1])
    oracle.batch_select_indices([0, 0, 1])
    bt = pool.block_table
    assert torch.equal(bt[0, :3], bt[1, :3]) and (bt[0, :3] <= -2).all()
    assert (pool.cold_shares[(-2 - bt[0, :3]).long()] == 1).all()
    assert torch.equal(bt[0, 3:5], hot0) and not set(bt[1, 3:5].tolist()) & set(hot0.tolist())
    check_accounting(pool)
    gk, gv = pool.gather(3)
    ok, ov = oracle.current_tensors()
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
    pool.crop(3, 6)
    oracle.crop(6)
    check_accounting(pool)
    k, v = hf_layout(3, H, 5, D, torch.bfloat16, gen), hf_layout(3, H, 5, D, torch.bfloat16, gen)
    gk, gv = pool.update(k, v)
    ok, ov = oracle.update(to_bits(k), to_bits(v))
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
    pool.free_rows([1])
    oracle.release_rows([1])
    check_accounting(pool)
    pool.free_rows([0, 2])
    assert int(pool.ctrl[2]) == pool.num_cold and int(pool.ctrl[0]) == pool.num_pages
    # a copy of the emptied pool: every page and cold page free, stacks extended
    grown = pool.copy_rows([0, 1, 2, 2])
    assert grown.max_batch == 4 and grown.free_count == grown.num_pages and grown.cold_free == grown.num_cold
    check_accounting(grown)


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


def test_beam_search_on_fp8_pages_matches_the_oracle_beam_by_beam(monkeypatch):
    """generate(num_beams=4) on a quantised cache: every layer's every update returns the oracle's
    K/V bit for bit, with every beam reordering applied to the oracle too (quant_shadow); the
    beams share quantised blocks."""
    pytest.importorskip("transformers")
    from barqtrain.kv_cache import create_paged_kv_cache
    from quant_shadow import shadow
    from test_generate import tiny_llama

    model, cfg = tiny_llama()
    model.config._attn_implementation = "eager"
    prompt, new = 21, 16
    ids = torch.randint(1, 512, (2, prompt), generator=torch.Generator().manual_seed(8))
    cache = create_paged_kv_cache(model, max_batch_size=8, max_cache_len=prompt + new, page_size=4,
                                  kv_quant="fp8_e4m3", residual_window=8)
    stats = shadow(cache, monkeypatch)
    out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False,
                         num_beams=4, num_return_sequences=2, past_key_values=cache,
                         return_dict_in_generate=True, output_scores=True)
    assert out.sequences.shape[0] == 4
    assert all(s["updates"] >= new - 1 and s["selections"] >= new - 2 for s in stats), stats
    assert all(layer.pool.shared and int(layer.pool.cold_shares.max()) > 0 for layer in cache.layers)
    for layer in cache.layers:
        check_accounting(layer.pool)


def test_quant_oracle_append_rows_equals_append_on_leading_rows():
    """QuantLayerOracle.append_rows pinned against append (already pinned): appending to rows
    0 .. b-1 through append_rows leaves the same bits, lengths and quantised frontiers."""
    gen = torch.Generator().manual_seed(11)
    a = QuantLayerOracle(3, 64, 4, 8, "bf16")
    b = QuantLayerOracle(3, 64, 4, 8, "bf16")
    for t in (13, 1, 9, 1, 20):
        k, v = to_bits(hf_layout(2, 2, t, 8, torch.bfloat16, gen)), to_bits(hf_layout(2, 2, t, 8, torch.bfloat16, gen))
        a.append(k, v)
        b.append_rows([0, 1], k, v)
        for x, y in zip(a.current_tensors(), b.current_tensors()):
            assert np.array_equal(x, y)
        assert np.array_equal(a.cold, b.cold) and np.array_equal(a.seq_lens, b.seq_lens)
    assert int(a.cold.max()) > 0


@pytest.mark.parametrize("dtype,page,window,seed", [(torch.bfloat16, 4, 8, 0), (torch.float32, 5, 0, 1),
                                                    (torch.float16, 16, 16, 2)])
def test_append_rows_refills_freed_rows_like_the_oracle(dtype, page, window, seed):
    """QuantPagePool.append_rows on a host pool: each step frees two rows, re-prefills them with a
    ragged number of tokens (several chunks, each quantising what leaves the window) while the
    others keep decoding -- bit for bit against the oracle, with the page accounting checked."""
    from barqtrain_amd.paged import QuantPagePool

    B, H, D, ctx, steps, cap = 5, 2, 8, 20, 14, 96
    pool = QuantPagePool(max_batch=B, max_blocks=-(-cap // page), page_size=page, kv_heads=H, head_dim=D,
                         dtype=dtype, device="cpu", window=window, chunk=6)
    oracle = QuantLayerOracle(B, cap, page, window, DT[dtype])
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    k, v = hf_layout(B, H, ctx, D, dtype, gen) * 3, hf_layout(B, H, ctx, D, dtype, gen)
    pool.append(k, v)
    oracle.append(to_bits(k), to_bits(v))
    for step in range(steps):
        rows = sorted(rng.choice(B, size=2, replace=False).tolist())
        pool.free_rows(rows)
        oracle.release_rows(rows)
        t = int(rng.integers(1, 2 * ctx))
        kr, vr = hf_layout(2, H, t, D, dtype, gen) * 3, hf_layout(2, H, t, D, dtype, gen)
        order = rows if step % 2 else rows[::-1]
        pool.append_rows(order, kr if step % 2 else kr.flip(0), vr if step % 2 else vr.flip(0))
        oracle.append_rows(rows, to_bits(kr), to_bits(vr))
        check_accounting(pool)
        k, v = hf_layout(B, H, 1, D, dtype, gen), hf_layout(B, H, 1, D, dtype, gen)
        got = pool.update(k, v)
        oracle.append(to_bits(k), to_bits(v))
        ok, ov = oracle.current_tensors()
        assert np.array_equal(to_bits(got[0]), ok) and np.array_equal(to_bits(got[1]), ov), step
        assert np.array_equal(pool.cold_blocks[:B], oracle.cold[:B])
        check_accounting(pool)


@pytest.mark.parametrize("dtype,page,window", [(torch.bfloat16, 4, 8), (torch.float16, 5, 0)])
def test_selection_larger_than_the_pool_grows_it(dtype, page, window):
    """A selection with more rows than a quantised pool holds (batch_repeat_interleave, a beam
    search's first expansion): the layer moves to a larger pool holding this one's state, which
    selects in place -- bit for bit against the oracle, then decoding on, with the accounting of
    shared quantised blocks checked."""
    from barqtrain_amd.kv_cache import BarqPagedKVCacheLayer

    H, D, cap = 2, 8, 64
    gen = torch.Generator().manual_seed(5)
    layer = BarqPagedKVCacheLayer(max_batch_size=2, max_cache_len=cap, page_size=page, kv_quant="fp8_e4m3",
                                  residual_window=window)
    oracle = QuantLayerOracle(2, cap, page, window, DT[dtype])
    k, v = hf_layout(2, H, 23, D, dtype, gen) * 3, hf_layout(2, H, 23, D, dtype, gen)
    layer.update(k, v)
    oracle.append(to_bits(k), to_bits(v))
    before = layer.pool
    layer.batch_repeat_interleave(3)  # 6 rows from a 2-row pool
    oracle.batch_repeat_interleave(3)
    assert layer.pool is not before and layer.pool.max_batch >= 6 and layer.current_batch_size == 6
    ok, ov = oracle.current_tensors()
    gk, gv = layer.pool.gather(6, ok.shape[2])
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
    check_accounting(layer.pool)
    layer.batch_select_indices(torch.tensor([5, 5, 0, 2, 3, 1]))
    oracle.batch_select_indices([5, 5, 0, 2, 3, 1])
    for _ in range(12):
        k, v = hf_layout(6, H, 1, D, dtype, gen), hf_layout(6, H, 1, D, dtype, gen)
        gk, gv = layer.update(k, v)
        oracle.append(to_bits(k), to_bits(v))
        ok, ov = oracle.current_tensors()
        assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
        check_accounting(layer.pool)
