"""GPU parity of the fp8 cold store (barq_kv_compress / barq_kv_gather_cold / barq_kv_update_cold /
barq_kv_free_rows_cold / barq_kv_select_rows_cold_layers / barq_kv_crop_cold), through the C ABI
and the layer API, against the oracle QuantLayerOracle: bit-exact (codes, scales and every
dequantised element), with page accounting -- shared cold pages included -- checked after every
operation."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from capi_pool import CColdPool
from kvgen import hf_layout, to_bits
from oracle import kv_quant_oracle as q

pytestmark = pytest.mark.gpu
DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def assert_same(pool, oracle, what):
    ok, ov = oracle.current_tensors()
    gk, gv = pool.gather(ok.shape[0], ok.shape[2])
    for g, w, name in ((gk, ok, "K"), (gv, ov, "V")):
        g = to_bits(g)
        if not np.array_equal(g, w):
            bad = np.argwhere(g != w)
            raise AssertionError(f"{what} {name}: {len(bad)} elements differ, first at {bad[0].tolist()}")


CASES = [
    # dtype, heads, dim, page, window
    (torch.bfloat16, 2, 16, 4, 8),
    (torch.float16, 3, 80, 16, 16),
    (torch.float32, 1, 12, 5, 0),
    (torch.bfloat16, 8, 128, 16, 32),
    (torch.bfloat16, 2, 6, 1, 3),   # 2-element vectors, one-token pages
    # the one-launch update (tokens <= window, token rows of 64 / 128 16-byte vectors)
    (torch.float16, 8, 128, 32, 48),
    (torch.bfloat16, 4, 128, 16, 16),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{DT[c[0]]}-h{c[1]}d{c[2]}p{c[3]}w{c[4]}")
@pytest.mark.parametrize("seed", [0, 1])
def test_random_programs_through_capi(capi, case, seed):
    dtype, H, D, P, W = case
    Bmax, cap = 4, 96
    rng = np.random.default_rng(seed * 7 + P)
    gen = torch.Generator().manual_seed(seed)
    pool = CColdPool(window=W, max_batch=Bmax, max_blocks=-(-cap // P), page_size=P, heads=H, dim=D, dtype=dtype)
    oracle = q.QuantLayerOracle(Bmax, cap, P, W, DT[dtype])
    for it in range(60):
        r = rng.random()
        if r < 0.55 or not oracle.is_initialized:
            b = int(rng.integers(1, (oracle.max_batch_size if oracle.is_initialized else Bmax) + 1))
            t = int(rng.integers(1, 30)) if rng.random() < 0.3 else 1
            if oracle.is_initialized and int(oracle.seq_lens[:b].max()) + t > cap:
                continue
            k, v = hf_layout(b, H, t, D, dtype, gen) * 4, hf_layout(b, H, t, D, dtype, gen)
            oracle.append(to_bits(k), to_bits(v))
            if rng.random() < 0.3:  # the three launches one by one
                pool.append(k.cuda(), v.cuda())
                pool.compress(b)
            else:
                got = pool.update(k.cuda(), v.cuda(), oracle.get_seq_length())
                ok, ov = oracle.current_tensors()
                assert np.array_equal(to_bits(got[0]), ok) and np.array_equal(to_bits(got[1]), ov), f"update it{it}"
        elif r < 0.7 and oracle.current_batch_size:
            cur = oracle.current_batch_size
            m = int(rng.integers(0, cap))  # below quantised blocks too: barq_kv_crop_cold re-opens them
            pool.crop(cur, m)
            oracle.crop(m)
        elif r < 0.85 and oracle.current_batch_size:
            rows = rng.integers(0, oracle.current_batch_size, size=int(rng.integers(1, Bmax + 1))).tolist()
            pool.select_rows(rows)  # repeats share quantised blocks; hot blocks move or are copied
            oracle.batch_select_indices(rows)
        elif oracle.current_batch_size:
            n = oracle.max_batch_size
            rows = sorted(rng.choice(n, size=min(int(rng.integers(1, 3)), n), replace=False).tolist())
            pool.free_rows(rows)
            oracle.release_rows(rows)
        if oracle.current_batch_size:
            assert_same(pool, oracle, f"it{it}")
        pool.check_invariants()
    assert pool.errors() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H", [4, 8, 16])
def test_lanes_kernels_decode_extreme_pages_like_the_oracle(capi, dtype, H):
    """The gather and the one-launch update over cold pages whose token rows are 64, 128 or 256
    16-byte vectors (H x 128): NaN and infinite values, signed zeros and (bf16) heads scaled by
    2^-100 and 2^100, whose scale bytes leave [64, 191], so that vectors the hardware decode does
    not cover take the element-wise path; bit-exact against the oracle."""
    D, P, W = 128, 16, 16
    rng = np.random.default_rng(H)
    x = rng.standard_normal((2, 3 * P, H, D)).astype(np.float32)
    x[0, 3, 1, 5] = np.nan
    x[1, 20, 1, 3] = np.nan
    x[1, 4, 0, 7] = np.inf
    x[1, 5, 2, 9] = -np.inf
    x[0, 6, 3, :] = -0.0
    if dtype == torch.bfloat16:
        x[0, :, 2, :] *= np.float32(2.0 ** -100)
        x[1, 17:, 3, :64] *= np.float32(2.0 ** 100)
    t = torch.from_numpy(x).to(dtype)
    k = t[0][None].permute(0, 2, 1, 3).contiguous()
    v = t[1][None].permute(0, 2, 1, 3).contiguous()
    pool = CColdPool(window=W, max_batch=1, max_blocks=4, page_size=P, heads=H, dim=D, dtype=dtype)
    oracle = q.QuantLayerOracle(1, 4 * P, P, W, DT[dtype])
    pool.append(k.cuda(), v.cuda())
    pool.compress(1)
    oracle.append(to_bits(k), to_bits(v))
    assert oracle.cold.tolist() == [2]
    assert_same(pool, oracle, "gather")
    gen = torch.Generator().manual_seed(H)
    k1, v1 = hf_layout(1, H, 1, D, dtype, gen), hf_layout(1, H, 1, D, dtype, gen)
    oracle.append(to_bits(k1), to_bits(v1))
    got = pool.update(k1.cuda(), v1.cuda(), oracle.get_seq_length())
    ok, ov = oracle.current_tensors()
    assert np.array_equal(to_bits(got[0]), ok) and np.array_equal(to_bits(got[1]), ov), "update"
    assert pool.errors() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_boundary_values_quantise_like_the_oracle(capi, dtype):
    """Groups whose values sit on E4M3 codes, on the midpoints between them (ties to even) and
    one float ulp either side, group maxima exactly at and just above 448 * 2^e, NaN, infinities,
    signed zeros, all-zero groups and groups at the far ends of the exponent range."""
    H, D, P, W = 2, 64, 16, 0
    vals = q.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    pts = np.concatenate([vals.astype(np.float32), mids, np.nextafter(mids, np.float32(0)),
                          np.nextafter(mids, np.float32(1e9))])
    rng = np.random.default_rng(3)
    page = rng.choice(pts, size=(2, P, H, D)).astype(np.float32) * np.where(rng.random((2, P, H, D)) < 0.5, -1, 1)
    page[0, 0] = 448.0                       # channel maxima exactly 448: exponent 0
    page[1, 0, 0] = np.float32(448.0) * np.float32(1 + 2 ** -7)   # just above: exponent 1
    page[0, 3, 1, 5] = np.nan
    page[1, 4, 0, 7] = np.inf
    page[1, 5, 1, 9] = -np.inf
    page[0, 6, 0, :] = 0.0
    page[0, 6, 1, :] = -0.0
    scale = np.float32(2.0 ** 20) if dtype == torch.float32 else np.float32(2.0 ** 4)
    page[1, :, 1, 32:] *= scale              # a loud half-head: per-token value scales follow it
    if dtype == torch.float32:
        page[0, 8:, 1, 40:] = np.float32(3e-39)  # a denormal float32 group
    t = torch.from_numpy(page).to(dtype)     # rounds to the element type first
    k = t[0][None].permute(0, 2, 1, 3)       # [1, H, P, D]
    v = t[1][None].permute(0, 2, 1, 3)
    pool = CColdPool(window=W, max_batch=1, max_blocks=2, page_size=P, heads=H, dim=D, dtype=dtype)
    oracle = q.QuantLayerOracle(1, 2 * P, P, W, DT[dtype])
    pool.append(k.contiguous().cuda(), v.contiguous().cuda())
    pool.compress(1)
    oracle.append(to_bits(k.contiguous()), to_bits(v.contiguous()))
    assert oracle.cold.tolist() == [1]
    c = -2 - int(pool.bt[0, 0])
    for key, codes, scales in ((True, pool.kc, pool.ks), (False, pool.vc, pool.vs)):
        want_codes, want_scales = oracle.quantized_page(0, 0, key)
        assert np.array_equal(codes[c].cpu().numpy(), want_codes), key
        assert np.array_equal(scales[c].cpu().numpy(), want_scales), key
    assert_same(pool, oracle, "boundary page")


def test_c2_shape_prefill_and_decode(capi):
    """The Llama-3-8B KV shape (8 heads x 128, bf16, page 16), 16 rows, window 128: a 512-token
    prefill and 24 decode steps, the last compared element for element."""
    B, H, D, P, W, cap = 16, 8, 128, 16, 128, 544
    pool = CColdPool(window=W, max_batch=B, max_blocks=cap // P, page_size=P, heads=H, dim=D, dtype=torch.bfloat16)
    oracle = q.QuantLayerOracle(B, cap, P, W, "bf16")
    gen = torch.Generator().manual_seed(12)
    k, v = hf_layout(B, H, 512, D, torch.bfloat16, gen), hf_layout(B, H, 512, D, torch.bfloat16, gen)
    oracle.append(to_bits(k), to_bits(v))
    pool.update(k.cuda(), v.cuda(), 512)
    for s in range(24):
        k, v = hf_layout(B, H, 1, D, torch.bfloat16, gen), hf_layout(B, H, 1, D, torch.bfloat16, gen)
        oracle.append(to_bits(k), to_bits(v))
        got = pool.update(k.cuda(), v.cuda(), 513 + s)
    ok, ov = oracle.current_tensors()
    assert np.array_equal(to_bits(got[0]), ok) and np.array_equal(to_bits(got[1]), ov)
    assert oracle.cold.tolist() == [(536 - W) // P] * B
    pool.check_invariants()
    assert pool.errors() == 0


def test_cold_store_exhaustion_keeps_blocks_hot(capi):
    P = 4
    pool = CColdPool(window=0, num_cold=3, max_batch=2, max_blocks=4, page_size=P, heads=1, dim=8,
                     dtype=torch.float32)
    gen = torch.Generator().manual_seed(1)
    k, v = hf_layout(2, 1, 9, 8, torch.float32, gen), hf_layout(2, 1, 9, 8, torch.float32, gen)
    oracle = q.QuantLayerOracle(2, 16, P, 0, "f32")
    pool.update(k.cuda(), v.cuda(), 9)      # 4 full blocks want 4 cold pages, 3 exist
    assert pool.errors() == 1               # POOL_EXHAUSTED
    pool.check_invariants()
    bt = pool.bt.cpu().numpy()
    assert int((bt[:, :2] <= -2).sum()) == 3
    # every block reads back either exactly (hot) or as the oracle's dequantised page (cold)
    oracle.append(to_bits(k), to_bits(v))
    gk, _ = pool.gather(2, 9)
    ok, _ = oracle.current_tensors()
    exact = to_bits(k)
    for r in range(2):
        for j in range(2):
            sl = slice(j * P, (j + 1) * P)
            want = ok[r, :, sl] if bt[r, j] <= -2 else exact[r, :, sl]
            assert np.array_equal(to_bits(gk)[r, :, sl], want), (r, j)


def test_layer_api_with_graph_replays(hip):
    """QuantPagePool through the torch binding, decode steps captured in a HIP graph
    (CapturedDecodeStep), every replay's output compared with the oracle."""
    from barqtrain_amd.graph import CapturedDecodeStep
    from barqtrain_amd.paged import QuantPagePool

    B, H, D, P, W = 3, 2, 64, 8, 16
    cap = 128
    pools = [QuantPagePool(max_batch=B, max_blocks=cap // P, page_size=P, kv_heads=H, head_dim=D,
                           dtype=torch.bfloat16, device="cuda", window=W, chunk=32) for _ in range(2)]
    oracles = [q.QuantLayerOracle(B, cap, P, W, "bf16") for _ in range(2)]
    gen = torch.Generator().manual_seed(7)
    for pool, o in zip(pools, oracles):
        k, v = hf_layout(B, H, 70, D, torch.bfloat16, gen), hf_layout(B, H, 70, D, torch.bfloat16, gen)
        pool.update(k.cuda(), v.cuda())
        o.append(to_bits(k), to_bits(v))
    step = CapturedDecodeStep(pools, B, 1)
    for s in range(30):
        for i, (pool, o) in enumerate(zip(pools, oracles)):
            k, v = hf_layout(B, H, 1, D, torch.bfloat16, gen), hf_layout(B, H, 1, D, torch.bfloat16, gen)
            step.key_in[i].copy_(k)
            step.value_in[i].copy_(v)
            o.append(to_bits(k), to_bits(v))
        outs = step.replay()
        for (gk, gv), o in zip(outs, oracles):
            ok, ov = o.current_tensors()
            assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov), s
    for pool in pools:
        assert pool.errors() == 0
        assert int(pool.ctrl[0]) == pool.free_count and int(pool.ctrl[2]) == pool.cold_free
        assert pool.cold_blocks.tolist() == [(100 - W) // P] * B


def test_beam_search_on_fp8_pages_matches_the_oracle_beam_by_beam(hip, monkeypatch):
    """generate(num_beams=4, kv_quant="fp8_e4m3") on GPU pools: every layer's every update returns
    the oracle's K/V bit for bit, every beam reordering (one barq_kv_select_rows_cold_layers
    launch set for all layers) applied to the oracle too; the beams share quantised blocks."""
    pytest.importorskip("transformers")
    from barqtrain import create_paged_kv_cache
    from quant_shadow import shadow
    from test_gpu_layer import tiny_llama

    model, cfg = tiny_llama()
    model = model.to("cuda")
    model.config._attn_implementation = "eager"
    prompt, new = 40, 24
    ids = torch.randint(1, 512, (2, prompt), generator=torch.Generator().manual_seed(9)).to("cuda")
    cache = create_paged_kv_cache(model, max_batch_size=8, max_cache_len=prompt + new, page_size=4,
                                  kv_quant="fp8_e4m3", residual_window=8)
    stats = shadow(cache, monkeypatch)
    out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False,
                         num_beams=4, num_return_sequences=2, past_key_values=cache,
                         return_dict_in_generate=True, output_scores=True)
    assert out.sequences.shape == (4, prompt + new)
    assert all(s["updates"] >= new - 1 and s["selections"] >= new - 2 for s in stats), stats
    for layer in cache.layers:
        pool = layer.pool
        assert pool.on_gpu and pool.errors() == 0 and pool.shared
        assert int(pool.cold_shares.max()) > 0  # beams hold quantised blocks in common


def test_model_on_gpu_with_fp8_pages_tracks_full_precision(hip):
    """A model's decode steps on fp8 pages (kv_quant="fp8_e4m3", 16-token window) against
    DynamicCache, teacher-forced on DynamicCache's greedy sequence so both see the same tokens:
    per-step logits within 5 % relative (L2) and the same argmax on at least 75 % of steps
    (random weights give near-flat logits).  Then generate() runs on the quantised cache."""
    pytest.importorskip("transformers")
    from transformers.cache_utils import DynamicCache

    from barqtrain import create_paged_kv_cache
    from test_gpu_layer import tiny_llama

    model, cfg = tiny_llama()
    model = model.to("cuda")
    prompt, new = 48, 32
    ids = torch.randint(1, 512, (2, prompt), generator=torch.Generator().manual_seed(3)).to("cuda")
    seq = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False,
                         past_key_values=DynamicCache(config=cfg))

    @torch.no_grad()
    def forced(cache):
        out = model(seq[:, :prompt], past_key_values=cache, use_cache=True)
        logits = [out.logits[:, -1]]
        for i in range(prompt, prompt + new - 1):
            out = model(seq[:, i:i + 1], past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1])
        return torch.stack(logits, 1)

    ref = forced(DynamicCache(config=cfg))
    cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=prompt + new, page_size=16,
                                  kv_quant="fp8_e4m3", residual_window=16)
    got = forced(cache)
    assert all(layer.pool.on_gpu and layer.pool.errors() == 0 and int(layer.pool.cold_blocks.min()) >= 3
               for layer in cache.layers)
    assert ((got - ref).norm() / ref.norm()) < 0.05
    assert (got.argmax(-1) == ref.argmax(-1)).float().mean() >= 0.75
    cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=prompt + new, page_size=16,
                                  kv_quant="fp8_e4m3", residual_window=16)
    out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False,
                         past_key_values=cache)
    assert out.shape == (2, prompt + new) and cache.get_seq_length() == prompt + new - 1


ATT_F32 = dict(rtol=2e-5, atol=2e-5)
ATT_OUT = {torch.bfloat16: dict(rtol=2.0 ** -8, atol=2e-5), torch.float16: dict(rtol=2.0 ** -11, atol=2e-5)}


@pytest.mark.parametrize("dtype,page,window,D", [(torch.bfloat16, 16, 0, 128), (torch.bfloat16, 16, 48, 128),
                                                 (torch.float16, 32, 32, 128), (torch.bfloat16, 32, 128, 128),
                                                 (torch.bfloat16, 16, 48, 64), (torch.float16, 32, 0, 64),
                                                 # pages not a multiple of 16 (dequantising gather + attention)
                                                 (torch.bfloat16, 5, 16, 128), (torch.float16, 8, 24, 64),
                                                 # head size 256 (dequantising gather + attention)
                                                 (torch.bfloat16, 16, 48, 256)])
def test_decode_attention_reads_quantised_pages(hip, dtype, page, window, D):
    """Attention over a quantised pool (barq_kv_decode_attention_cold: cold blocks read as codes
    and scales, dequantised in registers) against the float64 reference over the dequantising
    gather's K/V -- the values the cold store holds -- on ragged rows mixing cold and hot blocks,
    G = 1, 4, 8 and two query tokens; fp32 and cache-dtype outputs; head sizes 128, 64 and 256."""
    from attn_ref import decode_attention_reference, within_tolerance
    from barqtrain_amd.paged import QuantPagePool

    H = 4
    lens = [700, 333, 129, 64, 17, 1]
    B, cap = len(lens), 768
    pool = QuantPagePool(max_batch=B, max_blocks=cap // page, page_size=page, kv_heads=H, head_dim=D, dtype=dtype,
                         device="cuda", window=window)
    gen = torch.Generator().manual_seed(page + window)
    done = 0
    for b in range(B, 0, -1):           # rows [0, b) grow to the next length, longest first
        n = lens[b - 1] - done
        if n > 0:
            k, v = hf_layout(b, H, n, D, dtype, gen) * 3, hf_layout(b, H, n, D, dtype, gen)
            pool.append(k.cuda(), v.cuda())
            done += n
    assert int(pool.cold_blocks.max()) > 0
    kd, vd = (t.double().cpu().numpy() for t in pool.gather(B))
    for G, T in ((1, 1), (4, 1), (8, 1), (4, 2)):
        q = hf_layout(B, G * H, T, D, dtype, gen).cuda()
        want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, lens, D ** -0.5)
        got = pool.attend(q, out_dtype=torch.float32)
        ok, ratio = within_tolerance(got.double().cpu().numpy(), want, **ATT_F32)
        assert ok, f"G={G} T={T}: {ratio:.3g} x tolerance"
        got = pool.attend(q)
        ok, ratio = within_tolerance(got.double().cpu().numpy(), want, **ATT_OUT[dtype])
        assert ok, f"G={G} T={T} {dtype}: {ratio:.3g} x tolerance"
    assert pool.errors() == 0


@pytest.mark.parametrize("cap,D", [(640, 128), (1024, 128), (640, 64), (1024, 64)])
def test_decode_attention_on_quantised_pages_many_pairs(hip, cap, D):
    """Attention over a quantised pool with 128 (row, kv head) pairs of ragged rows (the one-launch
    pair kernel: up to 44 chunks, and with up to 4 query rows up to 64; at head size 64 a loop over
    the quantised chunks, then one over the window's, each chunk loaded whole and clamped): against
    the float64 reference over the dequantising gather's K/V.  Rows shorter than the window, rows
    whose pieces straddle the window's start, one and two query tokens."""
    from attn_ref import decode_attention_reference, within_tolerance
    from barqtrain_amd.paged import QuantPagePool

    H, P, W = 4, 16, 32
    rng = np.random.default_rng(77 + cap)
    top = cap - 40
    lens = sorted([top, top - 15, 1, 16, 33] + rng.integers(40, top, size=27).tolist(), reverse=True)
    B = len(lens)
    pool = QuantPagePool(max_batch=B, max_blocks=cap // P, page_size=P, kv_heads=H, head_dim=D,
                         dtype=torch.bfloat16, device="cuda", window=W)
    gen = torch.Generator().manual_seed(78)
    done = 0
    for b in range(B, 0, -1):
        n = lens[b - 1] - done
        if n > 0:
            k, v = hf_layout(b, H, n, D, torch.bfloat16, gen) * 3, hf_layout(b, H, n, D, torch.bfloat16, gen)
            pool.append(k.cuda(), v.cuda())
            done += n
    assert int(pool.cold_blocks.max()) > 0
    kd, vd = (t.double().cpu().numpy() for t in pool.gather(B))
    for G, T in ((4, 1), (2, 1), (2, 2), (8, 1)):
        q = hf_layout(B, G * H, T, D, torch.bfloat16, gen).cuda()
        want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, lens, D ** -0.5)
        got = pool.attend(q, out_dtype=torch.float32)
        ok, ratio = within_tolerance(got.double().cpu().numpy(), want, **ATT_F32)
        assert ok, f"G={G} T={T}: {ratio:.3g} x tolerance"
    assert pool.errors() == 0


@pytest.mark.parametrize("D", [128, 64])
def test_decode_attention_cold_through_capi(capi, D):
    """The C entry point on a CColdPool with a crafted cold page (zero, subnormal and NaN-free
    boundary codes take the exact per-element decode) next to hot pages."""
    from attn_ref import decode_attention_reference, within_tolerance
    from capi_pool import attend_cold

    B, H, P, W = 2, 2, 16, 16
    pool = CColdPool(window=W, max_batch=B, max_blocks=8, page_size=P, heads=H, dim=D, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(21)
    k, v = hf_layout(B, H, 70, D, torch.bfloat16, gen), hf_layout(B, H, 70, D, torch.bfloat16, gen)
    k[0, :, 3] = 0.0                     # a zero key: zero codes in a cold page
    v[1, 1, 5, :7] = 1e-30               # tiny values: subnormal codes
    pool.append(k.cuda(), v.cuda())
    pool.compress(B)
    assert pool.errors() == 0 and int((pool.bt[:, :3] <= -2).sum()) == 6
    kd, vd = (t.double().cpu().numpy() for t in pool.gather(B, 70))
    q = hf_layout(B, 4 * H, 1, D, torch.bfloat16, gen).cuda()
    out = attend_cold(pool, q)
    torch.cuda.synchronize()
    want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, [70, 70], D ** -0.5)
    ok, ratio = within_tolerance(out.double().cpu().numpy(), want, **ATT_F32)
    assert ok, ratio
    assert pool.errors() == 0


def test_fused_paged_attention_on_fp8_pages_in_a_model(hip):
    """A bf16 Llama whose decode attention reads the quantised pages directly (fused "barq_paged"
    attention + kv_quant), teacher-forced against the same model on DynamicCache: logits within
    5 % relative (L2), argmax agreeing on at least 75 % of steps."""
    pytest.importorskip("transformers")
    from transformers.cache_utils import DynamicCache

    from barqtrain import create_paged_kv_cache
    from barqtrain_amd import attention
    from test_gpu_layer import bf16_llama

    model, cfg = bf16_llama()
    model = model.to("cuda")
    prompt, new = 64, 32
    seq = torch.randint(1, 512, (2, prompt + new), generator=torch.Generator().manual_seed(8)).to("cuda")

    @torch.no_grad()
    def forced(cache):
        out = model(seq[:, :prompt], past_key_values=cache, use_cache=True)
        logits = [out.logits[:, -1].float()]
        for i in range(prompt, prompt + new - 1):
            out = model(seq[:, i:i + 1], past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1].float())
        return torch.stack(logits, 1)

    model.config._attn_implementation = "sdpa"
    ref = forced(DynamicCache(config=cfg))
    attention.enable_paged_attention(model)
    cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=prompt + new, page_size=16,
                                  kv_quant="fp8_e4m3", residual_window=16)
    got = forced(cache)
    assert all(layer.fused_attention and int(layer.pool.cold_blocks.min()) >= 3 for layer in cache.layers)
    assert all(layer.pool.errors() == 0 for layer in cache.layers)
    assert ((got - ref).norm() / ref.norm()) < 0.05
    assert (got.argmax(-1) == ref.argmax(-1)).float().mean() >= 0.75


def test_refill_freed_rows_on_fp8_pages_like_the_oracle(hip):
    """The serving pattern of C5 on fp8 pages: each step frees two rows, re-prefills them with a new
    sequence of 200..700 tokens (QuantPagePool.append_rows: per row, chunks of append + quantise on
    the row's one-row metadata view, the free stacks shared) while every row decodes -- against
    the oracle bit for bit, the stacks' tops against the host shadow."""
    from barqtrain_amd.paged import CTRL_COLD_TOP, CTRL_FREE_TOP, QuantPagePool
    from oracle.kv_quant_oracle import QuantLayerOracle

    B, H, D, P, W, ctx, steps = 6, 8, 128, 16, 64, 400, 10
    cap = 1200
    pool = QuantPagePool(max_batch=B, max_blocks=cap // P, page_size=P, kv_heads=H, head_dim=D, dtype=torch.bfloat16,
                         device="cuda", window=W)
    oracle = QuantLayerOracle(B, cap, P, W, "bf16")
    rng = np.random.default_rng(8)
    gen = torch.Generator().manual_seed(8)
    k, v = hf_layout(B, H, ctx, D, torch.bfloat16, gen) * 2, hf_layout(B, H, ctx, D, torch.bfloat16, gen)
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    for step in range(steps):
        rows = sorted(rng.choice(B, size=2, replace=False).tolist())
        pool.free_rows(rows)
        oracle.release_rows(rows)
        t = int(rng.integers(200, 700))
        kr, vr = hf_layout(2, H, t, D, torch.bfloat16, gen) * 2, hf_layout(2, H, t, D, torch.bfloat16, gen)
        pool.append_rows(rows, kr.cuda(), vr.cuda())
        oracle.append_rows(rows, to_bits(kr), to_bits(vr))
        k, v = hf_layout(B, H, 1, D, torch.bfloat16, gen), hf_layout(B, H, 1, D, torch.bfloat16, gen)
        got = pool.update(k.cuda(), v.cuda())
        oracle.append(to_bits(k), to_bits(v))
        assert pool.free_count == int(pool.ctrl[CTRL_FREE_TOP].item())
        assert pool.cold_free == int(pool.ctrl[CTRL_COLD_TOP].item())
        if step % 3 == 2 or step == steps - 1:
            ok, ov = oracle.current_tensors()
            assert np.array_equal(to_bits(got[0]), ok) and np.array_equal(to_bits(got[1]), ov), step
    assert np.array_equal(pool.cold_blocks, oracle.cold)
    assert pool.errors() == 0


def test_selection_larger_than_an_fp8_pool_on_gpu(hip):
    """batch_repeat_interleave past an fp8 pool's rows on the GPU: the layer moves to a grown pool
    that selects in place (quantised blocks shared, hot blocks copied) -- against the oracle, then
    decoding on."""
    from barqtrain_amd.kv_cache import BarqPagedKVCacheLayer
    from oracle.kv_quant_oracle import QuantLayerOracle

    H, D, P, W, cap = 8, 128, 16, 32, 320
    gen = torch.Generator().manual_seed(9)
    layer = BarqPagedKVCacheLayer(max_batch_size=2, max_cache_len=cap, page_size=P, kv_quant="fp8_e4m3",
                                  residual_window=W)
    oracle = QuantLayerOracle(2, cap, P, W, "bf16")
    k, v = hf_layout(2, H, 150, D, torch.bfloat16, gen) * 2, hf_layout(2, H, 150, D, torch.bfloat16, gen)
    layer.update(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    layer.batch_repeat_interleave(4)
    oracle.batch_repeat_interleave(4)
    assert layer.pool.max_batch >= 8 and layer.current_batch_size == 8
    for _ in range(20):
        k, v = hf_layout(8, H, 1, D, torch.bfloat16, gen), hf_layout(8, H, 1, D, torch.bfloat16, gen)
        gk, gv = layer.update(k.cuda(), v.cuda())
        oracle.append(to_bits(k), to_bits(v))
    ok, ov = oracle.current_tensors()
    assert np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov)
    assert layer.pool.errors() == 0


@pytest.mark.parametrize("D", [128, 64])
def test_decode_attention_on_quantised_pages_long_rows(hip, D):
    """Attention over a quantised pool whose rows pass one table window (the long-row pair kernel
    over cold blocks: 5,000 and 1,500 positions, 8 pairs), against the float64 reference over the
    dequantising gather's K/V."""
    from attn_ref import decode_attention_reference, within_tolerance
    from barqtrain_amd.paged import QuantPagePool

    H, P, W = 4, 16, 64
    lens = [5000, 1500]
    B, cap = len(lens), 5008
    pool = QuantPagePool(max_batch=B, max_blocks=cap // P, page_size=P, kv_heads=H, head_dim=D, dtype=torch.bfloat16,
                         device="cuda", window=W)
    gen = torch.Generator().manual_seed(91)
    done = 0
    for b in range(B, 0, -1):
        n = lens[b - 1] - done
        while n > 0:
            t = min(n, 1024)
            k, v = hf_layout(b, H, t, D, torch.bfloat16, gen) * 3, hf_layout(b, H, t, D, torch.bfloat16, gen)
            pool.append(k.cuda(), v.cuda())
            done += t
            n -= t
    assert int(pool.cold_blocks.max()) > 256
    kd, vd = (t.double().cpu().numpy() for t in pool.gather(B))
    for G in (4, 8):
        q = hf_layout(B, G * H, 1, D, torch.bfloat16, gen).cuda()
        want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, lens, D ** -0.5)
        got = pool.attend(q, out_dtype=torch.float32)
        ok, ratio = within_tolerance(got.double().cpu().numpy(), want, **ATT_F32)
        assert ok, f"G={G}: {ratio:.3g} x tolerance"
    assert pool.errors() == 0
