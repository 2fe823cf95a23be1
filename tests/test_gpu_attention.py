"""GPU parity of the paged decode-attention kernel (barq_kv_decode_attention) through the C ABI,
against the float64 reference over the oracle's gathered K/V (tests/attn_ref.py).

Tolerances: with float32 output, |out - ref| <= 2e-5 + 2e-5 |ref| (scores from exact bf16/fp16
products summed in fp32, fp32 softmax and P.V); with the cache's own 2-byte output, one rounding
of that value more: 2^-8 |ref| + 2e-5 for bf16, 2^-11 |ref| + 2e-5 for fp16.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from attn_ref import decode_attention_reference, within_tolerance
from capi_pool import CPool
from kvgen import hf_layout

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=2e-5, atol=2e-5)
OUT_TOL = {torch.bfloat16: dict(rtol=2.0**-8, atol=2e-5), torch.float16: dict(rtol=2.0**-11, atol=2e-5)}


def fill_pool(pool, kd, vd, lens, dtype):
    """Append each row's K/V: rows sorted by length, longest first, appended in rounds so each
    call appends `tokens` to rows [0, batch)."""
    B = len(lens)
    order = np.argsort(-np.asarray(lens), kind="stable")
    assert list(order) == list(range(B)), "rows must be given longest first"
    cur = 0
    while True:
        active = [b for b in range(B) if lens[b] > cur]
        if not active:
            break
        batch = len(active)
        nxt = min(lens[b] for b in active)
        k = torch.from_numpy(np.ascontiguousarray(kd[:batch, :, cur:nxt])).to(dtype).cuda()
        v = torch.from_numpy(np.ascontiguousarray(vd[:batch, :, cur:nxt])).to(dtype).cuda()
        pool.append(k, v)
        cur = nxt


def make_rows(B, Hkv, page, lens, dtype, seed, order_seed=None, cap=None, D=128):
    lens = sorted((int(x) for x in lens), reverse=True)
    cap = cap or max(max(lens), 1)
    gen = torch.Generator().manual_seed(seed)
    max_blocks = -(-cap // page)
    order = None
    n_pages = B * max_blocks
    if order_seed is not None:
        order = torch.from_numpy(np.random.default_rng(order_seed).permutation(n_pages).astype(np.int32))
    pool = CPool(max_batch=B, max_blocks=max_blocks, page_size=page, heads=Hkv, dim=D, dtype=dtype,
                 num_pages=n_pages, order=order)
    kd = torch.randn(B, Hkv, cap, D, generator=gen).to(dtype).double().numpy()
    vd = torch.randn(B, Hkv, cap, D, generator=gen).to(dtype).double().numpy()
    fill_pool(pool, kd, vd, lens, dtype)
    torch.cuda.synchronize()
    assert pool.errors() == 0
    return pool, kd, vd, lens


def check(pool, kd, vd, lens, G, T, dtype, seed, out_f32=True, split_tokens=0, max_seq=0, ws=None,
          scale=None, tol=None):
    B, Hkv, D = kd.shape[0], kd.shape[1], kd.shape[3]
    gen = torch.Generator().manual_seed(seed)
    q = hf_layout(B, G * Hkv, T, D, dtype, gen).cuda()
    scale = D ** -0.5 if scale is None else scale
    out, ws = pool.attend(q, scale=scale, out_f32=out_f32, split_tokens=split_tokens, max_seq=max_seq,
                          workspace=ws)
    torch.cuda.synchronize()
    want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, lens, scale)
    got = out.double().cpu().numpy()
    tol = tol or (F32_TOL if out_f32 else OUT_TOL[dtype])
    ok, ratio = within_tolerance(got, want, **tol)
    assert ok, f"G={G} T={T} lens={list(lens)[:8]} split={split_tokens}: error {ratio:.3g} x tolerance"
    return ws


@pytest.mark.parametrize("dtype,page", [(torch.bfloat16, 16), (torch.float16, 16), (torch.bfloat16, 32),
                                        (torch.float16, 32), (torch.bfloat16, 8), (torch.float16, 5),
                                        (torch.bfloat16, 1)])
def test_ragged_rows_gqa(dtype, page):
    """Ragged rows (1 .. 1100 positions, chunk, split and page boundaries on both sides), a
    random page order, grouped-query factors 1 / 4 / 8 / 16, one to five splits per row."""
    lens = [1100, 1025, 769, 513, 300, 257, 256, 255, 129, 64, 63, 17, 16, 1]
    pool, kd, vd, lens = make_rows(len(lens), 2, page, lens, dtype, seed=page, order_seed=page + 1)
    ws = None
    for i, (G, split) in enumerate([(4, 0), (1, 256), (8, 512), (16, 256), (4, 768)]):
        ws = check(pool, kd, vd, lens, G, 1, dtype, seed=100 + i, split_tokens=split, ws=ws)
    check(pool, kd, vd, lens, 4, 1, dtype, seed=7, out_f32=False)
    assert pool.errors() == 0


@pytest.mark.parametrize("G,T", [(4, 2), (4, 4), (2, 8), (1, 16), (8, 2)])
def test_multi_token_queries_causal(G, T):
    """T query tokens at the end of each row: token i sees positions up to len - T + i."""
    lens = [600, 200, 70, 64, 33, T]
    pool, kd, vd, lens = make_rows(len(lens), 2, 16, lens, torch.bfloat16, seed=G * T, order_seed=3)
    check(pool, kd, vd, lens, G, T, torch.bfloat16, seed=1, split_tokens=256)
    check(pool, kd, vd, lens, G, T, torch.bfloat16, seed=2)


@pytest.mark.parametrize("dtype,page", [(torch.bfloat16, 16), (torch.float16, 32), (torch.bfloat16, 5),
                                        (torch.float16, 1)])
def test_head_dim_64(dtype, page):
    """Head size 64 (Qwen2-0.5B: 14 query heads over 2 kv heads, G = 7): ragged rows with a random
    page order, G = 7 / 1 / 4 / 16, multi-token queries, fixed and automatic splits, both output
    types, and one long row whose pairs the merge launch folds from hundreds of records."""
    lens = [1100, 769, 513, 257, 256, 255, 64, 17, 16, 1, 0]
    pool, kd, vd, lens = make_rows(len(lens), 2, page, lens, dtype, seed=page + 64, order_seed=page + 65, D=64)
    ws = None
    for i, (G, T, split) in enumerate([(7, 1, 0), (1, 1, 256), (4, 1, 48), (16, 1, 0), (7, 2, 512), (2, 8, 0)]):
        ws = check(pool, kd, vd, lens, G, T, dtype, seed=300 + i, split_tokens=split, ws=ws)
    check(pool, kd, vd, lens, 7, 1, dtype, seed=9, out_f32=False)
    assert pool.errors() == 0
    pool, kd, vd, lens = make_rows(1, 2, page, [9001], dtype, seed=page + 66, order_seed=page + 67, D=64)
    check(pool, kd, vd, lens, 7, 1, dtype, seed=10)
    check(pool, kd, vd, lens, 7, 1, dtype, seed=11, out_f32=False)
    assert pool.errors() == 0


@pytest.mark.parametrize("dtype,page", [(torch.bfloat16, 16), (torch.float16, 32), (torch.bfloat16, 5)])
def test_head_dim_256(dtype, page):
    """Head size 256 (Gemma: 8 query heads over 1 kv head, or 16 over 8 -- G = 8 / 2 here) on
    two-byte pages, through the flat schedule at one wave per SIMD: ragged rows with a random page
    order (16-position chunks, pages of 16, 32 and 5), G = 8 / 2 / 4 / 16, two query tokens,
    fixed and automatic splits, both output types, and a long row folded from many records."""
    lens = [1100, 513, 257, 256, 255, 64, 17, 16, 1, 0]
    pool, kd, vd, lens = make_rows(len(lens), 2, page, lens, dtype, seed=page + 256, order_seed=page + 257, D=256)
    ws = None
    for i, (G, T, split) in enumerate([(8, 1, 0), (2, 1, 256), (4, 2, 48), (16, 1, 0), (8, 2, 0)]):
        ws = check(pool, kd, vd, lens, G, T, dtype, seed=900 + i, split_tokens=split, ws=ws)
    check(pool, kd, vd, lens, 8, 1, dtype, seed=9, out_f32=False)
    assert pool.errors() == 0
    pool, kd, vd, lens = make_rows(1, 2, page, [6001], dtype, seed=page + 258, order_seed=page + 259, D=256)
    check(pool, kd, vd, lens, 8, 1, dtype, seed=10)
    check(pool, kd, vd, lens, 2, 1, dtype, seed=11, out_f32=False)
    assert pool.errors() == 0


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64)])
def test_five_to_eight_rows_on_two_workgroups_a_pair(dtype, D):
    """5 to 8 query rows over 128 pairs of rows of 45 to 64 chunks: two workgroups a pair (the
    bound of up to 4 rows), ragged rows with empty, one-position and chunk-boundary lengths, one
    and two query tokens, both output types."""
    rng = np.random.default_rng(64 + D)
    lens = [1024, 1023, 1009, 720, 705, 704, 0, 1, 17] + rng.integers(0, 1025, size=23).tolist()
    pool, kd, vd, lens = make_rows(len(lens), 4, 16, lens, dtype, seed=640 + D, order_seed=641 + D, D=D)
    ws = None
    for i, (G, T) in enumerate([(8, 1), (5, 1), (3, 2), (4, 2)]):
        ws = check(pool, kd, vd, lens, G, T, dtype, seed=700 + i, ws=ws)
    check(pool, kd, vd, lens, 8, 1, dtype, seed=9, out_f32=False)
    assert pool.errors() == 0


@pytest.mark.parametrize("dtype,page,D", [(torch.bfloat16, 16, 128), (torch.float16, 32, 128), (torch.bfloat16, 16, 64)])
def test_many_short_pairs_one_launch(dtype, page, D):
    """128+ (row, kv head) pairs of at most 704 positions with the automatic split take one
    workgroup per pair that merges its waves' partials in LDS (one launch): ragged rows with
    empty, one-position and chunk-boundary lengths, G = 1 / 2 / 4 / 8, two query tokens, both
    output types; the flat schedule (a fixed split) over the same pool agrees."""
    rng = np.random.default_rng(page + D)
    lens = [700, 0, 1, 15, 16, 17, 31, 33] + rng.integers(0, 700, size=32).tolist()
    pool, kd, vd, lens = make_rows(len(lens), 4, page, lens, dtype, seed=page * 3 + D, order_seed=page + D, D=D)
    ws = None
    for i, (G, T) in enumerate([(4, 1), (1, 1), (8, 1), (2, 2), (4, 2)]):
        ws = check(pool, kd, vd, lens, G, T, dtype, seed=400 + i, ws=ws)
    check(pool, kd, vd, lens, 4, 1, dtype, seed=9, out_f32=False)
    check(pool, kd, vd, lens, 4, 1, dtype, seed=9, split_tokens=64)  # the flat schedule
    assert pool.errors() == 0


@pytest.mark.parametrize("rows,Hkv,cap,dtype,D,page", [(32, 4, 1024, torch.bfloat16, 128, 16),
                                                       (32, 8, 2048, torch.float16, 128, 16),
                                                       (16, 8, 1024, torch.bfloat16, 64, 16),
                                                       (32, 4, 1024, torch.float16, 128, 32),
                                                       (16, 8, 1024, torch.bfloat16, 128, 64)])
def test_long_pairs_one_launch(rows, Hkv, cap, dtype, D, page):
    """Up to 4 query rows take the one-launch pair kernel for longer rows: 128 pairs of up to 1024
    positions, 256 pairs of up to 2048, pages of 16, 32 and 64 positions.  Its loop loads the next
    chunk on every path, a partial last chunk with its positions past the row's end clamped to the
    last one, so lengths sit on and next to chunk boundaries (empty, 1, 15 .. 33, cap - 17 ..
    cap); G = 4 / 1 / 2, two tokens x 2 heads, the 2-byte output; the flat schedule (a fixed
    split) over the same pool agrees."""
    rng = np.random.default_rng(cap + D)
    edges = [cap, cap - 1, cap - 15, cap - 16, cap - 17, 0, 1, 15, 16, 17, 31, 32, 33]
    lens = edges + rng.integers(0, cap + 1, size=rows - len(edges)).tolist()
    pool, kd, vd, lens = make_rows(rows, Hkv, page, lens, dtype, seed=cap + 7, order_seed=cap + 8, D=D)
    ws = None
    for i, (G, T) in enumerate([(4, 1), (1, 1), (2, 2), (2, 1)]):
        ws = check(pool, kd, vd, lens, G, T, dtype, seed=500 + i, ws=ws)
    check(pool, kd, vd, lens, 4, 1, dtype, seed=9, out_f32=False)
    check(pool, kd, vd, lens, 4, 1, dtype, seed=9, split_tokens=256)  # the flat schedule
    assert pool.errors() == 0


def pair_words(pool, pairs):
    """The split pairs' arrival counts (BARQ_KV_CTRL_PAIR_WORD of include/barq_kv.h)."""
    idx = [64 + (q // 32) * 64 + 32 + q % 32 for q in range(pairs)]
    return pool.ctrl.cpu().numpy()[idx]


@pytest.mark.parametrize("dtype,D,G", [(torch.bfloat16, 128, 4), (torch.float16, 128, 8), (torch.bfloat16, 64, 2)])
def test_split_pairs_same_bits_every_call(dtype, D, G):
    """128 (row, kv head) pairs on 256 CUs: two workgroups a pair, each folding its waves in LDS;
    the second to arrive folds both halves' records into the output.  Rows from 22 chunks (337
    positions) are split with up to 4 query rows, from 28 (433) with 8, shorter ones taken by
    one workgroup, in the same launch (lengths on both sides of those bounds and of chunk
    boundaries).  Against the float64 reference; three
    calls in a row give the same bits (the fold does not depend on which half arrives second)
    and leave every pair's arrival count at 0; the flat schedule agrees."""
    rng = np.random.default_rng(D + G)
    lens = [704, 703, 433, 432, 337, 336, 385, 0, 1, 17] + rng.integers(0, 705, size=6).tolist()
    pool, kd, vd, lens = make_rows(16, 8, 16, lens, dtype, seed=D + G, order_seed=D + G + 1, D=D, cap=704)
    q = hf_layout(16, G * 8, 1, D, dtype, torch.Generator().manual_seed(G)).cuda()
    outs = []
    ws = None
    for _ in range(3):
        out, ws = pool.attend(q, out_f32=True, workspace=ws)
        torch.cuda.synchronize()
        outs.append(out.double().cpu().numpy())
        assert not pair_words(pool, 128).any()
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, lens, D ** -0.5)
    ok, ratio = within_tolerance(outs[0], want, **F32_TOL)
    assert ok, f"{ratio:.3g} x tolerance"
    check(pool, kd, vd, lens, G, 1, dtype, seed=5, out_f32=False)
    check(pool, kd, vd, lens, G, 1, dtype, seed=6, split_tokens=64)  # the flat schedule
    assert pool.errors() == 0


@pytest.mark.parametrize("B,Hkv,D", [(1, 8, 128), (3, 8, 128), (2, 2, 64)])
def test_few_pairs_one_launch(B, Hkv, D):
    """Fewer than 128 (row, kv head) pairs -- batch-1 decode -- take the one-launch pair kernel
    with up to 8 workgroups a pair (each at least 11 chunks of the row, 14 with 8 query rows): rows of up to 704
    positions on and next to chunk boundaries, G = 4 / 8 / 1, two query tokens, both output
    types; a row past the pair kernels' reach (36,865 positions, over 32 x 72 chunks) takes the flat
    schedule, which agrees."""
    rng = np.random.default_rng(B * 10 + D)
    lens = sorted([704, 17, 1][:B] + rng.integers(1, 705, size=max(B - 3, 0)).tolist(), reverse=True)
    pool, kd, vd, lens = make_rows(B, Hkv, 16, lens, torch.bfloat16, seed=B + D, order_seed=B + D + 1, D=D,
                                   cap=704)
    ws = None
    for i, (G, T) in enumerate([(4, 1), (8, 1), (1, 1), (2, 2)]):
        ws = check(pool, kd, vd, lens, G, T, torch.bfloat16, seed=800 + i, ws=ws)
    check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=9, out_f32=False)
    assert pool.errors() == 0
    pool, kd, vd, lens = make_rows(1, 2, 16, [36865], torch.bfloat16, seed=B + D + 2, order_seed=B + D + 3, D=D)
    check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=11)
    assert pool.errors() == 0


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64)])
def test_small_batch_pairs_over_many_workgroups(dtype, D):
    """8 (row, kv head) pairs on 256 CUs: up to 8 workgroups a pair (the grid's count), a row cut
    over as many as give each 11 chunks (14 with 8 query rows) -- with 4 rows 3072 positions over
    8, 1537 over 8, 385 over 2, 191 alone -- and the last to arrive folding the parts' records in
    their order.  Rows up to 3072
    positions take this one launch (the flat schedule before).  G = 4 / 8, two query tokens,
    against the float64 reference; three calls give the same bits and leave every arrival count
    at 0; the flat schedule agrees."""
    pool, kd, vd, lens = make_rows(4, 2, 16, [3072, 1537, 385, 191], dtype, seed=D, order_seed=D + 1, D=D)
    for i, (G, T) in enumerate([(4, 1), (8, 1), (2, 2)]):
        q = hf_layout(4, G * 2, T, D, dtype, torch.Generator().manual_seed(30 + i)).cuda()
        outs = []
        for _ in range(3):
            out, _ = pool.attend(q, out_f32=True)
            torch.cuda.synchronize()
            outs.append(out.double().cpu().numpy())
            assert not pair_words(pool, 8).any()
        assert all(np.array_equal(outs[0], o) for o in outs[1:])
        want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, lens, D ** -0.5)
        ok, ratio = within_tolerance(outs[0], want, **F32_TOL)
        assert ok, f"G={G} T={T}: {ratio:.3g} x tolerance"
    check(pool, kd, vd, lens, 4, 1, dtype, seed=7, out_f32=False)
    check(pool, kd, vd, lens, 4, 1, dtype, seed=8, split_tokens=256)  # the flat schedule
    assert pool.errors() == 0


@pytest.mark.parametrize("pattern", ["rising", "falling", "spikes"])
def test_running_maximum_moves_between_chunks(pattern):
    """Score ranges that move between chunks (up to 4 query rows, and 8 in the pair kernel, move
    the running maximum only when a score exceeds it by 2^8): keys scaled per position so that the scores of each of
    the first chunks pass the last maximum by more than that (a rescale at each), fall (none
    after the first), or spike at a few positions; 128 and 8 pairs (the pair kernel), and the
    flat schedule (a fixed split) over the 8, G = 4 and 8, one and two query tokens, both output
    types.  Scores reach ~25 here,
    whose fp32 sums carry ~1e-5 absolute error into the weights, so the float32 check allows
    1e-4 (a missed rescale is off by a factor of 2^8 or more)."""
    D, cap, page = 128, 704, 16
    for B, Hkv in ((32, 4), (4, 2)):
        rng = np.random.default_rng(len(pattern) * 100 + B)
        lens = sorted([cap, 1, 17, 255] + rng.integers(1, cap, size=B - 4).tolist(), reverse=True)
        gen = torch.Generator().manual_seed(B + 5)
        k = torch.randn(B, Hkv, cap, D, generator=gen)
        v = torch.randn(B, Hkv, cap, D, generator=gen)
        pos = torch.arange(cap, dtype=torch.float32)
        if pattern == "rising":  # +2.2 a chunk on the scores' spread: > 8 (log2) on the maximum
            f = 1 + 2.2 * torch.clamp(pos / 16, max=4.0)
        elif pattern == "falling":
            f = 1 + 2.2 * torch.clamp((cap - pos) / 16, max=4.0)
        else:
            f = torch.ones(cap)
            f[torch.from_numpy(rng.choice(cap, size=12, replace=False))] = 10.0
        k = k * f[None, None, :, None]
        kd = k.to(torch.bfloat16).double().numpy()
        vd = v.to(torch.bfloat16).double().numpy()
        order = torch.from_numpy(rng.permutation(B * (cap // page)).astype(np.int32))
        pool = CPool(max_batch=B, max_blocks=cap // page, page_size=page, heads=Hkv, dim=D, dtype=torch.bfloat16,
                     num_pages=B * (cap // page), order=order)
        fill_pool(pool, kd, vd, lens, torch.bfloat16)
        torch.cuda.synchronize()
        for i, (G, T) in enumerate([(4, 1), (2, 2), (8, 1)]):
            check(pool, kd, vd, lens, G, T, torch.bfloat16, seed=700 + i, tol=dict(rtol=1e-4, atol=1e-4))
        check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=9, out_f32=False)
        if B * Hkv < 128:
            check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=10, split_tokens=64, tol=dict(rtol=1e-4, atol=1e-4))
        assert pool.errors() == 0


def test_flat_schedule_with_ranges_of_two_sizes():
    """16 ragged rows of ~4200 positions over 8 kv heads (over 32k chunks: the automatic split's
    ranges hold 16+ chunks, so the first half of the waves take larger ones), G = 4 and 8; a
    fixed split over the same pool agrees."""
    rng = np.random.default_rng(4242)
    lens = sorted(rng.integers(4100, 4300, size=16).tolist(), reverse=True)
    assert sum(-(-x // 16) for x in lens) * 8 >= 16 * 2048
    pool, kd, vd, lens = make_rows(16, 8, 16, lens, torch.bfloat16, seed=4243, order_seed=4244)
    ws = check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=1)
    ws = check(pool, kd, vd, lens, 8, 1, torch.bfloat16, seed=2, ws=ws)
    check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=3, split_tokens=512)
    assert pool.errors() == 0


def test_llama3_8b_decode_shape():
    """The benchmark's C2 shape: 16 rows x 8 kv heads x 32 q heads, 513 positions, page 16."""
    lens = [513] * 16
    pool, kd, vd, lens = make_rows(16, 8, 16, lens, torch.bfloat16, seed=2002, order_seed=5, cap=768)
    check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=3, max_seq=513)
    check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=4, out_f32=False)


def test_long_row_many_records():
    """One long row (12,001 positions) over 2 kv heads: up to 8 query rows take the long-row pair
    kernel (16 workgroups a pair, each part's table window its own); 16 query rows and a fixed
    split take the flat schedule, whose many records a pair the merge launch folds with its wide
    workgroups (fewer merge workgroups than CUs)."""
    lens = [12001]
    pool, kd, vd, lens = make_rows(1, 2, 16, lens, torch.bfloat16, seed=77, order_seed=8)
    check(pool, kd, vd, lens, 4, 1, torch.bfloat16, seed=5)
    check(pool, kd, vd, lens, 2, 3, torch.bfloat16, seed=6, out_f32=False)
    check(pool, kd, vd, lens, 16, 1, torch.bfloat16, seed=7)    # 16 query rows per kv head
    check(pool, kd, vd, lens, 8, 2, torch.bfloat16, seed=8, split_tokens=48)  # fixed short ranges


def test_empty_rows_and_closed_forms():
    """A row of length 0 (and one shorter than T) gives zeros; equal V rows give that row; a zero
    query gives the mean of V."""
    D = 128
    lens = [40, 3, 0]
    pool, kd, vd, lens = make_rows(3, 1, 16, lens, torch.bfloat16, seed=9)
    gen = torch.Generator().manual_seed(1)
    q = hf_layout(3, 4, 4, D, torch.bfloat16, gen).cuda()
    out, _ = pool.attend(q, out_f32=True)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    assert np.all(got[2] == 0), "empty row"
    assert np.all(got[1, :, 0] == 0) and np.any(got[1, :, 1] != 0), "row 1 (3 positions, T=4): token 0 sees none"
    want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, lens, D ** -0.5)
    assert within_tolerance(got, want, **F32_TOL)[0]

    same = CPool(max_batch=1, max_blocks=4, page_size=16, heads=1, dim=D, dtype=torch.bfloat16)
    row = torch.randn(1, 1, 1, D, generator=gen).to(torch.bfloat16)
    same.append(row.expand(1, 1, 50, D).contiguous().cuda(), row.expand(1, 1, 50, D).contiguous().cuda())
    q = hf_layout(1, 8, 1, D, torch.bfloat16, gen).cuda() * 4
    out, _ = same.attend(q, out_f32=True)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out[0, :, 0].cpu().numpy(), row[0, 0].float().expand(8, D).numpy(), rtol=2e-6)

    zq = torch.zeros(1, 8, 1, D, dtype=torch.bfloat16, device="cuda")
    gk = torch.randn(1, 1, 50, D, generator=gen).to(torch.bfloat16)
    gv = torch.randn(1, 1, 50, D, generator=gen).to(torch.bfloat16)
    mean = CPool(max_batch=1, max_blocks=4, page_size=16, heads=1, dim=D, dtype=torch.bfloat16)
    mean.append(gk.cuda(), gv.cuda())
    out, _ = mean.attend(zq, out_f32=True)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out[0, 0, 0].cpu().numpy(), gv[0, 0].double().mean(0).numpy(), rtol=1e-5, atol=1e-6)


def test_short_max_seq_is_flagged():
    """max_seq 64 sizes the launch to one 256-position split; a 600-position row is flagged."""
    lens = [600, 50]
    pool, kd, vd, lens = make_rows(2, 2, 16, lens, torch.bfloat16, seed=4)
    gen = torch.Generator().manual_seed(0)
    q = hf_layout(2, 8, 1, 128, torch.bfloat16, gen).cuda()
    pool.attend(q, out_f32=True, max_seq=64)
    torch.cuda.synchronize()
    assert pool.errors() & 16, "ATTN_SHORT bit"


def test_page_pool_attend_and_graph_replays(hip):
    """PagePool.attend through the torch binding, then a captured graph of append + attend over
    3 layers replayed while rows grow: every replay against the reference."""
    from barqtrain_amd.paged import PagePool

    L, B, Hkv, G, D, P, prefill, steps = 3, 4, 2, 4, 128, 16, 60, 12
    cap = prefill + steps
    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(11)
    pools = [PagePool(max_batch=B, max_blocks=-(-cap // P), page_size=P, kv_heads=Hkv, head_dim=D,
                      dtype=torch.bfloat16, device=dev) for _ in range(L)]
    dense_k = np.zeros((L, B, Hkv, cap, D))
    dense_v = np.zeros((L, B, Hkv, cap, D))
    for li, pool in enumerate(pools):
        k = hf_layout(B, Hkv, prefill, D, torch.bfloat16, gen)
        v = hf_layout(B, Hkv, prefill, D, torch.bfloat16, gen)
        pool.append(k.to(dev), v.to(dev))
        dense_k[li, :, :, :prefill] = k.double().numpy()
        dense_v[li, :, :, :prefill] = v.double().numpy()
    q = hf_layout(B, G * Hkv, 1, D, torch.bfloat16, gen).to(dev)
    out = pools[0].attend(q, out_dtype=torch.float32)
    torch.cuda.synchronize()
    want = decode_attention_reference(q.double().cpu().numpy(), dense_k[0], dense_v[0], [prefill] * B, D ** -0.5)
    assert within_tolerance(out.double().cpu().numpy(), want, **F32_TOL)[0]

    kin = torch.zeros((L, B, Hkv, 1, D), dtype=torch.bfloat16, device=dev)
    vin = torch.zeros_like(kin)
    qin = torch.zeros((L, B, G * Hkv, 1, D), dtype=torch.bfloat16, device=dev)
    outs = [torch.zeros((B, 1, G * Hkv, D), dtype=torch.float32, device=dev).transpose(1, 2) for _ in range(L)]
    for pool in pools:  # workspaces sized for the capacity before capture
        pool.attention_workspace(hip.attention_workspace_bytes(pool.tensors, B, G * Hkv, 1, cap, 0))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for li, pool in enumerate(pools):
            hip.pool_append_(pool.tensors, kin[li], vin[li])
            hip.pool_decode_attention(pool.tensors, qin[li], outs[li], D ** -0.5, cap, 0,
                                      pool.attention_workspace(0))
    for s in range(steps):
        ks = [hf_layout(B, Hkv, 1, D, torch.bfloat16, gen) for _ in range(L)]
        vs = [hf_layout(B, Hkv, 1, D, torch.bfloat16, gen) for _ in range(L)]
        qs = [hf_layout(B, G * Hkv, 1, D, torch.bfloat16, gen) for _ in range(L)]
        for li in range(L):
            kin[li].copy_(ks[li].to(dev))
            vin[li].copy_(vs[li].to(dev))
            qin[li].copy_(qs[li].to(dev))
            dense_k[li, :, :, prefill + s] = ks[li][:, :, 0].double().numpy()
            dense_v[li, :, :, prefill + s] = vs[li][:, :, 0].double().numpy()
        _ = torch.randn(1 << 18, device=dev).sum().item()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        n = prefill + s + 1
        for li in range(L):
            want = decode_attention_reference(qs[li].double().numpy(), dense_k[li], dense_v[li], [n] * B, D ** -0.5)
            ok, ratio = within_tolerance(outs[li].double().cpu().numpy(), want, **F32_TOL)
            assert ok, f"replay {s} layer {li}: {ratio:.3g} x tolerance"
    assert all(p.errors() == 0 for p in pools)


@pytest.mark.parametrize("B,Hkv,prefill", [(16, 8, 400), (2, 4, 700)])
def test_split_pairs_in_graph_replays(hip, B, Hkv, prefill):
    """Split pairs under graph capture: append + attend over 2 layers captured once (128 pairs:
    two workgroups a pair; 8 pairs: up to 8), replayed while the rows grow, with eager work
    between replays; every replay against the reference, and every pair's arrival count back at
    0 after it (the last arrival resets it inside the launch: nothing in the graph clears it)."""
    from barqtrain_amd.paged import PagePool

    L, G, D, P, steps = 2, 4, 128, 16, 5
    cap = prefill + steps
    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(B + prefill)
    pools = [PagePool(max_batch=B, max_blocks=-(-cap // P), page_size=P, kv_heads=Hkv, head_dim=D,
                      dtype=torch.bfloat16, device=dev) for _ in range(L)]
    dense_k = np.zeros((L, B, Hkv, cap, D))
    dense_v = np.zeros((L, B, Hkv, cap, D))
    for li, pool in enumerate(pools):
        k = hf_layout(B, Hkv, prefill, D, torch.bfloat16, gen)
        v = hf_layout(B, Hkv, prefill, D, torch.bfloat16, gen)
        pool.append(k.to(dev), v.to(dev))
        dense_k[li, :, :, :prefill] = k.double().numpy()
        dense_v[li, :, :, :prefill] = v.double().numpy()
    kin = torch.zeros((L, B, Hkv, 1, D), dtype=torch.bfloat16, device=dev)
    vin = torch.zeros_like(kin)
    qin = torch.zeros((L, B, G * Hkv, 1, D), dtype=torch.bfloat16, device=dev)
    outs = [torch.zeros((B, 1, G * Hkv, D), dtype=torch.float32, device=dev).transpose(1, 2) for _ in range(L)]
    for pool in pools:
        pool.attention_workspace(hip.attention_workspace_bytes(pool.tensors, B, G * Hkv, 1, cap, 0))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for li, pool in enumerate(pools):
            hip.pool_append_(pool.tensors, kin[li], vin[li])
            hip.pool_decode_attention(pool.tensors, qin[li], outs[li], D ** -0.5, cap, 0,
                                      pool.attention_workspace(0))
    for s in range(steps):
        ks = [hf_layout(B, Hkv, 1, D, torch.bfloat16, gen) for _ in range(L)]
        vs = [hf_layout(B, Hkv, 1, D, torch.bfloat16, gen) for _ in range(L)]
        qs = [hf_layout(B, G * Hkv, 1, D, torch.bfloat16, gen) for _ in range(L)]
        for li in range(L):
            kin[li].copy_(ks[li].to(dev))
            vin[li].copy_(vs[li].to(dev))
            qin[li].copy_(qs[li].to(dev))
            dense_k[li, :, :, prefill + s] = ks[li][:, :, 0].double().numpy()
            dense_v[li, :, :, prefill + s] = vs[li][:, :, 0].double().numpy()
        _ = torch.randn(1 << 18, device=dev).sum().item()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        n = prefill + s + 1
        for li in range(L):
            want = decode_attention_reference(qs[li].double().numpy(), dense_k[li], dense_v[li], [n] * B, D ** -0.5)
            ok, ratio = within_tolerance(outs[li].double().cpu().numpy(), want, **F32_TOL)
            assert ok, f"replay {s} layer {li}: {ratio:.3g} x tolerance"
            assert not pair_words(pools[li], B * Hkv).any()
    assert all(p.errors() == 0 for p in pools)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64)])
def test_long_rows_over_many_workgroups(dtype, D):
    """Rows longer than one table window (256 blocks) at a small batch: the long-row pair kernel,
    up to 32 workgroups a pair.  8,192 positions: 16 contiguous parts of 32 chunks, those past block
    256 loading their own window; 3,001 positions in the same launch: 8 parts dealt in turn from
    the prologue's window.  G = 4 / 8, two query tokens, both output types, against the float64
    reference; three calls give the same bits and leave every arrival count at 0; the flat
    schedule agrees."""
    pool, kd, vd, lens = make_rows(2, 4, 16, [8192, 3001], dtype, seed=D + 3, order_seed=D + 4, D=D)
    for i, (G, T) in enumerate([(4, 1), (8, 1), (2, 2)]):
        q = hf_layout(2, G * 4, T, D, dtype, torch.Generator().manual_seed(60 + i)).cuda()
        outs = []
        for _ in range(3):
            out, _ = pool.attend(q, out_f32=True)
            torch.cuda.synchronize()
            outs.append(out.double().cpu().numpy())
            assert not pair_words(pool, 8).any()
        assert all(np.array_equal(outs[0], o) for o in outs[1:])
        want = decode_attention_reference(q.double().cpu().numpy(), kd, vd, lens, D ** -0.5)
        ok, ratio = within_tolerance(outs[0], want, **F32_TOL)
        assert ok, f"G={G} T={T}: {ratio:.3g} x tolerance"
    check(pool, kd, vd, lens, 4, 1, dtype, seed=9, out_f32=False)
    check(pool, kd, vd, lens, 4, 1, dtype, seed=10, split_tokens=256)  # the flat schedule
    assert pool.errors() == 0
