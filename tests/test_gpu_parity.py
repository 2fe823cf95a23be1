"""GPU parity of the gfx950 kernels, called through the C ABI, against the CPU oracle.

Bit-exact: every output is compared as raw element bits (np.array_equal), no tolerance.
Shapes: the five benchmark configurations at their real per-layer shapes (layers are
independent pools, so a subset of layers is run), plus edge cases of the reference's semantics.
"""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest
import torch

from capi_pool import SEPARATE_FINALIZE, SEQ_FROM_DEVICE, CPool
from kvgen import C1, config1_steps, hf_layout, normal, to_bits
from mirror import DeviceMirror
from oracle.kv_oracle import DenseLayerOracle, dense_append_reference

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def assert_bits_equal(got: torch.Tensor, want: np.ndarray, what=""):
    g = to_bits(got)
    assert g.shape == want.shape, (what, g.shape, want.shape)
    if not np.array_equal(g, want):
        bad = np.argwhere(g != want)
        raise AssertionError(f"{what}: {len(bad)} elements differ, first at {bad[0].tolist()}")


def make_pool(oracle_cap, batch, heads, dim, page, dtype, **kw):
    mb = -(-oracle_cap // page)
    return CPool(max_batch=batch, max_blocks=mb, page_size=page, heads=heads, dim=dim, dtype=dtype, **kw)


def compare_layer(pool: CPool, oracle: DenseLayerOracle, got=None, what=""):
    """The pool's gather of the current batch equals the oracle's materialised current_tensors."""
    ok, ov = oracle.current_tensors()
    if got is None:
        got = pool.gather(ok.shape[0], ok.shape[2])
    assert_bits_equal(got[0], ok, what + " K")
    assert_bits_equal(got[1], ov, what + " V")


# --------------------------------------------------------------------------- reference drop-in
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_dense_append_matches_reference_kernel(capi, dtype):
    """barq_kv_append_dense vs the restated paged_kv_append_cuda, HF-strided inputs."""
    gen = torch.Generator().manual_seed(7)
    B_cache, H, MB, P, D = 3, 4, 6, 8, 64
    kc = torch.zeros((B_cache, H, MB, P, D), dtype=dtype, device="cuda")
    vc = torch.zeros_like(kc)
    lens = torch.zeros(B_cache, dtype=torch.int32, device="cuda")
    okc, ovc = to_bits(kc), to_bits(vc)
    olens = np.zeros(B_cache, dtype=np.int64)
    stream = torch.cuda.current_stream().cuda_stream
    for b, t in [(3, 13), (2, 1), (3, 1), (1, 20), (3, 5)]:
        k = hf_layout(b, H, t, D, dtype, gen)
        v = hf_layout(b, H, t, D, dtype, gen)
        dense_append_reference(okc, ovc, olens, to_bits(k), to_bits(v))
        kd, vd = k.cuda(), v.cuda()
        rc = capi.barq_kv_append_dense(kc.data_ptr(), vc.data_ptr(), lens.data_ptr(), kd.data_ptr(),
                                       vd.data_ptr(), b, H, t, D, B_cache, MB, P, kd.element_size(),
                                       kd.stride(0), kd.stride(1), kd.stride(2), stream)
        assert rc == 0
        assert_bits_equal(kc, okc, "dense K")
        assert_bits_equal(vc, ovc, "dense V")
        assert lens.cpu().numpy().tolist() == olens.tolist()


def test_dense_binding_error_and_int64_lens(hip):
    """The torch binding keeps the reference's checks: capacity RuntimeError before any write,
    int64 seq_lens converted and incremented in place."""
    kc = torch.zeros((1, 2, 2, 4, 8), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    lens = torch.tensor([6], dtype=torch.int64, device="cuda")
    k = torch.ones((1, 2, 3, 8), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="requested 9 tokens, max_cache_len=8"):
        hip.paged_kv_append_(kc, vc, lens, k, k)
    assert not kc.any() and lens.item() == 6
    hip.paged_kv_append_(kc, vc, lens, k[:, :, :2], k[:, :, :2])
    assert lens.item() == 8 and lens.dtype == torch.int64
    assert kc[0, :, 1, 2:, :].eq(1).all() and not kc[0, :, 1, :2, :].any()


# --------------------------------------------------------------------------- configurations
def run_c1(flags):
    cap = C1["prefill"] + C1["decode"]
    pools = [make_pool(cap, C1["batch"], C1["heads"], C1["dim"], C1["page"], C1["dtype"]) for _ in range(C1["layers"])]
    with open(os.path.join(GOLDEN, "config1_digests.json")) as f:
        digests = json.load(f)["layers"]
    oracles = [DenseLayerOracle(C1["batch"], cap, C1["page"]) for _ in pools]
    for step, layers in enumerate(config1_steps()):
        for li, (k, v) in enumerate(layers):
            seq = oracles[li].get_seq_length() + k.shape[2]
            got = pools[li].update(k.cuda(), v.cuda(), seq, flags)
            ok, ov = oracles[li].update(to_bits(k), to_bits(v))
            assert_bits_equal(got[0], ok, f"C1 layer {li} step {step} K")
            assert_bits_equal(got[1], ov, f"C1 layer {li} step {step} V")
            h = hashlib.sha256(to_bits(got[0]).tobytes() + to_bits(got[1]).tobytes()).hexdigest()[:16]
            assert h == digests[li][step]
    for p in pools:
        p.check_invariants()
        assert p.errors() == 0


@pytest.mark.parametrize("flags", [0, SEPARATE_FINALIZE])
def test_config1_update_every_step(capi, flags):
    run_c1(flags)


def test_config2_llama8b_shape(capi):
    """B=16, 8 KV heads x 128, bf16, page 16: prefill 512, then 256 decode steps of fused
    append+gather; two layers, every step against the device mirror, every 32nd step and the
    last against the oracle."""
    B, H, D, P, prefill, decode = 16, 8, 128, 16, 512, 256
    cap = prefill + decode
    gen = torch.Generator().manual_seed(1002)
    for layer in range(2):
        pool = make_pool(cap, B, H, D, P, torch.bfloat16)
        oracle = DenseLayerOracle(B, cap, P)
        mirror = DeviceMirror(B, H, cap, D, torch.bfloat16)
        k = hf_layout(B, H, prefill, D, torch.bfloat16, gen)
        v = hf_layout(B, H, prefill, D, torch.bfloat16, gen)
        got = pool.update(k.cuda(), v.cuda(), prefill)
        oracle.append(to_bits(k), to_bits(v))
        mirror.append(k.cuda(), v.cuda())
        compare_layer(pool, oracle, got, f"C2 layer {layer} prefill")
        mirror.check(got, f"C2 layer {layer} prefill")
        for step in range(decode):
            k = hf_layout(B, H, 1, D, torch.bfloat16, gen)
            v = hf_layout(B, H, 1, D, torch.bfloat16, gen)
            got = pool.update(k.cuda(), v.cuda(), prefill + step + 1)
            oracle.append(to_bits(k), to_bits(v))
            mirror.append(k.cuda(), v.cuda())
            mirror.check(got, f"C2 layer {layer} step {step}")
            if step % 32 == 31 or step == decode - 1:
                compare_layer(pool, oracle, got, f"C2 layer {layer} step {step}")
        pool.check_invariants()
        assert pool.errors() == 0


def staircase(lengths_desc):
    """(batch, tokens) appends that give row i lengths_desc[i] tokens through the reference
    API, which appends to rows [0, batch): longest rows first."""
    calls = []
    done = 0
    n = len(lengths_desc)
    for b in range(n, 0, -1):
        need = lengths_desc[b - 1] - done
        if need > 0:
            calls.append((b, need))
            done += need
    return calls


@pytest.mark.parametrize("B,S", [(2, 2100), (8, 700), (16, 600), (32, 300), (1, 32900), (4, 8300)])
def test_cu_balanced_tail_pieces(capi, B, S):
    """Single-round gather launches whose tile count (2 * B * ceil(S / 32) at 8 KV heads x 128,
    bf16, page 16) is not a multiple of the CU count cut their tail into one piece per CU; (B = 1
    and 4) launches of several dispatch rounds with such tile counts keep whole tiles.
    Ragged rows (stale and zero-padded positions in the pieces), updates of 1 and 3 tokens, exact
    extents and device-side extents over a larger output; positions past the longest row are
    never written."""
    H, D, P = 8, 128, 16
    rng = np.random.default_rng(5000 + B)
    lengths = sorted(rng.integers(S // 2, S + 1, size=B).tolist(), reverse=True)
    lengths[0] = S
    cap = S + 40
    pool = make_pool(cap, B, H, D, P, torch.bfloat16)
    oracle = DenseLayerOracle(B, cap, P)
    gen = torch.Generator().manual_seed(B)
    for b, t in staircase(lengths):
        k = hf_layout(b, H, t, D, torch.bfloat16, gen)
        v = hf_layout(b, H, t, D, torch.bfloat16, gen)
        pool.append(k.cuda(), v.cuda())
        oracle.append(to_bits(k), to_bits(v))
    compare_layer(pool, oracle, None, f"B{B} prefill")
    sentinel = torch.full((B, H, cap, D), -7.0, dtype=torch.bfloat16, device="cuda")
    for step, t in enumerate([1, 3, 1, 1, 3]):
        k = hf_layout(B, H, t, D, torch.bfloat16, gen)
        v = hf_layout(B, H, t, D, torch.bfloat16, gen)
        oracle.append(to_bits(k), to_bits(v))
        seq = oracle.get_seq_length()
        if step % 2:
            ko, vo = sentinel.clone(), sentinel.clone()
            pool.update(k.cuda(), v.cuda(), cap, SEQ_FROM_DEVICE, out=(ko, vo))
            compare_layer(pool, oracle, (ko[:, :, :seq], vo[:, :, :seq]), f"B{B} step {step} device extent")
            untouched = to_bits(sentinel[:, :, seq:])
            assert_bits_equal(ko[:, :, seq:], untouched, f"B{B} step {step} K past the longest row")
            assert_bits_equal(vo[:, :, seq:], untouched, f"B{B} step {step} V past the longest row")
        else:
            got = pool.update(k.cuda(), v.cuda(), seq)
            compare_layer(pool, oracle, got, f"B{B} step {step}")
    got = pool.gather(B, oracle.get_seq_length())
    compare_layer(pool, oracle, got, f"B{B} gather")
    pool.check_invariants()
    assert pool.errors() == 0


@pytest.mark.parametrize("B,P,S", [(8, 16, 700), (8, 32, 700), (16, 16, 560), (16, 16, 700), (32, 16, 300),
                                   (2, 16, 2100)])
def test_balanced_lean_tiles_with_stale_rows(capi, B, P, S):
    """Single-round gather launches whose one-page tile count is not a multiple of the CU count
    cut each (row, K or V) into equal chunks that start anywhere in a page (touching up to two
    blocks); (16, 16, 700) takes page-aligned two-page tiles.  Ragged rows, a crop whose slots stay visible below the mark once a longer row sets
    the extent, appends of 1 and 3 tokens that map new blocks, exact extents (the positions past
    a row's end spread over its chunks) and device-side extents (written by the row's last chunk;
    nothing past the longest row written)."""
    H, D = 8, 128
    rng = np.random.default_rng(7000 + B + P)
    lengths = sorted(rng.integers(S // 2, S + 1, size=B).tolist(), reverse=True)
    lengths[0] = S
    cap = S + 40
    pool = make_pool(cap, B, H, D, P, torch.bfloat16, order=torch.from_numpy(
        np.random.default_rng(B).permutation(B * (-(-cap // P))).astype(np.int32)))
    oracle = DenseLayerOracle(B, cap, P)
    gen = torch.Generator().manual_seed(B * P)

    def tokens(b, t):
        return hf_layout(b, H, t, D, torch.bfloat16, gen), hf_layout(b, H, t, D, torch.bfloat16, gen)

    for b, t in staircase(lengths):
        k, v = tokens(b, t)
        pool.append(k.cuda(), v.cuda())
        oracle.append(to_bits(k), to_bits(v))
    k, v = tokens(B, 1)  # every row: the crop below applies to the whole batch
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    compare_layer(pool, oracle, None, f"B{B} P{P} prefill")
    cut = S // 2 + 7
    pool.crop(B, cut)
    oracle.crop(cut)
    k, v = tokens(2, 150)  # rows 0 and 1 grow past the others again: their stale slots show
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    sentinel = torch.full((B, H, cap, D), -7.0, dtype=torch.bfloat16, device="cuda")
    for step, t in enumerate([1, 3, 1, 3, 1, 1]):
        k, v = tokens(B, t)
        oracle.append(to_bits(k), to_bits(v))
        seq = oracle.get_seq_length()
        if step % 2:
            ko, vo = sentinel.clone(), sentinel.clone()
            pool.update(k.cuda(), v.cuda(), cap, SEQ_FROM_DEVICE, out=(ko, vo))
            compare_layer(pool, oracle, (ko[:, :, :seq], vo[:, :, :seq]), f"B{B} P{P} step {step} device extent")
            untouched = to_bits(sentinel[:, :, seq:])
            assert_bits_equal(ko[:, :, seq:], untouched, f"B{B} P{P} step {step} K past the longest row")
            assert_bits_equal(vo[:, :, seq:], untouched, f"B{B} P{P} step {step} V past the longest row")
        else:
            got = pool.update(k.cuda(), v.cuda(), seq)
            compare_layer(pool, oracle, got, f"B{B} P{P} step {step}")
    compare_layer(pool, oracle, pool.gather(B, oracle.get_seq_length()), f"B{B} P{P} gather")
    pool.check_invariants()
    assert pool.errors() == 0


def test_config3_ragged_random_pages(capi):
    """B=64, context lengths U{128..4096}, pages handed out in a seeded random permutation:
    a non-contiguous block table; 128 1-token append + gather steps, every one against the device
    mirror, the first and the last against the oracle."""
    B, H, D, P = 64, 8, 128, 16
    rng = np.random.default_rng(2003)
    lengths = sorted(rng.integers(128, 4097, size=B).tolist(), reverse=True)
    steps = 128
    cap = lengths[0] + steps
    mb = -(-cap // P)
    perm = torch.from_numpy(np.random.default_rng(3003).permutation(B * mb).astype(np.int32))
    pool = make_pool(cap, B, H, D, P, torch.bfloat16, order=perm)
    oracle = DenseLayerOracle(B, cap, P)
    mirror = DeviceMirror(B, H, cap, D, torch.bfloat16)
    gen = torch.Generator().manual_seed(1003)
    for b, t in staircase(lengths):
        k = hf_layout(b, H, t, D, torch.bfloat16, gen)
        v = hf_layout(b, H, t, D, torch.bfloat16, gen)
        pool.append(k.cuda(), v.cuda())
        oracle.append(to_bits(k), to_bits(v))
        mirror.append(k.cuda(), v.cuda())
    bt = pool.bt.cpu().numpy()
    assert (np.diff(bt[0, : lengths[0] // P]) != 1).any(), "block table should be non-contiguous"
    for step in range(steps):
        k = hf_layout(B, H, 1, D, torch.bfloat16, gen)
        v = hf_layout(B, H, 1, D, torch.bfloat16, gen)
        seq = lengths[0] + step + 1
        got = pool.update(k.cuda(), v.cuda(), seq)
        oracle.append(to_bits(k), to_bits(v))
        mirror.append(k.cuda(), v.cuda())
        mirror.check(got, f"C3 step {step}")
        if step in (0, steps - 1):
            compare_layer(pool, oracle, got, f"C3 step {step}")
    pool.check_invariants()
    assert pool.errors() == 0


def test_config4_chunked_prefill_32k(capi):
    """B=1, fp16, page 32: 16 chunked appends of 2048 tokens (gather after each), then 64
    decode appends; every chunk and every 16th decode step compared."""
    H, D, P, chunk, n_chunks, decode = 8, 128, 32, 2048, 16, 64
    cap = chunk * n_chunks + decode
    pool = make_pool(cap, 1, H, D, P, torch.float16)
    oracle = DenseLayerOracle(1, cap, P)
    gen = torch.Generator().manual_seed(1004)
    for c in range(n_chunks + decode):
        t = chunk if c < n_chunks else 1
        k = hf_layout(1, H, t, D, torch.float16, gen)
        v = hf_layout(1, H, t, D, torch.float16, gen)
        seq = oracle.get_seq_length() + t
        got = pool.update(k.cuda(), v.cuda(), seq)
        oracle.append(to_bits(k), to_bits(v))
        if c < n_chunks or (c - n_chunks) % 16 == 15:
            compare_layer(pool, oracle, got, f"C4 call {c}")
    pool.check_invariants()


def test_config5_pool_at_90_percent_with_churn(capi):
    """70B-class layer shape: B=32, context 8192, pool sized for 90% occupancy; before each 1-token
    append + gather of all rows, two seeded rows are freed and re-prefilled with 8192 new tokens
    (barq_kv_append over the row's one-row metadata view), which takes the pages those rows and
    earlier ones released: the pool stays near 90% for every step.  All 64 steps of the
    configuration, every one against the device mirror, steps 0, 31 and 63 against the oracle."""
    B, H, D, P, ctx, steps = 32, 8, 128, 16, 8192, 64
    cap = ctx + steps
    live = B * (ctx // P)
    num_pages = int(np.ceil(live / 0.9))
    pool = make_pool(cap, B, H, D, P, torch.bfloat16, num_pages=num_pages)
    oracle = DenseLayerOracle(B, cap, P)
    mirror = DeviceMirror(B, H, cap, D, torch.bfloat16)
    gen = torch.Generator().manual_seed(1005)
    k = hf_layout(B, H, ctx, D, torch.bfloat16, gen)
    v = hf_layout(B, H, ctx, D, torch.bfloat16, gen)
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    mirror.append(k.cuda(), v.cuda())
    del k, v
    assert pool.free_top() == num_pages - live
    churn = np.random.default_rng(4005)
    most_free = 0
    for step in range(steps):
        rows = sorted(churn.choice(B, size=2, replace=False).tolist())
        pool.free_rows(rows)
        oracle.release_rows(rows)
        mirror.release_rows(rows)
        kr = hf_layout(2, H, ctx, D, torch.bfloat16, gen)
        vr = hf_layout(2, H, ctx, D, torch.bfloat16, gen)
        pool.append_rows(rows, kr.cuda(), vr.cuda())
        oracle.append_rows(rows, to_bits(kr), to_bits(vr))
        mirror.append_rows(rows, kr.cuda(), vr.cuda())
        del kr, vr
        most_free = max(most_free, pool.free_top())
        k = hf_layout(B, H, 1, D, torch.bfloat16, gen)
        v = hf_layout(B, H, 1, D, torch.bfloat16, gen)
        seq = oracle.get_seq_length() + 1
        got = pool.update(k.cuda(), v.cuda(), seq)
        oracle.append(to_bits(k), to_bits(v))
        mirror.append(k.cuda(), v.cuda())
        mirror.check(got, f"C5 step {step}")
        if step in (0, 31, steps - 1):
            compare_layer(pool, oracle, got, f"C5 step {step}")
    # every decode step ran with >= 88% of the pool holding live tokens
    assert most_free <= 0.12 * num_pages, most_free
    pool.check_invariants()
    assert pool.errors() == 0


# --------------------------------------------------------------------------- edge cases
SHAPES = [
    # heads, dim, page, dtype
    (2, 4, 4, torch.float32),     # the reference test's geometry (16-byte rows)
    (3, 80, 5, torch.bfloat16),   # odd head count, 160-byte rows, page size not a power of two
    (1, 3, 1, torch.float16),     # 6-byte rows: 2-byte vectors, page size 1
    (4, 64, 16, torch.float64),
    (8, 128, 32, torch.bfloat16),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"h{s[0]}d{s[1]}p{s[2]}{str(s[3])[6:]}")
@pytest.mark.parametrize("seed", [0, 1])
def test_random_programs_through_capi(capi, shape, seed):
    """Ragged batches, multi-token appends, crop (stale slots visible), gather-only, separate
    and in-kernel commit, row release -- each step compared with the oracle."""
    H, D, P, dtype = shape
    rng = np.random.default_rng(seed * 31 + D)
    Bmax, cap = 4, 40
    pool = make_pool(cap, Bmax, H, D, P, dtype)
    oracle = DenseLayerOracle(Bmax, cap, P)
    gen = torch.Generator().manual_seed(seed)
    cur = 0
    for it in range(30):
        r = rng.random()
        if r < 0.55:
            b = int(rng.integers(1, Bmax + 1))
            t = int(rng.integers(1, 6))
            longest = int(oracle.seq_lens[:b].max()) if oracle.is_initialized else 0
            if longest + t > cap:
                continue
            k = hf_layout(b, H, t, D, dtype, gen)
            v = hf_layout(b, H, t, D, dtype, gen)
            flags = SEPARATE_FINALIZE if rng.random() < 0.3 else 0
            if rng.random() < 0.3:
                pool.append(k.cuda(), v.cuda())
                oracle.append(to_bits(k), to_bits(v))
                cur = b
                compare_layer(pool, oracle, None, f"append it{it}")
            else:
                oracle.append(to_bits(k), to_bits(v))
                cur = b
                got = pool.update(k.cuda(), v.cuda(), oracle.get_seq_length(), flags)
                compare_layer(pool, oracle, got, f"update it{it}")
        elif r < 0.7 and cur:
            m = int(rng.integers(0, cap))
            pool.crop(cur, m)
            oracle.crop(m)
            compare_layer(pool, oracle, None, f"crop it{it}")
        elif r < 0.8 and cur:
            rows = sorted(rng.choice(Bmax, size=int(rng.integers(1, 3)), replace=False).tolist())
            pool.free_rows(rows)
            oracle.release_rows(rows)
            compare_layer(pool, oracle, None, f"free it{it}")
        elif cur:
            seq = oracle.get_seq_length()
            got = pool.gather(cur, seq, SEQ_FROM_DEVICE)
            compare_layer(pool, oracle, got, f"gather it{it}")
    pool.check_invariants()
    assert pool.errors() == 0


def test_copy_rows_beam_select_and_repeat(capi):
    H, D, P, dtype = 4, 64, 8, torch.bfloat16
    cap, B = 50, 3
    pool = make_pool(cap, B, H, D, P, dtype)
    oracle = DenseLayerOracle(B, cap, P)
    gen = torch.Generator().manual_seed(11)
    for b, t in [(3, 9), (2, 7), (3, 1)]:
        k, v = hf_layout(b, H, t, D, dtype, gen), hf_layout(b, H, t, D, dtype, gen)
        pool.append(k.cuda(), v.cuda())
        oracle.append(to_bits(k), to_bits(v))
    pool.crop(3, 12)
    oracle.crop(12)
    for rows in ([2, 0, 0, 1, 2, 2], [1, 1, 1]):
        dst = make_pool(cap, len(rows), H, D, P, dtype)
        pool.copy_rows_into(dst, rows)
        o2 = DenseLayerOracle(B, cap, P)
        o2.__dict__.update({k_: (v_.copy() if isinstance(v_, np.ndarray) else v_) for k_, v_ in oracle.__dict__.items()})
        o2.batch_select_indices(rows)
        compare_layer(dst, o2, None, f"copy_rows {rows}")
        dst.check_invariants()
        k, v = hf_layout(len(rows), H, 2, D, dtype, gen), hf_layout(len(rows), H, 2, D, dtype, gen)
        o2.append(to_bits(k), to_bits(v))
        got = dst.update(k.cuda(), v.cuda(), o2.get_seq_length())
        compare_layer(dst, o2, got, f"after copy_rows {rows}")


def test_nan_payloads_are_bit_copied(capi):
    H, D, P = 2, 16, 4
    pool = make_pool(16, 2, H, D, P, torch.bfloat16)
    oracle = DenseLayerOracle(2, 16, P)
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 2**16, size=(2, H, 7, D), dtype=np.uint16)
    raw[..., 0] = 0x7FC1  # quiet NaN with payload
    raw[..., 1] = 0xFF81  # signalling-pattern NaN, sign set
    raw[..., 2] = 0x8000  # negative zero
    k = torch.from_numpy(raw.view(np.int16)).view(torch.bfloat16)
    v = torch.from_numpy(raw[::-1].copy().view(np.int16)).view(torch.bfloat16)
    got = pool.update(k.cuda(), v.cuda(), 7)
    oracle.append(to_bits(k), to_bits(v))
    compare_layer(pool, oracle, got, "nan payloads")


def test_misaligned_inputs_use_narrow_vectors(capi):
    """States that start 2 bytes into an allocation force 2-byte vectors; results unchanged."""
    H, D, P = 4, 64, 16
    pool = make_pool(64, 2, H, D, P, torch.bfloat16)
    oracle = DenseLayerOracle(2, 64, P)
    gen = torch.Generator().manual_seed(5)
    big = normal((2, 5, H, D + 1), torch.bfloat16, gen)
    k = big[..., 1:].transpose(1, 2)  # [2, H, 5, D]: data pointer + 2 bytes, token stride H*(D+1)
    v = big[..., :D].transpose(1, 2)
    dev = big.cuda()
    got = pool.update(dev[..., 1:].transpose(1, 2), dev[..., :D].transpose(1, 2), 5)
    oracle.append(to_bits(k), to_bits(v))
    compare_layer(pool, oracle, got, "misaligned")


@pytest.mark.parametrize("flags", [0, SEPARATE_FINALIZE])
def test_commits_that_map_thousands_of_blocks(capi, flags):
    """Commits that map many new blocks at once: 600 rows (wider than a wave: the workgroup
    commit, several chunks of rows and of ranks), then one 5000-token row (the one-wave commit,
    1250 ranks: several rounds of 64 and of the grouped stack reads), which is freed again
    (1250 block-table entries read back in groups)."""
    H, D, P = 2, 8, 4
    gen = torch.Generator().manual_seed(77)
    B, T = 600, 37
    cap = 2 * T + 1
    pool = make_pool(cap, B, H, D, P, torch.float32)
    oracle = DenseLayerOracle(B, cap, P)
    for t in (T, 1, T):
        k = hf_layout(B, H, t, D, torch.float32, gen)
        v = hf_layout(B, H, t, D, torch.float32, gen)
        got = pool.update(k.cuda(), v.cuda(), oracle.get_seq_length() + t, flags)
        oracle.append(to_bits(k), to_bits(v))
        compare_layer(pool, oracle, got, f"600 rows after {t}")
    pool.check_invariants()
    assert pool.errors() == 0

    T1 = 5000
    pool = make_pool(T1 + 1, 2, H, D, P, torch.float32)
    oracle = DenseLayerOracle(2, T1 + 1, P)
    k = hf_layout(1, H, T1, D, torch.float32, gen)
    v = hf_layout(1, H, T1, D, torch.float32, gen)
    pool.append(k.cuda(), v.cuda())
    oracle.append(to_bits(k), to_bits(v))
    k = hf_layout(2, H, 1, D, torch.float32, gen)
    got = pool.update(k.cuda(), k.cuda(), T1 + 1, flags)
    oracle.append(to_bits(k), to_bits(k))
    compare_layer(pool, oracle, got, "one long row")
    pool.check_invariants()
    pool.free_rows([0])
    oracle.release_rows([0])
    assert pool.free_top() == pool.num_pages - 1  # row 1 keeps its one page
    compare_layer(pool, oracle, None, "after freeing the long row")
    pool.check_invariants()
    assert pool.errors() == 0


def test_empty_batch_and_zero_tokens(capi):
    H, D, P = 2, 8, 4
    pool = make_pool(16, 2, H, D, P, torch.float32)
    k = torch.zeros((0, H, 3, D), device="cuda")
    pool.update(k, k, 0)
    k = torch.zeros((2, H, 0, D), device="cuda")
    pool.append(k, k)
    assert pool.lens.cpu().tolist() == [0, 0] and pool.free_top() == pool.num_pages
    ko, vo = pool.gather(2, 3)  # nothing written: zeros
    assert not ko.any() and not vo.any()


def test_pool_exhaustion_sets_error_bit_without_fault(capi):
    """Append needing 3 pages from a pool of 2: the kernels drop the unmappable block's tokens
    from the pages (the output still shows them from the input) and set the sticky bit."""
    H, D, P = 2, 8, 4
    pool = make_pool(12, 1, H, D, P, torch.float32, num_pages=2)
    gen = torch.Generator().manual_seed(1)
    k = hf_layout(1, H, 10, D, torch.float32, gen).cuda()
    got = pool.update(k, k, 10)
    assert torch.equal(got[0], k)
    assert pool.errors() & 1
    assert pool.free_top() == 0
    bt = pool.bt.cpu().tolist()[0]
    assert sorted(bt[:2]) == [0, 1] and bt[2] == -1


def test_large_pool_int64_offsets(capi):
    """A 5 GiB K pool: pages past 4 GiB are written and read back at the right place."""
    H, D, P = 8, 128, 16  # 32 KiB pages
    num_pages = 5 * 2**30 // (P * H * D * 2)
    pool = CPool(max_batch=1, max_blocks=4, page_size=P, heads=H, dim=D, dtype=torch.bfloat16,
                 num_pages=num_pages, order=torch.arange(num_pages - 1, -1, -1, dtype=torch.int32))
    oracle = DenseLayerOracle(1, 4 * P, P)
    gen = torch.Generator().manual_seed(2)
    k = hf_layout(1, H, 50, D, torch.bfloat16, gen)
    v = hf_layout(1, H, 50, D, torch.bfloat16, gen)
    got = pool.update(k.cuda(), v.cuda(), 50)
    oracle.append(to_bits(k), to_bits(v))
    assert pool.bt[0, 0].item() == num_pages - 1
    compare_layer(pool, oracle, got, "large pool")
    compare_layer(pool, oracle, None, "large pool regather")
    del pool
    torch.cuda.empty_cache()
