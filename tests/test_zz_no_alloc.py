"""GPU test of barq_kv_decode_attention_noalloc (the allocation-free variant whose workspace is the
library's static device scratch) through the C ABI: on the same pool and query it must return
exactly what barq_kv_decode_attention returns with a caller workspace -- the same kernels over
the same schedule, so bit for bit -- on two calls in a row, the second smaller than the first
(the scratch keeps the first call's records); a request beyond the scratch is refused before
any launch; the call allocates no device memory (torch's caching allocator and the device's
free memory are unchanged around it, after the first call on the device has resolved the
array's address)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from capi_pool import CPool
from kvgen import hf_layout

pytestmark = pytest.mark.gpu

ERR_SCRATCH = 3
SCRATCH_BYTES = 24 * 1024 * 1024


def make_pool(B, lens, page=16, Hkv=8, dtype=torch.bfloat16, seed=0):
    cap = max(lens)
    pool = CPool(max_batch=B, max_blocks=-(-cap // page), page_size=page, heads=Hkv, dim=128, dtype=dtype,
                 num_pages=B * -(-cap // page))
    gen = torch.Generator().manual_seed(seed)
    done = 0
    for b in range(B, 0, -1):  # rows longest first: append to rows [0, b) in rounds
        need = lens[b - 1] - done
        if need > 0:
            k = hf_layout(b, Hkv, need, 128, dtype, gen).cuda()
            v = hf_layout(b, Hkv, need, 128, dtype, gen).cuda()
            pool.append(k, v)
            done += need
    torch.cuda.synchronize()
    assert pool.errors() == 0
    return pool


def attend_both(capi, pool, B, G, T, dtype, seed, out_f32):
    """(workspace variant output, allocation-free variant output) for one query."""
    Hkv = pool.heads
    gen = torch.Generator().manual_seed(seed)
    q = hf_layout(B, G * Hkv, T, 128, dtype, gen).cuda()
    dt = torch.float32 if out_f32 else dtype
    flags = (1 if dtype == torch.float16 else 0) | (2 if out_f32 else 0)
    scale = 128 ** -0.5
    outs = []
    for variant in ("workspace", "noalloc"):
        out = torch.full((B, T, G * Hkv, 128), float("nan"), dtype=dt, device="cuda").transpose(1, 2)
        args = (pool.ref, q.data_ptr(), B, G * Hkv, T, q.stride(0), q.stride(1), q.stride(2), out.data_ptr(),
                out.stride(0), out.stride(1), out.stride(2), scale, 0, 0, flags)
        st = torch.cuda.current_stream().cuda_stream
        if variant == "workspace":
            need = capi.barq_kv_attention_workspace_bytes(pool.ref, B, G * Hkv, T, 0, 0)
            assert 0 < need <= SCRATCH_BYTES
            ws = torch.empty(need, dtype=torch.uint8, device="cuda")
            rc = capi.barq_kv_decode_attention(*args, ws.data_ptr(), need, st)
        else:
            rc = capi.barq_kv_decode_attention_noalloc(*args, st)
        assert rc == 0, capi.barq_kv_status_string(rc)
        torch.cuda.synchronize()
        outs.append(out)
    return outs


def bits(t):
    return t.contiguous().view(torch.int32 if t.dtype == torch.float32 else torch.int16).cpu().numpy()


def test_noalloc_matches_workspace_variant_twice_second_smaller(capi):
    # First call: the C2 shape (16 rows of 769 positions, G = 4); second: fewer rows, shorter
    # and ragged, other G -- it reuses the scratch the first call filled.
    cases = [
        dict(B=16, lens=[769] * 16, G=4, T=1, dtype=torch.bfloat16, out_f32=False, seed=11),
        dict(B=5, lens=[300, 211, 97, 40, 3], G=2, T=2, dtype=torch.float16, out_f32=True, seed=12),
    ]
    for c in cases:
        pool = make_pool(c["B"], c["lens"], dtype=c["dtype"], seed=c["seed"])
        ref, got = attend_both(capi, pool, c["B"], c["G"], c["T"], c["dtype"], c["seed"] + 100, c["out_f32"])
        assert not torch.isnan(ref).any()
        assert np.array_equal(bits(ref), bits(got)), f"allocation-free output differs: {c}"
        assert pool.errors() == 0


def test_noalloc_largest_documented_shape(capi):
    # Batch 64 with 8 KV heads at G * tokens = 16: (2048 + 512) records of 16 * 130 floats, 21.3 MB,
    # the largest workspace the header promises the scratch holds; then a smaller call after it.
    cases = [
        dict(B=64, lens=sorted(((37 * i) % 500 + 20 for i in range(64)), reverse=True), G=4, T=4, dtype=torch.bfloat16, out_f32=False,
             seed=21),
        dict(B=3, lens=[130, 64, 17], G=8, T=2, dtype=torch.bfloat16, out_f32=False, seed=22),
    ]
    need = None
    for c in cases:
        pool = make_pool(c["B"], c["lens"], dtype=c["dtype"], seed=c["seed"])
        if need is None:
            need = capi.barq_kv_attention_workspace_bytes(pool.ref, c["B"], c["G"] * 8, c["T"], 0, 0)
            assert 16 * 1024 * 1024 < need <= SCRATCH_BYTES
        ref, got = attend_both(capi, pool, c["B"], c["G"], c["T"], c["dtype"], c["seed"] + 100, c["out_f32"])
        assert not torch.isnan(ref).any()
        assert np.array_equal(bits(ref), bits(got)), f"allocation-free output differs: {c}"
        assert pool.errors() == 0


def test_noalloc_allocates_nothing(capi):
    pool = make_pool(4, [120, 90, 64, 1])
    attend_both(capi, pool, 4, 4, 1, torch.bfloat16, 3, False)  # resolves the scratch address
    q = hf_layout(4, 32, 1, 128, torch.bfloat16, torch.Generator().manual_seed(4)).cuda()
    out = torch.empty((4, 1, 32, 128), dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    torch.cuda.synchronize()
    alloc0 = torch.cuda.memory_allocated()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        rc = capi.barq_kv_decode_attention_noalloc(pool.ref, q.data_ptr(), 4, 32, 1, q.stride(0), q.stride(1),
                                                   q.stride(2), out.data_ptr(), out.stride(0), out.stride(1),
                                                   out.stride(2), 128 ** -0.5, 0, 0, 0,
                                                   torch.cuda.current_stream().cuda_stream)
        assert rc == 0
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert torch.cuda.memory_allocated() == alloc0
    assert free1 == free0


def test_noalloc_refuses_requests_beyond_scratch(capi):
    # 1024 rows x 8 KV heads with G * T = 16: (2048 + 8192) records of 8320 bytes > 24 MiB.
    pool = CPool(max_batch=1024, max_blocks=1, page_size=16, heads=8, dim=128, dtype=torch.bfloat16, num_pages=16)
    need = capi.barq_kv_attention_workspace_bytes(pool.ref, 1024, 128, 1, 0, 0)
    assert need > SCRATCH_BYTES
    rc = capi.barq_kv_decode_attention_noalloc(pool.ref, ctypes.c_void_p(16), 1024, 128, 1, 128, 128, 128,
                                               ctypes.c_void_p(16), 128, 128, 128, 1.0, 0, 0, 0,
                                               torch.cuda.current_stream().cuda_stream)
    assert rc == ERR_SCRATCH
    assert "scratch" in capi.barq_kv_status_string(rc).decode()


def test_noalloc_head_256_limits(capi):
    # Head size 256 doubles the records: batch 64 with 8 KV heads fits the scratch at G * tokens = 9
    # ((2048 + 512) records of 9 * 258 floats, 23.8 MB) but not at 10; G * tokens = 16 is refused
    # at any batch (33.9 MB at batch 1).
    pool = CPool(max_batch=64, max_blocks=1, page_size=16, heads=8, dim=256, dtype=torch.bfloat16, num_pages=16)
    assert capi.barq_kv_attention_workspace_bytes(pool.ref, 64, 9 * 8, 1, 0, 0) <= SCRATCH_BYTES
    assert capi.barq_kv_attention_workspace_bytes(pool.ref, 64, 10 * 8, 1, 0, 0) > SCRATCH_BYTES
    assert capi.barq_kv_attention_workspace_bytes(pool.ref, 1, 16 * 8, 1, 0, 0) > SCRATCH_BYTES
    rc = capi.barq_kv_decode_attention_noalloc(pool.ref, ctypes.c_void_p(16), 1, 128, 1, 256, 256, 256,
                                               ctypes.c_void_p(16), 256, 256, 256, 1.0, 0, 0, 0,
                                               torch.cuda.current_stream().cuda_stream)
    assert rc == ERR_SCRATCH
