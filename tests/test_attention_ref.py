"""CPU tests of the decode-attention checker and host path, and of the C ABI's argument checks.

* The float64 reference (tests/attn_ref.py) against torch's scaled_dot_product_attention:
  decode over the last T positions of a row equals the last T rows of square causal attention
  over the whole row (a library routine that shares no code with the reference), grouped-query
  heads included; ragged rows are independent rows.
* PagePool.attend on a host-memory pool against the reference.
* barq_kv_attention_workspace_bytes / barq_kv_decode_attention reject what the kernel cannot
  take before anything is launched (no GPU needed).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from attn_ref import decode_attention_reference, within_tolerance


def _sdpa_last_rows(q_full, k, v, T, scale):
    """q_full [Hq, n, D] queries of all n positions; k, v [Hkv, n, D]; last T rows of square
    causal attention, float64."""
    out = F.scaled_dot_product_attention(q_full[None], k[None], v[None], is_causal=True, scale=scale,
                                         enable_gqa=True)
    return out[0, :, -T:].numpy()


@pytest.mark.parametrize("G,T", [(1, 1), (4, 1), (4, 3), (8, 2), (16, 1)])
def test_reference_matches_sdpa_causal(G, T):
    gen = torch.Generator().manual_seed(10 * G + T)
    Hkv, D = 2, 16
    lens = [1 + T, 7, 33, 64]
    lens = [max(n, T) for n in lens]
    S = max(lens)
    B = len(lens)
    q_full = torch.randn(B, G * Hkv, S, D, generator=gen, dtype=torch.float64)
    k = torch.randn(B, Hkv, S, D, generator=gen, dtype=torch.float64)
    v = torch.randn(B, Hkv, S, D, generator=gen, dtype=torch.float64)
    scale = 0.37
    q = torch.zeros(B, G * Hkv, T, D, dtype=torch.float64)
    for b, n in enumerate(lens):
        q[b] = q_full[b, :, n - T:n]
    got = decode_attention_reference(q.numpy(), k.numpy(), v.numpy(), lens, scale)
    for b, n in enumerate(lens):
        want = _sdpa_last_rows(q_full[b, :, :n], k[b, :, :n], v[b, :, :n], T, scale)
        np.testing.assert_allclose(got[b], want, rtol=1e-12, atol=1e-12)


def test_reference_closed_forms():
    """Equal V rows give that row; a zero query averages V uniformly; a row that sees nothing
    gives zeros (lens < T)."""
    rng = np.random.default_rng(0)
    D = 8
    k = rng.standard_normal((1, 1, 5, D))
    v = np.repeat(rng.standard_normal((1, 1, 1, D)), 5, axis=2)
    q = rng.standard_normal((1, 2, 1, D))
    out = decode_attention_reference(q, k, v, [5], 1.0)
    np.testing.assert_allclose(out[0, :, 0], np.repeat(v[0, 0, :1], 2, axis=0), rtol=1e-14)
    v2 = rng.standard_normal((1, 1, 5, D))
    out = decode_attention_reference(np.zeros((1, 1, 1, D)), k, v2, [5], 1.0)
    np.testing.assert_allclose(out[0, 0, 0], v2[0, 0].mean(axis=0), rtol=1e-13)
    out = decode_attention_reference(q[:, :, :1].repeat(3, axis=2), k, v2, [2], 1.0)
    assert np.all(out[0, :, 0] == 0) and np.any(out[0, :, 2] != 0)


@pytest.mark.parametrize("page,dtype", [(16, torch.bfloat16), (5, torch.float16)])
def test_host_pool_attend_matches_reference(page, dtype):
    from barqtrain_amd.paged import PagePool

    gen = torch.Generator().manual_seed(page)
    B, Hkv, D, G, T = 3, 2, 128, 4, 2
    pool = PagePool(max_batch=B, max_blocks=-(-40 // page), page_size=page, kv_heads=Hkv, head_dim=D,
                    dtype=dtype, device="cpu")
    k = torch.randn(B, Hkv, 23, D, generator=gen).to(dtype)
    v = torch.randn(B, Hkv, 23, D, generator=gen).to(dtype)
    pool.append(k, v)
    pool.crop(B, 23)
    q = torch.randn(B, G * Hkv, T, D, generator=gen).to(dtype)
    out = pool.attend(q, out_dtype=torch.float32)
    want = decode_attention_reference(q.float().numpy(), k.float().numpy(), v.float().numpy(), [23] * B,
                                      D ** -0.5)
    ok, ratio = within_tolerance(out.numpy(), want, rtol=1e-5, atol=1e-5)
    assert ok, ratio


# ---------------------------------------------------------------------- C ABI argument checks


def _fake_pool(elem=2, dim=128, heads=8, page=16, blocks=8, batch=4, pages=None):
    from barqtrain_amd import _capi

    pages = pages or batch * blocks
    # Non-null but never dereferenced: every call below is rejected or sized on the host.
    p = 1 << 20
    return _capi.BarqKVPool(p, p, p, p, p, p, p, p, pages, batch, blocks, page, heads, dim, elem)


def test_workspace_bytes_and_rejections():
    from barqtrain_amd import _capi

    lib = _capi.load_library()
    ws = lib.barq_kv_attention_workspace_bytes
    pool = _fake_pool()
    ref = ctypes.byref(pool)
    # one record slot per (range + pair): automatic ranges are at most 2048 (the resident waves
    # of an MI355X); a fixed range of s positions gives ceil(pairs * ceil(max_seq / 16) / (s / 16))
    rec4 = 4 * 128 + 8
    pairs = 2 * 8
    assert ws(ref, 2, 32, 1, 100, 0) == (2048 + pairs) * rec4 * 4
    assert ws(ref, 2, 32, 1, 100, 64) == (pairs * 7 // 4 + pairs) * rec4 * 4  # 7 chunks/pair, 4 per range
    assert ws(ref, 2, 32, 1, 100, 50) == (pairs * 7 // 4 + pairs) * rec4 * 4  # 50 -> 64
    big = ctypes.byref(_fake_pool(blocks=64))                 # capacity 1024: 64 chunks per pair
    assert ws(big, 2, 32, 1, 0, 256) == (pairs * 64 // 16 + pairs) * rec4 * 4
    assert ws(big, 2, 128, 1, 0, 256) == (pairs * 4 + pairs) * (16 * 128 + 32) * 4  # G = 16
    assert ws(big, 2, 8, 1, 0, 256) == (pairs * 4 + pairs) * (128 + 4) * 4           # G = 1
    assert ws(ctypes.byref(_fake_pool(batch=1025, pages=1)), 1025, 32, 1, 0, 0) == -1  # batch > 1024
    assert ws(ref, 2, 128, 2, 100, 0) == -1   # 32 query rows per kv head
    assert ws(ref, 2, 12, 1, 100, 0) == -1    # q_heads not a multiple of kv_heads
    assert ws(ref, 5, 32, 1, 100, 0) == -1    # batch beyond the pool's rows
    assert ws(ref, 2, 32, 0, 100, 0) == -1    # no query tokens
    assert ws(ctypes.byref(_fake_pool(elem=4)), 2, 32, 1, 100, 0) == -1   # fp32 pool
    assert ws(ctypes.byref(_fake_pool(dim=64)), 2, 32, 1, 100, 0) == (2048 + pairs) * (4 * 64 + 8) * 4  # head_dim 64
    assert ws(ctypes.byref(_fake_pool(dim=96)), 2, 32, 1, 100, 0) == -1   # head_dim 96
    assert ws(ctypes.byref(_fake_pool(dim=256)), 2, 32, 1, 100, 0) == (2048 + pairs) * (4 * 256 + 8) * 4  # head_dim 256
    assert ws(ctypes.byref(_fake_pool(dim=512)), 2, 32, 1, 100, 0) == -1  # head_dim 512

    att = lib.barq_kv_decode_attention
    # Fake, aligned device addresses: every call below is rejected before any launch (batch 0
    # returns first), so nothing ever dereferences them.
    buf = 1 << 21

    def call(**kw):
        a = dict(batch=2, q_heads=32, tokens=1, qsb=32 * 128, qsh=128, qst=128, out=buf, osb=32 * 128,
                 osh=128, ost=128, flags=0, wsb=10**6, query=buf, ws=buf, max_seq=0)
        a.update(kw)
        return att(big, a["query"], a["batch"], a["q_heads"], a["tokens"], a["qsb"], a["qsh"], a["qst"],
                   a["out"], a["osb"], a["osh"], a["ost"], 0.1, a["max_seq"], 256, a["flags"], a["ws"],
                   a["wsb"], None)

    assert call(batch=0) == 0                   # nothing to do
    assert call(qsh=100) == 1                    # query head stride not a multiple of 8
    assert call(query=buf + 8) == 1              # query rows not 16-byte aligned
    assert call(out=buf + 2, batch=0) == 0       # batch 0 returns before pointer checks
    assert call(out=buf + 2) == 1                # output not aligned
    assert call(wsb=1000) == 1                   # workspace too small (splits of 256)
    assert call(ws=buf + 8) == 1                 # workspace not 16-byte aligned
    assert call(flags=4) == 1                    # unknown flag
    assert call(query=0) == 1                    # null query
