"""GPU test of barq_kv_update_known (the update whose row state -- lengths, marks, stack top --
comes from the caller's exact host shadow instead of device reads) through the C ABI: on twin
pools driven by the same random program, it returns and leaves exactly what barq_kv_update
returns and leaves -- outputs bit for bit, block tables, lengths, marks and stack top -- at
ragged lengths (rows of a call are [0, batch), so varying batches leave rows of different
lengths), page boundaries, shuffled page orders, multi-token appends, batch 1 at the Llama-3-8B
shape and a batch above the kernel's 64 rows (which runs the device-read path)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from capi_pool import CPool
from kvgen import hf_layout, to_bits

pytestmark = pytest.mark.gpu


def twin(B, cap, P, H, D, dtype, order=None):
    mb = -(-cap // P)
    pools = [CPool(max_batch=B, max_blocks=mb, page_size=P, heads=H, dim=D, dtype=dtype, num_pages=B * mb + 3,
                   order=order) for _ in range(2)]
    return pools


def step_both(capi, a, b, k, v, seq):
    ko_a, vo_a = a.new_out(k.shape[0], seq)
    ko_b, vo_b = b.new_out(k.shape[0], seq)
    st = torch.cuda.current_stream().cuda_stream
    rc = capi.barq_kv_update(a.ref, k.data_ptr(), v.data_ptr(), k.shape[0], k.shape[2], k.stride(0), k.stride(1),
                             k.stride(2), ko_a.data_ptr(), vo_a.data_ptr(), seq, ko_a.stride(0), ko_a.stride(1),
                             ko_a.stride(2), 0, st)
    assert rc == 0
    # the exact device state of pool b before its launch (what an eager caller's shadow holds)
    batch = k.shape[0]
    lens = b.lens[:batch].cpu().numpy().astype(np.int32)
    hw = b.hw[:batch].cpu().numpy().astype(np.int32)
    top = int(b.ctrl[0].item())
    rc = capi.barq_kv_update_known(b.ref, k.data_ptr(), v.data_ptr(), batch, k.shape[2], k.stride(0), k.stride(1),
                                   k.stride(2), ko_b.data_ptr(), vo_b.data_ptr(), seq, ko_b.stride(0),
                                   ko_b.stride(1), ko_b.stride(2), lens.ctypes.data, hw.ctypes.data, top, st)
    assert rc == 0
    torch.cuda.synchronize()
    for x, y, what in ((ko_a, ko_b, "K"), (vo_a, vo_b, "V")):
        assert np.array_equal(to_bits(x), to_bits(y)), what
    for x, y, what in ((a.bt, b.bt, "block table"), (a.lens, b.lens, "lengths"), (a.hw, b.hw, "marks"),
                       (a.ctrl, b.ctrl, "ctrl")):
        assert torch.equal(x, y), what


@pytest.mark.parametrize("P,H,D,dtype,seed", [(16, 8, 128, torch.bfloat16, 0), (5, 2, 64, torch.float16, 1),
                                              (16, 4, 64, torch.float32, 2)])
def test_known_state_update_matches_device_reads(capi, P, H, D, dtype, seed):
    rng = np.random.default_rng(seed)
    B, cap = 6, 200
    perm = torch.from_numpy(rng.permutation(B * -(-cap // P) + 3).astype(np.int32))
    a, b = twin(B, cap, P, H, D, dtype, order=perm)
    gen = torch.Generator().manual_seed(seed)
    longest = 0
    for _ in range(40):
        batch = int(rng.integers(1, B + 1))
        t = int(rng.choice([1, 1, 1, 2, 7, 19]))
        lens = a.lens[:batch].cpu().numpy()
        if int(lens.max()) + t > cap:
            break
        k = hf_layout(batch, H, t, D, dtype, gen).cuda()
        v = hf_layout(batch, H, t, D, dtype, gen).cuda()
        seq = int(lens.max()) + t
        step_both(capi, a, b, k, v, seq)
        longest = max(longest, seq)
    assert longest > 2 * P
    assert a.errors() == b.errors() == 0


def test_known_state_batch1_llama3_shape_and_wide_batch(capi):
    gen = torch.Generator().manual_seed(3)
    a, b = twin(1, 700, 16, 8, 128, torch.bfloat16)
    k = hf_layout(1, 8, 620, 128, torch.bfloat16, gen).cuda()
    step_both(capi, a, b, k, k, 620)
    for s in range(40):  # crosses the page boundaries at 624, 640 and 656
        k = hf_layout(1, 8, 1, 128, torch.bfloat16, gen).cuda()
        v = hf_layout(1, 8, 1, 128, torch.bfloat16, gen).cuda()
        step_both(capi, a, b, k, v, 621 + s)
    # 80 rows: more than the kernel's commit holds, so the entry point runs the device-read path
    a, b = twin(80, 40, 16, 2, 64, torch.bfloat16)
    for t in (17, 1, 1, 15):
        k = hf_layout(80, 2, t, 64, torch.bfloat16, gen).cuda()
        step_both(capi, a, b, k, k, int(a.lens[0].item()) + t)
