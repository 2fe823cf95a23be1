"""A page pool driven only through the C ABI (ctypes over libbarq_kv.so), for the GPU tests."""

from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np
import torch

from barqtrain_amd import _capi

CTRL_WORDS = 1088
SEQ_FROM_DEVICE = 1
SEPARATE_FINALIZE = 2


class CPool:
    def __init__(self, *, max_batch, max_blocks, page_size, heads, dim, dtype,
                 num_pages: Optional[int] = None, order: Optional[torch.Tensor] = None,
                 device="cuda"):
        self.lib = _capi.load_library()
        self.max_batch, self.max_blocks, self.page_size = max_batch, max_blocks, page_size
        self.heads, self.dim, self.dtype = heads, dim, dtype
        self.num_pages = num_pages or max_batch * max_blocks
        shape = (self.num_pages, page_size, heads, dim)
        self.kp = torch.empty(shape, dtype=dtype, device=device)
        self.vp = torch.empty(shape, dtype=dtype, device=device)
        i32 = dict(dtype=torch.int32, device=device)
        self.bt = torch.empty((max_batch, max_blocks), **i32)
        self.lens = torch.empty((max_batch,), **i32)
        self.hw = torch.empty((max_batch,), **i32)
        self.free = torch.empty((self.num_pages,), **i32)
        self.ctrl = torch.empty((CTRL_WORDS,), **i32)
        self.shares = torch.empty((self.num_pages,), **i32)
        elem = torch.empty(0, dtype=dtype).element_size()
        self.s = _capi.BarqKVPool(self.kp.data_ptr(), self.vp.data_ptr(), self.bt.data_ptr(),
                                  self.lens.data_ptr(), self.hw.data_ptr(), self.free.data_ptr(),
                                  self.ctrl.data_ptr(), self.shares.data_ptr(), self.num_pages,
                                  max_batch, max_blocks, page_size, heads, dim, elem)
        self.reset(order)

    @property
    def ref(self):
        return ctypes.byref(self.s)

    def _stream(self):
        return _capi.current_stream()

    def reset(self, order=None):
        self._order = None if order is None else order.to(device=self.kp.device, dtype=torch.int32).contiguous()
        ptr = self._order.data_ptr() if self._order is not None else None
        _capi.check(self.lib.barq_kv_pool_reset(self.ref, ptr, self._stream()))

    def append(self, k, v):
        _capi.check(self.lib.barq_kv_append(self.ref, k.data_ptr(), v.data_ptr(), k.shape[0], k.shape[2],
                                            k.stride(0), k.stride(1), k.stride(2), self._stream()))

    def append_rows(self, rows, k, v):
        """k[i], v[i] appended to row rows[i]: barq_kv_append over the one-row view of each row's
        metadata (block-table row, length, mark), the free stack shared."""
        for i, r in enumerate(rows):
            one = _capi.BarqKVPool(*[getattr(self.s, f) for f, _ in _capi.BarqKVPool._fields_])
            one.block_table = self.bt[r:r + 1].data_ptr()
            one.seq_lens = self.lens[r:r + 1].data_ptr()
            one.high_water = self.hw[r:r + 1].data_ptr()
            one.max_batch = 1
            ki, vi = k[i:i + 1], v[i:i + 1]
            _capi.check(self.lib.barq_kv_append(ctypes.byref(one), ki.data_ptr(), vi.data_ptr(), 1, ki.shape[2],
                                                ki.stride(0), ki.stride(1), ki.stride(2), self._stream()))

    def gather(self, batch, seq, flags=0, out=None):
        ko, vo = out or self.new_out(batch, seq)
        _capi.check(self.lib.barq_kv_gather(self.ref, ko.data_ptr(), vo.data_ptr(), batch, seq,
                                            ko.stride(0), ko.stride(1), ko.stride(2), flags, self._stream()))
        return ko, vo

    def update(self, k, v, seq, flags=0, out=None):
        ko, vo = out or self.new_out(k.shape[0], seq)
        _capi.check(self.lib.barq_kv_update(self.ref, k.data_ptr(), v.data_ptr(), k.shape[0], k.shape[2],
                                            k.stride(0), k.stride(1), k.stride(2), ko.data_ptr(), vo.data_ptr(),
                                            seq, ko.stride(0), ko.stride(1), ko.stride(2), flags, self._stream()))
        return ko, vo

    def crop(self, batch, max_length):
        _capi.check(self.lib.barq_kv_crop(self.ref, batch, max_length, self._stream()))

    def free_rows(self, rows):
        idx = torch.tensor(rows, dtype=torch.int32, device=self.kp.device)
        _capi.check(self.lib.barq_kv_free_rows(self.ref, idx.data_ptr(), len(rows), self._stream()))
        torch.cuda.current_stream().synchronize()

    def copy_rows_into(self, dst: "CPool", rows):
        idx = torch.tensor(rows, dtype=torch.int32, device=self.kp.device)
        _capi.check(self.lib.barq_kv_copy_rows(self.ref, dst.ref, idx.data_ptr(), len(rows), self._stream()))
        torch.cuda.current_stream().synchronize()

    def attend(self, q, *, scale=None, out_f32=False, max_seq=0, split_tokens=0, workspace=None):
        """barq_kv_decode_attention; returns (out [B, Hq, T, D], workspace)."""
        B, Hq, T, D = q.shape
        need = self.lib.barq_kv_attention_workspace_bytes(self.ref, B, Hq, T, max_seq, split_tokens)
        assert need >= 0, "attention arguments rejected"
        if workspace is None or workspace.numel() < need:
            workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=self.kp.device)
        dt = torch.float32 if out_f32 else self.dtype
        out = torch.full((B, T, Hq, D), float("nan"), dtype=dt, device=self.kp.device).transpose(1, 2)
        flags = (1 if self.dtype == torch.float16 else 0) | (2 if out_f32 else 0)
        scale = D ** -0.5 if scale is None else scale
        _capi.check(self.lib.barq_kv_decode_attention(
            self.ref, q.data_ptr(), B, Hq, T, q.stride(0), q.stride(1), q.stride(2), out.data_ptr(),
            out.stride(0), out.stride(1), out.stride(2), scale, max_seq, split_tokens, flags,
            workspace.data_ptr(), workspace.numel(), self._stream()))
        return out, workspace

    def select_rows(self, rows):
        idx = torch.tensor(rows, dtype=torch.int32, device=self.kp.device)
        words = self.lib.barq_kv_select_workspace_words(self.ref, 1, len(rows))
        assert words > 0
        ws = torch.empty(words, dtype=torch.int32, device=self.kp.device)
        _capi.check(self.lib.barq_kv_select_rows(self.ref, idx.data_ptr(), len(rows), ws.data_ptr(), ws.numel(),
                                                 self._stream()))
        torch.cuda.current_stream().synchronize()

    def new_out(self, batch, seq):
        shape = (batch, self.heads, seq, self.dim)
        return (torch.empty(shape, dtype=self.dtype, device=self.kp.device),
                torch.empty(shape, dtype=self.dtype, device=self.kp.device))

    def errors(self) -> int:
        return int(self.ctrl[1].item())

    def free_top(self) -> int:
        return int(self.ctrl[0].item())

    def check_invariants(self):
        check_pool_invariants(self.bt.cpu().numpy(), self.lens.cpu().numpy(), self.hw.cpu().numpy(),
                              self.free.cpu().numpy(), self.ctrl.cpu().numpy(), self.shares.cpu().numpy(),
                              self.page_size)


def check_pool_invariants(bt, lens, hw, free, ctrl, shares, P):
    """Block b of row r holds a page iff b * P < high_water[r]; a page is on the free stack iff
    no block holds it; page_shares = holders - 1 (0 when free); only blocks wholly below their
    row's length are shared; arrival counters are back at zero."""
    import collections

    num_pages = len(free)
    top = int(ctrl[0])
    free_set = set(free[:top].tolist())
    assert len(free_set) == top, "a page is on the free stack twice"
    holders = collections.defaultdict(list)
    for r in range(bt.shape[0]):
        n = -(-int(hw[r]) // P)
        assert (bt[r, :n] >= 0).all(), (r, bt[r, :n])
        assert (bt[r, n:] == -1).all(), r
        for b in range(n):
            holders[int(bt[r, b])].append((r, b))
    assert not (free_set & set(holders)), "a held page is on the free stack"
    assert len(free_set) + len(holders) == num_pages, "a page is neither free nor held"
    for page in range(num_pages):
        h = holders.get(page, [])
        assert int(shares[page]) == max(len(h) - 1, 0), (page, int(shares[page]), h)
        if len(h) > 1:
            for r, b in h:
                assert (b + 1) * P <= int(lens[r]), f"shared page {page} at row {r} block {b} can be written"
    assert ctrl[32] == 0, "arrival counter not reset"
    assert not ctrl[64:].any(), "arrival sub-counters not reset"


def bits(t: torch.Tensor) -> np.ndarray:
    from kvgen import to_bits

    return to_bits(t)


ELEMENT_TYPE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


class CColdPool(CPool):
    """A page pool with an fp8 cold store, driven through the C ABI (barq_kv_cold entry points)."""

    def __init__(self, *, window, num_cold=None, **kw):
        self.window = int(window)
        super().__init__(**kw)
        dev = self.kp.device
        n = num_cold or self.max_batch * self.max_blocks
        u8 = dict(dtype=torch.uint8, device=dev)
        self.kc = torch.empty((n, self.page_size, self.heads, self.dim), **u8)
        self.vc = torch.empty_like(self.kc)
        self.ks = torch.empty((n, self.heads, self.dim), **u8)
        self.vs = torch.empty((n, self.page_size, self.heads), **u8)
        self.free_cold = torch.empty((n,), dtype=torch.int32, device=dev)
        self.cold_shares = torch.empty((n,), dtype=torch.int32, device=dev)
        self.num_cold = n
        self.cs = _capi.BarqKVCold(self.kc.data_ptr(), self.vc.data_ptr(), self.ks.data_ptr(), self.vs.data_ptr(),
                                   self.free_cold.data_ptr(), self.cold_shares.data_ptr(), n, self.window,
                                   ELEMENT_TYPE[self.dtype])
        self.cold_reset()

    @property
    def cref(self):
        return ctypes.byref(self.cs)

    def cold_reset(self):
        _capi.check(self.lib.barq_kv_cold_reset(self.ref, self.cref, self._stream()))

    def reset(self, order=None):
        super().reset(order)
        if hasattr(self, "cs"):
            self.cold_reset()

    def compress(self, batch):
        _capi.check(self.lib.barq_kv_compress(self.ref, self.cref, batch, self._stream()))

    def append_rows(self, rows, k, v):
        """k[i], v[i] appended to row rows[i]: barq_kv_append over the one-row view of each row's
        metadata (block-table row, length, mark), the free stack shared."""
        for i, r in enumerate(rows):
            one = _capi.BarqKVPool(*[getattr(self.s, f) for f, _ in _capi.BarqKVPool._fields_])
            one.block_table = self.bt[r:r + 1].data_ptr()
            one.seq_lens = self.lens[r:r + 1].data_ptr()
            one.high_water = self.hw[r:r + 1].data_ptr()
            one.max_batch = 1
            ki, vi = k[i:i + 1], v[i:i + 1]
            _capi.check(self.lib.barq_kv_append(ctypes.byref(one), ki.data_ptr(), vi.data_ptr(), 1, ki.shape[2],
                                                ki.stride(0), ki.stride(1), ki.stride(2), self._stream()))

    def gather(self, batch, seq, flags=0, out=None):
        ko, vo = out or self.new_out(batch, seq)
        _capi.check(self.lib.barq_kv_gather_cold(self.ref, self.cref, ko.data_ptr(), vo.data_ptr(), batch, seq,
                                                 ko.stride(0), ko.stride(1), ko.stride(2), flags, self._stream()))
        return ko, vo

    def update(self, k, v, seq, flags=0, out=None):
        ko, vo = out or self.new_out(k.shape[0], seq)
        _capi.check(self.lib.barq_kv_update_cold(self.ref, self.cref, k.data_ptr(), v.data_ptr(), k.shape[0],
                                                 k.shape[2], k.stride(0), k.stride(1), k.stride(2), ko.data_ptr(),
                                                 vo.data_ptr(), seq, ko.stride(0), ko.stride(1), ko.stride(2), flags,
                                                 self._stream()))
        return ko, vo

    def free_rows(self, rows):
        idx = torch.tensor(rows, dtype=torch.int32, device=self.kp.device)
        _capi.check(self.lib.barq_kv_free_rows_cold(self.ref, self.cref, idx.data_ptr(), len(rows), self._stream()))
        torch.cuda.current_stream().synchronize()

    def select_rows(self, rows):
        idx = torch.tensor(rows or [0], dtype=torch.int32, device=self.kp.device)
        words = self.lib.barq_kv_select_workspace_words(self.ref, 1, len(rows))
        assert words > 0
        ws = torch.empty(words, dtype=torch.int32, device=self.kp.device)
        _capi.check(self.lib.barq_kv_select_rows_cold_layers(self.ref, self.cref, 1, idx.data_ptr(), len(rows),
                                                             ws.data_ptr(), ws.numel(), self._stream()))
        torch.cuda.current_stream().synchronize()

    def crop(self, batch, max_length):
        _capi.check(self.lib.barq_kv_crop_cold(self.ref, self.cref, batch, max_length, self._stream()))

    def check_invariants(self, window=None):
        """Per row: blocks below the high-water mark hold a page (cold ones first, as a prefix).
        Hot pages are held once; a cold page held by k blocks has cold_shares k - 1; each stack
        holds exactly the pages no block holds."""
        P = self.page_size
        bt = self.bt.cpu().numpy()
        hw = self.hw.cpu().numpy()
        ctrl = self.ctrl.cpu().numpy()
        hot, cold = [], []
        for r in range(self.max_batch):
            n = -(-int(hw[r]) // P)
            row = bt[r, :n]
            c = int((row <= -2).sum())
            assert (row[:c] <= -2).all() and (row[c:] >= 0).all(), (r, row)
            assert (bt[r, n:] == -1).all()
            cold += (-2 - row[:c]).tolist()
            hot += row[c:].tolist()
        free = set(self.free.cpu().numpy()[: int(ctrl[0])].tolist())
        free_c = set(self.free_cold.cpu().numpy()[: int(ctrl[2])].tolist())
        held_c = np.bincount(np.asarray(cold, dtype=np.int64), minlength=self.num_cold)
        shares_c = self.cold_shares.cpu().numpy()
        assert len(set(hot)) == len(hot)
        assert (shares_c == np.maximum(held_c - 1, 0)).all()
        assert not free & set(hot) and not free_c & set(cold)
        assert len(free) == int(ctrl[0]) and len(free_c) == int(ctrl[2])
        assert len(hot) + len(free) == self.num_pages and int((held_c > 0).sum()) + len(free_c) == self.num_cold


def attend_cold(pool: "CColdPool", q, *, scale=None, out_f32=True, max_seq=0, split_tokens=0):
    """barq_kv_decode_attention_cold over a CColdPool; returns out [B, Hq, T, D]."""
    B, Hq, T, D = q.shape
    need = pool.lib.barq_kv_attention_workspace_bytes(pool.ref, B, Hq, T, max_seq, split_tokens)
    assert need >= 0
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=pool.kp.device)
    dt = torch.float32 if out_f32 else pool.dtype
    out = torch.full((B, T, Hq, D), float("nan"), dtype=dt, device=pool.kp.device).transpose(1, 2)
    flags = (1 if pool.dtype == torch.float16 else 0) | (2 if out_f32 else 0)
    scale = D ** -0.5 if scale is None else scale
    _capi.check(pool.lib.barq_kv_decode_attention_cold(
        pool.ref, pool.cref, q.data_ptr(), B, Hq, T, q.stride(0), q.stride(1), q.stride(2), out.data_ptr(),
        out.stride(0), out.stride(1), out.stride(2), scale, max_seq, split_tokens, flags, ws.data_ptr(),
        ws.numel(), pool._stream()))
    return out
