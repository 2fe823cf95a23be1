"""The reference CPU path in torch -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` may import this module: it is the
CPU baseline the benchmark times on the host's cores, and is checked against the numpy oracle
(``oracle/kv_oracle.py``) by ``tests/test_oracle.py``.  The product never imports it.

``DenseLayerTorch`` restates, with torch CPU tensors in the cache's own dtype, the reference
layer's storage and CPU append exactly as ``python/barqtrain/kv_cache.py`` writes them: the dense
``[max_batch, kv_heads, max_blocks, page_size, head_dim]`` tensors of ``lazy_initialization``
(:53-73), one slice assignment per (row, token) in ``_python_append`` (:75-91), and
``current_tensors`` (:120-133) as the reference's view ``cache[:B].view(B, H, MB * P, D)[..., :S, :]``
followed by ``.contiguous()`` (the copy an attention kernel would read; torch runs it on its
intra-op threads).  Every operation is a copy, so results are bit-identical to the numpy oracle's.
"""

from __future__ import annotations

import math
from typing import Sequence

import torch


class DenseLayerTorch:
    def __init__(self, max_batch_size: int, max_cache_len: int, page_size: int = 16):
        # kv_cache.py:42-51
        self.max_batch_size = int(max_batch_size)
        self.max_cache_len = int(max_cache_len)
        self.page_size = int(page_size)
        self.max_blocks = math.ceil(self.max_cache_len / self.page_size)
        self.keys = self.values = self.seq_lens = None
        self.current_batch_size = 0

    def lazy_initialization(self, key_states: torch.Tensor) -> None:
        # kv_cache.py:53-73
        batch, heads, _, dim = key_states.shape
        if batch > self.max_batch_size:
            raise ValueError(f"batch_size={batch} exceeds max_batch_size={self.max_batch_size} for paged KV cache")
        shape = (self.max_batch_size, heads, self.max_blocks, self.page_size, dim)
        self.keys = torch.zeros(shape, dtype=key_states.dtype)
        self.values = torch.zeros_like(self.keys)
        self.seq_lens = torch.zeros((self.max_batch_size,), dtype=torch.int32)
        self.current_batch_size = batch

    def append(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        # kv_cache.py:93-118 (CPU branch) and _python_append :75-91
        if self.keys is None:
            self.lazy_initialization(key_states)
        key_states = key_states.contiguous()
        value_states = value_states.contiguous()
        batch, _, tokens, _ = key_states.shape
        for b in range(batch):
            start = int(self.seq_lens[b].item())
            end = start + tokens
            if end > self.max_cache_len:
                raise ValueError(f"paged KV cache capacity exceeded: requested {end}, max_cache_len={self.max_cache_len}")
            for t in range(tokens):
                pos = start + t
                blk, off = pos // self.page_size, pos % self.page_size
                self.keys[b, :, blk, off, :] = key_states[b, :, t, :]
                self.values[b, :, blk, off, :] = value_states[b, :, t, :]
            self.seq_lens[b] = end
        self.current_batch_size = batch

    def get_seq_length(self) -> int:
        # kv_cache.py:150-153
        if self.keys is None or self.current_batch_size == 0:
            return 0
        return int(self.seq_lens[: self.current_batch_size].max().item())

    def current_tensors(self) -> tuple[torch.Tensor, torch.Tensor]:
        # kv_cache.py:120-133, then the copy to contiguous K/V
        B = self.current_batch_size
        S = self.get_seq_length()
        H, D = self.keys.shape[1], self.keys.shape[-1]
        flat = self.max_blocks * self.page_size
        k = self.keys[:B].view(B, H, flat, D)[..., :S, :].contiguous()
        v = self.values[:B].view(B, H, flat, D)[..., :S, :].contiguous()
        return k, v

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        # kv_cache.py:135-142
        self.append(key_states, value_states)
        return self.current_tensors()

    def append_rows(self, rows: Sequence[int], key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Append states[i] to row rows[i]: the per-row body of _python_append (kv_cache.py:77-90)
        over a chosen set of rows (the page pool's append_rows)."""
        key_states = key_states.contiguous()
        value_states = value_states.contiguous()
        tokens = key_states.shape[2]
        for i, r in enumerate(rows):
            start = int(self.seq_lens[r].item())
            end = start + tokens
            if end > self.max_cache_len:
                raise ValueError(f"paged KV cache capacity exceeded: requested {end}, max_cache_len={self.max_cache_len}")
            for t in range(tokens):
                pos = start + t
                self.keys[r, :, pos // self.page_size, pos % self.page_size, :] = key_states[i, :, t, :]
                self.values[r, :, pos // self.page_size, pos % self.page_size, :] = value_states[i, :, t, :]
            self.seq_lens[r] = end

    def release_rows(self, rows: Sequence[int]) -> None:
        """A freed row returns to its lazy_initialization state (zero data, zero length)."""
        for r in rows:
            self.keys[r].zero_()
            self.values[r].zero_()
            self.seq_lens[r] = 0
