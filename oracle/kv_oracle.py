"""CPU oracle for the paged KV-cache path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module, and only as the checker.  The product (``barqtrain_amd``) never imports,
calls or falls back to it.

It restates, in numpy, the reference implementation of BarqTrain's paged KV cache:

* ``DenseLayerOracle`` -- ``BarqPagedKVCacheLayer`` (python/barqtrain/kv_cache.py:37-194) on
  its own dense layout ``[max_batch, kv_heads, max_blocks, page_size, head_dim]`` with the
  per-(row, token) CPU append ``_python_append`` (kv_cache.py:75-91) and the "gather"
  ``current_tensors`` (kv_cache.py:120-133) materialised with a copy.
* ``dense_append_reference`` -- the CUDA path ``paged_kv_append_cuda`` /
  ``paged_kv_append_kernel`` (csrc/kernels/paged_kv_cache.cu:15-54,58-128).

Element payloads are handled as raw bits: every array is an unsigned integer array of the
element width (uint16 for bf16 / fp16, uint32 for fp32, uint64 for fp64), because every
operation on this path is a copy and index computation.  Equality is therefore bit equality,
NaN payloads included.

Pinning (tests/test_oracle.py): the known-answer case of the reference's own test
(tests/test_kv_cache.py:24-47, fixture tests/golden/known_answer_update.json), the library
routine ``transformers.DynamicLayer.update`` (concatenation along the sequence axis) for
uniform appends, an independent slot-history replay for ragged appends, crop, reset and beam
operations, and invariants (``seq_lens`` arithmetic, capacity errors, zero padding).  Planted
mistakes in this module are shown to fail those checks.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np

__all__ = [
    "CapacityError",
    "DenseLayerOracle",
    "dense_append_reference",
    "bits_dtype",
]


class CapacityError(ValueError):
    """Raised where the reference raises ``ValueError`` for a full cache (kv_cache.py:80-83)."""


def bits_dtype(elem_bytes: int) -> np.dtype:
    """Unsigned integer dtype that carries one element's bits."""
    return {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[int(elem_bytes)]


class DenseLayerOracle:
    """Restatement of ``BarqPagedKVCacheLayer`` (python/barqtrain/kv_cache.py:37-194).

    Inputs ``key_states`` / ``value_states`` are numpy arrays ``[batch, kv_heads, tokens,
    head_dim]`` of an unsigned bits dtype.
    """

    def __init__(self, max_batch_size: int, max_cache_len: int, page_size: int = 16):
        # kv_cache.py:42-51
        self.max_batch_size = int(max_batch_size)
        self.max_cache_len = int(max_cache_len)
        self.page_size = int(page_size)
        self.max_blocks = math.ceil(self.max_cache_len / self.page_size)
        self.seq_lens: Optional[np.ndarray] = None
        self.keys: Optional[np.ndarray] = None
        self.values: Optional[np.ndarray] = None
        self.dtype = None
        self.current_batch_size = 0
        self.is_initialized = False

    # kv_cache.py:53-73
    def lazy_initialization(self, key_states: np.ndarray) -> None:
        if key_states.ndim != 4:
            raise ValueError("key_states must have shape [batch, kv_heads, seq, head_dim]")
        batch_size, num_kv_heads, _, head_dim = key_states.shape
        if batch_size > self.max_batch_size:
            raise ValueError(
                f"batch_size={batch_size} exceeds max_batch_size={self.max_batch_size} for paged KV cache"
            )
        self.dtype = key_states.dtype
        self.current_batch_size = batch_size
        shape = (self.max_batch_size, num_kv_heads, self.max_blocks, self.page_size, head_dim)
        self.keys = np.zeros(shape, dtype=self.dtype)
        self.values = np.zeros_like(self.keys)
        self.seq_lens = np.zeros((self.max_batch_size,), dtype=np.int32)
        self.is_initialized = True

    # kv_cache.py:75-91 -- the reference's CPU path: one slice assignment per (row, token).
    # A row that overflows raises after the rows before it were appended, as in the reference.
    def _python_append(self, key_states: np.ndarray, value_states: np.ndarray) -> None:
        batch_size, _, token_count, _ = key_states.shape
        for batch_idx in range(batch_size):
            start = int(self.seq_lens[batch_idx])
            end = start + token_count
            if end > self.max_cache_len:
                raise CapacityError(
                    f"paged KV cache capacity exceeded: requested {end}, max_cache_len={self.max_cache_len}"
                )
            for token_idx in range(token_count):
                absolute_pos = start + token_idx
                block_idx = absolute_pos // self.page_size
                page_offset = absolute_pos % self.page_size
                self.keys[batch_idx, :, block_idx, page_offset, :] = key_states[batch_idx, :, token_idx, :]
                self.values[batch_idx, :, block_idx, page_offset, :] = value_states[batch_idx, :, token_idx, :]
            self.seq_lens[batch_idx] = end
        self.current_batch_size = batch_size

    # kv_cache.py:93-118 (CPU branch, :118)
    def append(self, key_states: np.ndarray, value_states: np.ndarray) -> None:
        if not self.is_initialized:
            self.lazy_initialization(key_states)
        if key_states.shape != value_states.shape:
            raise ValueError("key_states and value_states must have identical shapes")
        if key_states.dtype != self.dtype or value_states.dtype != self.dtype:
            raise ValueError("key_states and value_states must stay in the cache dtype")
        if key_states.shape[0] > self.max_batch_size:
            raise ValueError("batch size exceeds the configured paged KV cache capacity")
        self._python_append(np.ascontiguousarray(key_states), np.ascontiguousarray(value_states))

    # kv_cache.py:120-127
    def _flatten_pages(self, cache_tensor: np.ndarray) -> np.ndarray:
        batch_size = self.current_batch_size or cache_tensor.shape[0]
        return cache_tensor[:batch_size].reshape(
            batch_size, cache_tensor.shape[1], self.max_blocks * self.page_size, cache_tensor.shape[-1]
        )

    # kv_cache.py:129-133, materialised (the reference returns a strided view; the copy is the
    # contiguous K/V an attention kernel would read)
    def current_tensors(self) -> tuple[np.ndarray, np.ndarray]:
        seq_len = self.get_seq_length()
        keys = np.ascontiguousarray(self._flatten_pages(self.keys)[..., :seq_len, :])
        values = np.ascontiguousarray(self._flatten_pages(self.values)[..., :seq_len, :])
        return keys, values

    # kv_cache.py:135-142
    def update(self, key_states: np.ndarray, value_states: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        self.append(key_states, value_states)
        return self.current_tensors()

    # kv_cache.py:144-148
    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + int(query_length), 0

    # kv_cache.py:150-153
    def get_seq_length(self) -> int:
        if not self.is_initialized or self.seq_lens is None or self.current_batch_size == 0:
            return 0
        return int(self.seq_lens[: self.current_batch_size].max())

    # kv_cache.py:155-156
    def get_max_cache_shape(self) -> int:
        return self.max_cache_len

    # kv_cache.py:158-164
    def crop(self, max_length: int) -> None:
        if not self.is_initialized or self.seq_lens is None:
            return
        if max_length < 0:
            max_length = self.get_seq_length() - abs(max_length)
        max_length = max(max_length, 0)
        np.minimum(self.seq_lens[: self.current_batch_size], max_length,
                   out=self.seq_lens[: self.current_batch_size])

    # kv_cache.py:166-173
    def batch_repeat_interleave(self, repeats: int) -> None:
        if not self.is_initialized or self.current_batch_size == 0:
            return
        self.keys = np.repeat(self.keys[: self.current_batch_size], repeats, axis=0)
        self.values = np.repeat(self.values[: self.current_batch_size], repeats, axis=0)
        self.seq_lens = np.repeat(self.seq_lens[: self.current_batch_size], repeats, axis=0)
        self.current_batch_size = self.keys.shape[0]
        self.max_batch_size = self.current_batch_size

    # kv_cache.py:175-183
    def batch_select_indices(self, indices: Sequence[int]) -> None:
        if not self.is_initialized or self.current_batch_size == 0:
            return
        indices = np.asarray(indices, dtype=np.int64)
        self.keys = np.take(self.keys[: self.current_batch_size], indices, axis=0)
        self.values = np.take(self.values[: self.current_batch_size], indices, axis=0)
        self.seq_lens = np.take(self.seq_lens[: self.current_batch_size], indices, axis=0)
        self.current_batch_size = self.keys.shape[0]
        self.max_batch_size = self.current_batch_size

    # kv_cache.py:185-186
    def reorder_cache(self, beam_idx: Sequence[int]) -> None:
        self.batch_select_indices(beam_idx)

    # kv_cache.py:188-194
    def reset(self) -> None:
        if not self.is_initialized:
            return
        self.keys[...] = 0
        self.values[...] = 0
        self.seq_lens[...] = 0
        self.current_batch_size = 0

    # Appending to chosen rows (the page pool's append_rows, no reference counterpart): for each
    # row, the per-row body of _python_append (kv_cache.py:77-90) -- the reference appends to
    # rows [0, batch) one row at a time, so this is the same loop over a chosen set of rows.
    def append_rows(self, rows: Sequence[int], key_states: np.ndarray, value_states: np.ndarray) -> None:
        if not self.is_initialized:
            self.lazy_initialization(key_states)
        token_count = key_states.shape[2]
        for i, r in enumerate(rows):
            start = int(self.seq_lens[r])
            end = start + token_count
            if end > self.max_cache_len:
                raise CapacityError(
                    f"paged KV cache capacity exceeded: requested {end}, max_cache_len={self.max_cache_len}"
                )
            for token_idx in range(token_count):
                pos = start + token_idx
                self.keys[r, :, pos // self.page_size, pos % self.page_size, :] = key_states[i, :, token_idx, :]
                self.values[r, :, pos // self.page_size, pos % self.page_size, :] = value_states[i, :, token_idx, :]
            self.seq_lens[r] = end

    # Free-and-reallocate of one row (the page pool's free_rows, no reference counterpart):
    # the row returns to the state lazy_initialization gives it -- zero data, zero length.
    def release_rows(self, rows: Sequence[int]) -> None:
        for r in rows:
            self.keys[r] = 0
            self.values[r] = 0
            self.seq_lens[r] = 0


def dense_append_reference(key_cache: np.ndarray, value_cache: np.ndarray, seq_lens: np.ndarray,
                           key_states: np.ndarray, value_states: np.ndarray) -> None:
    """In-place restatement of ``paged_kv_append_cuda`` (csrc/kernels/paged_kv_cache.cu:58-128).

    ``key_cache`` / ``value_cache``: ``[cache_batch, H, max_blocks, P, D]``; ``seq_lens`` int
    array ``[>= B]``; states ``[B, H, T, D]``.  Raises ``RuntimeError`` with the reference text
    when ``max(seq_lens[:B]) + T > max_blocks * P`` (:92-99) before touching anything; slots
    whose block is ``>= max_blocks`` are skipped (:42-44); then ``seq_lens[:B] += T`` (:127).
    """
    batch, heads, tokens, _ = key_states.shape
    max_blocks, page_size = key_cache.shape[2], key_cache.shape[3]
    max_cache_len = max_blocks * page_size
    if batch > key_cache.shape[0]:
        raise RuntimeError("key_cache batch dimension is too small")
    if batch > seq_lens.shape[0]:
        raise RuntimeError("seq_lens batch dimension is too small")
    if batch == 0:
        return
    max_start = int(seq_lens[:batch].astype(np.int64).max())
    if max_start + tokens > max_cache_len:
        raise RuntimeError(
            f"paged KV cache capacity exceeded: requested {max_start + tokens} tokens, max_cache_len={max_cache_len}"
        )
    for b in range(batch):  # paged_kv_cache.cu:36-53, one (b, t) at a time, all heads at once
        start = int(seq_lens[b])
        for t in range(tokens):
            pos = start + t
            blk, off = pos // page_size, pos % page_size
            if blk >= max_blocks:
                continue
            key_cache[b, :, blk, off, :] = key_states[b, :, t, :]
            value_cache[b, :, blk, off, :] = value_states[b, :, t, :]
    seq_lens[:batch] += tokens
