"""One layer's page pool: pages, block table, row lengths and the free-page stack.

Device layout (see include/barq_kv.h):

* ``key_pages`` / ``value_pages``: ``[num_pages, page_size, kv_heads, head_dim]`` -- one token's
  K (or V) over all heads is one contiguous run, the run HF attention produces.
* ``block_table``: int32 ``[max_batch, max_blocks]``, page id or -1.
* ``seq_lens`` / ``high_water``: int32 ``[max_batch]``.  Slots ``[0, high_water)`` of a row have
  been written; a gathered slot at or past ``high_water`` is zero, which reproduces the
  zero-initialised dense cache of the reference (python/barqtrain/kv_cache.py:66-71) and its
  crop that keeps data (:158-164).
* ``free_pages``: int32 stack, ``ctrl[0]`` entries free; ``ctrl``: int32 ``[64]``.

The host keeps a shadow of every row's length and high-water mark and of the free-page count.
The shadow is updated by the same arithmetic the kernels apply, so capacity and pool checks,
``get_seq_length`` and output shapes never read the device: a decode step issues no host sync.

GPU tensors (device type ``cuda`` on ROCm PyTorch) always go through the HIP kernels of
``barqtrain_cuda`` and raise if that module is missing.  Tensors in host memory -- which the
reference layer also accepts (kv_cache.py:107,118) -- are served by ``_HostOps``, the same
algorithm (same page-allocation order) written with torch CPU operators.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

CTRL_WORDS = 1088  # BARQ_KV_CTRL_WORDS of include/barq_kv.h: 64 + 16 arrival sub-counters x 64
CTRL_FREE_TOP = 0
CTRL_ERRORS = 1
CTRL_COLD_TOP = 2  # BARQ_KV_CTRL_COLD_TOP: free entries of a cold store's free_cold
ERRBIT_POOL_EXHAUSTED = 1
ERRBIT_CAPACITY = 2
ERRBIT_BAD_INDEX = 4
ERRBIT_OUT_SHORT = 8
ERRBIT_ATTN_SHORT = 16
SEQ_FROM_DEVICE = 1
NO_COMPRESS = 4  # BARQ_KV_NO_COMPRESS: an update of a quantised pool skips its compress launch
SEPARATE_FINALIZE = 2


class PagedKVCapacityError(ValueError, RuntimeError):
    """A row would exceed the cache capacity.

    The reference raises ``ValueError`` on its CPU path (kv_cache.py:80-83) and
    ``RuntimeError`` on its CUDA path (paged_kv_cache.cu:94-99); this class is both.
    """


class PagedKVPoolExhausted(PagedKVCapacityError):
    """The pool has fewer free pages than an append needs."""


def _gpu_backend():
    from barqtrain_amd import kv_cache

    backend = kv_cache._get_cuda_backend()
    if backend is None or not hasattr(backend, "pool_update_"):
        raise RuntimeError(
            "barqtrain: the HIP backend module barqtrain_cuda is not available; build it with "
            "`python -m barqtrain_amd.build` (GPU tensors have no other code path)"
        )
    return backend


class PagePool:
    """Page pool of one cache layer."""

    def __init__(
        self,
        *,
        max_batch: int,
        max_blocks: int,
        page_size: int,
        kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device | str,
        num_pages: Optional[int] = None,
        page_order: Optional[torch.Tensor] = None,
    ):
        self.max_batch = int(max_batch)
        self.max_blocks = int(max_blocks)
        self.page_size = int(page_size)
        self.kv_heads = int(kv_heads)
        self.head_dim = int(head_dim)
        self.dtype = dtype
        self.device = torch.device(device)
        # Default: every row at capacity, plus one page per row for the copies a beam selection
        # makes before the pages it drops return (at most one per row while no crop intervenes).
        self.num_pages = int(num_pages) if num_pages is not None else self.max_batch * (self.max_blocks + 1)
        if min(self.max_batch, self.max_blocks, self.page_size, self.kv_heads, self.head_dim, self.num_pages) < 1:
            raise ValueError("page pool dimensions must be positive")
        if self.num_pages >= 2**31 or self.max_batch * self.max_blocks >= 2**31:
            raise ValueError("page pool too large for int32 page ids")
        shape = (self.num_pages, self.page_size, self.kv_heads, self.head_dim)
        # Pages are not cleared: a slot is only ever read after it was written.
        self.key_pages = torch.empty(shape, dtype=dtype, device=self.device)
        self.value_pages = torch.empty(shape, dtype=dtype, device=self.device)
        i32 = dict(dtype=torch.int32, device=self.device)
        self.block_table = torch.empty((self.max_batch, self.max_blocks), **i32)
        self.seq_lens = torch.empty((self.max_batch,), **i32)
        self.high_water = torch.empty((self.max_batch,), **i32)
        self.free_pages = torch.empty((self.num_pages,), **i32)
        self.ctrl = torch.empty((CTRL_WORDS,), **i32)
        self.page_shares = torch.empty((self.num_pages,), **i32)
        self.lens = np.zeros(self.max_batch, dtype=np.int64)
        self.hw = np.zeros(self.max_batch, dtype=np.int64)
        self.free_count = self.num_pages
        self.free_exact = True   # free_count equals the device's free stack (else a lower bound)
        self.shared = False      # some page may be held by more than one block
        self.tails_shared = False  # a crop may have left shared pages in rows' tails
        self.generation = 0      # bumped whenever the tensors are replaced (cached pool groups)
        self.reset(page_order)

    # ------------------------------------------------------------------ plumbing
    @property
    def on_gpu(self) -> bool:
        return self.device.type == "cuda"

    @property
    def tensors(self) -> list[torch.Tensor]:
        return [self.key_pages, self.value_pages, self.block_table, self.seq_lens,
                self.high_water, self.free_pages, self.ctrl, self.page_shares]

    @property
    def capacity(self) -> int:
        return self.max_blocks * self.page_size

    def _ops(self):
        return _gpu_backend() if self.on_gpu else _HostOps

    def _index_tensor(self, rows: Sequence[int]) -> torch.Tensor:
        """Row indices as int32 on the pool's device, copied from pinned memory without waiting
        for the stream (a plain host-to-device copy would synchronise it)."""
        host = torch.tensor(rows, dtype=torch.int32)
        if not self.on_gpu:
            return host
        return host.pin_memory().to(self.device, non_blocking=True)

    # ------------------------------------------------------------------ host shadow
    def new_block_counts(self, batch: int, tokens: int) -> np.ndarray:
        """Blocks each row [0, batch) maps for the first time when `tokens` are appended."""
        if tokens <= 0 or batch <= 0:
            return np.zeros(max(batch, 0), dtype=np.int64)
        P = self.page_size
        first = -(-self.hw[:batch] // P)
        end = np.minimum(-(-(self.lens[:batch] + tokens) // P), self.max_blocks)
        return np.maximum(end - first, 0)

    def check_append(self, batch: int, tokens: int, max_length: Optional[int] = None) -> int:
        """Raise if appending would pass `max_length` (default: the block capacity) or drain the
        pool; return the number of pages the append takes."""
        return self._plan_append(batch, tokens, max_length)[0]

    def _plan_append(self, batch: int, tokens: int, max_length: Optional[int]) -> tuple[int, int]:
        """check_append's work, returning (pages taken, longest row after the append).  Every
        update passes here, so the arithmetic on the rows' shadow is kept to a few array ops
        (each costs about a microsecond on a decode batch)."""
        limit = self.capacity if max_length is None else int(max_length)
        if batch > self.max_batch:
            raise ValueError("batch size exceeds the configured paged KV cache capacity")
        if batch <= 0 or tokens <= 0:
            return 0, self.max_len(batch)
        lens = self.lens[:batch]
        worst = int(lens.max()) + tokens
        if worst > limit or worst > self.capacity:
            raise PagedKVCapacityError(
                f"paged KV cache capacity exceeded: requested {worst}, max_cache_len={limit}"
            )
        # blocks mapped for the first time: ceil((len + T) / P) - ceil(hw / P) where positive (no
        # row passes max_blocks: worst <= capacity was checked above)
        P = self.page_size
        end = lens + (tokens + P - 1)
        end //= P
        end -= (self.hw[:batch] + (P - 1)) // P
        need = int(np.maximum(end, 0, out=end).sum())
        self.ensure_free(need, "append")
        return need, worst

    def ensure_free(self, need: int, what: str) -> None:
        """Raise PagedKVPoolExhausted unless `need` pages are free.  After shared-page operations
        the host count is a lower bound; it is refreshed from the device (a synchronisation)
        only when it would refuse."""
        if need > self.free_count and not self.free_exact:
            self.free_count = int(self.ctrl[CTRL_FREE_TOP].item())
            self.free_exact = True
        if need > self.free_count:
            raise PagedKVPoolExhausted(
                f"paged KV page pool exhausted: {what} needs {need} pages, {self.free_count} free"
            )

    def _advance(self, batch: int, tokens: int, need: int) -> None:
        if batch <= 0 or tokens <= 0:
            return
        lens, hw = self.lens[:batch], self.hw[:batch]
        lens += tokens
        np.maximum(hw, lens, out=hw)
        self.free_count -= need

    def max_len(self, batch: int) -> int:
        return int(self.lens[:batch].max()) if batch > 0 else 0

    # ------------------------------------------------------------------ operations
    def reset(self, page_order: Optional[torch.Tensor] = None) -> None:
        """Free every page; row lengths and high-water marks to zero.  O(metadata)."""
        if page_order is not None:
            page_order = page_order.to(device=self.device, dtype=torch.int32).contiguous()
            if page_order.numel() != self.num_pages or not torch.equal(
                    torch.sort(page_order).values,
                    torch.arange(self.num_pages, dtype=torch.int32, device=self.device)):
                raise ValueError("page_order must list every page of the pool exactly once")
        self._ops().pool_reset_(self.tensors, page_order)
        self.lens[:] = 0
        self.hw[:] = 0
        self.free_count = self.num_pages
        self.free_exact = True
        self.shared = False
        self.tails_shared = False

    def _check_states(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        if key_states.dim() != 4 or key_states.shape != value_states.shape:
            raise ValueError("key_states and value_states must have identical [batch, kv_heads, seq, head_dim] shapes")
        if key_states.shape[1] != self.kv_heads or key_states.shape[3] != self.head_dim:
            raise ValueError("key_states kv_heads/head_dim do not match the cache")

    @staticmethod
    def _compatible_pair(key_states: torch.Tensor, value_states: torch.Tensor):
        """K and V as views the kernels take: unit stride along head_dim and one layout for both
        (strides of size-1 dimensions do not count: HF decode steps pass K and V that differ only
        in the stride of their size-1 sequence dimension).  Copies only when needed."""
        same = all(n == 1 or a == b for n, a, b in zip(key_states.shape, key_states.stride(), value_states.stride()))
        if key_states.stride(-1) != 1 or value_states.stride(-1) != 1 or not same:
            return key_states.contiguous(), value_states.contiguous()
        return key_states, value_states

    def _step(self, key_states, value_states, max_length, flags, gather):
        """One update (gather) or append with the host planning done in the binding (pool_step_):
        returns (key_out, value_out, pages taken), or pages taken < 0 when the call must take the
        checked path (which raises the exact error, or handles an empty call)."""
        backend = _gpu_backend()
        handle = self.__dict__.get("_handle")
        if handle is None or handle[0] != self.generation:
            handle = (self.generation, backend.pool_group([self.tensors]))
            self._handle = handle
        limit = self.capacity if max_length is None else int(max_length)
        ko, vo, need = backend.pool_step_(handle[1], self.key_pages, key_states, value_states, self.lens, self.hw,
                                          self.free_count, self.free_exact, limit, flags, gather)
        if need >= 0:
            self.free_count -= need
        return ko, vo, need

    def append(self, key_states: torch.Tensor, value_states: torch.Tensor,
               max_length: Optional[int] = None) -> None:
        if self.on_gpu and self._step(key_states, value_states, max_length, 0, False)[2] >= 0:
            return
        self._check_states(key_states, value_states)
        batch, _, tokens, _ = key_states.shape
        need = self.check_append(batch, tokens, max_length)
        if batch == 0 or tokens == 0:
            return
        k, v = self._compatible_pair(key_states, value_states)
        self._ops().pool_append_(self.tensors, k, v)
        self._advance(batch, tokens, need)

    def append_rows(self, rows: Sequence[int], key_states: torch.Tensor, value_states: torch.Tensor,
                    max_length: Optional[int] = None) -> None:
        """Append ``key_states[i]`` / ``value_states[i]`` to row ``rows[i]`` (distinct rows, not
        necessarily [0, batch)): a freed row takes a new sequence's prefill while the others keep
        decoding.  Checked in full first (capacity, free pages), then one append launch per row
        over the one-row view of the row metadata -- the same kernels, sharing the free stack,
        so pages come off it in the order of `rows`."""
        self._check_states(key_states, value_states)
        rows = [int(r) for r in rows]
        if len(rows) != key_states.shape[0]:
            raise ValueError("append_rows: one row index per batch entry of the states")
        if len(set(rows)) != len(rows):
            raise ValueError("append_rows: rows must be distinct")
        if any(r < 0 or r >= self.max_batch for r in rows):
            raise IndexError("append_rows: row out of range")
        tokens = key_states.shape[2]
        if not rows or tokens == 0:
            return
        r = np.asarray(rows)
        limit = self.capacity if max_length is None else int(max_length)
        worst = int(self.lens[r].max()) + tokens
        if worst > limit or worst > self.capacity:
            raise PagedKVCapacityError(f"paged KV cache capacity exceeded: requested {worst}, max_cache_len={limit}")
        P = self.page_size
        need = int(np.maximum(-(-(self.lens[r] + tokens) // P) - (-(-self.hw[r] // P)), 0).sum())
        self.ensure_free(need, "append_rows")
        k, v = self._compatible_pair(key_states, value_states)
        t = self.tensors
        ops = self._ops()
        for i, row in enumerate(rows):
            one = t[:2] + [t[2][row:row + 1], t[3][row:row + 1], t[4][row:row + 1]] + t[5:]
            ops.pool_append_(one, k[i:i + 1], v[i:i + 1])
        self.lens[r] += tokens
        self.hw[r] = np.maximum(self.hw[r], self.lens[r])
        self.free_count -= need

    def _new_out(self, batch: int, seq: int) -> tuple[torch.Tensor, torch.Tensor]:
        shape = (batch, self.kv_heads, seq, self.head_dim)
        return (torch.empty(shape, dtype=self.dtype, device=self.device),
                torch.empty(shape, dtype=self.dtype, device=self.device))

    def gather(self, batch: int, seq_out: Optional[int] = None,
               out: Optional[tuple[torch.Tensor, torch.Tensor]] = None,
               flags: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        """Materialise rows [0, batch) as contiguous ``[batch, kv_heads, seq_out, head_dim]``
        (default seq_out: the longest row)."""
        seq = self.max_len(batch) if seq_out is None else int(seq_out)
        if seq > self.capacity:
            raise ValueError("seq_out exceeds the cache capacity")
        ko, vo = out if out is not None else self._new_out(batch, seq)
        if batch > 0 and seq > 0:
            self._ops().pool_gather(self.tensors, ko, vo, batch, seq, flags)
        return ko, vo

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor,
               max_length: Optional[int] = None, out=None, seq_out: Optional[int] = None,
               flags: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        """Append, then materialise rows [0, batch) up to the longest row, in one pass."""
        if self.on_gpu and out is None and seq_out is None:
            ko, vo, need = self._step(key_states, value_states, max_length, flags, True)
            if need >= 0:
                return ko, vo
        self._check_states(key_states, value_states)
        batch, _, tokens, _ = key_states.shape
        need, worst = self._plan_append(batch, tokens, max_length)
        if tokens == 0:
            return self.gather(batch, seq_out, out, flags)
        seq = worst if seq_out is None else int(seq_out)
        ko, vo = out if out is not None else self._new_out(batch, seq)
        k, v = self._compatible_pair(key_states, value_states)
        self._ops().pool_update_(self.tensors, k, v, ko, vo, seq, flags)
        self._advance(batch, tokens, need)
        return ko, vo

    def crop(self, batch: int, max_length: int) -> None:
        """seq_lens[:batch] = min(seq_lens, max_length); data and pages are kept.  When rows
        share pages, the blocks the crop re-opens for writing are given pages of their own."""
        max_length = max(int(max_length), 0)
        if batch <= 0:
            return
        if self.shared:
            # Room for the identity selection below, from the lengths after the crop, before
            # anything changes: every tail block (re-opened for writing) may need a copy.
            lens = self.lens.copy()
            np.minimum(lens[:batch], max_length, out=lens[:batch])
            nb = np.minimum(-(-self.hw // self.page_size), self.max_blocks)
            self.ensure_free(int((nb - np.minimum(lens // self.page_size, nb)).sum()), "crop")
        self._ops().pool_crop_(self.tensors, batch, max_length)
        np.minimum(self.lens[:batch], max_length, out=self.lens[:batch])
        if self.shared:
            # the identity selection moves every exclusive tail page and copies the shared ones
            self.tails_shared = True
            self.select_rows(list(range(self.max_batch)))

    def free_rows(self, rows: Sequence[int]) -> None:
        """Return every page of `rows` to the pool; their lengths become 0."""
        rows = [int(r) for r in rows]
        if len(set(rows)) != len(rows):
            raise ValueError("free_rows: rows must be distinct")
        if any(r < 0 or r >= self.max_batch for r in rows):
            raise IndexError("free_rows: row out of range")
        if not rows:
            return
        self._ops().pool_free_rows_(self.tensors, self._index_tensor(rows))
        r = np.asarray(rows)
        if self.shared:
            self.free_exact = False  # shared pages stay held: the device knows how many returned
        else:
            self.free_count += int(np.minimum(-(-self.hw[r] // self.page_size), self.max_blocks).sum())
        self.lens[r] = 0
        self.hw[r] = 0

    def tail_block_counts(self, rows: np.ndarray) -> np.ndarray:
        """Tail blocks of each row: from the one holding seq_lens up to the high-water mark (the
        blocks an append or a crop can still write, which a selection moves or copies)."""
        nb = np.minimum(-(-self.hw[rows] // self.page_size), self.max_blocks)
        return nb - np.minimum(self.lens[rows] // self.page_size, nb)

    @staticmethod
    def repeated_mask(rows: np.ndarray) -> np.ndarray:
        """True where a selection takes a source row that an earlier new row already took."""
        mask = np.ones(len(rows), dtype=bool)
        mask[np.unique(rows, return_index=True)[1]] = False
        return mask

    def select_copy_bound(self, rows: np.ndarray) -> int:
        """Pages a selection copies, at most: the tails of repeated takers, plus the first
        takers' tails when a crop may have left shared pages there."""
        tails = self.tail_block_counts(rows)
        return int(tails.sum() if self.tails_shared else tails[self.repeated_mask(rows)].sum())

    def select_workspace_words(self, num_rows: int) -> int:
        """int32 words of a one-pool selection's workspace (barq_kv_select_workspace_words)."""
        return num_rows * (self.max_blocks + 3) + self.max_batch + 2

    def _selection(self, src_rows: Sequence[int]) -> np.ndarray:
        rows = np.asarray([int(r) for r in src_rows], dtype=np.int64)
        if len(rows) > self.max_batch:
            raise ValueError("select_rows: more rows than the pool holds")
        if len(rows) and (rows.min() < 0 or rows.max() >= self.max_batch):
            raise IndexError("select_rows: row out of range")
        return rows

    def _selected(self, lens: np.ndarray, hw: np.ndarray, need: int) -> None:
        """Host shadow after a selection: the new rows' lengths and marks (other rows empty).
        Written in place: a captured decode step keeps views of these arrays."""
        self.lens[:] = lens
        self.hw[:] = hw
        self.free_count -= need
        self.free_exact = False   # moves, copies and released pages are settled on the device
        self.shared = True
        self.tails_shared = False

    def select_rows(self, src_rows: Sequence[int]) -> None:
        """In place: row i becomes row src_rows[i] (repeats allowed), every other row empty.
        Full blocks are shared (copy-on-write), so the cost is the rows' partial last blocks,
        not their history (reference: kv_cache.py:166-186, which copies the whole cache)."""
        r = self._selection(src_rows)
        n = len(r)
        need = self.select_copy_bound(r) if n else 0
        self.ensure_free(need, "select_rows")
        words = self.select_workspace_words(n)
        ws = getattr(self, "_select_ws", None)
        if ws is None or ws.numel() < words:
            ws = torch.empty((words,), dtype=torch.int32, device=self.device)
            self._select_ws = ws
        self._ops().pool_select_rows_(self.tensors, self._index_tensor(r.tolist() or [0])[:n], ws)
        lens, hw = np.zeros_like(self.lens), np.zeros_like(self.hw)
        lens[:n], hw[:n] = self.lens[r], self.hw[r]
        self._selected(lens, hw, need)

    def copy_rows(self, src_rows: Sequence[int], num_pages: Optional[int] = None) -> "PagePool":
        """A new pool whose row i copies row src_rows[i] of this one (repeats allowed)."""
        src_rows = [int(r) for r in src_rows]
        if any(r < 0 or r >= self.max_batch for r in src_rows):
            raise IndexError("copy_rows: row out of range")
        n = len(src_rows)
        r = np.asarray(src_rows, dtype=np.int64)
        need = int(np.minimum(-(-self.hw[r] // self.page_size), self.max_blocks).sum()) if n else 0
        if num_pages is None:
            scaled = math.ceil(self.num_pages * max(n, 1) / self.max_batch)
            num_pages = max(need, scaled, 1)
        if need > num_pages:
            raise PagedKVPoolExhausted(f"copy_rows needs {need} pages, pool of {num_pages}")
        dst = PagePool(max_batch=max(n, 1), max_blocks=self.max_blocks, page_size=self.page_size,
                       kv_heads=self.kv_heads, head_dim=self.head_dim, dtype=self.dtype,
                       device=self.device, num_pages=num_pages)
        if n:
            self._ops().pool_copy_rows_(self.tensors, dst.tensors, self._index_tensor(src_rows))
            dst.lens[:n] = self.lens[r]
            dst.hw[:n] = self.hw[r]
            dst.free_count = num_pages - need
        return dst

    def attend(self, query: torch.Tensor, scale: Optional[float] = None, *,
               out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
               split_tokens: int = 0, max_seq: Optional[int] = None) -> torch.Tensor:
        """Decode attention of `query` ``[batch, q_heads, tokens, head_dim]`` over rows
        [0, batch), reading K and V from the pages through the block table (nothing is
        gathered).  Query token i of row b sits at position seq_lens[b] - tokens + i and sees
        positions [0, seq_lens[b] - tokens + i]; q head h reads kv head h // (q_heads //
        kv_heads).  Returns ``[batch, q_heads, tokens, head_dim]`` (a view of a
        ``[batch, tokens, q_heads, head_dim]`` buffer, the layout attention outputs take next)
        in `out_dtype` (default the query's).  `max_seq` bounds the rows' lengths (default:
        the host shadow's longest row; pass the capacity when capturing a graph)."""
        if query.dim() != 4 or query.shape[3] != self.head_dim or query.shape[1] % self.kv_heads:
            raise ValueError("query must be [batch, q_heads, tokens, head_dim] with q_heads a "
                             "multiple of the pool's kv_heads")
        batch, q_heads, tokens, _ = query.shape
        if batch > self.max_batch:
            raise ValueError("query batch exceeds the pool's rows")
        if query.dtype != self.dtype or query.device != self.key_pages.device:
            raise ValueError("query must have the pool's dtype and device")
        scale = 1.0 / math.sqrt(self.head_dim) if scale is None else float(scale)
        if out is None:
            dt = out_dtype or query.dtype
            out = torch.empty((batch, tokens, q_heads, self.head_dim), dtype=dt,
                              device=query.device).transpose(1, 2)
        if batch == 0 or tokens == 0:
            return out
        if max_seq is None:
            max_seq = int(self.lens[:batch].max())
        if not self.on_gpu:
            ko, vo = self.gather(batch, int(self.lens[:batch].max()))
            _HostOps.attention_over(ko, vo, self.lens, query, out, scale, batch)
            return out
        backend = _gpu_backend()
        if query.stride(3) != 1 or query.data_ptr() % 16 or any(s % 8 for s in query.stride()[:3]):
            query = query.contiguous()
        need = backend.attention_workspace_bytes(self.tensors, batch, q_heads, tokens,
                                                 max(int(max_seq), 1), int(split_tokens))
        if need < 0:
            raise ValueError(
                "paged decode attention takes bf16/fp16 pools with head_dim 64, 128 or 256 and at most 16 "
                f"query rows per kv head (got {self.dtype}, head_dim {self.head_dim}, "
                f"{q_heads // self.kv_heads} x {tokens} rows)")
        self._attention_call(backend, query, out, scale, max(int(max_seq), 1), int(split_tokens),
                             self.attention_workspace(need))
        return out

    def _attention_call(self, backend, query, out, scale, max_seq, split_tokens, ws):
        backend.pool_decode_attention(self.tensors, query, out, scale, max_seq, split_tokens, ws)

    def attention_workspace(self, nbytes: int) -> torch.Tensor:
        """The pool's decode-attention workspace (split records), at least `nbytes`; grown, never
        shrunk.  Launches on one stream may share it."""
        ws = getattr(self, "_attn_ws", None)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty((max(int(nbytes), 256),), dtype=torch.uint8, device=self.device)
            self._attn_ws = ws
        return ws

    def errors(self) -> int:
        """Sticky device error bits (reads the device: a synchronisation point)."""
        return int(self.ctrl[CTRL_ERRORS].item())

    def to(self, device) -> "PagePool":
        """Move every tensor of the pool (offload / prefetch)."""
        device = torch.device(device)
        for name in ("key_pages", "value_pages", "block_table", "seq_lens", "high_water", "free_pages", "ctrl",
                     "page_shares"):
            setattr(self, name, getattr(self, name).to(device, non_blocking=True))
        self.device = device
        self.generation += 1
        return self


KV_QUANT_FP8 = "fp8_e4m3"
_ELEMENT_TYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


class QuantPagePool(PagePool):
    """A page pool whose blocks behind each row's residual window are kept as fp8 codes.

    Format (``barq_kv_cold`` in include/barq_kv.h): OCP FP8 E4M3 codes, rounded to nearest even,
    with power-of-two scales stored as E8M0 bytes -- keys one per channel (head, dim) over a
    page's tokens, values one per token (token, head) over head_dim, KIVI's grouping
    (arXiv:2402.02750) -- each the smallest 2^e with max |x| <= 448 * 2^e.  Reads dequantise to
    the cache dtype.  The reference plans this cache (IMPLEMENTATION_PLAN.md:106-129: quantised
    storage, a full-precision residual window, dequant-on-read) and ships none.

    Full-precision ("hot") pages hold each row's last ``window`` tokens and its partial block: an
    append writes there, the blocks that left the window are quantised (``barq_kv_compress``)
    and reads dequantise (``barq_kv_gather_cold``).  Appends longer than ``chunk`` tokens
    (prefill) run in chunks, so a row holds at most ``ceil((window + chunk) / P) + 2`` hot pages,
    and ``ceil(window / P) + 1`` between appends.  The default pool is the sum of the two per row:
    a beam selection copies hot blocks before the ones it drops return, which takes at most the
    second term per row.  The cold store defaults to every block that can lie wholly before the
    window, ``max_batch * (max_blocks - window // P)``.

    Beam selection (``select_rows``) shares quantised blocks between rows by reference (they
    never change) and moves or copies the hot ones, so a hot page always has one holder.  A crop
    below a row's quantised blocks re-opens them: their dequantised contents become hot pages
    again (lossy, as any read of them is) and are quantised anew when they leave the window.
    """

    quantized = True

    def __init__(self, *, max_batch: int, max_blocks: int, page_size: int, kv_heads: int, head_dim: int,
                 dtype: torch.dtype, device: torch.device | str, window: int = 128, chunk: int = 64,
                 num_pages: Optional[int] = None, num_cold: Optional[int] = None,
                 page_order: Optional[torch.Tensor] = None):
        if dtype not in _ELEMENT_TYPES:
            raise ValueError("quantised KV pages need a bfloat16, float16 or float32 cache")
        if int(window) < 0 or int(chunk) < 1:
            raise ValueError("window must be >= 0 and chunk >= 1 tokens")
        self.window = int(window)
        self.chunk = int(chunk)
        P = int(page_size)
        if num_pages is None:
            per_row = (-(-(self.window + self.chunk) // P) + 2) + (-(-self.window // P) + 1)
            num_pages = min(int(max_batch) * per_row, int(max_batch) * (int(max_blocks) + 1))
        # A row's quantised blocks lie wholly before its last `window` tokens.
        default_cold = int(max_batch) * max(int(max_blocks) - self.window // P, 1)
        self.num_cold = int(num_cold) if num_cold is not None else default_cold
        if not 1 <= self.num_cold < 2**31 - 2:
            raise ValueError("num_cold out of range")
        if P * int(kv_heads) > 4096 or int(kv_heads) * int(head_dim) > 16384:
            raise ValueError("quantised pages need page_size * kv_heads <= 4096 and kv_heads * head_dim <= 16384")
        dev = torch.device(device)
        u8 = dict(dtype=torch.uint8, device=dev)
        self.key_codes = torch.empty((self.num_cold, P, int(kv_heads), int(head_dim)), **u8)
        self.value_codes = torch.empty_like(self.key_codes)
        self.key_scales = torch.empty((self.num_cold, int(kv_heads), int(head_dim)), **u8)
        self.value_scales = torch.empty((self.num_cold, P, int(kv_heads)), **u8)
        self.free_cold = torch.empty((self.num_cold,), dtype=torch.int32, device=dev)
        self.cold_shares = torch.empty((self.num_cold,), dtype=torch.int32, device=dev)
        self.cold_blocks = np.zeros(int(max_batch), dtype=np.int64)  # leading quantised blocks per row
        self.cold_free = self.num_cold
        self.cold_exact = True  # cold_free equals the device's cold stack (else a lower bound)
        super().__init__(max_batch=max_batch, max_blocks=max_blocks, page_size=page_size, kv_heads=kv_heads,
                         head_dim=head_dim, dtype=dtype, device=device, num_pages=num_pages,
                         page_order=page_order)

    @property
    def cold_tensors(self) -> list[torch.Tensor]:
        return [self.key_codes, self.value_codes, self.key_scales, self.value_scales, self.free_cold,
                self.cold_shares]

    def reset(self, page_order: Optional[torch.Tensor] = None) -> None:
        super().reset(page_order)
        self._ops().pool_cold_reset_(self.tensors, self.cold_tensors, self.window)
        self.cold_blocks[:] = 0
        self.cold_free = self.num_cold
        self.cold_exact = True

    def ensure_cold(self, need: int) -> None:
        """Raise PagedKVPoolExhausted unless `need` cold pages are free.  After selections the host
        count is a lower bound (a released cold page may still be shared); it is refreshed from
        the device only when it would refuse."""
        if need > self.cold_free and not self.cold_exact:
            self.cold_free = int(self.ctrl[CTRL_COLD_TOP].item())
            self.cold_exact = True
        if need > self.cold_free:
            raise PagedKVPoolExhausted(
                f"paged KV cold store exhausted: quantising needs {need} pages, {self.cold_free} free")

    def _cold_after(self, batch: int, tokens: int) -> tuple[np.ndarray, int]:
        """(frontier after appending `tokens` to rows [0, batch), blocks it newly quantises)."""
        frontier = np.maximum(self.lens[:batch] + tokens - self.window, 0) // self.page_size
        moved = int(np.maximum(frontier - self.cold_blocks[:batch], 0).sum())
        self.ensure_cold(moved)
        return frontier, moved

    def _quantised(self, batch: int, frontier: np.ndarray, moved: int) -> None:
        np.maximum(self.cold_blocks[:batch], frontier, out=self.cold_blocks[:batch])
        self.cold_free -= moved
        self.free_count += moved  # each quantised block returned its full-precision page

    def append(self, key_states: torch.Tensor, value_states: torch.Tensor,
               max_length: Optional[int] = None) -> None:
        self._check_states(key_states, value_states)
        batch, _, tokens, _ = key_states.shape
        if tokens > self.chunk:
            # Every chunk's capacity, hot-page and cold-page needs are checked up front, so an
            # append that cannot finish raises before its first chunk changes anything.
            self._check_chunked(batch, tokens, max_length)
            for s0 in range(0, tokens, self.chunk):
                self.append(key_states[:, :, s0:s0 + self.chunk], value_states[:, :, s0:s0 + self.chunk],
                            max_length)
            return
        need = self.check_append(batch, tokens, max_length)
        if batch == 0 or tokens == 0:
            return
        frontier, moved = self._cold_after(batch, tokens)
        k, v = self._compatible_pair(key_states, value_states)
        ops = self._ops()
        ops.pool_append_(self.tensors, k, v)
        ops.pool_compress_(self.tensors, self.cold_tensors, self.window, batch)
        self._advance(batch, tokens, need)
        self._quantised(batch, frontier, moved)

    def _check_chunked(self, batch: int, tokens: int, max_length: Optional[int],
                       rows: Optional[np.ndarray] = None) -> None:
        """Raise, changing nothing, unless appending `tokens` to rows [0, batch) (or to `rows`) in
        chunks of `chunk` fits: the same capacity rule, hot-page and cold-page arithmetic each
        chunk's append and quantisation apply, run on a copy of the host shadow."""
        limit = self.capacity if max_length is None else int(max_length)
        if batch > self.max_batch:
            raise ValueError("batch size exceeds the configured paged KV cache capacity")
        if batch <= 0 or tokens <= 0:
            return
        r = np.arange(batch) if rows is None else rows
        lens = self.lens[r].copy()
        hw = self.hw[r].copy()
        cold = self.cold_blocks[r].copy()
        worst = int(lens.max()) + tokens
        if worst > limit or worst > self.capacity:
            raise PagedKVCapacityError(
                f"paged KV cache capacity exceeded: requested {worst}, max_cache_len={limit}")
        if not self.free_exact:  # a lower bound: read the device's count once
            self.free_count = int(self.ctrl[CTRL_FREE_TOP].item())
            self.free_exact = True
        if not self.cold_exact:
            self.cold_free = int(self.ctrl[CTRL_COLD_TOP].item())
            self.cold_exact = True
        free, cold_free, P = self.free_count, self.cold_free, self.page_size
        for s0 in range(0, tokens, self.chunk):
            t = min(self.chunk, tokens - s0)
            end = np.minimum(-(-(lens + t) // P), self.max_blocks)
            need = int(np.maximum(end - (-(-hw // P)), 0).sum())
            if need > free:
                raise PagedKVPoolExhausted(
                    f"paged KV page pool exhausted: append needs {need} pages at token {s0}, {free} free")
            free -= need
            lens += t
            np.maximum(hw, lens, out=hw)
            frontier = np.maximum(lens - self.window, 0) // P
            moved = int(np.maximum(frontier - cold, 0).sum())
            if moved > cold_free:
                raise PagedKVPoolExhausted(
                    f"paged KV cold store exhausted: quantising needs {moved} pages, {cold_free} free")
            np.maximum(cold, frontier, out=cold)
            cold_free -= moved
            free += moved

    def gather(self, batch: int, seq_out: Optional[int] = None,
               out: Optional[tuple[torch.Tensor, torch.Tensor]] = None,
               flags: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        seq = self.max_len(batch) if seq_out is None else int(seq_out)
        if seq > self.capacity:
            raise ValueError("seq_out exceeds the cache capacity")
        ko, vo = out if out is not None else self._new_out(batch, seq)
        if batch > 0 and seq > 0:
            self._ops().pool_gather_cold(self.tensors, self.cold_tensors, self.window, ko, vo, batch, seq, flags)
        return ko, vo

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor,
               max_length: Optional[int] = None, out=None, seq_out: Optional[int] = None,
               flags: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        self._check_states(key_states, value_states)
        batch, _, tokens, _ = key_states.shape
        if tokens > self.chunk:
            self.append(key_states, value_states, max_length)
            return self.gather(batch, seq_out, out, flags)
        need = self.check_append(batch, tokens, max_length)
        if tokens == 0 or batch == 0:
            return self.gather(batch, seq_out, out, flags)
        frontier, moved = self._cold_after(batch, tokens)
        seq = int((self.lens[:batch] + tokens).max()) if seq_out is None else int(seq_out)
        ko, vo = out if out is not None else self._new_out(batch, seq)
        k, v = self._compatible_pair(key_states, value_states)
        skip = NO_COMPRESS if moved == 0 else 0  # no block leaves the window: no compress launch
        self._ops().pool_update_cold_(self.tensors, self.cold_tensors, self.window, k, v, ko, vo, seq, flags | skip)
        self._advance(batch, tokens, need)
        self._quantised(batch, frontier, moved)
        return ko, vo

    def crop(self, batch: int, max_length: int) -> None:
        """seq_lens[:batch] = min(seq_lens, max_length).  Quantised blocks from the one holding a
        row's new length on are re-opened as hot pages holding their dequantised contents
        (barq_kv_crop_cold); the room for them is checked before anything changes."""
        m = max(int(max_length), 0)
        if batch <= 0:
            return
        first = np.minimum(self.lens[:batch], m) // self.page_size
        reopened = np.maximum(self.cold_blocks[:batch] - first, 0)
        need = int(reopened.sum())
        self.ensure_free(need, "crop")
        self._ops().pool_crop_cold_(self.tensors, self.cold_tensors, self.window, batch, m)
        np.minimum(self.lens[:batch], m, out=self.lens[:batch])
        np.minimum(self.cold_blocks[:batch], first, out=self.cold_blocks[:batch])
        self.free_count -= need
        if self.shared:
            self.cold_exact = False  # a re-opened block's cold page may stay held by another row
        else:
            self.cold_free += need

    def free_rows(self, rows: Sequence[int]) -> None:
        rows = [int(r) for r in rows]
        if len(set(rows)) != len(rows):
            raise ValueError("free_rows: rows must be distinct")
        if any(r < 0 or r >= self.max_batch for r in rows):
            raise IndexError("free_rows: row out of range")
        if not rows:
            return
        self._ops().pool_free_rows_cold_(self.tensors, self.cold_tensors, self.window, self._index_tensor(rows))
        r = np.asarray(rows)
        nb = np.minimum(-(-self.hw[r] // self.page_size), self.max_blocks)
        cold = np.minimum(self.cold_blocks[r], nb)
        self.free_count += int((nb - cold).sum())  # hot pages have one holder
        if self.shared:
            self.cold_exact = False  # shared cold pages stay held
        else:
            self.cold_free += int(cold.sum())
        self.lens[r] = 0
        self.hw[r] = 0
        self.cold_blocks[r] = 0

    def memory_bytes(self) -> dict:
        """Bytes the pool holds on its device: hot pages, cold codes and scales, metadata."""
        def size(ts):
            return int(sum(t.numel() * t.element_size() for t in ts))

        return {"hot_pages": size(self.tensors[:2]), "cold_store": size(self.cold_tensors[:4]),
                "metadata": size(self.tensors[2:]) + size(self.cold_tensors[4:])}

    def append_rows(self, rows: Sequence[int], key_states: torch.Tensor, value_states: torch.Tensor,
                    max_length: Optional[int] = None) -> None:
        """Append ``key_states[i]`` / ``value_states[i]`` to row ``rows[i]`` (distinct rows): a
        freed row takes a new sequence's prefill while the others keep decoding.  Checked in full
        first (capacity, hot pages, cold pages, every chunk), then per row and per chunk of
        `chunk` tokens an append and a quantisation of what left the window, each over the
        row's one-row view of the row metadata -- the same kernels, sharing the free stacks."""
        self._check_states(key_states, value_states)
        rows = [int(r) for r in rows]
        if len(rows) != key_states.shape[0]:
            raise ValueError("append_rows: one row index per batch entry of the states")
        if len(set(rows)) != len(rows):
            raise ValueError("append_rows: rows must be distinct")
        if any(r < 0 or r >= self.max_batch for r in rows):
            raise IndexError("append_rows: row out of range")
        tokens = key_states.shape[2]
        if not rows or tokens == 0:
            return
        r = np.asarray(rows)
        self._check_chunked(len(rows), tokens, max_length, rows=r)
        k, v = self._compatible_pair(key_states, value_states)
        t = self.tensors
        ops = self._ops()
        P = self.page_size
        for i, row in enumerate(rows):
            one = t[:2] + [t[2][row:row + 1], t[3][row:row + 1], t[4][row:row + 1]] + t[5:]
            for s0 in range(0, tokens, self.chunk):
                n = min(self.chunk, tokens - s0)
                start = int(self.lens[row])
                need = max(min(-(-(start + n) // P), self.max_blocks) - (-(-int(self.hw[row]) // P)), 0)
                ops.pool_append_(one, k[i:i + 1, :, s0:s0 + n], v[i:i + 1, :, s0:s0 + n])
                ops.pool_compress_(one, self.cold_tensors, self.window, 1)
                self.lens[row] = start + n
                self.hw[row] = max(int(self.hw[row]), start + n)
                frontier = max(start + n - self.window, 0) // P
                moved = max(frontier - int(self.cold_blocks[row]), 0)
                self.cold_blocks[row] = max(int(self.cold_blocks[row]), frontier)
                self.free_count += moved - need
                self.cold_free -= moved

    def hot_block_counts(self, rows: np.ndarray) -> np.ndarray:
        """Hot blocks of each row: below the high-water mark and after the quantised ones (the
        blocks a selection moves or copies)."""
        nb = np.minimum(-(-self.hw[rows] // self.page_size), self.max_blocks)
        return nb - np.minimum(self.cold_blocks[rows], nb)

    def select_copy_bound(self, rows: np.ndarray) -> int:
        """Pages a selection copies, at most: the hot blocks of repeated takers."""
        return int(self.hot_block_counts(rows)[self.repeated_mask(rows)].sum())

    def select_rows(self, src_rows: Sequence[int]) -> None:
        """In place: row i becomes row src_rows[i] (repeats allowed), every other row empty.
        Quantised blocks are shared by reference; hot blocks move to the first taker of their
        row and are copied for the others (barq_kv_select_rows_cold_layers)."""
        select_rows_layers([self], src_rows)

    def _selected_cold(self, r: np.ndarray, need: int) -> None:
        n = len(r)
        lens, hw, cold = np.zeros_like(self.lens), np.zeros_like(self.hw), np.zeros_like(self.cold_blocks)
        lens[:n], hw[:n], cold[:n] = self.lens[r], self.hw[r], self.cold_blocks[r]
        self.lens[:] = lens  # in place: a captured decode step keeps views of these arrays
        self.hw[:] = hw
        self.cold_blocks[:] = cold
        self.free_count -= need
        self.free_exact = False  # moved and released pages are settled on the device
        self.cold_exact = False  # released cold pages return only when no row shares them
        self.shared = True       # cold pages may have several holders (hot pages never do)

    def copy_rows(self, src_rows: Sequence[int], num_pages: Optional[int] = None,
                  num_cold: Optional[int] = None) -> "QuantPagePool":
        """A new pool whose row i holds row src_rows[i] of this one (repeats allowed), for
        selections with more rows than this pool has (kv_cache.py:166-173 grows the batch): this
        pool's state is copied into a pool of max(len(src_rows), max_batch) rows -- page and cold
        page ids kept, the added pages and cold pages pushed on the free stacks -- which then
        selects in place (select_rows: quantised blocks shared by reference, hot blocks moved to
        their row's first taker and copied for the others).  Reads the stack tops (a
        synchronisation)."""
        src_rows = [int(r) for r in src_rows]
        if any(r < 0 or r >= self.max_batch for r in src_rows):
            raise IndexError("copy_rows: row out of range")
        n = len(src_rows)
        B2 = max(n, self.max_batch)
        P = self.page_size
        copies = self.select_copy_bound(np.asarray(src_rows, dtype=np.int64)) if n else 0
        if num_pages is None:
            per_row = (-(-(self.window + self.chunk) // P) + 2) + (-(-self.window // P) + 1)
            num_pages = max(math.ceil(self.num_pages * B2 / self.max_batch), min(B2 * per_row, B2 * (self.max_blocks + 1)))
        num_pages = max(int(num_pages), self.num_pages + copies)
        if num_cold is None:
            num_cold = max(self.num_cold, B2 * max(self.max_blocks - self.window // P, 1))
        num_cold = max(int(num_cold), self.num_cold)
        dst = QuantPagePool(max_batch=B2, max_blocks=self.max_blocks, page_size=P, kv_heads=self.kv_heads,
                            head_dim=self.head_dim, dtype=self.dtype, device=self.device, window=self.window,
                            chunk=self.chunk, num_pages=num_pages, num_cold=num_cold)
        N, C, B = self.num_pages, self.num_cold, self.max_batch
        top = int(self.ctrl[CTRL_FREE_TOP].item())
        ctop = int(self.ctrl[CTRL_COLD_TOP].item())
        i32 = dict(dtype=torch.int32, device=self.device)
        with torch.no_grad():
            dst.key_pages[:N].copy_(self.key_pages)
            dst.value_pages[:N].copy_(self.value_pages)
            dst.block_table.fill_(-1)
            dst.block_table[:B].copy_(self.block_table)
            for a, b in ((dst.seq_lens, self.seq_lens), (dst.high_water, self.high_water),
                         (dst.page_shares, self.page_shares), (dst.cold_shares, self.cold_shares)):
                a.zero_()
                a[:b.numel()].copy_(b)
            dst.free_pages[:top].copy_(self.free_pages[:top])
            dst.free_pages[top:top + num_pages - N].copy_(torch.arange(N, num_pages, **i32))
            for name in ("key_codes", "value_codes", "key_scales", "value_scales"):
                getattr(dst, name)[:C].copy_(getattr(self, name))
            dst.free_cold[:ctop].copy_(self.free_cold[:ctop])
            dst.free_cold[ctop:ctop + num_cold - C].copy_(torch.arange(C, num_cold, **i32))
            dst.ctrl.copy_(self.ctrl)
            dst.ctrl[CTRL_FREE_TOP] = top + num_pages - N
            dst.ctrl[CTRL_COLD_TOP] = ctop + num_cold - C
        dst.lens[:B] = self.lens
        dst.hw[:B] = self.hw
        dst.cold_blocks[:B] = self.cold_blocks
        dst.free_count, dst.free_exact = top + num_pages - N, True
        dst.cold_free, dst.cold_exact = ctop + num_cold - C, True
        dst.shared, dst.tails_shared = self.shared, self.tails_shared
        if n:
            dst.select_rows(src_rows)
        return dst

    def _attention_call(self, backend, query, out, scale, max_seq, split_tokens, ws):
        if self.page_size % 16 == 0 and self.head_dim in (64, 128):
            backend.pool_decode_attention_cold(self.tensors, self.cold_tensors, self.window, query, out, scale,
                                               max_seq, split_tokens, ws)
            return
        # Pages of other sizes: the kernel reads a 16-position chunk in one format, which such pages
        # do not give (nor does it decode codes at head size 256).  The dequantising gather instead
        # (the values the kernel would decode), then attention over the gathered K/V on the device,
        # in float32, with the row lengths read on the device (so a captured graph serves growing
        # rows).
        batch, q_heads, tokens, _ = query.shape
        ko, vo = self.gather(batch, max_seq)
        group = q_heads // self.kv_heads
        k = ko.float().repeat_interleave(group, dim=1)
        v = vo.float().repeat_interleave(group, dim=1)
        s = torch.matmul(query.float(), k.transpose(-1, -2).contiguous()) * scale  # [B, Hq, T, S]
        lens = self.seq_lens[:batch].clamp(max=max_seq).to(torch.int64)
        pos = torch.arange(max_seq, device=query.device)
        qpos = lens[:, None] - tokens + torch.arange(tokens, device=query.device)[None, :]  # [B, T]
        s = s.masked_fill((pos[None, None, :] > qpos[:, :, None])[:, None], float("-inf"))
        p = torch.softmax(s, dim=-1).nan_to_num(0.0)
        out.copy_(torch.matmul(p, v).to(out.dtype))

    def to(self, device) -> "QuantPagePool":
        super().to(device)
        for name in ("key_codes", "value_codes", "key_scales", "value_scales", "free_cold", "cold_shares"):
            setattr(self, name, getattr(self, name).to(self.device, non_blocking=True))
        return self


_GROUPS: dict = {}


def _select_rows_cold(pools: list, src_rows: Sequence[int]) -> None:
    """select_rows_layers for pools with quantised pages: one set of launches for pools of one
    device, geometry and window (else one per pool), every pool checked for room first."""
    if not all(getattr(p, "quantized", False) for p in pools):
        raise ValueError("a selection over quantised pools needs every pool quantised")
    if len({id(p) for p in pools}) != len(pools):
        raise ValueError("select_rows_layers: a pool is named twice")
    rows = [p._selection(src_rows) for p in pools]
    need = [p.select_copy_bound(r) if len(r) else 0 for p, r in zip(pools, rows)]
    for p, k in zip(pools, need):
        p.ensure_free(k, "select_rows")
    g = pools[0]
    key = lambda p: (p.device, p.max_batch, p.max_blocks, p.page_size, p.kv_heads, p.head_dim, p.dtype, p.window)
    groups = [pools] if all(key(p) == key(g) for p in pools) else [[p] for p in pools]
    r = rows[0]
    n = len(r)
    for group in groups:
        q = group[0]
        words = n * (q.max_blocks + 3) + q.max_batch + 2
        words *= min(len(group), 32)
        ws = getattr(q, "_select_ws", None)
        if ws is None or ws.numel() < words:
            ws = torch.empty((words,), dtype=torch.int32, device=q.device)
            q._select_ws = ws
        q._ops().pool_select_rows_cold_([p.tensors for p in group], [p.cold_tensors for p in group], q.window,
                                        q._index_tensor(r.tolist() or [0])[:n], ws)
    for p, k in zip(pools, need):
        p._selected_cold(r, k)


def _pool_group(pools: list[PagePool]):
    """(packed pool array, workspace) of a list of GPU pools, cached while their tensors stay."""
    key = tuple((id(p), p.generation) for p in pools)
    entry = _GROUPS.get(key)
    if entry is None:
        if len(_GROUPS) >= 8:
            _GROUPS.clear()
        # the entry holds the pools, so the ids in its key stay theirs
        entry = {"pools": list(pools), "group": _gpu_backend().pool_group([p.tensors for p in pools]),
                 "ws": None}
        _GROUPS[key] = entry
    return entry


def select_rows_layers(pools: Sequence[PagePool], src_rows: Sequence[int]) -> None:
    """``PagePool.select_rows(src_rows)`` on every pool -- a model's layers, as
    ``Cache.reorder_cache`` / ``batch_select_indices`` apply one selection to all of them
    (kv_cache.py:166-186 per layer) -- in one set of launches when the pools are GPU pools of one
    geometry; every pool is checked for room before any is changed."""
    pools = list(pools)
    if not pools:
        return
    if any(getattr(p, "quantized", False) for p in pools):
        _select_rows_cold(pools, src_rows)
        return
    g = pools[0]
    geom = (g.device, g.max_batch, g.max_blocks, g.page_size, g.kv_heads, g.head_dim, g.dtype)
    batched = (len(pools) > 1 and g.on_gpu and len({id(p) for p in pools}) == len(pools)
               and not any(getattr(p, "quantized", False) for p in pools)
               and all((p.device, p.max_batch, p.max_blocks, p.page_size, p.kv_heads, p.head_dim, p.dtype) == geom
                       for p in pools))
    if not batched:
        for p in pools:
            p._selection(src_rows)
        for p in pools:
            p.select_rows(src_rows)
        return
    r = g._selection(src_rows)
    n = len(r)
    lens = np.stack([p.lens for p in pools])
    hw = np.stack([p.hw for p in pools])
    P = g.page_size
    nb = np.minimum(-(-hw[:, r] // P), g.max_blocks)
    tails = nb - np.minimum(lens[:, r] // P, nb)
    repeated = PagePool.repeated_mask(r)
    need = np.where([p.tails_shared for p in pools], tails.sum(axis=1), tails[:, repeated].sum(axis=1))
    for p, k in zip(pools, need.tolist()):
        p.ensure_free(int(k), "select_rows")
    entry = _pool_group(pools)
    backend = _gpu_backend()
    words = int(backend.select_workspace_words(entry["group"], n))
    if entry["ws"] is None or entry["ws"].numel() < words:
        entry["ws"] = torch.empty((words,), dtype=torch.int32, device=g.device)
    backend.pool_group_select_rows_(entry["group"], g._index_tensor(r.tolist() or [0])[:n], entry["ws"])
    new_lens, new_hw = np.zeros_like(lens), np.zeros_like(hw)
    new_lens[:, :n], new_hw[:, :n] = lens[:, r], hw[:, r]
    for l, (p, k) in enumerate(zip(pools, need.tolist())):
        p._selected(new_lens[l], new_hw[l], int(k))


class _HostOps:
    """The pool operations for tensors in host memory, in torch CPU operators.

    Same semantics and page-allocation order as the HIP kernels (barq_kv.hip): new blocks are
    ranked in (row, block) order and rank k takes ``free_pages[top - 1 - k]``.
    """

    @staticmethod
    def _geometry(t):
        kp, _, bt = t[0], t[1], t[2]
        return kp.shape[1], bt.shape[1]

    @staticmethod
    def pool_reset_(t, page_order=None):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        n = kp.shape[0]
        order = page_order if page_order is not None else torch.arange(n, dtype=torch.int32)
        free.copy_(order.flip(0))
        shares.zero_()
        bt.fill_(-1)
        lens.zero_()
        hw.zero_()
        ctrl.zero_()
        ctrl[CTRL_FREE_TOP] = n

    @staticmethod
    def _map_new_blocks(t, batch, tokens):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        P, MB = _HostOps._geometry(t)
        top = int(ctrl[CTRL_FREE_TOP])
        used = 0
        err = 0
        for b in range(batch):
            ln, h = int(lens[b]), int(hw[b])
            first = -(-h // P)
            full_end = -(-(ln + tokens) // P)
            if full_end > MB:
                err |= ERRBIT_CAPACITY
            end = min(full_end, MB)
            for j in range(first, end):
                idx = top - 1 - used
                used += 1
                page = int(free[idx]) if idx >= 0 else -1
                if page < 0:
                    err |= ERRBIT_POOL_EXHAUSTED
                bt[b, j] = page
        ctrl[CTRL_FREE_TOP] = max(0, top - used)
        if err:
            ctrl[CTRL_ERRORS] |= err

    @staticmethod
    def _scatter(t, key_states, value_states, old_lens):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        P, MB = _HostOps._geometry(t)
        batch, _, tokens, _ = key_states.shape
        pos = old_lens[:, None] + torch.arange(tokens, dtype=torch.int64)[None, :]
        blk = pos // P
        ok = blk < MB
        rows = torch.arange(batch)[:, None].expand_as(pos)
        page = torch.full_like(pos, -1)
        page[ok] = bt[rows[ok], blk[ok]].long()
        ok &= page >= 0
        off = pos % P
        ks = key_states.permute(0, 2, 1, 3)  # [B, T, H, D]
        vs = value_states.permute(0, 2, 1, 3)
        kp[page[ok], off[ok]] = ks[ok]
        vp[page[ok], off[ok]] = vs[ok]

    @staticmethod
    def _commit(t, batch, tokens):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        lens[:batch] += tokens
        torch.maximum(hw[:batch], lens[:batch], out=hw[:batch])

    @staticmethod
    def pool_append_(t, key_states, value_states):
        batch, _, tokens, _ = key_states.shape
        old = t[3][:batch].long().clone()
        _HostOps._map_new_blocks(t, batch, tokens)
        _HostOps._scatter(t, key_states, value_states, old)
        _HostOps._commit(t, batch, tokens)

    @staticmethod
    def pool_gather(t, key_out, value_out, batch, seq_out, flags=0):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        P, MB = _HostOps._geometry(t)
        if flags & SEQ_FROM_DEVICE:
            seq_out = min(seq_out, int(lens[:batch].max())) if batch else 0
        s = torch.arange(seq_out, dtype=torch.int64)
        blk = torch.clamp(s // P, max=MB - 1)
        page = bt[:batch].long()[:, blk]  # [B, S]
        valid = (s[None, :] < hw[:batch].long()[:, None]) & (page >= 0) & (s[None, :] < MB * P)
        off = (s % P)[None, :].expand_as(page)
        for pages, out in ((kp, key_out), (vp, value_out)):
            vals = pages[page.clamp(min=0), off]  # [B, S, H, D]
            vals[~valid] = 0
            out[:batch, :, :seq_out, :] = vals.permute(0, 2, 1, 3)

    @staticmethod
    def pool_update_(t, key_states, value_states, key_out, value_out, seq_out, flags=0):
        _HostOps.pool_append_(t, key_states, value_states)
        _HostOps.pool_gather(t, key_out, value_out, key_states.shape[0], seq_out, flags)

    @staticmethod
    def pool_decode_attention(t, query, out, scale, batch):
        """Decode attention for a pool in host memory: the gathered rows, float32 arithmetic."""
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        seq = int(lens[:batch].max())
        shape = (batch, kp.shape[2], seq, query.shape[3])
        ko = torch.empty(shape, dtype=kp.dtype)
        vo = torch.empty(shape, dtype=kp.dtype)
        _HostOps.pool_gather(t, ko, vo, batch, seq)
        _HostOps.attention_over(ko, vo, lens, query, out, scale, batch)

    @staticmethod
    def attention_over(ko, vo, lens, query, out, scale, batch):
        """Attention of `query` over gathered rows ko / vo ``[batch, kv_heads, seq, D]`` (row b
        has lens[b] positions; query token i sees [0, lens[b] - tokens + i]), float32."""
        _, q_heads, tokens, D = query.shape
        group = q_heads // ko.shape[1]
        for b in range(batch):
            n = int(lens[b])
            k = ko[b, :, :n].float().repeat_interleave(group, dim=0)  # [q_heads, n, D]
            v = vo[b, :, :n].float().repeat_interleave(group, dim=0)
            s = torch.matmul(query[b].float(), k.transpose(1, 2)) * scale  # [q_heads, T, n]
            pos = torch.arange(n)[None, :]
            limit = n - tokens + torch.arange(tokens)[:, None]
            s = s.masked_fill(pos > limit, float("-inf"))
            p = torch.softmax(s, dim=-1).nan_to_num(0.0)  # a row that sees nothing gives zeros
            out[b] = torch.matmul(p, v).to(out.dtype)

    # -------------------------------------------------------------- fp8 cold store (host memory)
    @staticmethod
    def pool_cold_reset_(t, cold, window):
        free, shares = cold[4], cold[5]
        n = free.numel()
        free.copy_(torch.arange(n - 1, -1, -1, dtype=torch.int32))
        shares.zero_()
        t[6][CTRL_COLD_TOP] = n

    @staticmethod
    def _quantise(x: torch.Tensor, dim: int) -> tuple[torch.Tensor, torch.Tensor]:
        """float32 groups along `dim` -> (E4M3 codes, exponents): 2^e the smallest power of two
        with max |x| <= 448 * 2^e over finite elements; codes from torch's float8_e4m3fn
        conversion (round to nearest even) of the exactly scaled values."""
        a = x.abs()
        a = torch.where(torch.isfinite(a), a, torch.zeros_like(a)).amax(dim)
        m, e = torch.frexp(a)
        e = (e - 9 + (m > 0.875).to(e.dtype)).masked_fill(a == 0, 0).clamp(-127, 127)
        y = torch.ldexp(x, -e.unsqueeze(dim).to(torch.float32))
        return y.to(torch.float8_e4m3fn).view(torch.uint8), e

    @staticmethod
    def _dequantise(codes: torch.Tensor, e: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """code * 2^e in the cache dtype; NaN codes give the quiet NaN with the code's sign (the
        device's result, whatever payload the conversion library picks)."""
        x = torch.ldexp(codes.view(torch.float8_e4m3fn).float(), e.float())
        nan = (codes & 0x7F) == 0x7F
        y = x.masked_fill(nan, 0.0).to(dtype)
        if nan.any():
            quiet, width, bits_t = {torch.bfloat16: (0x7FC0, 16, torch.int16), torch.float16: (0x7E00, 16, torch.int16),
                                    torch.float32: (0x7FC00000, 32, torch.int32)}[dtype]
            sign = (codes >> 7).to(torch.int64) << (width - 1)
            bits = (sign | quiet).to(torch.int64)
            bits = torch.where(bits >= 1 << (width - 1), bits - (1 << width), bits)  # as signed
            y.view(bits_t)[nan] = bits[nan].to(bits_t)
        return y

    @staticmethod
    def pool_compress_(t, cold, window, batch):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        kc, vc, ks, vs, free_cold, _ = cold
        P, MB = _HostOps._geometry(t)
        for r in range(batch):
            jmax = min(max(int(lens[r]) - window, 0) // P, min(-(-int(hw[r]) // P), MB))
            for j in range(jmax):
                page = int(bt[r, j])
                if page < 0 or int(shares[page]) != 0:
                    continue
                top = int(ctrl[CTRL_COLD_TOP])
                if top <= 0:
                    ctrl[CTRL_ERRORS] |= ERRBIT_POOL_EXHAUSTED
                    continue
                c = int(free_cold[top - 1])
                ctrl[CTRL_COLD_TOP] = top - 1
                codes, e = _HostOps._quantise(kp[page].float(), 0)
                kc[c], ks[c] = codes, (e + 127).to(torch.uint8)
                codes, e = _HostOps._quantise(vp[page].float(), 2)
                vc[c], vs[c] = codes, (e + 127).to(torch.uint8)
                bt[r, j] = -2 - c
                free[int(ctrl[CTRL_FREE_TOP])] = page
                ctrl[CTRL_FREE_TOP] += 1

    @staticmethod
    def pool_gather_cold(t, cold, window, key_out, value_out, batch, seq_out, flags=0):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        kc, vc, ks, vs, _, _ = cold
        P, MB = _HostOps._geometry(t)
        if flags & SEQ_FROM_DEVICE:
            seq_out = min(seq_out, int(lens[:batch].max())) if batch else 0
        key_out[:batch, :, :seq_out].zero_()
        value_out[:batch, :, :seq_out].zero_()
        for b in range(batch):
            for j in range(min(-(-seq_out // P), MB)):
                lo = j * P
                n = min(P, min(seq_out, int(hw[b])) - lo)
                if n <= 0:
                    break
                e = int(bt[b, j])
                if e >= 0:
                    kpage, vpage = kp[e], vp[e]
                elif e <= -2:
                    c = -2 - e
                    kpage = _HostOps._dequantise(kc[c], ks[c].long()[None] - 127, kp.dtype)
                    vpage = _HostOps._dequantise(vc[c], vs[c].long()[..., None] - 127, kp.dtype)
                else:
                    continue
                key_out[b, :, lo:lo + n] = kpage[:n].permute(1, 0, 2)
                value_out[b, :, lo:lo + n] = vpage[:n].permute(1, 0, 2)

    @staticmethod
    def pool_update_cold_(t, cold, window, key_states, value_states, key_out, value_out, seq_out, flags=0):
        _HostOps.pool_append_(t, key_states, value_states)
        if not flags & NO_COMPRESS:
            _HostOps.pool_compress_(t, cold, window, key_states.shape[0])
        _HostOps.pool_gather_cold(t, cold, window, key_out, value_out, key_states.shape[0], seq_out, flags)

    @staticmethod
    def _release_cold(cold, ctrl, c):
        """Drop one reference to cold page c; push it on free_cold when none is left."""
        free_cold, cold_shares = cold[4], cold[5]
        if int(cold_shares[c]) > 0:
            cold_shares[c] -= 1
            return
        top = int(ctrl[CTRL_COLD_TOP])
        free_cold[top] = c
        ctrl[CTRL_COLD_TOP] = top + 1

    @staticmethod
    def pool_free_rows_cold_(t, cold, window, rows):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        P, MB = _HostOps._geometry(t)
        top = int(ctrl[CTRL_FREE_TOP])
        for r in rows.tolist():
            n = min(-(-int(hw[r]) // P), MB)
            for j in range(n):
                e = int(bt[r, j])
                if e >= 0:
                    top = _HostOps._release(t, e, top)
                elif e <= -2:
                    _HostOps._release_cold(cold, ctrl, -2 - e)
            bt[r, :n] = -1
            lens[r] = 0
            hw[r] = 0
        ctrl[CTRL_FREE_TOP] = top

    @staticmethod
    def pool_crop_cold_(t, cold, window, batch, max_length):
        """Lower lengths; re-open each row's quantised blocks from the one holding its new length
        (barq_kv_crop_cold): their dequantised contents go to pages popped from the stack."""
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        kc, vc, ks, vs = cold[:4]
        P, MB = _HostOps._geometry(t)
        for r in range(batch):
            m = min(int(lens[r]), max_length)
            for j in range(m // P, min(-(-int(hw[r]) // P), MB)):
                e = int(bt[r, j])
                if e > -2:
                    continue
                top = int(ctrl[CTRL_FREE_TOP])
                if top <= 0:
                    ctrl[CTRL_ERRORS] |= ERRBIT_POOL_EXHAUSTED
                    continue
                c, page = -2 - e, int(free[top - 1])
                ctrl[CTRL_FREE_TOP] = top - 1
                kp[page] = _HostOps._dequantise(kc[c], ks[c].long()[None] - 127, kp.dtype)
                vp[page] = _HostOps._dequantise(vc[c], vs[c].long()[..., None] - 127, kp.dtype)
                bt[r, j] = page
                _HostOps._release_cold(cold, ctrl, c)
            lens[r] = m

    @staticmethod
    def pool_select_rows_cold_(pools, colds, window, rows, workspace=None):
        """Selection over pools with cold stores (barq_kv_select_rows_cold_layers): quantised
        blocks shared by reference, every hot block moved to its row's first taker or copied."""
        for t, cold in zip(pools, colds):
            _HostOps._select_cold(t, cold, rows.tolist())

    @staticmethod
    def _select_cold(t, cold, rows):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        cold_shares = cold[5]
        P, MB = _HostOps._geometry(t)
        n, B = len(rows), bt.shape[0]
        nb = lambda r: min(-(-int(hw[r]) // P), MB)
        first = {}
        for i, r in enumerate(rows):
            first.setdefault(r, i)
        copies = 0
        for i, r in enumerate(rows):
            for j in range(nb(r)):
                e = int(bt[r, j])
                if e > -2 and not (first[r] == i and e >= 0 and int(shares[e]) == 0):
                    copies += 1
        top = int(ctrl[CTRL_FREE_TOP])
        if copies > top:
            ctrl[CTRL_ERRORS] |= ERRBIT_POOL_EXHAUSTED
            return
        new_bt = torch.full((n, MB), -1, dtype=torch.int32)
        used, moved = 0, set()
        for i, r in enumerate(rows):
            for j in range(nb(r)):
                e = int(bt[r, j])
                if e <= -2:
                    cold_shares[-2 - e] += 1
                    new_bt[i, j] = e
                elif first[r] == i and e >= 0 and int(shares[e]) == 0:
                    moved.add((r, j))
                    new_bt[i, j] = e
                else:
                    page = int(free[top - 1 - used])
                    used += 1
                    if e >= 0:
                        kp[page] = kp[e]
                        vp[page] = vp[e]
                    new_bt[i, j] = page
        new_lens = lens[rows].clone() if n else torch.zeros(0, dtype=torch.int32)
        new_hw = hw[rows].clone() if n else torch.zeros(0, dtype=torch.int32)
        top -= used
        ctrl[CTRL_FREE_TOP] = top
        for r in range(B):
            for j in range(nb(r)):
                e = int(bt[r, j])
                if e <= -2:
                    _HostOps._release_cold(cold, ctrl, -2 - e)
                elif e >= 0 and (r, j) not in moved:
                    ctrl[CTRL_FREE_TOP] = _HostOps._release(t, e, int(ctrl[CTRL_FREE_TOP]))
        bt.fill_(-1)
        lens.zero_()
        hw.zero_()
        bt[:n] = new_bt
        lens[:n] = new_lens
        hw[:n] = new_hw

    @staticmethod
    def pool_crop_(t, batch, max_length):
        t[3][:batch].clamp_(max=max_length)

    @staticmethod
    def _release(t, page, top):
        """Drop one reference to `page`; push it when none is left.  Returns the new top."""
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        if int(shares[page]) > 0:
            shares[page] -= 1
            return top
        free[top] = page
        return top + 1

    @staticmethod
    def pool_free_rows_(t, rows):
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        P, MB = _HostOps._geometry(t)
        top = int(ctrl[CTRL_FREE_TOP])
        for r in rows.tolist():
            n = min(-(-int(hw[r]) // P), MB)
            for j in range(n):
                top = _HostOps._release(t, int(bt[r, j]), top)
            bt[r, :n] = -1
            lens[r] = 0
            hw[r] = 0
        ctrl[CTRL_FREE_TOP] = top

    @staticmethod
    def pool_select_rows_(t, rows, workspace=None):
        """In-place selection with shared full blocks and moved or copied tails, all or nothing
        (the algorithm of select_plan / select_build / select_settle in barq_kv.hip)."""
        kp, vp, bt, lens, hw, free, ctrl, shares = t
        P, MB = _HostOps._geometry(t)
        rows = rows.tolist()
        n, B = len(rows), bt.shape[0]

        def tail(r):
            nb = min(-(-int(hw[r]) // P), MB)
            f = min(int(lens[r]) // P, nb)
            return f, nb

        first = {}
        for i, r in enumerate(rows):
            first.setdefault(r, i)
        moved = set()  # (old row, block) whose page its first taker keeps
        copies = 0
        for i, r in enumerate(rows):
            f, nb = tail(r)
            for j in range(f, nb):
                if first[r] == i and int(shares[int(bt[r, j])]) == 0:
                    moved.add((r, j))
                else:
                    copies += 1
        top = int(ctrl[CTRL_FREE_TOP])
        if copies > top:
            ctrl[CTRL_ERRORS] |= ERRBIT_POOL_EXHAUSTED
            return
        new_bt = torch.full((n, MB), -1, dtype=torch.int32)
        used = 0
        for i, r in enumerate(rows):
            f, nb = tail(r)
            for j in range(nb):
                old = int(bt[r, j])
                if j < f:
                    shares[old] += 1
                    new_bt[i, j] = old
                elif (r, j) in moved and first[r] == i:
                    new_bt[i, j] = old
                else:
                    page = int(free[top - 1 - used])
                    used += 1
                    kp[page] = kp[old]
                    vp[page] = vp[old]
                    new_bt[i, j] = page
        new_lens = lens[rows].clone() if n else torch.zeros(0, dtype=torch.int32)
        new_hw = hw[rows].clone() if n else torch.zeros(0, dtype=torch.int32)
        top -= used
        for r in range(B):
            _, nb = tail(r)
            for j in range(nb):
                if (r, j) not in moved:
                    top = _HostOps._release(t, int(bt[r, j]), top)
        ctrl[CTRL_FREE_TOP] = top
        bt.fill_(-1)
        lens.zero_()
        hw.zero_()
        bt[:n] = new_bt
        lens[:n] = new_lens
        hw[:n] = new_hw

    @staticmethod
    def pool_copy_rows_(src, dst, rows):
        skp, svp, sbt, slens, shw, _, _, _ = src
        dkp, dvp, dbt, dlens, dhw, dfree, dctrl, _ = dst
        P, MB = _HostOps._geometry(src)
        top = int(dctrl[CTRL_FREE_TOP])
        used = 0
        for i, r in enumerate(rows.tolist()):
            n = min(-(-int(shw[r]) // P), MB)
            for j in range(n):
                page = int(dfree[top - 1 - used])
                used += 1
                sp = int(sbt[r, j])
                dkp[page] = skp[sp]
                dvp[page] = svp[sp]
                dbt[i, j] = page
            dlens[i] = slens[r]
            dhw[i] = shw[r]
        dctrl[CTRL_FREE_TOP] = top - used
