"""HIP-graph capture of a decode step: every layer's append + gather replayed with one launch.

The captured kernels read row lengths, block tables and the free-page stack from device memory
and size their output extent on the device (``SEQ_FROM_DEVICE``), so a captured graph serves
every step while the sequences grow: no host work per layer and no host sync per step.  A graph's
grid covers a fixed extent, so the step keeps one graph per *bucket* of extent (captured on first
use) and replays the smallest bucket that holds the longest row: tiles past the rows' end are
never launched.  Inputs are static buffers the caller fills before ``replay`` (in a model, the K/V
projection writes them); outputs are persistent ``[batch, kv_heads, capacity, head_dim]`` buffers
whose ``[:, :, :seq]`` view is returned.  The host-side length shadow of each pool is advanced by
the same arithmetic the kernels apply.
"""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np
import torch

from barqtrain_amd.paged import NO_COMPRESS, SEPARATE_FINALIZE, SEQ_FROM_DEVICE, PagedKVCapacityError, PagePool


class CapturedDecodeStep:
    def __init__(self, pools: Sequence[PagePool], batch: int, tokens: int = 1,
                 max_length: Optional[int] = None, separate_commit: bool = False,
                 inputs: Optional[tuple[torch.Tensor, torch.Tensor]] = None,
                 bucket: Optional[int] = None):
        """`inputs`, if given, are stacked ``[layers, batch, kv_heads, tokens, head_dim]`` K and V
        buffers (one copy fills every layer); otherwise one buffer per layer is allocated.
        `bucket` is the extent granularity of the captured graphs (default: a sixteenth of the
        capacity, at least 64 positions); `bucket=0` captures one graph over the capacity."""
        if not pools or not all(p.on_gpu for p in pools):
            raise ValueError("graph capture needs GPU page pools")
        self.pools = list(pools)
        self.batch = int(batch)
        self.tokens = int(tokens)
        self.max_length = max_length
        p0 = self.pools[0]
        self.capacity = p0.capacity if max_length is None else min(p0.capacity, int(max_length))
        shape_in = (self.batch, p0.kv_heads, self.tokens, p0.head_dim)
        shape_out = (self.batch, p0.kv_heads, self.capacity, p0.head_dim)
        if inputs is not None:
            kin, vin = inputs
            if tuple(kin.shape) != (len(self.pools), *shape_in) or kin.shape != vin.shape:
                raise ValueError("stacked inputs must be [layers, batch, kv_heads, tokens, head_dim]")
            self.key_in = list(kin.unbind(0))
            self.value_in = list(vin.unbind(0))
        else:
            self.key_in = [torch.zeros(shape_in, dtype=p.dtype, device=p.device) for p in self.pools]
            self.value_in = [torch.zeros(shape_in, dtype=p.dtype, device=p.device) for p in self.pools]
        self.key_out = [torch.empty(shape_out, dtype=p.dtype, device=p.device) for p in self.pools]
        self.value_out = [torch.empty(shape_out, dtype=p.dtype, device=p.device) for p in self.pools]
        self.flags = SEQ_FROM_DEVICE | (SEPARATE_FINALIZE if separate_commit else 0)
        self.quantized = [bool(getattr(p, "quantized", False)) for p in self.pools]
        if separate_commit and any(self.quantized):
            raise ValueError("pools with quantised pages commit inside their append launch")
        geometry = {(p.page_size, p.max_blocks, p.max_batch) for p in self.pools}
        if len(geometry) != 1:
            raise ValueError("pools of one captured step must share page size, blocks and rows")
        if any(p.lens.base is not None or p.hw.base is not None for p in self.pools):
            raise ValueError("a page pool can belong to one captured step only")
        # One stacked host shadow for all pools (each pool keeps a row view of it), so a replay
        # checks and advances every layer with a handful of array operations.
        self._lens = np.stack([p.lens for p in self.pools])
        self._hw = np.stack([p.hw for p in self.pools])
        for i, p in enumerate(self.pools):
            p.lens = self._lens[i]
            p.hw = self._hw[i]
        # The quantised pools' leading-cold-block counts, stacked the same way.
        self._qidx = np.flatnonzero(self.quantized)
        if self._qidx.size:
            if any(self.pools[i].cold_blocks.base is not None for i in self._qidx):
                raise ValueError("a page pool can belong to one captured step only")
            self._cold = np.stack([self.pools[i].cold_blocks for i in self._qidx])
            for j, i in enumerate(self._qidx):
                self.pools[i].cold_blocks = self._cold[j]
            self._windows = np.array([self.pools[i].window for i in self._qidx], dtype=np.int64)
        if bucket is None:
            bucket = max(64, -(-self.capacity // 16))
        self.bucket = int(bucket) if bucket else self.capacity
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        # Captured launches hold the pools' device pointers: a pool whose tensors are replaced
        # (PagePool.to) bumps its generation, and the graphs are captured again.
        self._generations = [p.generation for p in self.pools]
        self._device = p0.key_pages.device

    def _graph(self, extent: int, compress: bool = False) -> torch.cuda.CUDAGraph:
        """The graph whose launches cover output positions [0, extent), captured on first use
        (with `compress`, quantised pools also run their compress launch).  Capture records the
        launches without running them: no pool state changes here."""
        graph = self.graphs.get((extent, compress))
        if graph is None:
            from barqtrain_amd.paged import _gpu_backend

            backend = _gpu_backend()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i, pool in enumerate(self.pools):
                    if self.quantized[i]:  # append, quantise what left the window, dequantising gather
                        backend.pool_update_cold_(pool.tensors, pool.cold_tensors, pool.window, self.key_in[i],
                                                  self.value_in[i], self.key_out[i], self.value_out[i], extent,
                                                  self.flags | (0 if compress else NO_COMPRESS))
                    else:
                        backend.pool_update_(pool.tensors, self.key_in[i], self.value_in[i],
                                             self.key_out[i], self.value_out[i], extent, self.flags)
            self.graphs[(extent, compress)] = graph
        return graph

    def prepare(self, longest_rows) -> None:
        """Capture now the graphs of the steps whose longest row (after the append) takes the
        given values, so that no replay of them captures (capture costs milliseconds)."""
        for worst in longest_rows:
            extent = min(self.capacity, -(-int(worst) // self.bucket) * self.bucket)
            self._graph(extent, False)
            if any(self.quantized):
                self._graph(extent, True)

    def replay(self, views: bool = True) -> Optional[list[tuple[torch.Tensor, torch.Tensor]]]:
        """Run one captured step; returns each layer's (K, V) views ``[batch, H, seq, D]`` of the
        persistent outputs (None with ``views=False``, for callers that read ``key_out`` /
        ``value_out`` themselves: two views per layer cost more host time than the replay).
        Raises, before anything runs, if any layer would pass its capacity or run out of pages."""
        B, T = self.batch, self.tokens
        p0 = self.pools[0]
        generations = [p.generation for p in self.pools]
        if generations != self._generations:
            if any(p.key_pages.device != self._device for p in self.pools):
                raise ValueError("a pool of this captured step left its device; capture a new step")
            self.graphs.clear()
            self._generations = generations
        lens = self._lens[:, :B]
        hw = self._hw[:, :B]
        ends = lens + T
        worst = int(ends.max())
        if worst > self.capacity:
            raise PagedKVCapacityError(
                f"paged KV cache capacity exceeded: requested {worst}, max_cache_len={self.capacity}")
        P = p0.page_size
        need = np.maximum(np.minimum(-(-ends // P), p0.max_blocks) - (-(-hw // P)), 0).sum(axis=1)
        grows = bool(need.any())
        if grows:
            for p, n in zip(self.pools, need):
                p.ensure_free(int(n), "append")
        # Blocks leaving the residual window, for every quantised pool at once (the per-pool
        # _cold_after / _quantised arithmetic on the stacked shadows).
        moved = None
        if self._qidx.size:
            frontier = np.maximum(ends[self._qidx] - self._windows[:, None], 0) // P
            cold_b = self._cold[:, :B]
            moved = np.maximum(frontier - cold_b, 0).sum(axis=1)
            movers = np.flatnonzero(moved)
            for j in movers:
                self.pools[self._qidx[j]].ensure_cold(int(moved[j]))
        compress = moved is not None and movers.size > 0
        self._graph(min(self.capacity, -(-worst // self.bucket) * self.bucket), compress).replay()
        lens += T
        np.maximum(hw, lens, out=hw)
        if grows:
            for p, n in zip(self.pools, need):
                p.free_count -= int(n)
        if compress:
            np.maximum(cold_b, frontier, out=cold_b)
            for j in movers:
                p = self.pools[self._qidx[j]]
                p.cold_free -= int(moved[j])
                p.free_count += int(moved[j])  # each quantised block returned its full-precision page
        if not views:
            return None
        seqs = ends.max(axis=1).tolist()
        return [(k[:, :, :n], v[:, :, :n]) for k, v, n in zip(self.key_out, self.value_out, seqs)]
