"""Independent model of the KV-cache value semantics, used to pin the oracle.

Each row is a list of slot records ``slot -> (call, row, token)`` naming which input element
was last stored in that slot; gathering looks the records up.  It shares no code or data
layout with ``oracle.kv_oracle``: no pages, no blocks, no dense reservation.

Semantics (python/barqtrain/kv_cache.py:66-71,75-91,120-133,158-194): an append of T tokens to
row b stores token t at slot len[b] + t and sets len[b] += T; crop lowers lengths and keeps
slots; reset forgets everything; gather returns, for each row of the current batch, slots
[0, max len) with unwritten slots as zero.
"""

from __future__ import annotations

import numpy as np


class SlotHistory:
    def __init__(self, max_batch: int):
        self.rows = [dict() for _ in range(max_batch)]
        self.lens = [0] * max_batch
        self.inputs = []  # per call: (keys, values) raw-bit arrays [B, H, T, D]
        self.current = 0

    def append(self, keys: np.ndarray, values: np.ndarray) -> None:
        call = len(self.inputs)
        self.inputs.append((keys, values))
        batch, _, tokens, _ = keys.shape
        for b in range(batch):
            for t in range(tokens):
                self.rows[b][self.lens[b] + t] = (call, b, t)
            self.lens[b] += tokens
        self.current = batch

    def append_rows(self, rows, keys: np.ndarray, values: np.ndarray) -> None:
        """Entry i of the call goes to row rows[i] (the current batch is unchanged)."""
        call = len(self.inputs)
        self.inputs.append((keys, values))
        tokens = keys.shape[2]
        for i, r in enumerate(rows):
            for t in range(tokens):
                self.rows[r][self.lens[r] + t] = (call, i, t)
            self.lens[r] += tokens

    def crop(self, max_length: int) -> None:
        for b in range(self.current):
            self.lens[b] = min(self.lens[b], max_length)

    def select(self, rows) -> None:
        self.rows = [dict(self.rows[r]) for r in rows]
        self.lens = [self.lens[r] for r in rows]
        self.current = len(rows)

    def release(self, rows) -> None:
        for r in rows:
            self.rows[r] = {}
            self.lens[r] = 0

    def reset(self) -> None:
        self.rows = [dict() for _ in self.rows]
        self.lens = [0] * len(self.lens)
        self.current = 0

    def seq_length(self) -> int:
        return max(self.lens[: self.current]) if self.current else 0

    def gather(self, heads: int, dim: int, dtype) -> tuple[np.ndarray, np.ndarray]:
        seq = self.seq_length()
        out = [np.zeros((self.current, heads, seq, dim), dtype=dtype) for _ in range(2)]
        for b in range(self.current):
            for s, (call, row, t) in self.rows[b].items():
                if s < seq:
                    for kv in range(2):
                        out[kv][b, :, s, :] = self.inputs[call][kv][row, :, t, :]
        return out[0], out[1]
