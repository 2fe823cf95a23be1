"""A dense device-side copy of a paged layer, for checking every step of long GPU programs.

``DeviceMirror`` keeps ``[batch, kv_heads, capacity, head_dim]`` K and V on the GPU, written with
plain torch indexing: an append of T tokens to rows [0, batch) stores them at positions
len[b] .. len[b] + T - 1 of each row; releasing a row zeroes it.  For programs of appends and row
releases (no crop), the reference's materialised cache (kv_cache.py:120-133: slots below a row's
length hold what was stored there, the rest zeros) is ``mirror[:, :, :seq]``, so every update can
be compared bit for bit on the device between the oracle's checkpoints.  The mirror itself is
checked against the oracle wherever the tests compare both with the kernels' output.
"""

from __future__ import annotations

import numpy as np
import torch

_BITS = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(_BITS[t.element_size()])


class DeviceMirror:
    def __init__(self, batch: int, heads: int, capacity: int, dim: int, dtype: torch.dtype, device="cuda"):
        self.k = torch.zeros((batch, heads, capacity, dim), dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.lens = np.zeros(batch, dtype=np.int64)

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: [batch, H, T, D] on the mirror's device, appended to rows [0, batch)."""
        batch, T = k.shape[0], k.shape[2]
        starts = self.lens[:batch]
        if (starts == starts[0]).all():
            s = int(starts[0])
            self.k[:batch, :, s:s + T] = k
            self.v[:batch, :, s:s + T] = v
        else:
            rows = torch.arange(batch, device=k.device).repeat_interleave(T)
            pos = torch.from_numpy((starts[:, None] + np.arange(T)[None, :]).ravel()).to(k.device)
            H, D = k.shape[1], k.shape[3]
            self.k[rows, :, pos] = k.permute(0, 2, 1, 3).reshape(batch * T, H, D)
            self.v[rows, :, pos] = v.permute(0, 2, 1, 3).reshape(batch * T, H, D)
        self.lens[:batch] += T

    def release_rows(self, rows) -> None:
        for r in rows:
            self.k[r].zero_()
            self.v[r].zero_()
            self.lens[r] = 0

    def append_rows(self, rows, k: torch.Tensor, v: torch.Tensor) -> None:
        """k[i], v[i] ([H, T, D]) appended to row rows[i]."""
        for i, r in enumerate(rows):
            s, T = int(self.lens[r]), k.shape[2]
            self.k[r, :, s:s + T] = k[i]
            self.v[r, :, s:s + T] = v[i]
            self.lens[r] += T

    def check(self, got, what: str = "") -> None:
        """got = (K, V) [batch, H, seq, D]: bit-equal to the mirror's first batch rows and seq
        positions."""
        for name, g, m in (("K", got[0], self.k), ("V", got[1], self.v)):
            b, _, seq, _ = g.shape
            want = m[:b, :, :seq]
            if not torch.equal(_bits(g), _bits(want)):
                bad = (_bits(g) != _bits(want)).nonzero()
                raise AssertionError(f"{what} {name}: {bad.shape[0]} elements differ from the device mirror, "
                                     f"first at {bad[0].tolist()}")
