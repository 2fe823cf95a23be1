"""Seeded inputs and raw-bit views shared by the tests, smoke() and bench.py."""

from __future__ import annotations

import numpy as np
import torch

_SIGNED = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32,
           torch.float64: torch.int64}
_UNSIGNED = {torch.int16: np.uint16, torch.int32: np.uint32, torch.int64: np.uint64}
_NP_SIGNED = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32, np.dtype(np.uint64): np.int64}


def to_bits(t: torch.Tensor) -> np.ndarray:
    """Raw element bits of a tensor (copied to host) as an unsigned numpy array."""
    signed = _SIGNED[t.dtype]
    return t.detach().contiguous().view(signed).cpu().numpy().view(_UNSIGNED[signed])


def from_bits(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    """Tensor of `dtype` with the given raw bits."""
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(_NP_SIGNED[a.dtype])).view(dtype)


def normal(shape, dtype: torch.dtype, gen: torch.Generator) -> torch.Tensor:
    """N(0, 1) drawn in float32 on the CPU, rounded to nearest-even into `dtype`."""
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(dtype)


def hf_layout(batch: int, heads: int, tokens: int, dim: int, dtype, gen) -> torch.Tensor:
    """[B, H, T, D] view of a [B, T, H, D] tensor: the layout HF attention hands to Cache.update
    (key_states.view(B, T, H, D).transpose(1, 2))."""
    return normal((batch, tokens, heads, dim), dtype, gen).transpose(1, 2)


# Configuration 1 of the benchmark set: 2 layers, batch 1, 4 KV heads, head_dim 64, page 16,
# fp32; prefill 32 tokens, then 128 single-token appends, gathering after each.
C1 = dict(layers=2, batch=1, heads=4, dim=64, page=16, dtype=torch.float32, prefill=32, decode=128,
          seed=1001)


def config1_steps():
    """Yield, for each step (the prefill, then each decode), a list over layers of (k, v)."""
    c = C1
    gen = torch.Generator().manual_seed(c["seed"])
    for step in range(1 + c["decode"]):
        tokens = c["prefill"] if step == 0 else 1
        yield [
            (hf_layout(c["batch"], c["heads"], tokens, c["dim"], c["dtype"], gen),
             hf_layout(c["batch"], c["heads"], tokens, c["dim"], c["dtype"], gen))
            for _ in range(c["layers"])
        ]
