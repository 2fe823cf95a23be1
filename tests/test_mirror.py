"""The device mirror the long GPU parity programs check every step against, run here on CPU
tensors: it must agree with the oracle's materialised cache on append / release programs, and its
check must catch a single wrong element."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvgen import from_bits, hf_layout, to_bits
from mirror import DeviceMirror
from oracle.kv_oracle import DenseLayerOracle


def _as_tensors(oracle: DenseLayerOracle, dtype):
    ok, ov = oracle.current_tensors()
    return from_bits(ok, dtype), from_bits(ov, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mirror_matches_oracle_on_append_and_release_programs(dtype):
    B, H, D, P, cap = 5, 3, 16, 4, 64
    rng = np.random.default_rng(11)
    gen = torch.Generator().manual_seed(12)
    oracle = DenseLayerOracle(B, cap, P)
    mirror = DeviceMirror(B, H, cap, D, dtype, device="cpu")
    # staircase prefill: rows [0, b) grow together, so the later decode appends are ragged
    for b, t in [(5, 7), (3, 5), (1, 9)]:
        k, v = hf_layout(b, H, t, D, dtype, gen), hf_layout(b, H, t, D, dtype, gen)
        oracle.append(to_bits(k), to_bits(v))
        mirror.append(k, v)
        mirror.check(_as_tensors(oracle, dtype), f"prefill {b}x{t}")
    for step in range(30):
        if step % 7 == 6:
            rows = sorted(rng.choice(B, size=2, replace=False).tolist())
            oracle.release_rows(rows)
            mirror.release_rows(rows)
            t = int(rng.integers(1, 6))
            k, v = hf_layout(2, H, t, D, dtype, gen), hf_layout(2, H, t, D, dtype, gen)
            oracle.append_rows(rows, to_bits(k), to_bits(v))
            mirror.append_rows(rows, k, v)
        t = 1 if step % 3 else 2
        k, v = hf_layout(B, H, t, D, dtype, gen), hf_layout(B, H, t, D, dtype, gen)
        oracle.append(to_bits(k), to_bits(v))
        mirror.append(k, v)
        assert mirror.lens.tolist() == oracle.seq_lens.tolist()
        mirror.check(_as_tensors(oracle, dtype), f"step {step}")


def test_mirror_check_catches_one_wrong_element():
    B, H, D, P, cap = 2, 2, 8, 4, 16
    gen = torch.Generator().manual_seed(3)
    oracle = DenseLayerOracle(B, cap, P)
    mirror = DeviceMirror(B, H, cap, D, torch.bfloat16, device="cpu")
    k, v = hf_layout(B, H, 6, D, torch.bfloat16, gen), hf_layout(B, H, 6, D, torch.bfloat16, gen)
    oracle.append(to_bits(k), to_bits(v))
    mirror.append(k, v)
    ok, ov = oracle.current_tensors()
    ok[1, 0, 5, 3] ^= 1  # one bit of one element of the oracle's K
    with pytest.raises(AssertionError, match="K: 1 elements differ"):
        mirror.check((from_bits(ok, torch.bfloat16), from_bits(ov, torch.bfloat16)))
    ok[1, 0, 5, 3] ^= 1
    ov[0, 1, 0, 0] ^= 0x8000  # a sign flip in V
    with pytest.raises(AssertionError, match="V: 1 elements differ"):
        mirror.check((from_bits(ok, torch.bfloat16), from_bits(ov, torch.bfloat16)))
