"""Float64 decode attention over gathered K/V: the checker of the paged decode-attention kernel.

Test infrastructure only.  Row b's query token i sits at position lens[b] - T + i and sees
positions [0, lens[b] - T + i]; q head h reads kv head h // (Hq // Hkv).  A row that sees no
position gives zeros.  Pinned against torch's scaled_dot_product_attention (square causal
attention, grouped-query) in tests/test_attention_ref.py.
"""

from __future__ import annotations

import numpy as np


def decode_attention_reference(q: np.ndarray, k: np.ndarray, v: np.ndarray, lens, scale: float) -> np.ndarray:
    """q [B, Hq, T, D]; k, v [B, Hkv, S, D] (S >= max(lens)); returns float64 [B, Hq, T, D]."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, T, D = q.shape
    G = Hq // k.shape[1]
    out = np.zeros((B, Hq, T, D))
    for b in range(B):
        n = int(lens[b])
        for h in range(Hq):
            kk = k[b, h // G, :n]
            vv = v[b, h // G, :n]
            for i in range(T):
                visible = n - T + i + 1
                if visible <= 0:
                    continue
                s = kk[:visible] @ q[b, h, i] * scale
                p = np.exp(s - s.max())
                out[b, h, i] = (p / p.sum()) @ vv[:visible]
    return out


def within_tolerance(got: np.ndarray, want: np.ndarray, rtol: float, atol: float) -> tuple[bool, float]:
    """|got - want| <= atol + rtol * |want| everywhere; also returns the worst excess ratio."""
    err = np.abs(np.asarray(got, dtype=np.float64) - want)
    bound = atol + rtol * np.abs(want)
    ratio = float((err / bound).max()) if err.size else 0.0
    return bool(np.all(err <= bound)), ratio
