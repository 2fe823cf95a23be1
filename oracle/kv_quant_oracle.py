"""CPU oracle for quantised (fp8 e4m3) KV pages -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module, and only as the checker.  The product (``barqtrain_amd``) never imports,
calls or falls back to it.

The reference plans a quantised KV cache -- "residual full-precision window plus compressed older
pages", "dequant-on-read" (IMPLEMENTATION_PLAN.md:106-129, after KIVI, arXiv:2402.02750) -- and
ships no implementation, so this module states the algorithm the product implements, in numpy:

* codes: OCP FP8 E4M3 ("e4m3fn": exponent bias 7, no infinities, 0x7F / 0xFF are NaN), rounded
  to nearest, ties to even; finite values beyond 448 saturate to +-448, non-finite values encode
  as NaN with their sign, and NaN codes read back as the quiet NaN 0x7FC00000 with that sign.
* scales: powers of two 2^e, stored as E8M0 bytes e + 127 (as OCP MX formats store them), one
  per group: for a page of P tokens, keys per channel (head, dim) over the page's tokens and
  values per token (token, head) over head_dim -- KIVI's key-per-channel / value-per-token
  grouping.  e is the smallest integer with max|x| <= 448 * 2^e over the group's finite
  elements (0 for a group without a finite non-zero element), clamped to [-127, 127].  Scaling by
  a power of two is exact, so a code depends only on the element and its group's maximum.
* a row's block j is quantised once it lies wholly before the row's residual window,
  (j + 1) * P <= len - W, from its content at that time (a full block never changes again).
* reads dequantise: decode(code) * 2^e, rounded to the cache dtype (ties to even).
* a crop below a row's quantised blocks re-opens them: from the block holding the row's new
  length on, a quantised block's stored content becomes its dequantised read (the bits a
  gather returned before the crop), which is what the row then holds there -- quantised again,
  from that content, once the block leaves the window anew.
* a selection (beam reordering) copies rows whole, quantised blocks included: a shared
  quantised block reads the same for every row holding it.

Pinning (tests/test_quant_oracle.py): every finite float32 code point and rounding boundary of
the encoder against torch's float8_e4m3fn conversion (an independent library routine); the
decode table against the closed form of the OCP E4M3 definition; the exponent rule against its
definition by brute force; the error bound |x - deq(x)| <= 2^(e+4) on random groups;
round trips of values already on the grid; planted mistakes shown to fail.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np

from oracle.kv_oracle import DenseLayerOracle

__all__ = [
    "E4M3_MAX",
    "e4m3_encode",
    "e4m3_decode",
    "group_exponent",
    "quantize_key_page",
    "quantize_value_page",
    "dequantize",
    "bits_to_float32",
    "float32_to_bits",
    "QuantLayerOracle",
]

E4M3_MAX = 448.0


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> E4M3 codes (uint8), round to nearest even, saturating, NaN for non-finite."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 31) & 1).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)  # exact copy of the float32 magnitude
    code = np.zeros(x.shape, dtype=np.int64)
    sub = a < 2.0 ** -6
    # subnormal codes: a / 2^-9 rounded to an integer (8 rounds up into the first normal code)
    code[sub] = np.rint(a[sub] * 512.0).astype(np.int64)
    norm = ~sub & np.isfinite(a)
    if norm.any():
        an = a[norm]
        e = np.floor(np.log2(an)).astype(np.int64)
        # guard log2 rounding: make 2^e <= an < 2^(e+1) exact
        e = np.where(np.ldexp(1.0, e) > an, e - 1, e)
        e = np.where(np.ldexp(1.0, e + 1) <= an, e + 1, e)
        m = an / np.ldexp(1.0, e) * 8.0 - 8.0  # 3-bit mantissa, as a real in [0, 8)
        mi = np.rint(m).astype(np.int64)      # ties to even
        carry = mi == 8
        e = np.where(carry, e + 1, e)
        mi = np.where(carry, 0, mi)
        c = ((e + 7) << 3) | mi
        c = np.where(c > 0x7E, 0x7E, c)       # saturate at 448
        code[norm] = c
    code[~np.isfinite(a)] = 0x7F
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e4m3_decode(code: np.ndarray) -> np.ndarray:
    """E4M3 codes -> float32 (exact); the NaN codes give the quiet NaN 0x7FC00000 with the
    code's sign."""
    c = np.asarray(code, dtype=np.uint8).astype(np.int64)
    E = (c >> 3) & 0xF
    M = c & 7
    mag = np.where(E == 0, M * 2.0 ** -9, (1.0 + M / 8.0) * np.ldexp(1.0, E - 7)).astype(np.float32)
    bits = mag.view(np.uint32)
    bits = np.where((c & 0x7F) == 0x7F, np.uint32(0x7FC00000), bits) | ((c & 0x80).astype(np.uint32) << 24)
    return bits.astype(np.uint32).view(np.float32)


def group_exponent(absmax: np.ndarray) -> np.ndarray:
    """Smallest e with absmax <= 448 * 2^e (0 for absmax 0), clamped to [-127, 127].

    With absmax = m * 2^x, m in [0.5, 1): e = x - 9, plus 1 when m > 0.875 (448 = 0.875 * 2^9).
    """
    a = np.asarray(absmax, dtype=np.float32)
    m, x = np.frexp(a)
    e = x.astype(np.int64) - 9 + (m > 0.875)
    e = np.where(a == 0, 0, e)
    return np.clip(e, -127, 127)


def _finite_abs(x: np.ndarray) -> np.ndarray:
    a = np.abs(x)
    return np.where(np.isfinite(a), a, 0).astype(np.float32)


def quantize_key_page(page: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Keys [P, H, D] float32 -> (codes [P, H, D] uint8, E8M0 bytes [H, D]): per channel."""
    e = group_exponent(_finite_abs(page).max(axis=0))
    codes = e4m3_encode(np.ldexp(page, -e[None]).astype(np.float32))
    return codes, (e + 127).astype(np.uint8)


def quantize_value_page(page: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Values [P, H, D] float32 -> (codes [P, H, D] uint8, E8M0 bytes [P, H]): per token."""
    e = group_exponent(_finite_abs(page).max(axis=2))
    codes = e4m3_encode(np.ldexp(page, -e[..., None]).astype(np.float32))
    return codes, (e + 127).astype(np.uint8)


def dequantize(codes: np.ndarray, scale_bytes: np.ndarray) -> np.ndarray:
    """decode(code) * 2^(s - 127), float32 (scale_bytes broadcast against codes)."""
    return np.ldexp(e4m3_decode(codes), scale_bytes.astype(np.int64) - 127).astype(np.float32)


def _bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def _f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (NaN kept quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def bits_to_float32(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Raw element bits of the cache dtype ('bf16', 'f16', 'f32') -> float32."""
    if dtype == "bf16":
        return _bf16_bits_to_f32(bits)
    if dtype == "f16":
        return bits.astype(np.uint16).view(np.float16).astype(np.float32)
    return bits.astype(np.uint32).view(np.float32)


def float32_to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> raw element bits of the cache dtype, round to nearest even."""
    if dtype == "bf16":
        return _f32_to_bf16_bits(x)
    if dtype == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)
    return np.asarray(x, dtype=np.float32).view(np.uint32)


class QuantLayerOracle(DenseLayerOracle):
    """``DenseLayerOracle`` whose blocks older than the residual window read back quantised.

    ``window`` is the residual window W in tokens; ``dtype`` the cache dtype ('bf16', 'f16',
    'f32') of the bit arrays.  ``cold[r]`` counts row r's leading quantised blocks; it grows
    after every append to floor((len - W) / P), and falls to floor(new len / P) when a crop
    re-opens blocks (their content replaced by its dequantised read), or to 0 when the row is
    released or the cache reset.
    """

    def __init__(self, max_batch_size: int, max_cache_len: int, page_size: int, window: int, dtype: str):
        super().__init__(max_batch_size, max_cache_len, page_size)
        self.window = int(window)
        self.qdtype = dtype
        self.cold = np.zeros(self.max_batch_size, dtype=np.int64)

    def append(self, key_states: np.ndarray, value_states: np.ndarray) -> None:
        super().append(key_states, value_states)
        b = key_states.shape[0]
        frontier = np.maximum((self.seq_lens[:b].astype(np.int64) - self.window) // self.page_size, 0)
        self.cold[:b] = np.maximum(self.cold[:b], np.minimum(frontier, self.max_blocks))

    def append_rows(self, rows: Sequence[int], key_states: np.ndarray, value_states: np.ndarray) -> None:
        """``DenseLayerOracle.append_rows`` (a new sequence's tokens into freed rows), then the same
        frontier rule as ``append`` for those rows: every block wholly before a row's window is
        quantised, whether its tokens came in one call or in chunks."""
        super().append_rows(rows, key_states, value_states)
        r = np.asarray(rows, dtype=np.int64)
        frontier = np.maximum((self.seq_lens[r].astype(np.int64) - self.window) // self.page_size, 0)
        self.cold[r] = np.maximum(self.cold[r], np.minimum(frontier, self.max_blocks))

    def crop(self, max_length: int) -> None:
        if not self.is_initialized:
            return
        m = max_length if max_length >= 0 else self.get_seq_length() - abs(max_length)
        m = max(m, 0)
        for r in range(self.current_batch_size):
            first = min(int(self.seq_lens[r]), m) // self.page_size
            for j in range(first, int(self.cold[r])):  # re-opened: the block now holds its read
                for cache, key in ((self.keys, True), (self.values, False)):
                    cache[r, :, j] = self._dequantised_block(cache[r, :, j], key)
            self.cold[r] = min(int(self.cold[r]), first)
        super().crop(max_length)

    def _dequantised_block(self, block: np.ndarray, key: bool) -> np.ndarray:
        """A block's bits [H, P, D] as a read of it quantised returns them."""
        page = np.ascontiguousarray(bits_to_float32(block, self.qdtype).transpose(1, 0, 2))  # [P, H, D]
        codes, scales = quantize_key_page(page) if key else quantize_value_page(page)
        deq = dequantize(codes, scales[None] if key else scales[..., None])
        return float32_to_bits(deq.transpose(1, 0, 2), self.qdtype)

    def batch_select_indices(self, indices: Sequence[int]) -> None:
        if not self.is_initialized or self.current_batch_size == 0:
            return
        cold = self.cold[: self.current_batch_size][np.asarray(indices, dtype=np.int64)]
        super().batch_select_indices(indices)
        self.cold = np.zeros(self.max_batch_size, dtype=np.int64)
        self.cold[: len(cold)] = cold

    def batch_repeat_interleave(self, repeats: int) -> None:
        if not self.is_initialized or self.current_batch_size == 0:
            return
        self.batch_select_indices([b for b in range(self.current_batch_size) for _ in range(int(repeats))])

    def reset(self) -> None:
        super().reset()
        self.cold[:] = 0

    def release_rows(self, rows: Sequence[int]) -> None:
        super().release_rows(rows)
        for r in rows:
            self.cold[r] = 0

    def _read(self, cache: np.ndarray, key: bool) -> np.ndarray:
        """The cache as read back: quantised blocks replaced by their dequantised content."""
        out = cache.copy()
        P = self.page_size
        for r in range(self.current_batch_size or cache.shape[0]):
            for j in range(int(self.cold[r])):
                out[r, :, j] = self._dequantised_block(cache[r, :, j], key)
        return out

    def current_tensors(self) -> tuple[np.ndarray, np.ndarray]:
        seq_len = self.get_seq_length()
        b = self.current_batch_size or self.keys.shape[0]
        shape = (b, self.keys.shape[1], self.max_blocks * self.page_size, self.keys.shape[-1])
        keys = self._read(self.keys[:b], True).reshape(shape)[..., :seq_len, :]
        values = self._read(self.values[:b], False).reshape(shape)[..., :seq_len, :]
        return np.ascontiguousarray(keys), np.ascontiguousarray(values)

    def quantized_page(self, row: int, block: int, key: bool) -> tuple[np.ndarray, np.ndarray]:
        """(codes [P, H, D], E8M0 bytes) of a quantised block, as the pool stores them."""
        cache = self.keys if key else self.values
        page = np.ascontiguousarray(bits_to_float32(cache[row, :, block], self.qdtype).transpose(1, 0, 2))
        return quantize_key_page(page) if key else quantize_value_page(page)


def max_abs_error_bound(scale_bytes: np.ndarray) -> np.ndarray:
    """|x - dequant(quant(x))| <= 2^(e + 4) for a finite x of a group with exponent e: half the
    code spacing of the largest binade, 2^(8 - 3) / 2 * 2^e."""
    return np.ldexp(1.0, scale_bytes.astype(np.int64) - 127 + 4)
