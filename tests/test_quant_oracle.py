"""Pinning of the fp8 (E4M3, E8M0-scaled) KV quantisation oracle, oracle/kv_quant_oracle.py.

The reference has no quantised cache (IMPLEMENTATION_PLAN.md:106-129 plans one), so the oracle
is pinned against an independent library routine (torch's float8_e4m3fn conversion), the closed
form of the OCP E4M3 format, the definition of the scale exponent, error bounds and round trips;
planted mistakes are shown to fail.  CPU only.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_quant_oracle as q


def torch_encode(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def boundary_values() -> np.ndarray:
    """Every code value, every midpoint between neighbouring codes (the ties), and the float32
    neighbours of both, over both signs."""
    vals = q.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    pts = np.concatenate([vals, mids, [448.0, 456.0, 464.0, 500.0, 1e6]]).astype(np.float32)
    pts = np.concatenate([pts, np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(0))])
    return np.concatenate([pts, -pts])


def test_encoder_matches_torch_on_boundaries_and_a_dense_sweep():
    x = boundary_values()
    inside = np.abs(x) <= 464.0  # torch turns finite overflow into NaN; this encoder saturates
    assert np.array_equal(q.e4m3_encode(x[inside]), torch_encode(x[inside]))
    assert (q.e4m3_encode(x[~inside]) & 0x7F == 0x7E).all()
    u = np.arange(0, 0x43E80000, 211, dtype=np.uint32)  # every 211th float32 in [0, 464]
    x = np.concatenate([u.view(np.float32), -u.view(np.float32)])
    assert np.array_equal(q.e4m3_encode(x), torch_encode(x))


def test_decoder_matches_the_ocp_definition_and_torch():
    c = np.arange(256, dtype=np.uint8)
    got = q.e4m3_decode(c)
    for code in range(256):
        s, E, M = code >> 7, (code >> 3) & 15, code & 7
        if E == 15 and M == 7:
            assert np.isnan(got[code])
            continue
        want = (2.0 ** -6) * (M / 8) if E == 0 else 2.0 ** (E - 7) * (1 + M / 8)
        assert got[code] == (-want if s else want), code
    t = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()
    ok = ~np.isnan(t)
    assert np.array_equal(np.isnan(got), ~ok) and np.array_equal(got[ok], t[ok])


def test_nan_codes_read_back_as_signed_quiet_nan():
    got = q.e4m3_decode(np.array([0x7F, 0xFF], dtype=np.uint8)).view(np.uint32)
    assert got.tolist() == [0x7FC00000, 0xFFC00000]
    assert q.float32_to_bits(got.view(np.float32), "bf16").tolist() == [0x7FC0, 0xFFC0]


def test_non_finite_and_saturation():
    x = np.array([np.nan, -np.nan, np.inf, -np.inf, 449.0, -1e30, 0.0, -0.0], dtype=np.float32)
    codes = q.e4m3_encode(x)
    assert (codes[:4] & 0x7F).tolist() == [0x7F] * 4
    assert codes[4:].tolist() == [0x7E, 0xFE, 0x00, 0x80]


def test_group_exponent_is_the_smallest_fitting_power_of_two():
    rng = np.random.default_rng(0)
    a = np.concatenate([
        np.exp(rng.uniform(-60, 60, 20000)).astype(np.float32),
        np.ldexp(np.float32(448.0), np.arange(-100, 100)).astype(np.float32),  # exact fits
        np.nextafter(np.ldexp(np.float32(448.0), np.arange(-100, 100)).astype(np.float32), np.float32(np.inf)),
    ])
    e = q.group_exponent(a)
    a64 = a.astype(np.float64)
    assert (a64 <= 448.0 * np.ldexp(1.0, e)).all()
    assert (a64 > 448.0 * np.ldexp(1.0, e - 1)).all()
    assert q.group_exponent(np.float32(0.0)) == 0
    assert q.group_exponent(np.float32(3e38)) == 120 and q.group_exponent(np.float32(1e-44)) == -127


def _groups(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32)
    x[rng.random(shape) < 0.01] *= 50.0  # outliers, as K channels have
    return x


def test_pages_meet_the_error_bound_and_group_as_kivi():
    rng = np.random.default_rng(1)
    page = _groups(rng, (16, 8, 128))
    kc, ks = q.quantize_key_page(page)
    vc, vs = q.quantize_value_page(page)
    assert ks.shape == (8, 128) and vs.shape == (16, 8)
    kd = q.dequantize(kc, ks[None])
    vd = q.dequantize(vc, vs[..., None])
    assert (np.abs(kd - page) <= q.max_abs_error_bound(ks)[None]).all()
    assert (np.abs(vd - page) <= q.max_abs_error_bound(vs)[..., None]).all()
    # every group's largest element maps into the top binade: its exponent is the tightest
    assert (np.abs(page).max(axis=0) > 224.0 * np.ldexp(1.0, ks.astype(int) - 127)).all()
    assert (np.abs(page).max(axis=2) > 224.0 * np.ldexp(1.0, vs.astype(int) - 127)).all()
    # relative error of normal-range codes: at most 2^-4
    big = np.abs(kd) >= np.ldexp(2.0 ** -6, ks.astype(int) - 127)[None]
    assert (np.abs(kd - page)[big] <= np.abs(page)[big] / 16).all()


def test_values_on_the_grid_round_trip_exactly():
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 0x7F, size=(16, 4, 64)).astype(np.uint8) | (rng.integers(0, 2, (16, 4, 64)) << 7).astype(np.uint8)
    codes[0] = 0x7E  # a 448 in every channel fixes each channel's exponent at 0
    page = q.e4m3_decode(codes) * np.float32(2.0 ** 5)
    kc, ks = q.quantize_key_page(page)
    assert (ks == 127 + 5).all()
    assert np.array_equal(q.dequantize(kc, ks[None]), page)


def test_dtype_roundings():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3e38, np.nan], dtype=np.float32)
    bf = q.float32_to_bits(x, "bf16")
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf[:-1], want[:-1]) and np.isnan(q.bits_to_float32(bf[-1:], "bf16")).all()
    h = q.float32_to_bits(x[:4], "f16")
    assert np.array_equal(q.bits_to_float32(h, "f16"), x[:4].astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("mistake", ["encode_truncates", "exponent_off_by_one", "value_scale_per_channel",
                                     "decode_bias_8"])
def test_planted_mistakes_fail(monkeypatch, mistake):
    rng = np.random.default_rng(3)
    page = _groups(rng, (16, 4, 64))
    if mistake == "encode_truncates":
        real = q.e4m3_encode

        def trunc(x):
            x = np.asarray(x, dtype=np.float32)
            return real(np.trunc(x * 8) / 8)  # drops rounding information

        monkeypatch.setattr(q, "e4m3_encode", trunc)
        x = boundary_values()
        x = x[np.abs(x) <= 464.0]
        assert not np.array_equal(q.e4m3_encode(x), torch_encode(x))
    elif mistake == "exponent_off_by_one":
        real = q.group_exponent
        monkeypatch.setattr(q, "group_exponent", lambda a: real(a) - 1)
        a = np.float32([1.0, 300.0, 5e-3])
        e = q.group_exponent(a)
        assert not (a.astype(np.float64) <= 448.0 * np.ldexp(1.0, e)).all()
    elif mistake == "value_scale_per_channel":
        # one loud token: per-token value scales keep the quiet tokens' precision; grouping the
        # values per channel (the keys' rule) does not, so its codes differ from the oracle's
        page[3] *= 1000.0
        wrong_codes, _ = q.quantize_key_page(page)
        codes, _ = q.quantize_value_page(page)
        assert not np.array_equal(wrong_codes, codes)
    else:
        c = np.arange(256, dtype=np.uint8)
        E, M = (c >> 3) & 15, c & 7
        wrong = np.where(E == 0, M * 2.0 ** -10, (1 + M / 8) * np.ldexp(1.0, E.astype(int) - 8))
        assert not np.array_equal(wrong[:0x7F].astype(np.float32), q.e4m3_decode(c)[:0x7F])


def test_layer_oracle_quantises_blocks_behind_the_window():
    from kvgen import hf_layout, to_bits

    P, W = 4, 8
    o = q.QuantLayerOracle(2, 40, P, W, "bf16")
    gen = torch.Generator().manual_seed(0)
    k, v = hf_layout(2, 2, 21, 16, torch.bfloat16, gen), hf_layout(2, 2, 21, 16, torch.bfloat16, gen)
    o.append(to_bits(k), to_bits(v))
    assert o.cold.tolist() == [(21 - W) // P] * 2   # blocks 0..2 wholly before positions 13..20
    gk, gv = o.current_tensors()
    assert np.array_equal(gk[:, :, 12:], to_bits(k)[:, :, 12:])  # the window and block 3 exact
    assert not np.array_equal(gk[:, :, :12], to_bits(k)[:, :, :12])
    kc, ks = o.quantized_page(0, 1, True)
    want = q.float32_to_bits(q.dequantize(kc, ks[None]).transpose(1, 0, 2), "bf16")
    assert np.array_equal(gk[0, :, 4:8], want)
    o.crop(13)
    assert o.cold.tolist() == [3, 3]
    o.release_rows([1])
    assert o.cold.tolist() == [3, 0]


def test_crop_reopens_quantised_blocks_with_their_read():
    """A crop to 10 tokens re-opens block 2 (positions 8..11): afterwards every position reads
    the bits it read before the crop (the re-opened block holds its dequantised read), and
    quantising that content again when the block leaves the window anew reads the same bits
    once more (power-of-two scales put a dequantised group on its own grid, and bf16 holds
    every code * 2^e exactly)."""
    from kvgen import hf_layout, to_bits

    P, W = 4, 8
    o = q.QuantLayerOracle(1, 64, P, W, "bf16")
    gen = torch.Generator().manual_seed(1)
    k, v = hf_layout(1, 2, 21, 16, torch.bfloat16, gen), hf_layout(1, 2, 21, 16, torch.bfloat16, gen)
    o.append(to_bits(k), to_bits(v))
    before = o.current_tensors()
    stored = o.keys[0, :, 2].copy()
    o.crop(10)
    assert o.cold.tolist() == [2]
    assert not np.array_equal(o.keys[0, :, 2], stored)  # the content itself changed ...
    got = o._read(o.keys[:1], True).reshape(1, 2, -1, 16)[..., :21, :]
    assert np.array_equal(got, before[0])               # ... to what was read
    o.append(to_bits(k[:, :, :12]), to_bits(v[:, :, :12]))  # to 22: blocks 0..2 quantised again
    assert o.cold.tolist() == [3]
    after = o.current_tensors()
    assert np.array_equal(after[0][..., :10, :], before[0][..., :10, :])
    assert np.array_equal(after[1][..., :10, :], before[1][..., :10, :])
