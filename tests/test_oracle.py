"""Pins the CPU oracle (oracle/kv_oracle.py) before anything is compared with it.

Each reference behaviour is checked against something that does not share the oracle's code:
the reference's own known-answer case (fixture), the transformers library routine
DynamicLayer.update (concatenation), the slot-history model (tests/slot_history.py), the
config-1 golden digests, and invariants.  The last tests plant plausible mistakes in the
oracle and show that these checks catch each one.
"""

from __future__ import annotations

import copy
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from kvgen import C1, config1_steps, from_bits, to_bits
from oracle.kv_oracle import CapacityError, DenseLayerOracle, dense_append_reference
from slot_history import SlotHistory

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ----------------------------------------------------------------------------- checks
def check_known_answer(oracle_cls=DenseLayerOracle):
    with open(os.path.join(GOLDEN, "known_answer_update.json")) as f:
        fx = json.load(f)
    layer = oracle_cls(**fx["layer"])
    for call in fx["calls"]:
        k = np.asarray(call["keys"], dtype=np.float32).view(np.uint32)
        v = np.asarray(call["values"], dtype=np.float32).view(np.uint32)
        gk, gv = layer.update(k, v)
        assert np.array_equal(gk, np.asarray(call["expect_keys"], dtype=np.float32).view(np.uint32))
        assert np.array_equal(gv, np.asarray(call["expect_values"], dtype=np.float32).view(np.uint32))
        assert layer.get_seq_length() == call["expect_seq_length"]


def check_against_dynamic_layer(oracle_cls=DenseLayerOracle, seed=0):
    """Uniform appends (every row the same length): the cache equals torch.cat along the
    sequence axis, which is transformers' DynamicLayer.update."""
    from transformers.cache_utils import DynamicLayer

    rng = np.random.default_rng(seed)
    batch, heads, dim, page = 3, 2, 8, 4
    chunks = [int(x) for x in rng.integers(1, 7, size=6)]
    oracle = oracle_cls(max_batch_size=batch, max_cache_len=sum(chunks) + 3, page_size=page)
    dyn = DynamicLayer()
    gen = torch.Generator().manual_seed(seed)
    for t in chunks:
        k = torch.randn((batch, heads, t, dim), generator=gen).to(torch.bfloat16)
        v = torch.randn((batch, heads, t, dim), generator=gen).to(torch.bfloat16)
        dk, dv = dyn.update(k, v)
        ok, ov = oracle.update(to_bits(k), to_bits(v))
        assert np.array_equal(ok, to_bits(dk)) and np.array_equal(ov, to_bits(dv))
        assert oracle.get_seq_length() == dyn.get_seq_length()


def random_program(seed, batch_max=4, heads=2, dim=4, cap=24, page=4, steps=40):
    """A seeded sequence of layer calls: ragged appends (varying batch), crop, beam select,
    repeat-interleave, reset and row release."""
    rng = np.random.default_rng(seed)
    ops = []
    cur_rows = batch_max
    for _ in range(steps):
        r = rng.random()
        if r < 0.6:
            b = int(rng.integers(1, cur_rows + 1))
            t = int(rng.integers(1, 5))
            k = rng.integers(0, 2**16, size=(b, heads, t, dim), dtype=np.uint16)
            v = rng.integers(0, 2**16, size=(b, heads, t, dim), dtype=np.uint16)
            ops.append(("append", k, v))
        elif r < 0.72:
            ops.append(("crop", int(rng.integers(-3, cap))))
        elif r < 0.80:
            ops.append(("select", None))
        elif r < 0.84:
            ops.append(("repeat", 2))
        elif r < 0.90:
            ops.append(("release", None))
        else:
            ops.append(("reset",))
    return ops, dict(batch_max=batch_max, heads=heads, dim=dim, cap=cap, page=page)


def stale_program():
    """Two rows reach 10 tokens, both are cropped to 5, then only row 0 grows; a later append to
    both rows leaves row 1 shorter than row 0, so its pre-crop slots 6..8 are visible padding."""
    rng = np.random.default_rng(99)
    geo = dict(batch_max=2, heads=2, dim=4, cap=24, page=4)

    def kv(b, t):
        return (rng.integers(0, 2**16, size=(b, 2, t, 4), dtype=np.uint16),
                rng.integers(0, 2**16, size=(b, 2, t, 4), dtype=np.uint16))

    ops = [("append", *kv(2, 10)), ("crop", 5), ("append", *kv(1, 3)), ("append", *kv(2, 1))]
    return ops, geo


def run_program_oracle_vs_history(ops, geo, oracle_cls=DenseLayerOracle, seed=0):
    rng = np.random.default_rng(seed + 1)
    oracle = oracle_cls(max_batch_size=geo["batch_max"], max_cache_len=geo["cap"], page_size=geo["page"])
    hist = SlotHistory(geo["batch_max"])
    for op in ops:
        if op[0] == "append":
            k, v = op[1], op[2]
            if k.shape[0] > oracle.max_batch_size:
                continue
            ends = [hist.lens[b] + k.shape[2] for b in range(k.shape[0])]
            if max(ends) > geo["cap"]:
                with pytest.raises(CapacityError):
                    oracle.update(k, v)
                # the reference appends the rows before the first overflowing one (kv_cache.py:77-90)
                first_bad = next(i for i, e in enumerate(ends) if e > geo["cap"])
                if first_bad:
                    hist.append(k[:first_bad], v[:first_bad])
                # rows past first_bad keep their length; current batch is not updated
                hist.current = oracle.current_batch_size
                continue
            gk, gv = oracle.update(k, v)
            hist.append(k, v)
            hk, hv = hist.gather(geo["heads"], geo["dim"], np.uint16)
            assert gk.shape == hk.shape
            assert np.array_equal(gk, hk) and np.array_equal(gv, hv)
            assert oracle.get_seq_length() == hist.seq_length()
        elif op[0] == "crop":
            if not oracle.is_initialized:
                continue
            m = op[1]
            if m < 0:
                m = hist.seq_length() - abs(m)
            oracle.crop(op[1])
            hist.crop(max(m, 0))
        elif op[0] in ("select", "repeat"):
            if not oracle.is_initialized or oracle.current_batch_size == 0:
                continue
            cur = oracle.current_batch_size
            if op[0] == "select":
                rows = [int(x) for x in rng.integers(0, cur, size=cur)]
                oracle.batch_select_indices(rows)
            else:
                rows = [b for b in range(cur) for _ in range(op[1])]
                oracle.batch_repeat_interleave(op[1])
            hist.select(rows)
            hist.rows += [dict() for _ in range(max(0, oracle.max_batch_size - len(hist.rows)))]
        elif op[0] == "release":
            if not oracle.is_initialized:
                continue
            rows = [0] if oracle.max_batch_size else []
            oracle.release_rows(rows)
            hist.release(rows)
        elif op[0] == "reset":
            oracle.reset()
            hist.reset()
        if oracle.is_initialized and oracle.current_batch_size:
            ok, ov = oracle.current_tensors()
            hk, hv = hist.gather(geo["heads"], geo["dim"], np.uint16)
            assert np.array_equal(ok, hk) and np.array_equal(ov, hv)


def check_config1_digests(oracle_cls=DenseLayerOracle):
    with open(os.path.join(GOLDEN, "config1_digests.json")) as f:
        fx = json.load(f)
    cap = C1["prefill"] + C1["decode"]
    layers = [oracle_cls(C1["batch"], cap, C1["page"]) for _ in range(C1["layers"])]
    for step_idx, step in enumerate(config1_steps()):
        for li, (k, v) in enumerate(step):
            gk, gv = layers[li].update(to_bits(k), to_bits(v))
            h = hashlib.sha256(gk.tobytes() + gv.tobytes()).hexdigest()[:16]
            assert h == fx["layers"][li][step_idx], (li, step_idx)


# ----------------------------------------------------------------------------- tests
def test_known_answer_fixture():
    check_known_answer()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_uniform_appends_equal_dynamic_layer_concat(seed):
    check_against_dynamic_layer(seed=seed)


@pytest.mark.parametrize("seed", range(12))
def test_random_programs_match_slot_history(seed):
    ops, geo = random_program(seed)
    run_program_oracle_vs_history(ops, geo, seed=seed)


def test_crop_keeps_stale_slots_visible():
    ops, geo = stale_program()
    run_program_oracle_vs_history(ops, geo)


def test_config1_golden_digests():
    check_config1_digests()


def test_fixture_dtype_roundtrip():
    t = torch.tensor([1.5, -0.0, float("nan"), float("inf")], dtype=torch.bfloat16)
    assert torch.equal(from_bits(to_bits(t), torch.bfloat16).view(torch.int16), t.view(torch.int16))


def test_capacity_error_and_partial_append():
    layer = DenseLayerOracle(max_batch_size=2, max_cache_len=5, page_size=2)
    layer.update(np.ones((2, 1, 2, 2), np.uint16), np.ones((2, 1, 2, 2), np.uint16))
    layer.update(np.full((1, 1, 3, 2), 7, np.uint16), np.full((1, 1, 3, 2), 7, np.uint16))  # row 0 -> 5
    with pytest.raises(CapacityError, match="requested 6, max_cache_len=5"):
        layer.update(np.full((2, 1, 1, 2), 9, np.uint16), np.full((2, 1, 1, 2), 9, np.uint16))
    assert list(layer.seq_lens) == [5, 2]
    # rows are appended in order: a failure at row 1 leaves row 0 appended
    layer2 = DenseLayerOracle(max_batch_size=2, max_cache_len=4, page_size=2)
    layer2.update(np.zeros((2, 1, 1, 2), np.uint16), np.zeros((2, 1, 1, 2), np.uint16))
    layer2.update(np.zeros((2, 1, 2, 2), np.uint16)[1:], np.zeros((1, 1, 2, 2), np.uint16))  # row 0 -> 3
    layer2.seq_lens[:] = [1, 3]
    with pytest.raises(CapacityError):
        layer2.update(np.zeros((2, 1, 2, 2), np.uint16), np.zeros((2, 1, 2, 2), np.uint16))
    assert list(layer2.seq_lens) == [3, 3]


def test_mask_sizes_and_crop_negative():
    layer = DenseLayerOracle(max_batch_size=1, max_cache_len=16, page_size=4)
    layer.update(np.zeros((1, 1, 6, 2), np.uint16), np.zeros((1, 1, 6, 2), np.uint16))
    assert layer.get_mask_sizes(3) == (9, 0)
    layer.crop(-2)
    assert layer.get_seq_length() == 4
    layer.crop(10)
    assert layer.get_seq_length() == 4
    layer.crop(-10)
    assert layer.get_seq_length() == 0


def test_dense_append_reference_against_history():
    rng = np.random.default_rng(5)
    B, H, MB, P, D = 3, 2, 4, 4, 8
    kc = np.zeros((B, H, MB, P, D), np.uint32)
    vc = np.zeros_like(kc)
    lens = np.zeros(B, np.int64)
    hist = SlotHistory(B)
    for _ in range(5):
        b = int(rng.integers(1, B + 1))
        t = int(rng.integers(1, 4))
        if int(lens[:b].max()) + t > MB * P:
            break
        k = rng.integers(0, 2**32, size=(b, H, t, D), dtype=np.uint32)
        v = rng.integers(0, 2**32, size=(b, H, t, D), dtype=np.uint32)
        dense_append_reference(kc, vc, lens, k, v)
        hist.append(k, v)
        assert list(lens) == hist.lens
    flat_k = kc.reshape(B, H, MB * P, D)
    hist.current = B
    seq = MB * P
    for b in range(B):
        for s in range(seq):
            rec = hist.rows[b].get(s)
            want = hist.inputs[rec[0]][0][rec[1], :, rec[2], :] if rec else np.zeros((H, D), np.uint32)
            assert np.array_equal(flat_k[b, :, s, :], want)


def test_dense_append_reference_capacity_message_and_no_mutation():
    kc = np.zeros((1, 1, 2, 2, 2), np.uint16)
    vc = np.zeros_like(kc)
    lens = np.array([3], np.int32)
    with pytest.raises(RuntimeError, match=r"requested 5 tokens, max_cache_len=4"):
        dense_append_reference(kc, vc, lens, np.ones((1, 1, 2, 2), np.uint16), np.ones((1, 1, 2, 2), np.uint16))
    assert lens[0] == 3 and not kc.any()


# ----------------------------------------------------------------------------- planted mistakes
class _OffByOnePage(DenseLayerOracle):
    def _python_append(self, key_states, value_states):
        batch_size, _, token_count, _ = key_states.shape
        for b in range(batch_size):
            start = int(self.seq_lens[b])
            for t in range(token_count):
                pos = start + t
                blk, off = pos // self.page_size, (pos + 1) % self.page_size  # wrong offset
                self.keys[b, :, blk, off, :] = key_states[b, :, t, :]
                self.values[b, :, blk, off, :] = value_states[b, :, t, :]
            self.seq_lens[b] = start + token_count
        self.current_batch_size = batch_size


class _SwappedKV(DenseLayerOracle):
    def current_tensors(self):
        k, v = super().current_tensors()
        return v, k


class _NoZeroInit(DenseLayerOracle):
    def lazy_initialization(self, key_states):
        super().lazy_initialization(key_states)
        self.keys[...] = 1  # stale bits instead of zeros
        self.values[...] = 1


class _CropZeroes(DenseLayerOracle):
    def crop(self, max_length):
        super().crop(max_length)
        for b in range(self.current_batch_size):  # clearing data the reference keeps
            n = int(self.seq_lens[b])
            flat = self.keys[b].reshape(self.keys.shape[1], -1, self.keys.shape[-1])
            flat[:, n:, :] = 0


class _SeqLenFromAllRows(DenseLayerOracle):
    def get_seq_length(self):
        if not self.is_initialized:
            return 0
        return int(self.seq_lens.max())  # ignores current_batch_size


class _SelectIgnoresIndices(DenseLayerOracle):
    def batch_select_indices(self, indices):
        n = len(indices)
        super().batch_select_indices(list(range(min(n, self.current_batch_size))) + [0] * max(0, n - self.current_batch_size))


def _ragged_programs_fail(cls):
    programs = [random_program(seed) for seed in range(12)] + [stale_program()]
    for seed, (ops, geo) in enumerate(programs):
        try:
            run_program_oracle_vs_history(ops, geo, oracle_cls=cls, seed=seed)
        except AssertionError:
            return True
    return False


@pytest.mark.parametrize("cls", [_OffByOnePage, _SwappedKV])
def test_planted_mistakes_fail_known_answer(cls):
    with pytest.raises(AssertionError):
        check_known_answer(cls)


@pytest.mark.parametrize("cls", [_OffByOnePage, _SwappedKV, _NoZeroInit, _CropZeroes,
                                 _SeqLenFromAllRows, _SelectIgnoresIndices])
def test_planted_mistakes_fail_slot_history(cls):
    assert _ragged_programs_fail(cls)


def test_planted_mistake_fails_dynamic_layer_check():
    with pytest.raises(AssertionError):
        check_against_dynamic_layer(_OffByOnePage)


def test_planted_mistake_fails_golden_digests():
    with pytest.raises(AssertionError):
        check_config1_digests(_OffByOnePage)


# ----------------------------------------------------------------------------- torch restatement
# oracle/kv_oracle_torch.py is the CPU baseline bench.py times on the host's cores; it must give
# the numpy oracle's bits.  It is fed the same raw bits as signed-integer tensors (its operations
# are copies, so the element type does not matter).
_SIGNED_NP = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32, np.dtype(np.uint64): np.int64}


class TorchBits:
    """DenseLayerTorch behind the numpy oracle's bits interface."""

    def __init__(self, max_batch_size, max_cache_len, page_size=16):
        from oracle.kv_oracle_torch import DenseLayerTorch

        self.layer = DenseLayerTorch(max_batch_size, max_cache_len, page_size)

    def update(self, k, v):
        u = k.dtype
        gk, gv = self.layer.update(torch.from_numpy(np.ascontiguousarray(k).view(_SIGNED_NP[u])),
                                   torch.from_numpy(np.ascontiguousarray(v).view(_SIGNED_NP[u])))
        return gk.numpy().view(u), gv.numpy().view(u)

    def release_rows(self, rows):
        self.layer.release_rows(rows)

    def get_seq_length(self):
        return self.layer.get_seq_length()


def test_torch_restatement_known_answer_and_golden_digests():
    check_known_answer(TorchBits)
    check_config1_digests(TorchBits)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_torch_restatement_matches_numpy_oracle(seed):
    rng = np.random.default_rng(500 + seed)
    Bmax, H, D, cap, P = 5, 2, 8, 40, 4
    a, b = DenseLayerOracle(Bmax, cap, P), TorchBits(Bmax, cap, P)
    for _ in range(40):
        if rng.random() < 0.15 and a.is_initialized:
            rows = sorted(rng.choice(Bmax, size=int(rng.integers(1, 3)), replace=False).tolist())
            a.release_rows(rows)
            b.release_rows(rows)
            continue
        n = int(rng.integers(1, Bmax + 1))
        t = int(rng.integers(1, 6))
        if a.is_initialized and int(a.seq_lens[:n].max()) + t > cap:
            continue
        k = rng.integers(0, 2**16, size=(n, H, t, D), dtype=np.uint16)
        v = rng.integers(0, 2**16, size=(n, H, t, D), dtype=np.uint16)
        ak, av = a.update(k, v)
        bk, bv = b.update(k, v)
        assert np.array_equal(ak, bk) and np.array_equal(av, bv)
        assert a.get_seq_length() == b.get_seq_length()


def test_torch_restatement_capacity_error():
    b = TorchBits(2, 6, 4)
    b.update(np.zeros((2, 1, 5, 2), np.uint16), np.zeros((2, 1, 5, 2), np.uint16))
    with pytest.raises(ValueError, match="capacity exceeded"):
        b.update(np.zeros((1, 1, 2, 2), np.uint16), np.zeros((1, 1, 2, 2), np.uint16))


@pytest.mark.parametrize("seed", [0, 1])
def test_append_rows_matches_slot_history_in_both_oracles(seed):
    """append_rows (a new sequence's prefill into freed rows while others decode) in the numpy
    and torch restatements, against the slot-history model (no pages, no dense layout)."""
    rng = np.random.default_rng(700 + seed)
    Bmax, H, D, cap, P = 6, 2, 4, 48, 4
    a, b = DenseLayerOracle(Bmax, cap, P), TorchBits(Bmax, cap, P)
    hist = SlotHistory(Bmax)
    k = rng.integers(0, 2**16, size=(Bmax, H, 5, D), dtype=np.uint16)
    for layer in (a, b):
        layer.update(k, k)
    hist.append(k, k)
    for _ in range(25):
        if rng.random() < 0.4:
            rows = sorted(rng.choice(Bmax, size=int(rng.integers(1, 3)), replace=False).tolist())
            for layer in (a, b):
                layer.release_rows(rows)
            hist.release(rows)
            t = int(rng.integers(1, 9))
            kr = rng.integers(0, 2**16, size=(len(rows), H, t, D), dtype=np.uint16)
            vr = rng.integers(0, 2**16, size=(len(rows), H, t, D), dtype=np.uint16)
            if max(hist.lens[r] for r in rows) + t > cap:
                continue
            a.append_rows(rows, kr, vr)
            b.layer.append_rows(rows, torch.from_numpy(kr.view(np.int16)), torch.from_numpy(vr.view(np.int16)))
            hist.append_rows(rows, kr, vr)
        if max(hist.lens) + 1 > cap:
            break
        k = rng.integers(0, 2**16, size=(Bmax, H, 1, D), dtype=np.uint16)
        ak, av = a.update(k, k)
        bk, bv = b.update(k, k)
        hist.append(k, k)
        hk, hv = hist.gather(H, D, np.uint16)
        assert np.array_equal(ak, hk) and np.array_equal(av, hv)
        assert np.array_equal(bk, hk) and np.array_equal(bv, hv)
