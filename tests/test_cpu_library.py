"""CPU-side checks of the backend library: it loads, exports every entry
point the header declares, and its pure host logic (edit sets, the edit
table, the Q4_0 split, rope turns, the synthetic weights) behaves as the
reference's. No compute call here needs a GPU."""
import ctypes
import re
import struct
from pathlib import Path

import numpy as np
import pytest

import _oracle as orc
import frizzle_amd as fz

ROOT = Path(__file__).resolve().parent.parent


def header_symbols():
    text = (ROOT / "include" / "frizzle_hip.h").read_text()
    return sorted(set(re.findall(r"\b(frz_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = fz.load()
    declared = header_symbols()
    assert len(declared) > 40
    for name in declared:
        assert hasattr(lib, name), name
    assert set(fz.exported_symbols()) == set(declared)


def test_open_without_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(fz.FrzError):
        fz.Device(0)


def test_q4_0_split_streams():
    rng = np.random.default_rng(0)
    blocks = rng.integers(0, 256, (10, 18), dtype=np.uint8)
    codes, scales = fz.q4_0_split(blocks.reshape(-1))
    assert np.array_equal(codes.reshape(10, 16), blocks[:, 2:])
    assert np.array_equal(scales.reshape(10, 2), blocks[:, :2])


@pytest.mark.parametrize("fmt,bb,sb", [(2, 18, 2), (3, 20, 4), (8, 34, 2)])
def test_block_split_streams(fmt, bb, sb):
    # A block is its scale halves (d; Q4_1 d then m) and then its codes
    # (device_layout.h:114-119 keeps them as two streams).
    rng = np.random.default_rng(fmt)
    blocks = rng.integers(0, 256, (10, bb), dtype=np.uint8)
    codes, scales = fz.block_split(fmt, blocks.reshape(-1))
    assert np.array_equal(codes.reshape(10, bb - sb), blocks[:, sb:])
    assert np.array_equal(scales.reshape(10, sb), blocks[:, :sb])


def test_block_split_refuses_other_formats():
    with pytest.raises(fz.FrzError):
        fz.block_split(0, np.zeros(64, dtype=np.uint8))


def test_rope_turns_match_oracle_and_f64():
    for base in (1e4, 1e6):
        t = fz.rope_turns(base, 256)
        assert np.array_equal(t, orc.rope_turns(base, 256))
        k = np.arange(128)
        want = (base ** (-2.0 * k / 256) / (2 * np.pi)).astype(np.float32)
        assert np.array_equal(t, want)


# ---- edits (tests/contracts/edits/edit_specs_test.cpp) --------------------------

E = fz.Edit
K = fz.EditKind


def test_edit_check_refusals():
    L, F = 26, 6912
    ok = [E(0, 1, K.SET, 1.0, 0, 5), E(0, 1, K.SCALE, 2.0, 5, 9), E(25, 6911, K.ZERO, 0.0)]
    assert fz.edit_check(ok, L, F) == (fz.EditError.OK, 0)
    cases = [
        ([E(26, 0, K.SET, 1.0)], fz.EditError.LAYER, 0),
        ([E(0, 0, K.SET, 1.0), E(0, 6912, K.SET, 1.0)], fz.EditError.NEURON, 1),
        ([E(0, 0, K.SET, float("nan"))], fz.EditError.NOT_FINITE, 0),
        ([E(0, 0, K.SET, float("inf"))], fz.EditError.NOT_FINITE, 0),
        ([E(0, 0, K.ZERO, 1.0)], fz.EditError.ZERO_VALUE, 0),
        ([E(0, 0, K.SET, 1.0, 3, 3)], fz.EditError.RANGE, 0),
        ([E(0, 0, K.SET, 1.0, 0, 5), E(0, 0, K.SET, 2.0, 4, 8)], fz.EditError.OVERLAP, 1),
        ([E(0, 0, K.SET, 1.0, 4, 8), E(0, 0, K.SET, 2.0, 0, 5)], fz.EditError.OVERLAP, 1),
        # a long range given late overlaps two short ones: the late one is named
        ([E(0, 0, K.SET, 1.0, 0, 2), E(0, 0, K.SET, 1.0, 5, 7), E(0, 0, K.SET, 1.0, 1, 9)],
         fz.EditError.OVERLAP, 2),
    ]
    for edits, err, idx in cases:
        assert fz.edit_check(edits, L, F) == (err, idx), edits
    bad_kind = [fz._lib.Edit(0, 0, 3, 1.0, 0, 1)]
    off = ctypes.c_uint32()
    arr = (fz._lib.Edit * 1)(*bad_kind)
    assert fz.load().frz_edit_check(arr, 1, L, F, ctypes.byref(off)) == fz.EditError.KIND
    many = [E(0, n % 6912, K.SET, 1.0, n // 6912, n // 6912 + 1) for n in range(4097)]
    assert fz.edit_check(many, L, F)[0] == fz.EditError.TOO_MANY
    # adjacent ranges of one neuron do not overlap
    assert fz.edit_check([E(0, 0, K.SET, 1.0, 0, 5), E(0, 0, K.SET, 1.0, 5, 9)], L, F)[0] == 0


def test_edit_table_layout():
    layers = 3
    edits = [E(2, 9, K.SCALE, -1.75, 1, 4), E(0, 3, K.SET, 2.5), E(2, 1, K.ZERO, 0.0, 0, 2),
             E(2, 9, K.SET, 4.0, 4, fz.TO_THE_END)]
    t = fz.edit_table(edits, layers, origin=10)
    assert t.size == 2 * layers + 5 * len(edits)
    # layer heads: [first, count]
    assert list(t[0:6]) == [6, 1, 0, 0, 11, 3]
    f = lambda v: struct.unpack("<I", struct.pack("<f", v))[0]
    assert list(t[6:11]) == [3, 0, f(2.5), 10, 0xFFFFFFFF]
    # layer 2 by neuron, then first step
    assert list(t[11:16]) == [1, 2, f(0.0), 10, 12]
    assert list(t[16:21]) == [9, 1, f(-1.75), 11, 14]
    assert list(t[21:26]) == [9, 0, f(4.0), 14, 0xFFFFFFFF]
    # saturation near the end of positions
    t2 = fz.edit_table([E(0, 0, K.SET, 1.0, 5, 0xFFFFFFF0)], 1, origin=100)
    assert t2[5] == 105 and t2[6] == 0xFFFFFFFF


def test_edit_apply_is_the_oracle():
    sub = np.array([0x123], dtype=np.uint32).view(np.float32)[0]
    assert fz.edit_apply(K.SET, 3.0, 7.0) == 3.0
    assert fz.edit_apply(K.ZERO, 0.0, 7.0) == 0.0
    assert fz.edit_apply(K.SCALE, -1.75, 2.0) == -3.5
    got = np.float32(fz.edit_apply(K.SCALE, 1.0, float(sub)))
    assert got.view(np.uint32) == 0x123


def test_synthetic_weights_are_seeded_and_shaped():
    cfg = fz.gemma3_1b_config(layers=2, vocab=4096)
    a = fz.synth_tensor(cfg, 5, 0, "gate")
    b = fz.synth_tensor(cfg, 5, 0, "gate")
    c = fz.synth_tensor(cfg, 6, 0, "gate")
    d = fz.synth_tensor(cfg, 5, 1, "gate")
    assert a.size == 6912 * 1152 // 32 * 18
    assert np.array_equal(a, b) and not np.array_equal(a, c) and not np.array_equal(a, d)
    blocks = a.reshape(-1, 18)
    scales = blocks[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    assert (scales >= 0).all()
    # |N(0, 0.02)|: mean 0.02 * sqrt(2 / pi), rms 0.02
    assert abs(scales.mean() - 0.02 * np.sqrt(2 / np.pi)) < 2e-4
    assert abs(np.sqrt((scales ** 2).mean()) - 0.02) < 2e-4
    codes = np.concatenate([blocks[:, 2:] & 15, blocks[:, 2:] >> 4]).ravel()
    counts = np.bincount(codes, minlength=16)
    assert counts.min() > 0.98 * counts.mean() and counts.max() < 1.02 * counts.mean()
    g = fz.synth_tensor(cfg, 5, 0, "attn_norm")
    assert g.dtype == np.float32 and g.size == 1152
    assert abs(g.mean() - 1.0) < 0.02 and abs(g.std() - 0.1) < 0.01
