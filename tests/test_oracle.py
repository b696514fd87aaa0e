"""Pins the CPU oracle (oracle/kquant_ref.c) before anything is checked against it.

Each function of the oracle is checked against something other than its own
formula: the reference's known-answer tests, exhaustive comparison with
numpy's IEEE half conversion, a round trip through an encoder written from
the GGML scale-packing description, hand-worked values, exact rational
arithmetic, and a second vectorised restatement that is structured
differently (tests/numpy_ref.py).
"""
import json
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import numpy_ref
import oracle_lib as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (bits(a) == bits(b))))


# ---- a2: f16 -> f32 ----------------------------------------------------------
def test_f16_to_f32_exhaustive_matches_ieee_half():
    pats = np.arange(65536, dtype=np.uint32)
    ours = np.array([O.f16_to_f32_bits(int(p)) for p in pats], dtype=np.uint32).view(np.float32)
    ref = pats.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(bits(ours[finite]), bits(ref[finite]))
    # NaNs: quant.rs keeps sign and payload (fraction << 13) without quieting
    nan_pats = pats[~finite]
    expect = ((nan_pats & 0x8000) << 16) | 0x7F800000 | ((nan_pats & 0x3FF) << 13)
    assert np.array_equal(bits(ours[~finite]), expect.astype(np.uint32))


def test_f16_subnormals_and_specials():
    assert O.f16_to_f32(0x0001) == 2.0 ** -24
    assert O.f16_to_f32(0x03FF) == 1023 * 2.0 ** -24
    assert O.f16_to_f32(0x0400) == 2.0 ** -14
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0xC000) == -2.0
    assert O.f16_to_f32(0x7BFF) == 65504.0
    assert O.f16_to_f32(0x7C00) == float("inf")
    assert np.signbit(np.float32(O.f16_to_f32(0x8000)))


# ---- a3: get_scale_min ---------------------------------------------------------
def test_get_scale_min_round_trips_an_independent_encoder():
    rng = np.random.default_rng(7)
    for _ in range(2000):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        packed = numpy_ref.encode_k4_scales(sc, mn)
        for j in range(8):
            assert O.get_scale_min(j, packed) == (sc[j], mn[j])
    # every 6-bit value at every position
    for j in range(8):
        for v in range(64):
            sc = [0] * 8
            mn = [0] * 8
            sc[j] = v
            mn[j] = 63 - v
            packed = numpy_ref.encode_k4_scales(sc, mn)
            got = [O.get_scale_min(k, packed) for k in range(8)]
            assert got == list(zip(sc, mn))


def test_get_scale_min_hand_worked_values():
    # scale bytes of metal.rs:7549 worked out bit by bit
    s = bytes([7, 19, 31, 43, 55, 67, 79, 91, 103, 115, 127, 139])
    assert O.get_scale_min(0, s) == (7, 55)      # s0&63, s4&63
    assert O.get_scale_min(3, s) == (43, 27)     # 91&63 = 27
    assert O.get_scale_min(4, s) == (7, 6)       # (103&15)|0, (103>>4)|((55>>6)<<4)
    assert O.get_scale_min(5, s) == (3, 23)      # (115&15)|((19>>6)<<4)=3; 7|((67>>6)<<4)=23
    assert O.get_scale_min(7, s) == (11, 24)     # (139&15)|0=11; 8|((91>>6)<<4)=24


def test_get_scale_min_exhaustive_low_indices():
    # j < 4 depends on two bytes only: check all 65,536 pairs for j = 0
    for a in range(0, 256, 3):
        for b in range(256):
            s = bytes([a, 0, 0, 0, b, 0, 0, 0, 0, 0, 0, 0])
            assert O.get_scale_min(0, s) == (a & 63, b & 63)


# ---- a4-a7: dequantisers --------------------------------------------------------
def test_reference_known_answer_tests():
    kats = json.loads((GOLDEN / "quant_kats.json").read_text())
    for k in kats["kats"]:
        got = O.dequantize(k["ggml_type"], bytes.fromhex(k["bytes"]), k["elements"])
        assert np.array_equal(got, np.array(k["expected"], dtype=np.float32)), k["name"]


def test_reference_rejections():
    kats = json.loads((GOLDEN / "quant_kats.json").read_text())
    for r in kats["rejections"]:
        assert O.dequantize_rc(r["ggml_type"], bytes(r["byte_len"]), r["elements"]) != O.KQ_OK
    assert O.dequantize_rc(12, b"", 0) == O.KQ_ERR_ELEMENTS
    assert O.dequantize_rc(12, bytes(144), 255) == O.KQ_ERR_ELEMENTS
    assert O.dequantize_rc(13, bytes(175), 256) == O.KQ_ERR_BYTES
    assert O.dequantize_rc(14, bytes(211), 256) == O.KQ_ERR_BYTES
    assert O.dequantize_rc(15, bytes(210), 256) == O.KQ_ERR_TYPE


@pytest.mark.parametrize("t,name", [(12, "q4_k"), (13, "q5_k"), (14, "q6_k")])
def test_committed_block_fixtures(t, name):
    fx = json.loads((GOLDEN / f"blocks_{name}.json").read_text())
    got = O.dequantize(t, bytes.fromhex(fx["bytes"]), fx["n_blocks"] * 256)
    exp = np.array(fx["expected_bits"], dtype=np.uint32).view(np.float32)
    assert same_bits(got, exp)


@pytest.mark.parametrize("t", [12, 13, 14])
def test_oracle_matches_independent_numpy_restatement(t):
    rng = np.random.default_rng(100 + t)
    bb = numpy_ref.BLOCK[t]
    data = rng.integers(0, 256, 12000 * bb, dtype=np.uint8)
    # keep most d/dmin finite so values are exercised, not only NaNs
    halves = rng.choice(np.array([0x3C00, 0x2E66, 0x1400, 0x0003, 0x8123, 0x0400], np.uint16), 24000)
    blocks = data.reshape(-1, bb)
    if t == 14:
        blocks[:, 208:210] = halves[:12000].view(np.uint8).reshape(-1, 2)
    else:
        blocks[:, 0:2] = halves[:12000].view(np.uint8).reshape(-1, 2)
        blocks[:, 2:4] = halves[12000:].view(np.uint8).reshape(-1, 2)
    got = O.dequantize(t, blocks.tobytes(), 12000 * 256)
    exp = numpy_ref.dequant(t, blocks.tobytes())
    assert same_bits(got, exp)


def test_q4_k_element_layout_by_construction():
    # one block, d=1, dmin=0, every scale 1: value k of group g is the nibble
    # placed at byte g*32 + (k % 32), low half for k < 32, high half otherwise
    blk = bytearray(144)
    blk[0:2] = struct.pack("<H", 0x3C00)
    blk[4:16] = numpy_ref.encode_k4_scales([1] * 8, [0] * 8)
    for g in range(4):
        for i in range(32):
            blk[16 + 32 * g + i] = (i % 16) | (((i + g) % 16) << 4)
    v = O.dequantize(12, bytes(blk), 256)
    for g in range(4):
        for i in range(32):
            assert v[64 * g + i] == i % 16
            assert v[64 * g + 32 + i] == (i + g) % 16


def test_q6_k_element_layout_by_construction():
    # d=1, all scales 1, q = element index mod 64 encoded by hand
    blk = bytearray(210)
    blk[208:210] = struct.pack("<H", 0x3C00)
    blk[192:208] = bytes([1] * 16)
    want = np.zeros(256)
    for h in range(2):
        for i in range(32):
            qs = [(h * 128 + i + 32 * k) % 64 for k in range(4)]
            blk[64 * h + i] = (qs[0] & 15) | ((qs[2] & 15) << 4)
            blk[64 * h + 32 + i] = (qs[1] & 15) | ((qs[3] & 15) << 4)
            blk[128 + 32 * h + i] = (qs[0] >> 4) | ((qs[1] >> 4) << 2) | ((qs[2] >> 4) << 4) | ((qs[3] >> 4) << 6)
            for k in range(4):
                want[128 * h + 32 * k + i] = qs[k] - 32
    assert np.array_equal(O.dequantize(14, bytes(blk), 256), want.astype(np.float32))


def test_q5_k_high_bit_masks_by_construction():
    # qh bit 2g lifts low nibbles of group g, bit 2g+1 the high ones
    blk = bytearray(176)
    blk[0:2] = struct.pack("<H", 0x3C00)
    blk[4:16] = numpy_ref.encode_k4_scales([1] * 8, [0] * 8)
    for i in range(32):
        blk[16 + i] = 1 << (i % 8)
    v = O.dequantize(13, bytes(blk), 256)
    for g in range(4):
        for i in range(32):
            assert v[64 * g + i] == (16 if i % 8 == 2 * g else 0)
            assert v[64 * g + 32 + i] == (16 if i % 8 == 2 * g + 1 else 0)


# ---- a8: dots ---------------------------------------------------------------------
def test_f64_dot_is_exact_for_small_integers_and_matches_fractions():
    rng = np.random.default_rng(3)
    w = rng.standard_normal(300).astype(np.float32)
    x = rng.standard_normal(300).astype(np.float32)
    lib = O.lib()
    fp = lambda a: a.ctypes.data_as(O._FP)
    exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(w, x))
    got = lib.kq_dot_f64(fp(w), fp(x), 300)
    assert abs(Fraction(got) - exact) <= Fraction(300 * 2 ** -52) * sum(abs(Fraction(float(a) * float(b))) for a, b in zip(w, x))
    assert lib.kq_abs_dot_f64(fp(w), fp(x), 300) == pytest.approx(float(np.sum(np.abs(w.astype(np.float64) * x))), rel=1e-12)


def test_f32_sequential_dot_matches_a_left_fold():
    rng = np.random.default_rng(4)
    w = rng.standard_normal(1000).astype(np.float32)
    x = rng.standard_normal(1000).astype(np.float32)
    acc = np.float32(-0.0)
    for p in (w * x):
        acc = np.float32(acc + p)
    lib = O.lib()
    got = lib.kq_dot_f32_sequential(w.ctypes.data_as(O._FP), x.ctypes.data_as(O._FP), 1000)
    assert np.float32(got).view(np.uint32) == acc.view(np.uint32)
    # cumsum in float32 is the same sequential fold
    assert np.float32(got) == np.cumsum(w * x, dtype=np.float32)[-1]


@pytest.mark.parametrize("t", [12, 13, 14])
def test_matvec_ref_threads_agree_and_match_dequant_plus_dot(t):
    import si_hip
    rows, cols = 37, 1024
    data = si_hip.synth_matrix(t, seed=9, rows=rows, cols=cols)
    x = si_hip.synth_normal(11, cols)
    y32a, y64a, aba = O.matvec(t, data, rows, cols, x, threads=1)
    y32b, y64b, abb = O.matvec(t, data, rows, cols, x, threads=5)
    assert np.array_equal(y32a, y32b) and np.array_equal(y64a, y64b) and np.array_equal(aba, abb)
    w = numpy_ref.dequant(t, data.tobytes()).reshape(rows, cols)
    assert np.allclose(y64a, w.astype(np.float64) @ x.astype(np.float64), rtol=0, atol=1e-9)
    for r in range(rows):
        assert y32a[r] == np.cumsum(w[r] * x, dtype=np.float32)[-1]


# ---- a12/a16: SiLU and argmax ------------------------------------------------------
def test_silu_matches_definition():
    for v in [-20.0, -1.5, -0.0, 0.0, 0.25, 3.0, 40.0]:
        ref = np.float32(v) / (np.float32(1.0) + np.exp(np.float32(-v), dtype=np.float32))
        assert O.silu(v) == pytest.approx(float(ref), rel=2e-7, abs=1e-30)


def test_argmax_rules_on_crafted_vectors():
    inf, nan = float("inf"), float("nan")
    cases = [
        # values,                      last-finite, first-greater
        ([1.0, 3.0, 3.0, 2.0],              2, 1),
        ([nan, 5.0, nan, 5.0],              3, 1),
        ([-0.0, 0.0, -0.0],                 1, 0),   # total_cmp: +0 > -0; '>' treats them equal
        ([0.0, -0.0],                       0, 0),
        ([1.0, inf, 2.0],                   2, 1),   # inf filtered out / inf allowed
        ([-inf, -inf],                      None, 0),
        ([nan, nan],                        None, 0),
        ([-inf, -3.0, nan],                 1, 1),
        ([-1e30, -1e30],                    1, 0),
        ([7.0],                             0, 0),
    ]
    for vals, last, first in cases:
        assert O.argmax_last_finite(vals) == last, vals
        assert O.argmax_first_greater(vals) == first, vals
