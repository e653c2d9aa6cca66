"""Pins of the oracle's FP8 E4M3 codec (oracle/nflow_oracle.c, restating
cpp/include/neuroflow/fp8_e4m3.h): the reference's own known-answer tests,
the reference build itself (oracle/_ref), and what the mathematics fixes
(nearest representable value, ties to even, saturation)."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

KATS = json.loads((Path(__file__).parent / "golden" / "fp8_e4m3_kats.json").read_text())
FIX = np.load(Path(__file__).parent / "golden" / "ref_int8_vectors.npz")


def _f(hexbits):
    return np.array([int(hexbits, 16)], np.uint32).view(np.float32)


@pytest.mark.parametrize("kat", KATS["encode"], ids=lambda k: k["cite"])
def test_encode_known_answers(kat):
    assert int(O.e4m3_encode(_f(kat["x"]))[0]) == kat["byte"]


@pytest.mark.parametrize("kat", KATS["decode"], ids=lambda k: k["cite"])
def test_decode_known_answers(kat):
    got = O.e4m3_decode(np.array([kat["byte"]], np.uint8))
    assert got.view(np.uint32)[0] == int(kat["x"], 16)


def test_decode_nan_bytes():
    for kat in KATS["decode_nan"]:
        assert np.isnan(O.e4m3_decode(np.array([kat["byte"]], np.uint8))[0])
    assert np.isfinite(O.e4m3_decode(np.array([0x7E, 0xFE], np.uint8))).all()


def test_subnormal_roundtrip():
    b = np.array(KATS["subnormal_roundtrip_bytes"]["bytes"], np.uint8)
    v = O.e4m3_decode(b)
    assert (v > 0).all() and (v < 2.0 ** -6).all()
    assert np.array_equal(O.e4m3_encode(v), b)


def test_noise_floor():
    k = KATS["noise_floor"]
    x = np.linspace(k["lo"], k["hi"], k["n"], dtype=np.float32)
    y = O.fp8_fake_quant(x, k["scale"])
    assert np.abs(y - x).max() <= k["max_abs_err"] + k["slack"]


def test_fake_quant_idempotent():
    k = KATS["idempotence"]
    i = np.arange(k["n"])
    x = (((i % 32) - 16) * 30.0 + np.where(i & 1, 0.01, -0.01)).astype(np.float32)
    y1 = O.fp8_fake_quant(x, k["scale"])
    y2 = O.fp8_fake_quant(y1, k["scale"])
    assert np.abs(y1 - y2).max() <= k["tol"]


def test_bulk_matches_scalar():
    i = np.arange(KATS["bulk_matches_scalar"]["n"], dtype=np.float64)
    x = (((i % 7) - 3) * 0.137 + np.where(i == 0, 0.0, 100.0 / np.maximum(i, 1))).astype(np.float32)
    lib = O.lib()
    scalar = np.array([lib.orc_e4m3_encode(float(v)) for v in x], np.uint8)
    assert np.array_equal(O.e4m3_encode(x), scalar)


def test_matches_reference_fixture():
    """Bytes and fake-quant values written by the reference's own code."""
    x = FIX["fp8_x"]
    assert np.array_equal(O.e4m3_encode(x), FIX["fp8_bytes"])
    assert np.array_equal(O.fp8_fake_quant(x, 2.5).view(np.uint32), FIX["fp8_fq_2p5"].view(np.uint32))


def _nearest_e4m3(x):
    """Brute force: the finite E4M3 value nearest to x, ties to the even
    mantissa (the textbook RNE the reference's normal range implements)."""
    vals = O.e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64)
    fin = np.isfinite(vals)
    codes = np.arange(256)[fin]
    v = vals[fin]
    d = np.abs(x[:, None].astype(np.float64) - v[None, :])
    best = d.min(axis=1, keepdims=True)
    cand = np.where(d == best, codes[None, :], 999)
    # ties: prefer the even mantissa, then the code with the sign of x
    even = np.where((cand & 1) == 0, cand, 999)
    pick = np.where((even != 999).any(axis=1), even.min(axis=1), cand.min(axis=1))
    return pick.astype(np.uint8)


def test_normal_range_is_round_to_nearest_even():
    """For 2^-6 <= |x| <= 448 the encoder picks the nearest E4M3 value, ties
    to even.  (This pins the mantissa rounding independently of the
    reference; a truncating or half-away encoder fails it.)"""
    rng = np.random.default_rng(5)
    mag = np.exp2(rng.uniform(-6, np.log2(448), 20000)).astype(np.float32)
    ties = np.array([1.0625, 1.1875, 3.25 * 2 ** -3, 1.9375, 432.0, 2 ** -6 * 1.0625], np.float32)
    x = np.concatenate([mag, -mag, ties, -ties]).astype(np.float32)
    x = x[(np.abs(x) >= 2 ** -6) & (np.abs(x) <= 448)]
    got = O.e4m3_encode(x)
    want = _nearest_e4m3(x)
    same_value = O.e4m3_decode(got) == O.e4m3_decode(want)
    assert same_value.all()


def test_reference_choices_below_normal_range_and_above_448():
    """What the reference does that differs from textbook RNE: below 2^-6 the
    subnormal branch is chosen before rounding and capped at 7 * 2^-9
    (fp8_e4m3.h:192-211), and (464, 496) -- mantissa 0b111 at exponent 15 --
    encodes as the NaN byte (fp8_e4m3.h:182-191)."""
    x = np.array([7.5 * 2 ** -9, 7.9 * 2 ** -9, 2 ** -6 * 0.999, 470.0, -470.0, 480.0, 495.0,
                  496.0, 464.0], np.float32)
    assert list(O.e4m3_encode(x)) == [0x07, 0x07, 0x07, 0x7F, 0xFF, 0x7F, 0x7F, 0x7E, 0x7E]
    # brute-force nearest would give the min normal for the first three
    assert list(_nearest_e4m3(x[:3])) == [0x08, 0x08, 0x08]


@pytest.mark.skipif(not O.ref_available("vnni") and not O.ref_available("avx2"),
                    reason="oracle/_ref not built on this host")
def test_matches_reference_build_strided_all_patterns():
    """Every 97th fp32 bit pattern (all exponents, signs and low-bit residues)."""
    n, stride = (1 << 32) // 97, 97
    chunk = 1 << 24
    for c0 in range(0, n, chunk):
        cnt = min(chunk, n - c0)
        start = (c0 * stride) & 0xFFFFFFFF
        bits = (np.arange(cnt, dtype=np.uint64) * stride + start).astype(np.uint32)
        got = O.e4m3_encode_bits_stride(start, stride, cnt)
        want = O.ref_e4m3_encode(bits.view(np.float32))
        assert np.array_equal(got, want), hex(start)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built on this host")
def test_fake_quant_matches_reference_build():
    rng = np.random.default_rng(3)
    x = ((rng.random(200000) - 0.5) * 2000).astype(np.float32)
    for s in (1.0, 0.37, 0.0, 3e-3):
        assert np.array_equal(O.fp8_fake_quant(x, s).view(np.uint32),
                              O.ref_fp8_fake_quant(x, s).view(np.uint32))
