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


# ---- the FP8 layer: per-token / per-channel quantise, exact GEMM, composition ----

def _fp8_rows(seed, M, K):
    rng = np.random.default_rng(seed)
    x = (2.0 * rng.standard_normal((M, K))).astype(np.float32)
    x = np.where(rng.random((M, K)) < 0.01, 20.0 * x, x).astype(np.float32)
    x[0] = 0.0
    x[1] = 1e-41
    x[2, :3] = [448.0, -3e5, 7.6 * 2.0 ** -9]
    return x


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built on this host")
def test_per_token_fp8_is_reference_fake_quant_per_row():
    """Scale absmax/448 (1 for an all-zero row); decode(code) * scale equals the
    reference's own fp8_e4m3_per_tensor_fake_quant of the row with that scale
    (fp8_e4m3.h:312-334), element for element."""
    x = _fp8_rows(11, 300, 64)
    q, s = O.quantise_per_token_fp8(x)
    am = np.abs(x).max(axis=1)
    assert np.array_equal(_bits(s), _bits(np.where(am == 0, np.float32(1), am / np.float32(448))))
    for m in range(x.shape[0]):
        want = O.ref_fp8_fake_quant(x[m], float(s[m]))
        assert np.array_equal(_bits(O.e4m3_decode(q[m]) * s[m]), _bits(want)), m


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built on this host")
def test_fp8_weight_blob_is_reference_fake_quant_per_channel():
    W = ((np.random.default_rng(12).random((96, 64)) - 0.5) * 0.25).astype(np.float32)
    q, s = O.quantise_weight_fp8(W)
    for n in range(W.shape[0]):
        assert np.array_equal(_bits(O.e4m3_decode(q[n]) * s[n]),
                              _bits(O.ref_fp8_fake_quant(W[n], float(s[n]))))


def test_fp8_exact_gemm_is_the_float64_dot_product():
    """E4M3 x E4M3 products are exact in float64 and a 64-term sum of them
    spans fewer than 53 bits, so numpy's float64 product is the exact sum in
    any summation order."""
    rng = np.random.default_rng(13)
    codes = np.array([b for b in range(256) if b not in (0x7F, 0xFF)], np.uint8)
    qa = rng.choice(codes, (70, 64))
    qw = rng.choice(codes, (40, 64))
    want = O.e4m3_decode(qa).astype(np.float64) @ O.e4m3_decode(qw).astype(np.float64).T
    assert np.array_equal(O.gemm_fp8_exact(qa, qw), want)
    qa[5, 7] = 0x7F                                    # a NaN code poisons its row
    got = O.gemm_fp8_exact(qa, qw)
    assert np.isnan(got[5]).all() and not np.isnan(np.delete(got, 5, axis=0)).any()


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built on this host")
def test_fp8_composed_layer_follows_reference_primitives():
    """The composition: the reference build's fake-quant per row and per
    channel, then the fp32 Linear loop of fno.cpp:68-79 (acc = bias, then
    acc += a_k * w_k in k order), no activation: bit for bit."""
    x = _fp8_rows(14, 48, 64)
    W = ((np.random.default_rng(15).random((24, 64)) - 0.5) * 0.25).astype(np.float32)
    b = ((np.random.default_rng(16).random(24) - 0.5) * 0.25).astype(np.float32)
    got, sa, sw = O.layer_fp8_composed(x, W, b, O.ACT_NONE)
    af = np.stack([O.ref_fp8_fake_quant(x[m], float(sa[m])) for m in range(x.shape[0])])
    wf = np.stack([O.ref_fp8_fake_quant(W[n], float(sw[n])) for n in range(W.shape[0])])
    acc = np.broadcast_to(b, got.shape).astype(np.float32)
    for k in range(x.shape[1]):
        acc = (acc + (af[:, k:k + 1] * wf[None, :, k])).astype(np.float32)
    assert np.array_equal(_bits(got), _bits(acc))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built on this host")
def test_fp8_exact_layer_is_composition_without_accumulation_rounding():
    """The exact-product layer differs from the reference composition only by
    the composition's own fp32 accumulation: |diff| <= K 2^-24 sum|terms| + a
    few ulp of the result."""
    x = _fp8_rows(17, 64, 64)
    W = ((np.random.default_rng(18).random((32, 64)) - 0.5) * 0.25).astype(np.float32)
    b = ((np.random.default_rng(19).random(32) - 0.5) * 0.25).astype(np.float32)
    composed, sa, sw = O.layer_fp8_composed(x, W, b, O.ACT_NONE)
    qa, sa2 = O.quantise_per_token_fp8(x)
    qw, sw2 = O.quantise_weight_fp8(W)
    assert np.array_equal(_bits(sa), _bits(sa2)) and np.array_equal(_bits(sw), _bits(sw2))
    exact = O.layer_fp8_exact(qa, sa2, qw, sw2, b, O.ACT_NONE).astype(np.float64)
    terms = (np.abs(O.e4m3_decode(qa)) * sa2[:, None]).astype(np.float64) @ \
        (np.abs(O.e4m3_decode(qw)) * sw2[:, None]).astype(np.float64).T
    bound = 64 * 2.0 ** -24 * (terms + np.abs(b)) + 4 * 2.0 ** -24 * np.abs(exact) + 1e-30
    assert np.all(np.abs(exact - composed) <= bound)
