"""Pins of the oracle's INT8 path (oracle/nflow_oracle.c, restating
cpp/src/int8_gemm.cpp and cpp/src/fno.cpp): vectors written by the reference's
own compiled code (tests/golden/ref_int8_vectors.npz), the reference build
where it runs, and closed forms (ties, saturation, brute-force sums, float
operation order, the GELU formula evaluated in float64)."""
from pathlib import Path

import numpy as np
import pytest

from neuroflow_amd import workloads as WL
from oracle import oracle as O

FIX = np.load(Path(__file__).parent / "golden" / "ref_int8_vectors.npz")


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


# ---- against the reference's own outputs ------------------------------------------

def test_quantise_activation_fixture():
    A = FIX["qa_A"]
    for i, (s, zp) in enumerate(FIX["qa_cases"]):
        assert np.array_equal(O.quantise_activation(A, np.float32(s), int(zp)), FIX[f"qa_out_{i}"])


@pytest.mark.parametrize("K", [64, 100, 4100])
def test_linear_forward_fixtures(K):
    q, s, zps, b, X = (FIX[f"lf{K}_{n}"] for n in ("Wq", "sW", "zpW", "b", "X"))
    assert np.array_equal(O.precompute_sum_w(q, zps), FIX[f"lf{K}_sumW_ref"])
    for zpa in (0, 5):
        for use_sum in (0, 1):
            sumW = FIX[f"lf{K}_sumW_ref"] if use_sum else None
            rc, rows = O.linear_forward_rows(X, q, s, zps, b, 0.02, zpa, sumW)
            assert rc == 0 and _same(rows, FIX[f"lf{K}_rows_zp{zpa}_sum{use_sum}"])
            rc, bat = O.linear_forward_batched(X, q, s, zps, b, 0.02, zpa, sumW)
            assert rc == 0 and _same(bat, FIX[f"lf{K}_batched_zp{zpa}_sum{use_sum}"])


def test_per_token_fixture():
    out, sa = O.layer_per_token_i8(FIX["pt_X"], FIX["pt_Wq"], FIX["pt_sW"], None, FIX["pt_b"],
                                   FIX["pt_sumW"], O.ACT_NONE)
    assert _same(sa, FIX["pt_sA"])
    assert _same(out, FIX["pt_out"])


@pytest.mark.skipif(not O.ref_available("vnni"), reason="reference VNNI build not runnable here")
def test_random_cases_match_reference_build():
    rng = np.random.default_rng(9)
    for K in (4, 64, 96, 256, 1000):
        N = 40
        W = rng.standard_normal((N, K)).astype(np.float32)
        s = O.per_channel_scales(W, 127.0)
        zps = rng.integers(-4, 5, N).astype(np.int32)
        q, sw = O.quantise_weight_2d(W, s, zps)
        b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
        X = (rng.standard_normal((5, K)) * 2).astype(np.float32)
        for zpa in (0, -3):
            for sumW in (None, sw):
                a = O.linear_forward_rows(X, q, s, zps, b, 0.013, zpa, sumW)[1]
                r = O.ref_linear_forward_rows(X, q, s, zps, b, 0.013, zpa, sumW, variant="vnni")[1]
                assert _same(a, r)
                a = O.linear_forward_batched(X, q, s, zps, b, 0.013, zpa, sumW)[1]
                r = O.ref_linear_forward_batched(X, q, s, zps, b, 0.013, zpa, sumW, variant="vnni")[1]
                assert _same(a, r)


def test_status_codes_of_reference_interface():
    """int8_gemm.cpp:203-208 (null / bad dims -> InvalidArg = 1) and
    :533-535 (bsz <= 0 -> Ok; null A or C -> InvalidArg)."""
    import ctypes as C
    q = np.zeros((4, 8), np.int8)
    p, keep = O.make_params(q, np.ones(4, np.float32), np.zeros(4, np.int32))
    x = np.zeros(8, np.float32)
    y = np.zeros(4, np.float32)
    L = O.lib()
    assert L.orc_linear_forward(C.byref(p), None, y.ctypes.data_as(C.c_void_p)) == 1
    p2 = O.LinearParams.from_buffer_copy(p)
    p2.in_features = 0
    assert L.orc_linear_forward(C.byref(p2), x.ctypes.data_as(C.c_void_p),
                                y.ctypes.data_as(C.c_void_p)) == 1
    assert L.orc_linear_forward_batched(C.byref(p), 0, None, None) == 0
    assert L.orc_linear_forward_batched(C.byref(p), 1, None, None) == 1
    del keep


# ---- closed forms ------------------------------------------------------------------

def test_quantise_ties_round_half_away_from_zero():
    # scale 1 makes x / s exact; k + 0.5 ties go away from zero (std::round).
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.5, 0.49999997], np.float32)
    assert list(O.quantise_activation(x[None, :], 1.0, 0)[0]) == [1, 2, 3, -1, -2, -3, 127, -128, 0]


def test_quantise_saturation_and_x86_conversion():
    # |q| >= 2^31 and NaN convert to INT32_MIN (cvttss2si), then + zp and clamp.
    x = np.array([1e30, -1e30, np.nan, np.inf, 200.0, -200.0], np.float32)
    assert list(O.quantise_activation(x[None, :], 1.0, 0)[0]) == [-128, -128, -128, -128, 127, -128]
    # INT32_MIN + (-1) wraps to INT32_MAX -> clamps to 127
    assert list(O.quantise_activation(x[None, :3], 1.0, -1)[0]) == [127, 127, 127]


def test_quantise_division_is_correctly_rounded():
    """The code uses the correctly rounded quotient: pick x, s where
    x * (1/s) and x / s round to different sides of a tie."""
    rng = np.random.default_rng(1)
    s = np.float32(0.0123)
    x = (rng.standard_normal(200000) * 1.5).astype(np.float32)
    q = O.quantise_activation(x[None, :], s, 0)[0].astype(np.int32)
    exact = np.round((x.astype(np.float64) / np.float64(s)).astype(np.float32).astype(np.float64) + 0)
    # numpy rounds half to even; use explicit half-away on the float32 quotient
    quot = (x / s).astype(np.float32)
    half_away = np.where(quot >= 0, np.floor(quot + np.float32(0.5)), np.ceil(quot - np.float32(0.5)))
    want = np.clip(np.where(np.abs(quot - np.trunc(quot)) == 0.5, half_away, exact), -128, 127)
    assert np.array_equal(q, want.astype(np.int32))


def test_per_token_scales_and_codes():
    A = WL.normal(1, (300, 64)) * 3
    A[0] = 0.0
    q, s, sa = O.quantise_per_token_i8(A)
    absmax = np.abs(A).max(axis=1)
    want = np.where(absmax == 0, np.float32(1.0), (absmax / np.float32(127.0)).astype(np.float32))
    assert _same(s, want)
    # the absmax element maps to +-127
    idx = np.abs(A[1:]).argmax(axis=1)
    assert np.all(np.abs(q[1:][np.arange(299), idx]) == 127)
    assert np.array_equal(sa, q.astype(np.int32).sum(axis=1))
    assert np.all(np.abs(q.astype(np.int32)) <= 127)


def test_gemm_i32_is_the_integer_dot_product():
    rng = np.random.default_rng(2)
    A = rng.integers(-128, 128, (50, 300)).astype(np.int8)
    W = rng.integers(-128, 128, (30, 300)).astype(np.int8)
    assert np.array_equal(O.gemm_i8_i32(A, W), A.astype(np.int64) @ W.astype(np.int64).T)


def test_symmetric_layer_is_scaled_dot_plus_bias():
    """zp = 0: y = (s_w * s_a) * float(acc) + b, in float32, in that order."""
    A = WL.normal(3, (200, 64))
    W = WL.uniform(4, (48, 64), -0.125, 0.125)
    s = O.per_channel_scales(W, 127.0)
    q, sw = O.quantise_weight_2d(W, s)
    b = WL.uniform(5, (48,), -0.1, 0.1)
    out, sa = O.layer_per_token_i8(A, q, s, None, b, sw, O.ACT_NONE)
    qa, sa2, _ = O.quantise_per_token_i8(A)
    acc = (qa.astype(np.int64) @ q.astype(np.int64).T).astype(np.float32)
    want = (s[None, :] * sa2[:, None]).astype(np.float32) * acc
    want = (want.astype(np.float32) + b[None, :]).astype(np.float32)
    assert _same(sa, sa2) and _same(out, want)


def test_weight_quantisation_closed_form():
    W = WL.uniform(6, (64, 64), -0.125, 0.125)
    s = O.per_channel_scales(W, 127.0)
    q, sw = O.quantise_weight_2d(W, s)
    quot = (W / s[:, None]).astype(np.float32)
    half_away = np.where(quot >= 0, np.floor(quot + np.float32(0.5)), np.ceil(quot - np.float32(0.5)))
    assert np.array_equal(q.astype(np.int32), np.clip(half_away, -128, 127).astype(np.int32))
    assert np.array_equal(sw, q.astype(np.int32).sum(axis=1))
    assert np.all(np.abs(q).max(axis=1) == 127)
    # idempotent: re-quantising the dequantised weights gives the same codes
    q2, _ = O.quantise_weight_2d((q.astype(np.float32) * s[:, None]).astype(np.float32), s)
    assert np.array_equal(q, q2)


def test_gelu_matches_float64_evaluation_of_the_tanh_form():
    z = np.concatenate([np.linspace(-10, 10, 20001), [0.0, -0.0, 1e-30, 50.0, -50.0]]).astype(np.float32)
    got = O.apply_activation(z, O.ACT_GELU_TANH).astype(np.float64)
    z64 = z.astype(np.float64)
    want = 0.5 * z64 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (z64 + 0.044715 * z64 ** 3)))
    # float32 evaluation of the same formula: a few ulp where it is well
    # conditioned; where 1 + tanh cancels (z ~ -3 .. -6) the relative error
    # reaches ~5e-5 but the absolute error stays below 5e-7
    err = np.abs(got - want)
    assert np.all(err <= 4e-7 * np.abs(want) + 5e-7)
    good = z64 > -1.0
    assert np.all(err[good] <= 4e-7 * np.abs(want[good]) + 1e-12)
    assert np.all(got[z == 0] == 0.0)
    assert np.all(got[z >= 6] == z[z >= 6])


def test_relu():
    z = np.array([-1.0, -0.0, 0.0, 2.0, np.nan], np.float32)
    got = O.apply_activation(z, O.ACT_RELU)
    assert list(got[:4]) == [0.0, 0.0, 0.0, 2.0] and np.isnan(got[4])
