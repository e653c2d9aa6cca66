"""The oracle's FNO1d forward (oracle/fno1d.py over oracle/nflow_oracle_fno.c)
pinned bit for bit against the reference runtime itself: InferenceRuntime
(cpp/src/runtime.cpp, fno.cpp, fft.cpp, int8_gemm.cpp compiled from its
sources into oracle/_ref/ref_fno_run) on the same IR file and input.

The FFT is also pinned against numpy's to tolerance (an independent
algorithm: a dropped twiddle, a wrong sign or bin order fails it), and its
inverse against the round trip."""
from __future__ import annotations

import subprocess
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import fno1d as OF
from oracle import oracle as O
from tests import nir_format as F

REF_RUN = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "ref_fno_run"
needs_run = pytest.mark.skipif(not REF_RUN.exists(), reason="oracle/_ref/ref_fno_run not built")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("n", [1, 2, 4, 8, 64, 1024])
def test_rfft_matches_numpy(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    got = O.rfft(x).reshape(-1, 2)
    want = np.fft.rfft(x.astype(np.float64))
    np.testing.assert_allclose(got[:, 0] + 1j * got[:, 1], want, rtol=0, atol=1e-5 * max(1.0, np.sqrt(n)))


@pytest.mark.parametrize("n", [2, 16, 256])
def test_irfft_inverts_rfft(n):
    rng = np.random.default_rng(n + 1)
    x = rng.standard_normal(n).astype(np.float32)
    np.testing.assert_allclose(O.irfft(O.rfft(x), n), x, rtol=0, atol=1e-5)


def _f32_exact(q: Fraction) -> np.float32:
    """q rounded to the nearest float32 (ties to even), from the exact rational."""
    if q == 0:
        return np.float32(0.0)
    sign, a = (-1, -q) if q < 0 else (1, q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    scaled = a * Fraction(2) ** (23 - e)
    n = scaled.numerator // scaled.denominator
    r = scaled - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(sign * float(Fraction(n) * Fraction(2) ** (e - 23)))


@pytest.mark.parametrize("k", [3, 7, 8, 15, 16, 24, 29, 64])
def test_linear_f32_summation_order(k):
    # The reference build's order (fno.cpp:75 vectorised by g++ -O3 -mfma):
    # from the bias, blocks of 16 then one of 8 add rounded products one by
    # one; the last k % 8 terms are fused, acc = fma(x, w, acc).  Plain
    # mul + add everywhere, or fma everywhere, fails this for some k.
    rng = np.random.default_rng(k)
    x = rng.standard_normal((6, k)).astype(np.float32)
    W = rng.standard_normal((4, k)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    y = O.linear_f32(x, W, b)
    tail = k % 8
    for i in range(6):
        for j in range(4):
            acc = np.float32(b[j])
            for p in range(k - tail):
                acc = np.float32(acc + np.float32(x[i, p] * W[j, p]))
            for p in range(k - tail, k):
                acc = _f32_exact(Fraction(float(x[i, p])) * Fraction(float(W[j, p])) + Fraction(float(acc)))
            assert _bits(y[i, j]) == _bits(acc)


def test_log2_snap_special_values():
    # |v| < 2^-6 passes; 2^e after the truncating exponent; 448 cap; NaN / Inf -> 0.
    s = np.float32(0.5)
    assert O.lib().orc_log2_snap_one(np.float32(0.001), s) == np.float32(0.001)
    assert O.lib().orc_log2_snap_one(np.float32(1.5), s) == np.float32(2.0) * s      # v = 3 -> e = 1
    assert O.lib().orc_log2_snap_one(np.float32(-0.75), s) == -np.float32(1.0) * s   # v = -1.5 -> e = 0
    assert O.lib().orc_log2_snap_one(np.float32(1e6), s) == np.float32(448.0) * s
    assert O.lib().orc_log2_snap_one(np.float32(np.inf), s) == 0.0
    assert O.lib().orc_log2_snap_one(np.float32(np.nan), s) == 0.0


# ---- whole runs against the reference runtime --------------------------------------------------

def _qrec_bytes(recs):
    out = []
    for kind, name, *p in recs:
        if kind == 1:
            out.append(F.qparam_record(1, name, p[0], p[1], p[2]))
        elif kind == 2:
            out.append(F.qparam_record(2, name, p[0], p[1], p[2]))
        else:
            out.append(F.qparam_record(kind, name, *p))
    return out


def ref_run(tmp_path, ir: bytes, x: np.ndarray, out_ch: int, int8: bool):
    b, n, c = x.shape
    (tmp_path / "m.nneuroir").write_bytes(ir)
    np.ascontiguousarray(x, np.float32).tofile(tmp_path / "x.f32")
    cmd = [str(REF_RUN), str(tmp_path / "m.nneuroir"), str(tmp_path / "x.f32"), str(b), str(n), str(c),
           str(out_ch), str(tmp_path / "y.f32")] + (["int8"] if int8 else [])
    out = subprocess.run(cmd, capture_output=True, text=True, check=True)
    assert out.stdout.split() == ["status", "0"], out.stdout
    return np.fromfile(tmp_path / "y.f32", np.float32).reshape(b, n, out_ch)


def quant_records(rng, weights, n_layers, width, n, kinds):
    """Per-channel weight qparams for every 2-D / spectral weight, per-tensor
    for biases, activation qparams for lift.output and every locs.{i}.output
    of the kinds asked for ("tensor", "token", "fp8")."""
    recs = []
    for name, Wt in weights.items():
        if Wt.ndim == 2:
            s, z = F.symmetric_per_channel(Wt)
            recs.append((1, name, s, z, 0))
        elif Wt.ndim == 3:
            s = (np.abs(Wt).max(axis=(0, 2)) / 127.0).astype(np.float32)
            recs.append((1, name, s, np.zeros_like(s, np.int32), 1))
        else:
            recs.append((0, name, float(np.abs(Wt).max() / 127.0), 0))
    recs.append((0, "lift.output", 0.03, 0))
    for i in range(n_layers):
        kind = kinds[i % len(kinds)]
        key = f"locs.{i}.output"
        recs.append((0, key, float(rng.uniform(0.01, 0.05)), int(rng.integers(-3, 4))))
        if kind == "token":
            cnt = n * width
            recs.append((2, key, rng.uniform(0.01, 0.05, cnt).astype(np.float32),
                         rng.integers(-4, 5, cnt).astype(np.int32), width))
        elif kind == "fp8":
            recs.append((3, key, float(rng.uniform(0.005, 0.02))))
    return recs


CASES = [
    # (b, n, in, out, width, modes, layers, pad, relu, quant kinds or None, int8)
    (2, 16, 2, 1, 8, 4, 2, 1, True, None, False),
    (2, 16, 2, 1, 8, 4, 2, 1, False, None, False),
    (3, 32, 1, 2, 16, 6, 3, 1, False, ["tensor"], False),
    (3, 32, 1, 2, 16, 6, 3, 1, False, ["tensor"], True),
    (2, 64, 3, 1, 12, 8, 4, 1, True, ["tensor", "token", "fp8"], True),
    (2, 64, 3, 1, 12, 8, 4, 1, False, ["token", "tensor", "fp8"], True),
    (1, 4, 1, 1, 4, 2, 2, 8, False, ["tensor"], True),
    (4, 256, 1, 1, 32, 12, 4, 1, False, ["tensor"], True),
]


@needs_run
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"b{c[0]}n{c[1]}w{c[4]}L{c[6]}p{c[7]}"
                         f"{'relu' if c[8] else 'gelu'}{'-'.join(c[9] or ['fp32'])}{'-int8' if c[10] else ''}")
def test_forward_matches_reference_runtime(tmp_path, case):
    b, n, ci, co, w, modes, L, pad, relu, kinds, int8 = case
    rng = np.random.default_rng([b, n, w, L, pad, int(relu), int(int8), len(kinds or [])])
    weights = F.fno1d_weights(rng, ci, co, w, modes, L)
    n_pad = n + ((pad - n % pad) % pad if pad > 1 else 0)
    recs = None if kinds is None else quant_records(rng, weights, L, w, n_pad, kinds)
    cfg = [ci, co, w, modes, L, pad, 0]
    ir = F.fno1d_file(weights, cfg, None if recs is None else _qrec_bytes(recs), act=1 if relu else 0)
    x = rng.standard_normal((b, n, ci)).astype(np.float32)
    y_ref = ref_run(tmp_path, ir, x, co, int8)
    m = OF.from_records(cfg, relu, weights, recs)
    if int8:
        OF.enable_int8_gemm(m)
    y = OF.forward(m, x)
    assert np.array_equal(_bits(y), _bits(y_ref))
