"""The oracle's FNO x2 fake-quant (orc_x2_fake_quant, fno.cpp:572-648)
pinned two ways:
- per element against the reference's own QuantiseActivation (oracle/_ref,
  int8_gemm.cpp:507-520), which rounds and clamps the same quotient:
  fq(v) = (q - zp) * s;
- end to end against the reference runtime itself (oracle/_ref/ref_fno_run):
  an FNO1d IR with identity lift / local / projection weights, zero spectral
  weights and ReLU makes InferenceRuntime::Run return relu(fq(x)) exactly,
  which exposes the per-position indexing of fno.cpp:615-633."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from tests import nir_format as F

REF_RUN = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "ref_fno_run"
needs_run = pytest.mark.skipif(not REF_RUN.exists(), reason="oracle/_ref/ref_fno_run not built")


@pytest.mark.skipif(not O.ref_available(), reason="reference build not available")
@pytest.mark.parametrize("scale,zp", [(0.05, 0), (0.013, 7), (0.2, -3), (1.0, 0), (3e-3, 100)])
def test_per_tensor_matches_reference_quantise_activation(scale, zp):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((300, 64)) * 2.0).astype(np.float32)
    x[0, :16] = (np.arange(16, dtype=np.float32) - 8.0 + 0.5) * np.float32(scale)   # exact ties
    x[1, :4] = [1e6, -1e6, 0.0, -0.0]
    q = O.ref_quantise_activation(x, scale, zp).astype(np.int32)
    want = ((q - zp).astype(np.float32) * np.float32(scale)).astype(np.float32)
    got = O.x2_fake_quant(x, scale, zp)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_nan_passes_and_infinities_clamp():
    x = np.array([[np.nan, np.inf, -np.inf, 0.5]], np.float32)
    got = O.x2_fake_quant(x, 0.25, 2)
    assert np.isnan(got[0, 0])
    assert got[0, 1] == np.float32((127 - 2) * 0.25) and got[0, 2] == np.float32((-128 - 2) * 0.25)


def _identity_fno1d(w, n_points, qrecords):
    """FNO1d with in = out = width w, one layer: every weight the identity or zero."""
    eye = np.eye(w, dtype=np.float32)
    zero = np.zeros(w, np.float32)
    weights = {"lift.weight": eye, "lift.bias": zero,
               "specs.0.weights_real": np.zeros((w, w, 2), np.float32),
               "specs.0.weights_imag": np.zeros((w, w, 2), np.float32),
               "locs.0.weight": eye, "locs.0.bias": zero,
               "proj_q.weight": eye, "proj_q.bias": zero,
               "proj_out.weight": eye, "proj_out.bias": zero}
    return F.fno1d_file(weights, [w, w, w, 2, 1, 1, 0], qrecords, act=1)


def _ref_run(tmp_path, ir: bytes, x: np.ndarray) -> np.ndarray:
    b, n, c = x.shape
    (tmp_path / "m.nneuroir").write_bytes(ir)
    x.astype(np.float32).tofile(tmp_path / "x.f32")
    out = subprocess.run([str(REF_RUN), str(tmp_path / "m.nneuroir"), str(tmp_path / "x.f32"), str(b), str(n),
                          str(c), str(c), str(tmp_path / "y.f32")], capture_output=True, text=True, check=True)
    assert out.stdout.split() == ["status", "0"], out.stdout
    return np.fromfile(tmp_path / "y.f32", np.float32).reshape(b, n, c)


@needs_run
@pytest.mark.parametrize("b,n,w", [(2, 8, 4), (3, 16, 8), (1, 32, 16)])
def test_per_position_matches_reference_runtime(tmp_path, b, n, w):
    rng = np.random.default_rng(b * 100 + n)
    scales = rng.uniform(0.01, 0.2, n * w).astype(np.float32)
    zps = rng.integers(-20, 20, n * w).astype(np.int32)
    ir = _identity_fno1d(w, n, [F.qparam_record(2, "locs.0.output", scales, zps, w)])
    x = (rng.standard_normal((b, n, w)) * 3.0).astype(np.float32)
    y_ref = _ref_run(tmp_path, ir, x)
    fq = O.x2_fake_quant(x.reshape(b * n, w), scales=scales, zps=zps, points=n)
    want = O.apply_activation(fq, O.ACT_RELU).reshape(b, n, w)
    assert np.array_equal(y_ref.view(np.uint32), want.view(np.uint32))
    # The indexing is not the "natural" one (position-major): it differs.
    nat = np.empty_like(x)
    flat = x.reshape(b, n * w)
    for i in range(n * w):
        nat.reshape(b, n * w)[:, i] = [O.x2_fake_quant(np.array([[v]], np.float32), scales[i], zps[i])[0, 0]
                                       for v in flat[:, i]]
    assert not np.array_equal(O.apply_activation(nat.reshape(b * n, w), O.ACT_RELU).reshape(b, n, w), y_ref)


@needs_run
def test_per_tensor_matches_reference_runtime(tmp_path):
    b, n, w = 2, 16, 8
    rng = np.random.default_rng(9)
    ir = _identity_fno1d(w, n, [F.qparam_record(0, "locs.0.output", 0.07, -5)])
    x = (rng.standard_normal((b, n, w)) * 3.0).astype(np.float32)
    y_ref = _ref_run(tmp_path, ir, x)
    want = O.apply_activation(O.x2_fake_quant(x.reshape(b * n, w), 0.07, -5), O.ACT_RELU).reshape(b, n, w)
    assert np.array_equal(y_ref.view(np.uint32), want.view(np.uint32))
