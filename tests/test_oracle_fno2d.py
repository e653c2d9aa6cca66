"""The oracle's FNO2d forward (oracle/fno2d.py over oracle/nflow_oracle_fno.c)
pinned bit for bit against the reference runtime itself: InferenceRuntime
over FNO2d::Forward (cpp/src/runtime.cpp, fno.cpp, fft.cpp compiled from
their sources into oracle/_ref/ref_fno_run) on the same IR file and input.

The 2-D FFT is also pinned against numpy's to tolerance (an independent
algorithm: a transposed axis, a dropped column or a wrong conjugate fails
it), its inverse against the round trip, and the spectral convolution
against a float64 numpy restatement of fno.cpp:717-771."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import fno2d as OF2
from oracle import oracle as O
from tests import nir_format as F

REF_RUN = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "ref_fno_run"
needs_run = pytest.mark.skipif(not REF_RUN.exists(), reason="oracle/_ref/ref_fno_run not built")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("H,W", [(1, 1), (1, 8), (8, 1), (4, 8), (16, 16), (32, 8)])
def test_rfft2_matches_numpy(H, W):
    rng = np.random.default_rng(H * 100 + W)
    x = rng.standard_normal((H, W)).astype(np.float32)
    got = O.rfft2(x)
    want = np.fft.rfft2(x.astype(np.float64))
    np.testing.assert_allclose(got[..., 0] + 1j * got[..., 1], want, rtol=0, atol=2e-5 * max(1.0, np.sqrt(H * W)))


@pytest.mark.parametrize("H,W", [(2, 4), (8, 8), (16, 32)])
def test_irfft2_inverts_rfft2(H, W):
    rng = np.random.default_rng(H + W)
    x = rng.standard_normal((H, W)).astype(np.float32)
    np.testing.assert_allclose(O.irfft2(O.rfft2(x), H, W), x, rtol=0, atol=2e-5)


def test_spectral_conv2d_matches_float64():
    # Only the (mh, mw) corner of rfft2 is mixed; the rest of the output
    # spectrum is zero (fno.cpp:723-767), so the result is irfft2 of the
    # mixed corner.
    rng = np.random.default_rng(7)
    b, w, H, W, mh, mw = 2, 3, 8, 16, 3, 5
    h = rng.standard_normal((b, w, H, W)).astype(np.float32)
    wr = rng.standard_normal((w, w, mh, mw)).astype(np.float32)
    wi = rng.standard_normal((w, w, mh, mw)).astype(np.float32)
    got = O.spectral_conv2d(h, wr, wi, mh, mw)
    spec = np.fft.rfft2(h.astype(np.float64))                  # (b, w, H, W/2+1)
    out = np.zeros_like(spec)
    wc = wr.astype(np.float64) + 1j * wi.astype(np.float64)
    out[:, :, :mh, :mw] = np.einsum("bimn,iomn->bomn", spec[:, :, :mh, :mw], wc)
    want = np.fft.irfft2(out, s=(H, W))
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-4)


# ---- whole runs against the reference runtime --------------------------------------------------

def ref_run(tmp_path, ir: bytes, x: np.ndarray, out_ch: int):
    b, H, W, c = x.shape
    (tmp_path / "m.nneuroir").write_bytes(ir)
    np.ascontiguousarray(x, np.float32).tofile(tmp_path / "x.f32")
    cmd = [str(REF_RUN), str(tmp_path / "m.nneuroir"), str(tmp_path / "x.f32"), str(b), f"{H}x{W}", str(c),
           str(out_ch), str(tmp_path / "y.f32")]
    out = subprocess.run(cmd, capture_output=True, text=True, check=True)
    assert out.stdout.split() == ["status", "0"], out.stdout
    return np.fromfile(tmp_path / "y.f32", np.float32).reshape(b, H, W, out_ch)


def quant_records(rng, weights, n_layers, kinds):
    """Per-channel qparams for the 2-D weights (axis 0), per-tensor for the
    biases and the 4-D spectral weights, and activation qparams for
    lift.output, every locs.{i}.output, proj_q.output and proj_out.output of
    the kinds asked for ("tensor", "fp8", "fp8zero": an FP8 record whose
    scale is 0, which disables the snap and hides the INT8 record)."""
    recs = []
    for name, Wt in weights.items():
        if Wt.ndim == 2:
            s, z = F.symmetric_per_channel(Wt)
            recs.append((1, name, s, z, 0))
        else:
            recs.append((0, name, float(np.abs(Wt).max() / 127.0), 0))
    keys = ["lift.output"] + [f"locs.{i}.output" for i in range(n_layers)] + ["proj_q.output", "proj_out.output"]
    for j, key in enumerate(keys):
        kind = kinds[j % len(kinds)]
        recs.append((0, key, float(rng.uniform(0.01, 0.05)), int(rng.integers(-3, 4))))
        if kind == "fp8":
            recs.append((3, key, float(rng.uniform(0.005, 0.02))))
        elif kind == "fp8zero":
            recs.append((3, key, 0.0))
    return recs


def qrec_bytes(recs):
    return [F.qparam_record(kind, name, *p) for kind, name, *p in recs]


CASES = [
    # (b, H, W, in, out, width, mh, mw, layers, pad, relu, quant kinds or None)
    (2, 8, 8, 2, 1, 8, 3, 3, 2, 1, True, None),
    (2, 8, 16, 3, 2, 8, 4, 5, 2, 1, False, None),
    (1, 16, 8, 1, 1, 12, 5, 4, 3, 1, False, ["tensor"]),
    (2, 16, 16, 3, 1, 8, 6, 6, 4, 1, False, ["fp8", "tensor", "fp8zero"]),
    (1, 4, 4, 1, 1, 4, 2, 2, 2, 8, False, ["tensor", "fp8"]),
    (1, 1, 8, 1, 1, 4, 1, 3, 1, 1, True, None),
    (2, 32, 32, 1, 1, 16, 8, 8, 2, 1, False, ["fp8"]),
]


@needs_run
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"b{c[0]}H{c[1]}W{c[2]}w{c[5]}m{c[6]}x{c[7]}L{c[8]}p{c[9]}"
                         f"{'relu' if c[10] else 'gelu'}{'-'.join(c[11] or ['fp32'])}")
def test_forward_matches_reference_runtime(tmp_path, case):
    b, H, W, ci, co, w, mh, mw, L, pad, relu, kinds = case
    rng = np.random.default_rng([b, H, W, w, L, pad, int(relu), len(kinds or [])])
    weights = F.fno2d_weights(rng, ci, co, w, mh, mw, L)
    recs = None if kinds is None else quant_records(rng, weights, L, kinds)
    cfg = [ci, co, w, mh, mw, L, pad]
    ir = F.fno2d_file(weights, cfg, None if recs is None else qrec_bytes(recs), act=1 if relu else 0)
    x = rng.standard_normal((b, H, W, ci)).astype(np.float32)
    y_ref = ref_run(tmp_path, ir, x, co)
    m = OF2.from_records(cfg, relu, weights, recs)
    y = OF2.forward(m, x)
    assert np.array_equal(_bits(y), _bits(y_ref))
