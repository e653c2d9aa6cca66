"""Write tests/golden/ref_fno_models.npz from the reference's own runtime.

Runs NeuroFlow's InferenceRuntime (cpp/src/runtime.cpp over fno.cpp and
fft.cpp, compiled from the reference sources into oracle/_ref/ref_fno_run
by `make -C oracle ref`) on small seeded FNO1d and FNO2d models, and stores
each model's IR file, input and output.  The fixture is data only; the tests
compare the oracle and the device runtime against it, also where oracle/_ref
is not built.

    python tests/golden/make_fno_fixtures.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from tests import nir_format as F  # noqa: E402
from tests import test_oracle_fno1d as T1  # noqa: E402
from tests import test_oracle_fno2d as T2  # noqa: E402

OUT = Path(__file__).resolve().parent / "ref_fno_models.npz"

# FNO1d: (b, n, in, out, width, modes, layers, pad, relu, quant kinds or None, int8)
CASES_1D = [
    (2, 16, 2, 1, 8, 4, 2, 1, False, None, False),
    (2, 32, 1, 2, 8, 6, 3, 1, False, ["tensor", "token", "fp8"], True),
    (1, 4, 1, 1, 4, 2, 2, 8, True, ["tensor"], True),
]
# FNO2d: (b, H, W, in, out, width, mh, mw, layers, pad, relu, quant kinds or None)
CASES_2D = [
    (1, 8, 8, 2, 1, 8, 3, 3, 2, 1, False, None),
    (2, 8, 16, 1, 2, 8, 4, 5, 2, 1, False, ["fp8", "tensor", "fp8zero"]),
    (1, 4, 4, 1, 1, 4, 2, 2, 2, 8, True, ["tensor", "fp8"]),
]


def model_1d(i: int):
    """Case i of CASES_1D: (ir bytes, x, cfg, weights, qrecords, relu, int8)."""
    b, n, ci, co, w, modes, L, pad, relu, kinds, int8 = CASES_1D[i]
    rng = np.random.default_rng([5100 + i])
    weights = F.fno1d_weights(rng, ci, co, w, modes, L)
    n_pad = n + ((pad - n % pad) % pad if pad > 1 else 0)
    recs = None if kinds is None else T1.quant_records(rng, weights, L, w, n_pad, kinds)
    cfg = [ci, co, w, modes, L, pad, 0]
    ir = F.fno1d_file(weights, cfg, None if recs is None else T1._qrec_bytes(recs), act=1 if relu else 0)
    x = rng.standard_normal((b, n, ci)).astype(np.float32)
    return ir, x, cfg, weights, recs, relu, int8


def model_2d(i: int):
    """Case i of CASES_2D: (ir bytes, x, cfg, weights, qrecords, relu)."""
    b, H, W, ci, co, w, mh, mw, L, pad, relu, kinds = CASES_2D[i]
    rng = np.random.default_rng([5200 + i])
    weights = F.fno2d_weights(rng, ci, co, w, mh, mw, L)
    recs = None if kinds is None else T2.quant_records(rng, weights, L, kinds)
    cfg = [ci, co, w, mh, mw, L, pad]
    ir = F.fno2d_file(weights, cfg, None if recs is None else T2.qrec_bytes(recs), act=1 if relu else 0)
    x = rng.standard_normal((b, H, W, ci)).astype(np.float32)
    return ir, x, cfg, weights, recs, relu


def main(tmp: Path) -> None:
    d = {}
    for i in range(len(CASES_1D)):
        ir, x, cfg, _, _, _, int8 = model_1d(i)
        d[f"fno1d_{i}_ir"] = np.frombuffer(ir, np.uint8)
        d[f"fno1d_{i}_x"] = x
        d[f"fno1d_{i}_y"] = T1.ref_run(tmp, ir, x, cfg[1], int8)
    for i in range(len(CASES_2D)):
        ir, x, cfg, _, _, _ = model_2d(i)
        d[f"fno2d_{i}_ir"] = np.frombuffer(ir, np.uint8)
        d[f"fno2d_{i}_x"] = x
        d[f"fno2d_{i}_y"] = T2.ref_run(tmp, ir, x, cfg[1])
    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(CASES_1D)} FNO1d and {len(CASES_2D)} FNO2d models)")


if __name__ == "__main__":
    import tempfile
    with tempfile.TemporaryDirectory() as t:
        main(Path(t))
