"""Whole FNO1d / FNO2d models against outputs the reference's own runtime
wrote (tests/golden/ref_fno_models.npz, from oracle/_ref/ref_fno_run by
tests/golden/make_fno_fixtures.py): the oracle on the CPU, the device
runtime on the GPU, every output bit equal.  These run also where
oracle/_ref is not built."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import fno1d as OF
from oracle import fno2d as OF2
from tests.golden import make_fno_fixtures as MF

FIX = np.load(Path(__file__).resolve().parent / "golden" / "ref_fno_models.npz")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("i", range(len(MF.CASES_1D)))
def test_oracle_fno1d_matches_fixture(i):
    ir, x, cfg, weights, recs, relu, int8 = MF.model_1d(i)
    assert ir == FIX[f"fno1d_{i}_ir"].tobytes() and np.array_equal(x, FIX[f"fno1d_{i}_x"])
    m = OF.from_records(cfg, relu, weights, recs)
    if int8:
        OF.enable_int8_gemm(m)
    assert np.array_equal(_bits(OF.forward(m, x)), _bits(FIX[f"fno1d_{i}_y"]))


@pytest.mark.parametrize("i", range(len(MF.CASES_2D)))
def test_oracle_fno2d_matches_fixture(i):
    ir, x, cfg, weights, recs, relu = MF.model_2d(i)
    assert ir == FIX[f"fno2d_{i}_ir"].tobytes() and np.array_equal(x, FIX[f"fno2d_{i}_x"])
    m = OF2.from_records(cfg, relu, weights, recs)
    assert np.array_equal(_bits(OF2.forward(m, x)), _bits(FIX[f"fno2d_{i}_y"]))


@pytest.mark.gpu
@pytest.mark.parametrize("name", [f"fno1d_{i}" for i in range(len(MF.CASES_1D))] +
                         [f"fno2d_{i}" for i in range(len(MF.CASES_2D))])
def test_runtime_matches_fixture(gpu, tmp_path, name):
    from neuroflow_amd.runtime import load
    ncpp = load()
    path = tmp_path / "m.nneuroir"
    path.write_bytes(FIX[f"{name}_ir"].tobytes())
    x, want = FIX[f"{name}_x"], FIX[f"{name}_y"]
    rt = ncpp.InferenceRuntime(str(path))
    if name.startswith("fno1d") and MF.CASES_1D[int(name[-1])][10]:
        rt.enable_int8_gemm()
    y = np.zeros_like(want)
    rt.run(x, y)
    assert np.array_equal(_bits(y), _bits(want))
