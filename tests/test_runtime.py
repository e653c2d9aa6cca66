"""The neuroflow_cpp module and the runtime C-ABI without a GPU: the module
builds and exposes the reference module's surface (pybind_module.cpp:58-238,
fp8_e4m3_pybind.h:24-66), and creation fails with the reference loader's
status codes and RuntimeError messages before any device call."""
import ctypes as C

import numpy as np
import pytest

from neuroflow_amd import _lib
from neuroflow_amd.runtime import load
from tests import nir_format as F


@pytest.fixture(scope="module")
def ncpp():
    return load()


def test_module_surface(ncpp):
    for name in ["infer", "infer_arrays", "infer_deeponet_arrays", "InferenceRuntime", "fp8_e4m3_fake_quant",
                 "fp8_e4m3_to_bits", "fp8_e4m3_from_bits"]:
        assert hasattr(ncpp, name), name
    for meth in ["op", "enable_int8_gemm", "is_int8_gemm_enabled", "run", "run_device"]:
        assert hasattr(ncpp.InferenceRuntime, meth), meth


def test_create_missing_file(ncpp, tmp_path):
    with pytest.raises(RuntimeError, match="create runtime failed"):
        ncpp.InferenceRuntime(str(tmp_path / "nope.nneuroir"))
    h = C.c_void_p(5)
    assert _lib.lib().nflow_runtime_create(str(tmp_path / "nope").encode(), C.byref(h)) == _lib.FILE_NOT_FOUND
    assert h.value is None


def test_create_bad_magic(tmp_path):
    p = tmp_path / "bad.nneuroir"
    p.write_bytes(b"XXXX" + bytes(40))
    h = C.c_void_p()
    assert _lib.lib().nflow_runtime_create(str(p).encode(), C.byref(h)) == _lib.PARSE_ERROR


@pytest.mark.parametrize("op", [3, 4, 5, 6, 7, 8])
def test_other_ops_are_unsupported(ncpp, tmp_path, op):
    p = tmp_path / "m.nneuroir"
    p.write_bytes(F.header(op, [1, 1, 4, 2, 2, 1, 1]))
    h = C.c_void_p()
    assert _lib.lib().nflow_runtime_create(str(p).encode(), C.byref(h)) == _lib.UNSUPPORTED_OP
    with pytest.raises(RuntimeError, match="create runtime failed"):
        ncpp.InferenceRuntime(str(p))


def test_missing_weight_is_a_parse_error(tmp_path):
    rng = np.random.default_rng(1)
    w = F.fno1d_weights(rng, 2, 1, 8, 4, 2)
    del w["locs.1.bias"]
    p = tmp_path / "m.nneuroir"
    p.write_bytes(F.fno1d_file(w, [2, 1, 8, 4, 2, 1, 0]))
    h = C.c_void_p()
    assert _lib.lib().nflow_runtime_create(str(p).encode(), C.byref(h)) == _lib.PARSE_ERROR
    assert b"locs.1.bias" in _lib.lib().nflow_last_error()


def test_wrong_weight_shape_is_a_parse_error(tmp_path):
    rng = np.random.default_rng(2)
    w = F.fno1d_weights(rng, 2, 1, 8, 4, 1)
    w["specs.0.weights_real"] = w["specs.0.weights_real"][:, :, :3]
    p = tmp_path / "m.nneuroir"
    p.write_bytes(F.fno1d_file(w, [2, 1, 8, 4, 1, 1, 0]))
    h = C.c_void_p()
    assert _lib.lib().nflow_runtime_create(str(p).encode(), C.byref(h)) == _lib.PARSE_ERROR


def test_fno2d_weights_are_checked(tmp_path):
    # FNO2d is served: its weights are read in LoadBinary's order with the
    # (in, out, modes_h, modes_w) spectral shape (ir_loader.h:298-322).
    rng = np.random.default_rng(5)
    cfg = [2, 1, 8, 3, 4, 2, 1]
    p = tmp_path / "m.nneuroir"
    p.write_bytes(F.header(2, cfg))
    h = C.c_void_p()
    assert _lib.lib().nflow_runtime_create(str(p).encode(), C.byref(h)) == _lib.PARSE_ERROR
    assert b"lift.weight" in _lib.lib().nflow_last_error()
    w = F.fno2d_weights(rng, 2, 1, 8, 3, 4, 2)
    w["specs.1.weights_imag"] = w["specs.1.weights_imag"][:, :, :, :3]
    p.write_bytes(F.fno2d_file(w, cfg))
    assert _lib.lib().nflow_runtime_create(str(p).encode(), C.byref(h)) == _lib.PARSE_ERROR
    assert b"specs.1.weights_imag" in _lib.lib().nflow_last_error()


def test_deeponet_arrays_messages(ncpp, tmp_path):
    rng = np.random.default_rng(3)
    p = tmp_path / "m.nneuroir"
    p.write_bytes(F.fno1d_file(F.fno1d_weights(rng, 2, 1, 8, 4, 1), [2, 1, 8, 4, 1, 1, 0]))
    u = np.zeros((1, 4, 2), np.float32)
    with pytest.raises(RuntimeError, match="model op is FNO1d, not DeepONet"):
        ncpp.infer_deeponet_arrays(str(p), u, u)


def test_infer_arrays_rank_check(ncpp, tmp_path):
    rng = np.random.default_rng(4)
    p = tmp_path / "m.nneuroir"
    p.write_bytes(F.fno1d_file(F.fno1d_weights(rng, 2, 1, 8, 4, 1), [2, 1, 8, 4, 1, 1, 0]))
    with pytest.raises(RuntimeError, match="input rank mismatch for op FNO1d"):
        ncpp.infer_arrays(str(p), np.zeros((4, 2), np.float32))
