"""The FNO2d runtime on the GPU (neuroflow_cpp / include/nflow_runtime.h)
against the oracle's restatement of InferenceRuntime over FNO2d::Forward
(oracle/fno2d.py, pinned bit for bit to the reference runtime in
tests/test_oracle_fno2d.py) and, where oracle/_ref was built, the reference
runtime itself: every output bit equal, for ReLU and GELU models, without
and with fake-quants (INT8 per-tensor, the log2 "FP8" snap, an FP8 record
of scale 0), padding, grids from 1 x 8 to 256 x 256, and through every
entry point (run on host arrays, run_device on torch CUDA tensors,
infer_arrays)."""
import numpy as np
import pytest

from neuroflow_amd import _lib
from neuroflow_amd.runtime import load
from oracle import fno2d as OF2
from tests import nir_format as F
from tests.test_oracle_fno2d import REF_RUN, qrec_bytes, quant_records, ref_run

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _model(case, seed=11):
    b, H, W, ci, co, w, mh, mw, L, pad, relu, kinds = case
    rng = np.random.default_rng([b, H, W, w, L, pad, int(relu), len(kinds or []), seed])
    weights = F.fno2d_weights(rng, ci, co, w, mh, mw, L)
    recs = None if kinds is None else quant_records(rng, weights, L, kinds)
    cfg = [ci, co, w, mh, mw, L, pad]
    ir = F.fno2d_file(weights, cfg, None if recs is None else qrec_bytes(recs), act=1 if relu else 0)
    x = rng.standard_normal((b, H, W, ci)).astype(np.float32)
    return ir, x, OF2.from_records(cfg, relu, weights, recs)


CASES = [
    # (b, H, W, in, out, width, mh, mw, layers, pad, relu, quant kinds or None)
    (2, 8, 8, 2, 1, 8, 3, 3, 2, 1, True, None),
    (2, 8, 16, 3, 2, 8, 4, 5, 2, 1, False, None),
    (1, 16, 8, 1, 1, 12, 5, 4, 3, 1, False, ["tensor"]),
    (2, 16, 16, 3, 1, 8, 6, 6, 4, 1, False, ["fp8", "tensor", "fp8zero"]),
    (1, 4, 4, 1, 1, 4, 2, 2, 2, 8, False, ["tensor", "fp8"]),
    (1, 1, 8, 1, 1, 4, 1, 3, 1, 1, True, None),
    (2, 32, 32, 1, 1, 16, 8, 8, 2, 1, False, ["fp8"]),
    (2, 64, 32, 2, 1, 32, 12, 12, 2, 1, False, ["tensor", "fp8"]),
    (1, 128, 64, 1, 1, 64, 12, 12, 1, 1, False, ["fp8"]),
    (1, 256, 256, 1, 1, 64, 12, 12, 1, 1, False, ["fp8"]),
    # 512 whole 32-point tiles at width 64: the fp32 local linear and the
    # tail in one launch.
    (4, 64, 64, 1, 1, 64, 12, 12, 2, 1, True, ["tensor", "fp8"]),
    (4, 64, 64, 2, 1, 64, 12, 12, 2, 1, False, None),
    # Row lengths 128 and 512 on the fixed-length row FFTs, 12 rows (a
    # part-filled row set of 8 at 128 points).
    (1, 4, 128, 1, 1, 3, 3, 20, 1, 1, False, ["tensor"]),
    (2, 4, 512, 1, 1, 4, 2, 6, 1, 1, True, None),
    # Column lengths 256 (mh above 16: every group of the forward's later
    # passes and every stored row of the inverse), 512 and 1024 on the
    # fixed-length column FFTs.
    (1, 256, 8, 1, 1, 4, 20, 3, 1, 1, False, None),
    (1, 512, 4, 1, 1, 4, 6, 2, 1, 1, True, None),
    (1, 1024, 2, 1, 1, 4, 70, 2, 1, 1, False, ["tensor"]),
    (2, 8, 8, 1, 1, 8, 8, 5, 1, 1, False, None),            # all H rows and all W/2 + 1 bins
    (1, 4, 2, 1, 1, 4, 2, 2, 0, 1, False, ["tensor"]),       # no layers
    # Output element counts that are not a multiple of 4 (the fake-quant
    # passes' one-by-one remainder): 3 x 1 x 2 x 1 and 3 x 1 x 2 x 3.
    (3, 1, 2, 1, 1, 4, 1, 2, 1, 1, False, ["tensor", "fp8"]),
    (3, 1, 2, 2, 3, 4, 1, 2, 1, 1, True, ["fp8", "tensor"]),
]


def _ids(c):
    return (f"b{c[0]}H{c[1]}W{c[2]}w{c[5]}m{c[6]}x{c[7]}L{c[8]}p{c[9]}{'relu' if c[10] else 'gelu'}"
            f"{'-'.join(c[11] or ['fp32'])}")


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_run_bit_exact(gpu, tmp_path, case):
    ncpp = load()
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    rt = ncpp.InferenceRuntime(str(path))
    assert rt.op() == "FNO2d"
    rt.enable_int8_gemm()                       # a no-op for FNO2d, as in the reference
    assert not rt.is_int8_gemm_enabled()
    b, H, W, _ = x.shape
    y = np.zeros((b, H, W, case[4]), np.float32)
    rt.run(x, y)
    want = OF2.forward(m, x)
    assert np.array_equal(_bits(y), _bits(want)), int((_bits(y) != _bits(want)).sum())
    if REF_RUN.exists() and x.size * case[5] <= 1 << 20:
        assert np.array_equal(_bits(y), _bits(ref_run(tmp_path, ir, x, case[4])))


@pytest.mark.parametrize("case", [(2, 64, 64, 1, 1, 16, 12, 12, 2, 1, False, ["fp8"]),
                                  (1, 256, 8, 1, 1, 4, 20, 3, 1, 1, True, None)], ids=_ids)
def test_fixed_size_kernels_equal_generic(gpu, tmp_path, case):
    """The fixed-length row and column FFTs and the LDS-staged channel mix
    against the any-size kernels (kernel path generic_fft) and the oracle."""
    import ctypes as C
    ncpp = load()
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    want = OF2.forward(m, x)
    L = _lib.lib()
    b, H, W, _ = x.shape
    for flag in (0, 1):
        prev = C.c_int(0)
        _lib.check(L.nflow_debug_set_kernel_path(b"generic_fft", flag, C.byref(prev)), "kernel path")
        try:
            rt = ncpp.InferenceRuntime(str(path))
            y = np.zeros((b, H, W, case[4]), np.float32)
            rt.run(x, y)
        finally:
            _lib.check(L.nflow_debug_set_kernel_path(b"generic_fft", prev.value, None), "kernel path")
        assert np.array_equal(_bits(y), _bits(want)), (flag, int((_bits(y) != _bits(want)).sum()))


@pytest.mark.parametrize("relu,kinds", [(False, ["tensor", "fp8"]), (True, ["fp8", "tensor"]),
                                        (False, ["fp8zero", "tensor", "fp8"]), (False, None)])
def test_fused_launches_equal_separate(gpu, tmp_path, relu, kinds):
    """The width-64 local linear + tail (k_linear_tail) and the projection
    head (k_proj_tail) in one launch each against their separate launches
    (kernel path no_layer_tail) and the oracle, with proj_q / proj_out
    fake-quants off, per tensor, log2 snap and disabled by an FP8 record of
    scale 0."""
    import ctypes as C
    case = (4, 64, 64, 1, 1, 64, 12, 12, 2, 1, relu, kinds)
    ncpp = load()
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    want = OF2.forward(m, x)
    L = _lib.lib()
    b, H, W, _ = x.shape
    for flag in (0, 1):
        prev = C.c_int(0)
        _lib.check(L.nflow_debug_set_kernel_path(b"no_layer_tail", flag, C.byref(prev)), "kernel path")
        try:
            rt = ncpp.InferenceRuntime(str(path))
            y = np.zeros((b, H, W, 1), np.float32)
            rt.run(x, y)
        finally:
            _lib.check(L.nflow_debug_set_kernel_path(b"no_layer_tail", prev.value, None), "kernel path")
        assert np.array_equal(_bits(y), _bits(want)), (flag, int((_bits(y) != _bits(want)).sum()))


def test_run_device_and_infer_arrays(gpu, tmp_path):
    import torch
    ncpp = load()
    case = (3, 32, 16, 2, 2, 16, 6, 5, 2, 1, False, ["fp8", "tensor"])
    ir, x, m = _model(case, seed=12)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    want = OF2.forward(m, x)
    rt = ncpp.InferenceRuntime(str(path))
    dev = torch.device("cuda:0")
    xt = torch.from_numpy(x).to(dev)
    yt = torch.full((3, 32, 16, 2), float("nan"), device=dev)
    stream = torch.cuda.current_stream(dev)
    rt.run_device(xt.data_ptr(), list(xt.shape), yt.data_ptr(), list(yt.shape), stream.cuda_stream)
    torch.cuda.synchronize(dev)
    assert np.array_equal(_bits(yt.cpu().numpy()), _bits(want))
    # A second run with a smaller batch reuses the workspace.
    y2 = torch.full((1, 32, 16, 2), float("nan"), device=dev)
    rt.run_device(xt[:1].data_ptr(), [1, 32, 16, 2], y2.data_ptr(), [1, 32, 16, 2], stream.cuda_stream)
    torch.cuda.synchronize(dev)
    assert np.array_equal(_bits(y2.cpu().numpy()), _bits(want[:1]))
    # An output 4 bytes past a 16-byte boundary (the output fake-quant's
    # one-element-at-a-time form); the element before it stays untouched.
    big = torch.full((1 + 3 * 32 * 16 * 2,), float("nan"), device=dev)
    big[0] = 7.0
    y3 = big[1:].view(3, 32, 16, 2)
    rt.run_device(xt.data_ptr(), list(xt.shape), y3.data_ptr(), list(y3.shape), stream.cuda_stream)
    torch.cuda.synchronize(dev)
    assert np.array_equal(_bits(y3.cpu().numpy()), _bits(want))
    assert big[0].item() == 7.0
    assert np.array_equal(_bits(ncpp.infer_arrays(str(path), x)), _bits(want))
    with pytest.raises(RuntimeError, match="input rank mismatch for op FNO2d"):
        ncpp.infer_arrays(str(path), x[0])


def test_shape_errors(gpu, tmp_path):
    ncpp = load()
    ir, x, m = _model((2, 8, 8, 2, 1, 8, 3, 3, 2, 1, True, None))
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    rt = ncpp.InferenceRuntime(str(path))
    z = lambda *s: np.zeros(s, np.float32)
    with pytest.raises(RuntimeError, match="expected 4D input"):
        rt.run(z(2, 8, 2), z(2, 8, 8, 1))
    with pytest.raises(RuntimeError, match="input channels mismatch"):
        rt.run(z(2, 8, 8, 3), z(2, 8, 8, 1))
    with pytest.raises(RuntimeError, match="output buffer shape mismatch"):
        rt.run(z(2, 8, 8, 2), z(2, 8, 4, 1))
    with pytest.raises(RuntimeError, match="H and W must each be a power of two"):
        rt.run(z(2, 8, 6, 2), z(2, 8, 6, 1))
    with pytest.raises(RuntimeError, match="modes exceed"):
        rt.run(z(2, 2, 8, 2), z(2, 2, 8, 1))       # modes_h 3 > H 2
    rt.run(z(0, 8, 8, 2), z(0, 8, 8, 1))            # empty batch: Ok, nothing to do


def test_padded_grid_must_be_a_power_of_two(gpu, tmp_path):
    # pad_factor 3 pads 4 to 6, which the reference's radix-2 FFT cannot take
    # (fft.cpp asserts a power of two); the runtime reports it.
    ncpp = load()
    ir, x, m = _model((1, 4, 4, 1, 1, 4, 2, 2, 1, 3, False, None))
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    rt = ncpp.InferenceRuntime(str(path))
    with pytest.raises(RuntimeError, match="padded grid is not a power of two"):
        rt.run(x, np.zeros((1, 4, 4, 1), np.float32))


INT8_CASES = [
    # (b, H, W, in, out, width, mh, mw, layers, pad, relu, quant kinds)
    (2, 16, 16, 2, 1, 16, 4, 4, 3, 1, False, ["tensor"]),
    (2, 16, 8, 1, 2, 8, 3, 3, 4, 1, True, ["tensor", "fp8"]),      # fp8 inputs keep those layers fp32
    (1, 4, 4, 1, 1, 4, 2, 2, 2, 8, False, ["tensor"]),             # padded
    (2, 64, 64, 1, 1, 64, 12, 12, 2, 1, False, ["tensor"]),
    # Enough 32-point tiles for the layer and its tail in one launch.
    (4, 64, 64, 1, 1, 64, 12, 12, 2, 1, True, ["tensor"]),
]


@pytest.mark.parametrize("case", INT8_CASES, ids=_ids)
def test_int8_opt_in_bit_exact(gpu, tmp_path, case):
    """The FNO2d INT8 opt-in (no counterpart in the reference): each
    dispatched locs.{i} runs as LinearForwardBatched + bias with its input
    key's per-tensor qparam, bit-exact against the oracle composed of the
    reference's primitives; the reference's own enable_int8_gemm stays a
    no-op."""
    import ctypes as C
    ncpp = load()
    ir, x, m = _model(case, seed=13)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    b, H, W, _ = x.shape
    rt = ncpp.InferenceRuntime(str(path))
    rt.enable_int8_gemm()
    y_fp32 = np.zeros((b, H, W, case[4]), np.float32)
    rt.run(x, y_fp32)
    assert np.array_equal(_bits(y_fp32), _bits(OF2.forward(m, x)))
    rt.enable_int8_gemm_fno2d()
    assert rt.is_int8_gemm_enabled()
    OF2.enable_int8_gemm_fno2d(m)
    y = np.zeros_like(y_fp32)
    rt.run(x, y)
    want = OF2.forward(m, x)
    assert np.array_equal(_bits(y), _bits(want)), int((_bits(y) != _bits(want)).sum())
    # The per-layer decision is the one FNO1d's dispatch would take.
    h = C.c_void_p()
    _lib.check(_lib.lib().nflow_runtime_create(str(path).encode(), C.byref(h)), "runtime_create")
    _lib.check(_lib.lib().nflow_runtime_enable_int8_gemm_fno2d(h), "enable_int8_gemm_fno2d")
    for i in range(case[8]):
        used = C.c_int32()
        _lib.check(_lib.lib().nflow_runtime_layer_dispatch(h, i, C.byref(used)), "layer_dispatch")
        in_key = "lift.output" if i == 0 else f"locs.{i - 1}.output"
        assert bool(used.value) == (in_key in m.act_tensor and in_key not in m.fp8)
    _lib.lib().nflow_runtime_destroy(h)


def test_int8_opt_in_rejects_fno1d(gpu, tmp_path):
    ncpp = load()
    rng = np.random.default_rng(9)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(F.fno1d_file(F.fno1d_weights(rng, 2, 1, 8, 4, 1), [2, 1, 8, 4, 1, 1, 0]))
    rt = ncpp.InferenceRuntime(str(path))
    with pytest.raises(RuntimeError, match="enable_int8_gemm_fno2d failed"):
        rt.enable_int8_gemm_fno2d()
