"""The FNO1d runtime on the GPU (neuroflow_cpp / include/nflow_runtime.h)
against the oracle's restatement of InferenceRuntime (oracle/fno1d.py, pinned
bit for bit to the reference runtime in tests/test_oracle_fno1d.py) and,
where oracle/_ref was built, the reference runtime itself: every output bit
equal, for ReLU and GELU models, fp32 and INT8 local-linear layers, every
x2 fake-quant kind, padding, and through every entry point (run on host
arrays, run_device on torch CUDA tensors, infer_arrays, infer)."""
import ctypes as C

import numpy as np
import pytest

from neuroflow_amd import _lib
from neuroflow_amd.runtime import load
from oracle import fno1d as OF
from tests import nir_format as F
from tests.test_oracle_fno1d import REF_RUN, _qrec_bytes, quant_records, ref_run

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _model(case):
    b, n, ci, co, w, modes, L, pad, relu, kinds, int8 = case
    rng = np.random.default_rng([b, n, w, L, pad, int(relu), int(int8), len(kinds or []), 7])
    weights = F.fno1d_weights(rng, ci, co, w, modes, L)
    n_pad = n + ((pad - n % pad) % pad if pad > 1 else 0)
    recs = None if kinds is None else quant_records(rng, weights, L, w, n_pad, kinds)
    cfg = [ci, co, w, modes, L, pad, 0]
    ir = F.fno1d_file(weights, cfg, None if recs is None else _qrec_bytes(recs), act=1 if relu else 0)
    x = rng.standard_normal((b, n, ci)).astype(np.float32)
    m = OF.from_records(cfg, relu, weights, recs)
    if int8:
        OF.enable_int8_gemm(m)
    return ir, x, m


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
    (2, 1, 1, 1, 8, 1, 1, 1, False, ["tensor"], True),
    (2, 2048, 1, 1, 20, 16, 2, 1, False, ["fp8", "tensor"], True),
    (1, 8192, 2, 3, 8, 32, 1, 1, False, ["tensor"], True),
    (8, 1024, 1, 1, 64, 16, 4, 1, False, ["tensor"], True),
    # Batches large enough for the layer tail's 32-token tiles (at least
    # two tiles per CU): whole tiles, a partial channel tile (width 40) with
    # every x2 kind, and half-filled token tiles (16 points).
    (20, 1024, 1, 1, 64, 16, 2, 1, False, ["tensor"], True),
    (40, 1024, 1, 1, 40, 16, 3, 1, True, ["token", "tensor", "fp8"], True),
    (600, 16, 2, 1, 8, 4, 2, 1, False, ["fp8", "tensor"], True),
    # A batch whose lift (one input channel, width 64) takes several passes
    # of the grid: each thread's columns stay fixed from pass to pass.
    (160, 1024, 1, 1, 64, 16, 1, 1, False, ["tensor"], True),
    # The fixed-length row FFTs (64 .. 1024 points): modes up to the first
    # pass's group size (only element 0 of later groups kept) and above it,
    # and row counts that leave the last row set part-filled (15 rows).
    (3, 512, 1, 1, 16, 8, 2, 1, False, ["tensor"], False),
    (2, 512, 2, 1, 12, 20, 2, 1, True, None, False),
    (4, 128, 1, 2, 16, 24, 2, 1, False, ["fp8"], False),
    (3, 128, 1, 1, 5, 9, 1, 1, False, None, False),
    (3, 256, 1, 1, 5, 40, 2, 1, True, ["tensor"], False),
    (1, 1024, 1, 1, 8, 100, 1, 1, False, None, False),
    (3, 64, 1, 1, 5, 4, 1, 1, False, None, False),
    (3, 64, 1, 1, 5, 33, 1, 1, True, None, False),
    (2, 128, 1, 1, 8, 6, 1, 1, False, None, False),
    (1, 512, 1, 1, 4, 80, 1, 1, True, None, False),
]


def _ids(c):
    return (f"b{c[0]}n{c[1]}w{c[4]}L{c[6]}p{c[7]}{'relu' if c[8] else 'gelu'}"
            f"{'-'.join(c[9] or ['fp32'])}{'-int8' if c[10] else ''}")


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_run_bit_exact(gpu, tmp_path, case):
    ncpp = load()
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    rt = ncpp.InferenceRuntime(str(path))
    assert rt.op() == "FNO1d"
    assert not rt.is_int8_gemm_enabled()
    if case[10]:
        rt.enable_int8_gemm()
        assert rt.is_int8_gemm_enabled()
    y = np.zeros((x.shape[0], x.shape[1], case[3]), np.float32)
    rt.run(x, y)
    want = OF.forward(m, x)
    assert np.array_equal(_bits(y), _bits(want)), int((_bits(y) != _bits(want)).sum())
    if REF_RUN.exists() and x.size * case[4] <= 1 << 22:
        assert np.array_equal(_bits(y), _bits(ref_run(tmp_path, ir, x, case[3], case[10])))


@pytest.mark.parametrize("kinds,relu,int8", [(["tensor"], False, True), (["token", "tensor", "fp8"], True, True),
                                             (["fp8", "token"], False, True), (["tensor"], False, False),
                                             (["token", "tensor", "fp8"], True, False), (None, False, False)])
def test_layer_tail_fused_equals_two_launches(gpu, tmp_path, kinds, relu, int8):
    """The width-64 local-linear layer and its tail in one launch
    (k_layer_tail for INT8, k_linear_tail for fp32) against the two
    launches (the layer + k_post_rt, kernel path no_layer_tail) and the
    oracle: every x2 fake-quant kind, with and without zero points on the
    INT8 layer's input, and no fake-quant at all."""
    case = (20, 1024, 1, 1, 64, 16, 3, 1, relu, kinds, int8)
    ncpp = load()
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    want = OF.forward(m, x)
    L = _lib.lib()
    outs = []
    for flag in (0, 1):
        prev = C.c_int(0)
        _lib.check(L.nflow_debug_set_kernel_path(b"no_layer_tail", flag, C.byref(prev)), "kernel path")
        try:
            rt = ncpp.InferenceRuntime(str(path))
            if int8:
                rt.enable_int8_gemm()
            y = np.zeros((x.shape[0], x.shape[1], 1), np.float32)
            rt.run(x, y)
            outs.append(y)
        finally:
            _lib.check(L.nflow_debug_set_kernel_path(b"no_layer_tail", prev.value, None), "kernel path")
    for y in outs:
        assert np.array_equal(_bits(y), _bits(want)), int((_bits(y) != _bits(want)).sum())


@pytest.mark.parametrize("case", [(3, 256, 1, 1, 16, 12, 2, 1, False, ["tensor"], False),
                                  (2, 1024, 1, 1, 16, 16, 2, 1, True, None, False),
                                  (3, 256, 1, 1, 5, 40, 1, 1, False, None, False)], ids=_ids)
def test_fixed_length_ffts_equal_generic(gpu, tmp_path, case):
    """The fixed-length row FFT kernels against the any-length ones (kernel
    path generic_fft) and the oracle."""
    ncpp = load()
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    want = OF.forward(m, x)
    L = _lib.lib()
    for flag in (0, 1):
        prev = C.c_int(0)
        _lib.check(L.nflow_debug_set_kernel_path(b"generic_fft", flag, C.byref(prev)), "kernel path")
        try:
            rt = ncpp.InferenceRuntime(str(path))
            y = np.zeros((x.shape[0], x.shape[1], case[3]), np.float32)
            rt.run(x, y)
        finally:
            _lib.check(L.nflow_debug_set_kernel_path(b"generic_fft", prev.value, None), "kernel path")
        assert np.array_equal(_bits(y), _bits(want)), (flag, int((_bits(y) != _bits(want)).sum()))


def test_dispatch_matches_the_reference_decision(gpu, tmp_path):
    case = (2, 64, 3, 1, 12, 8, 4, 1, False, ["tensor", "token", "fp8"], True)
    ir, x, m = _model(case)
    h = C.c_void_p()
    L = _lib.lib()
    assert L.nflow_runtime_create_memory(ir, len(ir), C.byref(h)) == 0
    try:
        assert L.nflow_runtime_enable_int8_gemm(h) == 0
        for i in range(4):
            u = C.c_int(-1)
            assert L.nflow_runtime_layer_dispatch(h, i, C.byref(u)) == 0
            in_key = "lift.output" if i == 0 else f"locs.{i - 1}.output"
            want = (in_key in m.act_tensor and in_key not in m.per_token and in_key not in m.fp8
                    and f"locs.{i}.weight" in m.int8_cache)
            assert bool(u.value) == want, i
    finally:
        L.nflow_runtime_destroy(h)


def test_run_device_on_torch_tensors(gpu, tmp_path):
    import torch
    ncpp = load()
    case = (4, 256, 1, 1, 32, 12, 4, 1, False, ["tensor"], True)
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    rt = ncpp.InferenceRuntime(str(path))
    rt.enable_int8_gemm()
    xd = torch.from_numpy(x).to(gpu)
    yd = torch.full((4, 256, 1), float("nan"), device=gpu)
    s = torch.cuda.current_stream()
    rt.run_device(xd.data_ptr(), list(xd.shape), yd.data_ptr(), list(yd.shape), s.cuda_stream)
    s.synchronize()
    assert np.array_equal(_bits(yd.cpu().numpy()), _bits(OF.forward(m, x)))
    # A second run with another batch reuses the workspace.
    x2 = x[:3].copy() * 2
    yd2 = torch.empty((3, 256, 1), device=gpu)
    rt.run_device(torch.from_numpy(x2).to(gpu).data_ptr(), [3, 256, 1], yd2.data_ptr(), [3, 256, 1], 0)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(yd2.cpu().numpy()), _bits(OF.forward(m, x2)))


def test_run_host_buffers_across_batch_sizes(gpu, tmp_path):
    """run() on host arrays keeps its device copies of the input and output
    between calls and grows them on demand: a batch of 2, a larger one, a
    smaller one and the first again each equal the oracle bit for bit."""
    ncpp = load()
    case = (8, 256, 1, 1, 32, 12, 4, 1, False, ["tensor"], True)
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    rt = ncpp.InferenceRuntime(str(path))
    rt.enable_int8_gemm()
    for b, scale in ((2, 1.0), (8, 0.5), (1, 2.0), (2, 1.0)):
        xb = np.ascontiguousarray(x[:b] * np.float32(scale))
        y = np.full((b, 256, 1), np.nan, np.float32)
        rt.run(xb, y)
        assert np.array_equal(_bits(y), _bits(OF.forward(m, xb))), b


def test_infer_and_infer_arrays(gpu, tmp_path):
    ncpp = load()
    case = (3, 32, 1, 2, 16, 6, 3, 1, False, ["tensor"], False)
    ir, x, m = _model(case)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    want = OF.forward(m, x)
    assert np.array_equal(_bits(ncpp.infer_arrays(str(path), x)), _bits(want))
    np.save(tmp_path / "x.npy", x)
    assert ncpp.infer(str(path), str(tmp_path / "x.npy"), str(tmp_path / "y.npy")) == "ok"
    assert np.array_equal(_bits(np.load(tmp_path / "y.npy")), _bits(want))


def test_gelu_sweep_bit_exact(gpu, tmp_path):
    """Identity lift / projections and no layers: y = gelu(x) element by
    element, over a dense sweep of magnitudes (the reference's GELU with
    glibc tanhf, fno.cpp:41-46)."""
    ncpp = load()
    w = 64
    eye = np.eye(w, dtype=np.float32)
    zero = np.zeros(w, np.float32)
    weights = {"lift.weight": eye, "lift.bias": zero, "proj_q.weight": eye, "proj_q.bias": zero,
               "proj_out.weight": eye, "proj_out.bias": zero}
    ir = F.fno1d_file(weights, [w, w, w, 1, 0, 1, 0])
    path = tmp_path / "g.nneuroir"
    path.write_bytes(ir)
    rng = np.random.default_rng(11)
    mags = np.exp(rng.uniform(np.log(1e-30), np.log(1e4), 2 ** 20)).astype(np.float32)
    x = (mags * rng.choice([-1.0, 1.0], mags.size)).astype(np.float32)
    x[:8] = [0.5, -0.5, 3.0, -3.0, 10.0, -10.0, 1e-40, -9.5]
    x = x.reshape(1, -1, w)[:, :8192]            # 8192 points x 64 channels
    m = OF.from_records([w, w, w, 1, 0, 1], False, weights, None)
    y = np.zeros_like(x)
    ncpp.InferenceRuntime(str(path)).run(x, y)
    assert np.array_equal(_bits(y), _bits(OF.forward(m, x)))


def test_shape_errors(gpu, tmp_path):
    ncpp = load()
    ir, x, m = _model((2, 16, 2, 1, 8, 4, 2, 1, True, None, False))
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    rt = ncpp.InferenceRuntime(str(path))
    with pytest.raises(RuntimeError, match="expected 3D input"):
        rt.run(np.zeros((16, 2), np.float32), np.zeros((2, 16, 1), np.float32))
    with pytest.raises(RuntimeError, match="input channels mismatch"):
        rt.run(np.zeros((2, 16, 3), np.float32), np.zeros((2, 16, 1), np.float32))
    with pytest.raises(RuntimeError, match="output buffer shape mismatch"):
        rt.run(np.zeros((2, 16, 2), np.float32), np.zeros((2, 16, 2), np.float32))
    with pytest.raises(RuntimeError, match="power of two"):
        rt.run(np.zeros((2, 12, 2), np.float32), np.zeros((2, 12, 1), np.float32))
    y = np.zeros((0, 16, 1), np.float32)
    rt.run(np.zeros((0, 16, 2), np.float32), y)   # empty batch: Ok, nothing to do


def test_fp8_codec_functions(gpu):
    from oracle import oracle as O
    ncpp = load()
    x = np.random.default_rng(5).standard_normal(4097).astype(np.float32) * 100
    x[:4] = [np.nan, np.inf, -np.inf, 470.0]
    b = ncpp.fp8_e4m3_to_bits(x)
    assert np.array_equal(b, O.e4m3_encode(x))
    assert np.array_equal(_bits(ncpp.fp8_e4m3_from_bits(b)), _bits(O.e4m3_decode(b)))
    assert np.array_equal(_bits(ncpp.fp8_e4m3_fake_quant(x[4:], 0.5)), _bits(O.fp8_fake_quant(x[4:], 0.5)))


@pytest.mark.parametrize("relu", [False, True])
def test_exported_symmetric_ir_runs_int8(gpu, tmp_path, relu):
    """An FNO1d IR given symmetric qparams by neuroflow_amd.ir.export_symmetric
    (per-channel weights, per-tensor inputs of every local-linear layer)
    sends every locs.{i} to the INT8 GEMM with zero points 0, and the
    runtime equals the oracle and the reference runtime bit for bit."""
    from neuroflow_amd import ir as IRM
    ncpp = load()
    b, n, ci, co, w, modes, L = 4, 256, 2, 1, 32, 12, 4
    rng = np.random.default_rng([w, L, int(relu), 11])
    weights = F.fno1d_weights(rng, ci, co, w, modes, L)
    cfg = [ci, co, w, modes, L, 1, 0]
    plain = F.fno1d_file(weights, cfg, None, act=1 if relu else 0)
    acts = {"lift.output": 1.5, **{f"locs.{i}.output": 2.0 + i for i in range(L)}}
    ir = IRM.export_symmetric(plain, activations=acts)
    x = rng.standard_normal((b, n, ci)).astype(np.float32)
    names = [k for k, v in weights.items() if v.ndim == 2 and k.endswith(".weight")]
    recs = IRM._qparam_tuples(IRM.symmetric_quant(weights, names, acts))
    m = OF.from_records(cfg, relu, weights, recs)
    OF.enable_int8_gemm(m)
    path = tmp_path / "m.nneuroir"
    path.write_bytes(ir)
    rt = ncpp.InferenceRuntime(str(path))
    rt.enable_int8_gemm()
    h = C.c_void_p()
    lib = _lib.lib()
    assert lib.nflow_runtime_create_memory(ir, len(ir), C.byref(h)) == 0
    try:
        assert lib.nflow_runtime_enable_int8_gemm(h) == 0
        for i in range(L):
            u = C.c_int(-1)
            assert lib.nflow_runtime_layer_dispatch(h, i, C.byref(u)) == 0
            assert u.value == 1, i
    finally:
        lib.nflow_runtime_destroy(h)
    y = np.zeros((b, n, co), np.float32)
    rt.run(x, y)
    want = OF.forward(m, x)
    assert np.array_equal(_bits(y), _bits(want)), int((_bits(y) != _bits(want)).sum())
    if REF_RUN.exists():
        assert np.array_equal(_bits(y), _bits(ref_run(tmp_path, ir, x, co, True)))
