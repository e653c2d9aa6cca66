"""GPU tests of the device-resident layer handles (nflow_layer_*): the same
bits as the parameter-block entry points, for both formats and shapes on
both kernels, and create / destroy cycles."""
import numpy as np
import pytest
import torch

from neuroflow_amd import quant as Q
from neuroflow_amd import workloads as WL
from oracle import oracle as O

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-5, 1e-6


def _cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(1000, 64, 64), (700, 768, 256), (64, 1024, 1024)])
@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_layer_handle_matches_parameter_entry_points(gpu, M, N, K, fmt):
    W = WL.kaiming_uniform(60, N, K)
    b = WL.uniform(61, (N,), -0.05, 0.05)
    x = _cu(WL.normal(62, (M, K)))
    layer = Q.Layer(W, b, fmt)
    assert (layer.out_features, layer.in_features, layer.fmt) == (N, K, fmt)
    ref = (Q.Int8Linear if fmt == "int8" else Q.Fp8Linear)(W, b)
    y, s = layer(x, "gelu", return_scales=True)
    y_ref = ref(x, "gelu")
    assert _same(_host(y), _host(y_ref))
    qmax = 127.0 if fmt == "int8" else 448.0
    assert _same(_host(s), O.per_token_scales(_host(x), qmax))
    layer.close()


def test_layer_from_int8_blob_with_zero_points(gpu):
    M, N, K = 300, 256, 256
    W = WL.uniform(63, (N, K), -0.125, 0.125)
    s = O.per_channel_scales(W, 127.0)
    zps = WL.uniform(64, (N,), -6, 6).astype(np.int32)
    q, sw = O.quantise_weight_2d(W, s, zps)
    b = WL.uniform(65, (N,), -0.1, 0.1)
    A = WL.normal(66, (M, K))
    for sumW in (None, sw):
        layer = Q.Layer.from_int8_blob(q, s, zps, b, sumW)
        out = _host(layer(_cu(A), "none"))
        ref, _ = O.layer_per_token_i8(A, q, s, zps, b, sumW, 0)
        assert _same(out, ref)


@pytest.mark.parametrize("K,N", [(64, 64), (256, 256), (1024, 512)])
def test_layer_symmetric_blob_detection(gpu, K, N):
    """A handle built from a symmetric blob (zero points 0, sum_W the code
    sums) runs its per-token calls without the integer-epilogue terms; a
    blob with one nonzero zero point, or with a sum_W that differs from the
    code sums, keeps them.  Each output equals the oracle with the blob as
    given, bit for bit (no activation), on the K = 64, one-pass and
    persistent-GEMM kernels."""
    M = 700
    W = WL.uniform(69, (N, K), -0.125, 0.125)
    s = O.per_channel_scales(W, 127.0)
    zps = np.zeros(N, np.int32)
    q, sw = O.quantise_weight_2d(W, s, zps)
    b = WL.uniform(70, (N,), -0.1, 0.1)
    A = WL.normal(71, (M, K))
    sw_off = (sw + np.arange(N, dtype=np.int32) % 5 - 2).astype(np.int32)
    zp_one = zps.copy()
    zp_one[N // 3] = 2
    outs = []
    for zp_b, sw_b in ((zps, sw), (zps, sw_off), (zp_one, sw)):
        layer = Q.Layer.from_int8_blob(q, s, zp_b, b, sw_b)
        out = _host(layer(_cu(A), "none"))
        layer.close()
        ref, _ = O.layer_per_token_i8(A, q, s, zp_b, b, sw_b, 0)
        assert _same(out, ref)
        outs.append(out)
    # The terms show: the nonsymmetric blobs give other outputs.
    assert not _same(outs[1], outs[0]) and not _same(outs[2], outs[0])


def test_layer_create_destroy_cycles(gpu):
    W = WL.kaiming_uniform(67, 64, 64)
    x = _cu(WL.normal(68, (128, 64)))
    first = None
    for i in range(50):
        layer = Q.Layer(W, None, "int8" if i % 2 == 0 else "fp8")
        y = _host(layer(x, "relu"))
        if i == 0:
            first = y
        elif i % 2 == 0:
            assert _same(y, first)
        layer.close()
        layer.close()                          # closing twice is harmless


# ---- the FNO layer form act(x1 + x2) ------------------------------------------

@pytest.mark.parametrize("M,N,K", [(3000, 64, 64), (257, 768, 256), (300, 96, 100)])
@pytest.mark.parametrize("act", ["none", "relu", "gelu"])
def test_fno_layer_int8(gpu, M, N, K, act):
    """y = act(x1 + (W q(h) + b)) (fno.cpp:541-549, 650-654): the fused K = N = 64
    kernel and the two-pass form of the other shapes give the reference's
    operation order, so none / relu are bit-exact against the oracle layer."""
    W = WL.uniform(70, (N, K), -0.125, 0.125)
    s = O.per_channel_scales(W, 127.0)
    q, sw = O.quantise_weight_2d(W, s)
    b = WL.uniform(71, (N,), -0.1, 0.1)
    h = WL.normal(72, (M, K))
    x1 = (0.5 * WL.normal(73, (M, N))).astype(np.float32)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(np.zeros(N, np.int32)), _cu(b), sum_W_per_row=_cu(sw))
    y = _host(Q.fno_layer_per_token(p, _cu(h), _cu(x1), act))
    x2, _ = O.layer_per_token_i8(h, q, s, None, b, sw, 0)
    ref = O.apply_activation((x1 + x2).astype(np.float32), {"none": 0, "relu": 1, "gelu": 2}[act])
    if act == "gelu":
        np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)
    else:
        assert _same(y, ref)


@pytest.mark.parametrize("M,N,K", [(3000, 64, 64), (100, 768, 256)])
def test_fno_layer_fp8_and_handle(gpu, M, N, K):
    W = WL.kaiming_uniform(74, N, K)
    b = WL.uniform(75, (N,), -0.05, 0.05)
    h = _cu(2.0 * WL.normal(76, (M, K)))
    x1 = _cu(WL.normal(77, (M, N)))
    fp8 = Q.Fp8Linear(W, b)
    y = _host(Q.fp8_fno_layer_per_token(fp8.params, h, x1, "none"))
    x2 = _host(fp8(h, "none"))
    assert _same(y, (_host(x1) + x2).astype(np.float32))
    for fmt in ("int8", "fp8"):
        layer = Q.Layer(W, b, fmt)
        yl = _host(layer(h, "relu", residual=x1))
        x2l = _host(layer(h, "none"))
        assert _same(yl, O.apply_activation((_host(x1) + x2l).astype(np.float32), 1))
    with pytest.raises(Exception):
        Q.fno_layer_per_token(Q.Int8Linear(W, b).params, h, x1, "none", out=x1)


# ---- the FNO layer's x2 fake-quant (fno.cpp:572-648) ------------------------

def _x2q_params(kind, N, points, seed):
    rng = np.random.default_rng(seed)
    if kind == "per_tensor":
        return Q.X2Quant("per_tensor", scale=0.031, zero_point=-4), dict(scale=0.031, zp=-4)
    s = rng.uniform(0.01, 0.08, N * points).astype(np.float32)
    z = rng.integers(-10, 10, N * points).astype(np.int32)
    return (Q.X2Quant("per_position", scales=_cu(s), zero_points=_cu(z), width=N, points=points),
            dict(scales=s, zps=z, points=points))


@pytest.mark.parametrize("M,N,K", [(2048, 64, 64), (512, 256, 256), (256, 64, 100), (128, 1024, 1024)])
@pytest.mark.parametrize("kind", ["per_tensor", "per_position"])
@pytest.mark.parametrize("act,with_x1", [("relu", True), ("none", False), ("gelu", True)])
def test_fno_layer_x2_fake_quant_int8(gpu, M, N, K, kind, act, with_x1):
    points = 64
    x = (WL.normal(60, (M, K)) * 2.0).astype(np.float32)
    x1 = WL.normal(61, (M, N)).astype(np.float32) if with_x1 else None
    W = WL.uniform(62, (N, K), -0.25, 0.25)
    b = WL.uniform(63, (N,), -0.1, 0.1)
    layer = Q.Int8Linear(W, b)
    xq, oq = _x2q_params(kind, N, points, 64)
    out = _host(Q.fno_layer_per_token(layer.params, _cu(x), None if x1 is None else _cu(x1), act, x2_quant=xq))
    x2, _ = O.layer_per_token_i8(x, layer.W_q, layer.scale_W, None, b, layer.sum_W, O.ACT_NONE)
    fq = O.x2_fake_quant(x2, **oq)
    pre = fq if x1 is None else (x1 + fq).astype(np.float32)
    ref = O.apply_activation(pre, {"none": 0, "relu": 1, "gelu": 2}[act])
    if act == "gelu":
        np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)
    else:
        assert _same(out, ref)


@pytest.mark.parametrize("M,N,K", [(2048, 64, 64), (320, 256, 256)])
@pytest.mark.parametrize("kind", ["per_tensor", "per_position"])
def test_fno_layer_x2_fake_quant_fp8(gpu, M, N, K, kind):
    """FP8 x2 agrees with the exact-product oracle to 1e-5 / 1e-6, so a fake-quant
    step can flip where x2 sits at a rounding boundary: outputs equal the
    oracle's up to one quantisation step, and almost all exactly."""
    points = 32
    x = (2.0 * WL.normal(65, (M, K))).astype(np.float32)
    x1 = WL.normal(66, (M, N)).astype(np.float32)
    W = WL.uniform(67, (N, K), -0.125, 0.125)
    b = WL.uniform(68, (N,), -0.1, 0.1)
    layer = Q.Fp8Linear(W, b)
    xq, oq = _x2q_params(kind, N, points, 69)
    out = _host(Q.fp8_fno_layer_per_token(layer.params, _cu(x), _cu(x1), "relu", x2_quant=xq))
    qa, sa = O.quantise_per_token_fp8(x)
    x2 = O.layer_fp8_exact(qa, sa, layer.W_q, layer.scale_W, b, O.ACT_NONE)
    ref = O.apply_activation((x1 + O.x2_fake_quant(x2, **oq)).astype(np.float32), O.ACT_RELU)
    step = oq["scale"] if kind == "per_tensor" else float(oq["scales"].max())
    assert np.all(np.abs(out - ref) <= step * 1.001 + 1e-5)
    assert np.mean(out != ref) < 0.01


def test_fno_layer_x2_fake_quant_on_handles_and_errors(gpu):
    from neuroflow_amd._lib import NflowError, SHAPE_MISMATCH, UNSUPPORTED_OP
    M, N, K = 1024, 64, 64
    x = WL.normal(70, (M, K)).astype(np.float32)
    x1 = WL.normal(71, (M, N)).astype(np.float32)
    W = WL.uniform(72, (N, K), -0.25, 0.25)
    b = WL.uniform(73, (N,), -0.1, 0.1)
    h = Q.Layer(W, b, fmt="int8")
    p = Q.Int8Linear(W, b)
    xq, _ = _x2q_params("per_position", N, 16, 74)
    y_h = _host(h(_cu(x), "relu", residual=_cu(x1), x2_quant=xq))
    y_p = _host(Q.fno_layer_per_token(p.params, _cu(x), _cu(x1), "relu", x2_quant=xq))
    assert _same(y_h, y_p)
    bad = [Q.X2Quant("fp8_log2", scale=0.5),
           Q.X2Quant("per_position", scales=xq.scales, zero_points=xq.zero_points, width=N + 1, points=16),
           Q.X2Quant("per_position", scales=xq.scales, zero_points=xq.zero_points, width=N, points=17)]
    for q, code in zip(bad, [UNSUPPORTED_OP, SHAPE_MISMATCH, SHAPE_MISMATCH]):
        with pytest.raises(NflowError) as e:
            h(_cu(x), "relu", residual=_cu(x1), x2_quant=q)
        assert e.value.code == code
    h.close()


# ---- the K = N = 64 kernel's per-CU tile queue ---------------------------------

@pytest.fixture
def _queue_off():
    """Context: the K = 64 kernel with its static tile deal
    (nflow_debug_set_kernel_path("no_rows64_queue", 1))."""
    import contextlib
    import ctypes

    from neuroflow_amd import _lib

    @contextlib.contextmanager
    def ctx():
        L = _lib.lib()
        prev = ctypes.c_int(0)
        _lib.check(L.nflow_debug_set_kernel_path(b"no_rows64_queue", 1, ctypes.byref(prev)), "path")
        try:
            yield
        finally:
            _lib.check(L.nflow_debug_set_kernel_path(b"no_rows64_queue", prev.value, None), "path")
    return ctx


@pytest.mark.parametrize("M", [262144 + 37, 1 << 20])
@pytest.mark.parametrize("form", ["int8_gelu", "int8_none", "fp8_gelu", "fno_relu", "fno_x2q", "batched"])
def test_rows64_tile_queue_matches_static_deal(gpu, _queue_off, M, form):
    """Layers of 256 Ki+ rows run on one 16-wave block per CU whose waves take
    tiles from an LDS counter; every output equals the static deal's bit for
    bit (each tile is computed once, by whichever wave takes it), and sampled
    rows equal the oracle."""
    N = K = 64
    W = WL.uniform(90, (N, K), -0.125, 0.125)
    b = WL.uniform(91, (N,), -0.1, 0.1)
    h = WL.normal(92, (M, K))
    h[M // 3] = np.nan
    s = O.per_channel_scales(W, 127.0)
    q, sw = O.quantise_weight_2d(W, s)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(np.zeros(N, np.int32)), _cu(b), sum_W_per_row=_cu(sw))
    x1 = _cu((0.5 * WL.normal(93, (M, N))).astype(np.float32)) if form.startswith("fno") else None
    hd = _cu(h)

    def run():
        if form == "int8_gelu":
            return Q.linear_forward_per_token(p, hd, "gelu")
        if form == "int8_none":
            return Q.linear_forward_per_token(p, hd, "none")
        if form == "fp8_gelu":
            return Q.Fp8Linear(W, b)(hd, "gelu")
        if form == "fno_relu":
            return Q.fno_layer_per_token(p, hd, x1, "relu")
        if form == "fno_x2q":
            return Q.fno_layer_per_token(p, hd, x1, "gelu", x2_quant=Q.X2Quant("per_tensor", scale=0.031, zero_point=-4))
        pb = Q.Int8LinearParams(_cu(q), _cu(s), _cu(np.zeros(N, np.int32)), _cu(b), scale_A=0.021, zp_A=3)
        return Q.linear_forward_batched(pb, hd)

    y = _host(run())
    with _queue_off():
        y_static = _host(run())
    assert _same(y, y_static)
    if form == "int8_none":
        rows = np.unique(np.concatenate([np.arange(0, M, 997), [M // 3, M - 1]]))
        ref, _ = O.layer_per_token_i8(h[rows], q, s, None, b, sw, 0)
        fin = np.isfinite(ref)
        assert _same(y[rows][fin], ref[fin])
