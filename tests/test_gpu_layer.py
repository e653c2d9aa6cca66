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
