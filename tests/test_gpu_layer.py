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
