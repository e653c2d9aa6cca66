"""GPU tests of the IR-driven device layers: EnableInt8Gemm from a NeuroIR
file's per-channel qparams (nflow_ir_layer_create; fno.cpp:325-406), run as
the per-tensor INT8 layer of LinearDispatchTryInt8 (nflow_layer_forward_per_
tensor; fno.cpp:125-159, 541-549) and as the fused per-token layer."""
import numpy as np
import pytest
import torch

from neuroflow_amd.ir import IR
from oracle import oracle as O
from tests import nir_format as F

pytestmark = pytest.mark.gpu


def _cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _ir(width, n_layers, zp_layer=None, seed=5):
    rng = np.random.default_rng(seed)
    w = F.fno1d_weights(rng, 2, 1, width, 4, n_layers)
    recs = [F.qparam_record(0, "lift.output", 0.031, 0)]
    zps = {}
    for i in range(n_layers):
        s, z = F.symmetric_per_channel(w[f"locs.{i}.weight"])
        if i == zp_layer:
            z = (np.arange(width) % 7 - 3).astype(np.int32)
        zps[i] = (s, z)
        recs.append(F.qparam_record(1, f"locs.{i}.weight", s, z, 0))
        recs.append(F.qparam_record(0, f"locs.{i}.output", 0.02 * (i + 1), i - 1))
    return IR(data=F.fno1d_file(w, [2, 1, width, 4, n_layers, 1, 0], recs)), w, zps


@pytest.mark.parametrize("width,M", [(64, 5000), (256, 777), (1024, 300)])
@pytest.mark.parametrize("zp_layer", [None, 1])
def test_ir_layer_per_tensor_matches_reference_formula(gpu, width, M, zp_layer):
    ir, w, zps = _ir(width, 2, zp_layer)
    for i in range(2):
        dispatch = ir.fno_int8_dispatch(i)
        assert dispatch is not None
        scale_A, zp_A = dispatch
        layer = ir.layer(f"locs.{i}.weight", f"locs.{i}.bias")
        x = np.random.default_rng(10 + i).normal(0, 1.5, (M, width)).astype(np.float32)
        y = _host(layer.forward_per_tensor(_cu(x), scale_A, zp_A))
        s, z = zps[i]
        W_q, sum_W = O.quantise_weight_2d(w[f"locs.{i}.weight"], s, z)
        rc, ref = O.linear_forward_batched(x, W_q, s, z, w[f"locs.{i}.bias"], scale_A, zp_A, sum_W)
        assert rc == 0
        assert _same(y, ref)
        layer.close()
    ir.close()


@pytest.mark.parametrize("width", [64, 256])
def test_ir_layer_per_token_matches_oracle(gpu, width):
    ir, w, zps = _ir(width, 1, zp_layer=0)
    layer = ir.layer("locs.0.weight", "locs.0.bias")
    x = np.random.default_rng(3).normal(0, 1, (2000, width)).astype(np.float32)
    y = _host(layer(_cu(x), "relu"))
    s, z = zps[0]
    W_q, sum_W = O.quantise_weight_2d(w["locs.0.weight"], s, z)
    ref, _ = O.layer_per_token_i8(x, W_q, s, z, w["locs.0.bias"], sum_W, O.ACT_RELU)
    assert _same(y, ref)
    layer.close()
    ir.close()


def test_ir_layer_rejects_what_enable_int8_gemm_skips(gpu):
    from neuroflow_amd._lib import NflowError
    rng = np.random.default_rng(1)
    w = F.fno1d_weights(rng, 2, 1, 8, 4, 1)
    s, z = F.symmetric_per_channel(w["locs.0.weight"])
    recs = [F.qparam_record(1, "locs.0.weight", s, z, 1),                 # channel axis 1
            F.qparam_record(1, "specs.0.weights_real", np.ones(8, np.float32), np.zeros(8, np.int32), 0)]
    with IR(data=F.fno1d_file(w, [2, 1, 8, 4, 1, 1, 0], recs)) as ir:
        for args in [("locs.0.weight", None), ("specs.0.weights_real", None), ("proj_q.weight", None),
                     ("nope.weight", None), ("locs.0.weight", "nope.bias")]:
            with pytest.raises(NflowError):
                ir.layer(*args)


def test_ir_x2_fake_quant_drives_the_layer(gpu):
    """IR.fno_x2_quant's precedence (FP8, per-token, per-tensor; fno.cpp:575-648)
    and the per-position layer it feeds."""
    rng = np.random.default_rng(8)
    w, n = 64, 32
    W = F.fno1d_weights(rng, 2, 1, w, 4, 3)
    s, z = F.symmetric_per_channel(W["locs.0.weight"])
    ps = rng.uniform(0.01, 0.05, n * w).astype(np.float32)
    pz = rng.integers(-5, 5, n * w).astype(np.int32)
    recs = [F.qparam_record(1, "locs.0.weight", s, z, 0),
            F.qparam_record(2, "locs.0.output", ps, pz, w),
            F.qparam_record(0, "locs.0.output", 0.5, 0),
            F.qparam_record(0, "locs.1.output", 0.25, 3),
            F.qparam_record(3, "locs.2.output", 0.125),
            F.qparam_record(0, "locs.2.output", 0.5, 0)]
    with IR(data=F.fno1d_file(W, [2, 1, w, 4, 3, 1, 0], recs)) as ir:
        q0, q1, q2 = ir.fno_x2_quant(0, points=n), ir.fno_x2_quant(1), ir.fno_x2_quant(2)
        assert q0.kind == "per_position" and q0.width == w
        assert (q1.kind, q1.scale, q1.zero_point) == ("per_tensor", 0.25, 3)
        assert q2.kind == "fp8_log2" and ir.fno_x2_quant(5) is None
        layer = ir.layer("locs.0.weight", "locs.0.bias")
        x = rng.normal(0, 1, (4 * n, w)).astype(np.float32)
        x1 = rng.normal(0, 1, (4 * n, w)).astype(np.float32)
        y = _host(layer(_cu(x), "relu", residual=_cu(x1), x2_quant=q0))
        W_q, sum_W = O.quantise_weight_2d(W["locs.0.weight"], s, z)
        x2, _ = O.layer_per_token_i8(x, W_q, s, z, W["locs.0.bias"], sum_W, O.ACT_NONE)
        ref = O.apply_activation((x1 + O.x2_fake_quant(x2, scales=ps, zps=pz, points=n)).astype(np.float32),
                                 O.ACT_RELU)
        assert _same(y, ref)
        layer.close()
