"""Every workload configuration at its full size, through the product entry
points, against the oracle on sampled rows (oracle/parity.py says which rows
and why a sample of rows is an exact check of them):

  C1 standalone INT8         32768 x 64 -> 64, GELU
  C2 FNO1d INT8 stack        262144 x 64 -> 64, 4 chained layers, GELU
                             (16384 tiles: 4-6 per persistent wave)
  C3 FNO2d FP8 stack         1048576 x 64 -> 64, 4 chained layers, GELU
                             (65536 tiles: the doubled grid, 8-11 per wave)
  C4 TokenMixer INT8         32768 x 256 -> 768 / 256, 6 blocks (one-pass kernel)
  C5 DeepONet INT8 trunk     65536 x 1024 -> 1024 (3, ReLU) -> 256
                             (128 x 256 and 128 x 128 tiles of the tiled GEMM)
  C5 DeepONet INT8 branch    4096 x 1024 -> 1024 (4, ReLU) (64 x 128 tiles)

Each layer runs at full size with the workload's activation; its input is
the workload's input or the device output of the previous layer, so every
layer of a chain is checked on what it really read.  INT8 layers with an
activation run a second time without it, and those outputs must equal the
oracle's bits: codes, int32 accumulators and the dequantise are exact, and
only the activation carries the 1e-5 / 1e-6 tolerance.
"""
import numpy as np
import pytest
import torch

from neuroflow_amd import quant as Q
from neuroflow_amd import workloads as WL
from oracle import parity as P

pytestmark = pytest.mark.gpu


def _run_layer(obj, fmt, x, act):
    fn = Q.linear_forward_per_token if fmt == "int8" else Q.fp8_linear_forward_per_token
    return fn(obj.params, x, act, return_scales=True)


def _check_workload(wl, dev):
    ins = [torch.from_numpy(x).to(dev) for x in wl.inputs]
    outs = []
    report = []
    for l, L in enumerate(wl.layers):
        obj = (Q.Fp8Linear if L.fmt == "fp8" else Q.Int8Linear)(L.W, L.bias, device=dev)
        kind, k = wl.source(l)
        x = ins[k] if kind == "input" else outs[k]
        y, s = _run_layer(obj, L.fmt, x, L.act)
        outs.append(y)
        N, K = L.W.shape
        rows = P.sample_rows(wl.M, K, N)
        idx = torch.from_numpy(rows).to(dev)
        x_rows = x.index_select(0, idx).cpu().numpy()
        want, s_want = P.layer_ref(L.fmt, obj.W_q, obj.scale_W, getattr(obj, "sum_W", None), L.bias,
                                   x_rows, L.act)
        torch.cuda.synchronize()
        got = y.index_select(0, idx).cpu().numpy()
        s_got = s.index_select(0, idx).cpu().numpy()
        tag = f"layer {l} ({wl.M} x {K} -> {N}, {L.fmt}, {L.act}, {rows.size} rows)"
        assert np.array_equal(s_got.view(np.uint32), s_want.view(np.uint32)), f"{tag}: per-row scales"
        r = P.compare(got, want, L.fmt, L.act)
        assert r["ok"], f"{tag}: {r}"
        if L.fmt == "int8" and L.act != "none":
            y0, _ = _run_layer(obj, L.fmt, x, "none")
            want0, _ = P.layer_ref(L.fmt, obj.W_q, obj.scale_W, obj.sum_W, L.bias, x_rows, "none")
            torch.cuda.synchronize()
            r0 = P.compare(y0.index_select(0, idx).cpu().numpy(), want0, "int8", "none")
            assert r0["ok"], f"{tag}, no activation: {r0}"
            del y0
        report.append((tag, r["bit_exact_frac"], r["max_abs"]))
    return report


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5_trunk", "c5_branch"])
def test_config_full_size(gpu, name):
    wl = WL.WORKLOADS[name]()
    print(f"\n{wl.name}", flush=True)
    for tag, frac, mx in _check_workload(wl, gpu):
        print(f"  {tag}: bit-exact {frac:.4f}, max |diff| {mx:.3g}", flush=True)
    torch.cuda.empty_cache()
