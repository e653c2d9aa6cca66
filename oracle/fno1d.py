"""FNO1d inference restated on the oracle's C pieces: what
nflow::InferenceRuntime::Create / EnableInt8Gemm / Run do for an FNO1d IR
(cpp/src/runtime.cpp:21-101), i.e. ir_native::LoadBinary's maps
(cpp/include/neuroflow/ir_loader.h:556-650), FNO1d's weight fake-quant
(cpp/src/fno.cpp:209-300), its INT8 weight cache (fno.cpp:325-406) and
FNO1d::Forward (fno.cpp:408-700), in the reference's own (batch, width,
points) layout with its permutes.

TEST INFRASTRUCTURE ONLY: the reference results for the device runtime; the product
never imports it.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

from oracle import oracle as O


@dataclass
class Fno1dModel:
    in_ch: int
    out_ch: int
    width: int
    modes: int
    n_layers: int
    pad_factor: int
    act: int                                  # O.ACT_RELU or O.ACT_GELU_TANH
    weights: Dict[str, np.ndarray]
    quant_enabled: bool = False
    act_tensor: Dict[str, Tuple[float, int]] = field(default_factory=dict)
    weight_tensor: Dict[str, Tuple[float, int]] = field(default_factory=dict)
    per_channel: Dict[str, Tuple[np.ndarray, np.ndarray, int]] = field(default_factory=dict)
    per_token: Dict[str, Tuple[np.ndarray, np.ndarray, int]] = field(default_factory=dict)
    fp8: Dict[str, float] = field(default_factory=dict)
    int8_cache: Dict[str, Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]] = field(default_factory=dict)
    int8_enabled: bool = False


def from_records(cfg, act_relu: bool, weights: Dict[str, np.ndarray],
                 qrecords: Optional[List[tuple]] = None) -> Fno1dModel:
    """cfg = [in_ch, out_ch, width, modes, n_layers, pad_factor]; qrecords
    None (no NIRQ block) or a list of (kind, name, *payload) in file order,
    the payloads of tests/nir_format.qparam_record.  Later records of a
    name replace earlier ones (ir_loader.h:583-645); per-tensor records
    whose name ends in ".output" are activation qparams."""
    m = Fno1dModel(*[int(c) for c in cfg[:6]], O.ACT_RELU if act_relu else O.ACT_GELU_TANH,
                   {k: np.array(v, np.float32, copy=True) for k, v in weights.items()})
    if qrecords is not None:
        m.quant_enabled = True
        for kind, name, *p in qrecords:
            if kind == 0:
                tgt = m.act_tensor if name.endswith(".output") else m.weight_tensor
                tgt[name] = (np.float32(p[0]), int(p[1]))
            elif kind == 1:
                m.per_channel[name] = (np.asarray(p[0], np.float32), np.asarray(p[1], np.int32), int(p[2]))
            elif kind == 2:
                m.per_token[name] = (np.asarray(p[0], np.float32), np.asarray(p[1], np.int32), int(p[2]))
            elif kind == 3:
                m.fp8[name] = np.float32(p[0])
        _dequantise_weights(m)
    return m


def _weight_names(m: Fno1dModel):
    names = ["lift.weight", "lift.bias", "proj_q.weight", "proj_q.bias", "proj_out.weight", "proj_out.bias"]
    for i in range(m.n_layers):
        names += [f"specs.{i}.weights_real", f"specs.{i}.weights_imag"]
    for i in range(m.n_layers):
        names += [f"locs.{i}.weight", f"locs.{i}.bias"]
    return names


def _dequantise_weights(m: Fno1dModel):
    """fno.cpp:209-300 (EnablePerChannelWeightDequant): per-channel qparams
    for 2-D weights on axis 0 and 3-D spectral weights on axis 1, else the
    per-tensor qparam of the name, else nothing."""
    for name in _weight_names(m):
        t = m.weights[name]
        pc = m.per_channel.get(name)
        if pc is not None:
            scales, zps, axis = pc
            if t.ndim == 2 and axis == 0:
                n_ch = scales.size
                t[:n_ch] = O.fake_quant_elementwise(t[:n_ch], scales[:n_ch, None], zps[:n_ch, None])
                continue
            if t.ndim == 3 and axis == 1:
                out_dim = t.shape[1]
                m.weights[name] = O.fake_quant_elementwise(t, scales[None, :out_dim, None],
                                                           zps[None, :out_dim, None])
                continue
        pt = m.weight_tensor.get(name)
        if pt is not None:
            m.weights[name] = O.fake_quant_elementwise(t, pt[0], pt[1])


def enable_int8_gemm(m: Fno1dModel):
    """fno.cpp:360-406: an INT8 blob (QuantiseWeight2D, fno.cpp:325-358) for
    every Linear whose weight has a 2-D axis-0 per-channel qparam."""
    m.int8_enabled = True
    m.int8_cache = {}
    names = ["lift.weight"] + [f"locs.{i}.weight" for i in range(m.n_layers)] + ["proj_q.weight",
                                                                                 "proj_out.weight"]
    for name in names:
        pc = m.per_channel.get(name)
        W = m.weights[name]
        if pc is None or W.ndim != 2 or pc[2] != 0:
            continue
        scales = np.ascontiguousarray(pc[0][:W.shape[0]], np.float32)
        zps = np.ascontiguousarray(pc[1][:W.shape[0]], np.int32)
        Wq, sumw = O.quantise_weight_2d(W, scales, zps)
        m.int8_cache[name] = (Wq, scales, zps, sumw)


def _permute_bnw_to_bwn(a):
    return np.ascontiguousarray(a.transpose(0, 2, 1))


def forward(m: Fno1dModel, x: np.ndarray) -> np.ndarray:
    """FNO1d::Forward (fno.cpp:408-700) on x (batch, n, in_ch)."""
    x = np.ascontiguousarray(x, np.float32)
    b, n, in_ch = x.shape
    assert in_ch == m.in_ch and n > 0 and (n & (n - 1)) == 0
    w, L = m.width, m.n_layers
    W = m.weights
    h = O.linear_f32(x.reshape(b * n, in_ch), W["lift.weight"], W["lift.bias"]).reshape(b, n, w)
    h_perm = _permute_bnw_to_bwn(h)
    pad_len = 0
    if m.pad_factor > 1:
        r = n % m.pad_factor
        pad_len = 0 if r == 0 else m.pad_factor - r
        if pad_len:
            h_perm = np.concatenate([h_perm, np.zeros((b, w, pad_len), np.float32)], axis=2)
            n += pad_len
    for i in range(L):
        in_key = "lift.output" if i == 0 else f"locs.{i - 1}.output"
        if m.quant_enabled and in_key in m.act_tensor:
            s, zp = m.act_tensor[in_key]
            h_perm = O.fake_quant_elementwise(h_perm, s, zp)
        x1 = O.spectral_conv1d(h_perm, W[f"specs.{i}.weights_real"], W[f"specs.{i}.weights_imag"], m.modes)
        x2_in = np.ascontiguousarray(h_perm.transpose(0, 2, 1)).reshape(b * n, w)
        cache_key = f"locs.{i}.weight"
        use_int8 = (m.int8_enabled and in_key not in m.per_token and in_key not in m.fp8
                    and cache_key in m.int8_cache and in_key in m.act_tensor)
        if use_int8:
            Wq, sw, zw, sumw = m.int8_cache[cache_key]
            s_a, zp_a = m.act_tensor[in_key]
            rc, x2_out = O.linear_forward_batched(x2_in, Wq, sw, zw, None, s_a, zp_a, sumw)
            assert rc == 0
            x2_out = (x2_out + W[f"locs.{i}.bias"][None, :]).astype(np.float32)
        else:
            x2_out = O.linear_f32(x2_in, W[f"locs.{i}.weight"], W[f"locs.{i}.bias"])
        x2 = _permute_bnw_to_bwn(x2_out.reshape(b, n, w))
        if m.quant_enabled:
            key = f"locs.{i}.output"
            if key in m.fp8:
                if m.fp8[key] > 0.0:
                    x2 = O.log2_snap(x2, m.fp8[key])
            elif key in m.per_token:
                scales, zps, w_axis = m.per_token[key]
                cnt = n * w_axis
                assert w_axis == w and scales.size >= cnt
                flat = x2.reshape(b, n * w)
                x2 = O.fake_quant_elementwise(flat, scales[None, :cnt], zps[None, :cnt]).reshape(b, w, n)
            elif key in m.act_tensor:
                s, zp = m.act_tensor[key]
                x2 = O.fake_quant_elementwise(x2, s, zp)
        add = (x1 + x2).astype(np.float32)
        h_perm = O.apply_activation(add, m.act)
    if pad_len:
        n -= pad_len
        h_perm = np.ascontiguousarray(h_perm[:, :, :n])
    h_back = np.ascontiguousarray(h_perm.transpose(0, 2, 1)).reshape(b * n, w)
    q = O.linear_f32(h_back, W["proj_q.weight"], W["proj_q.bias"])
    q = O.apply_activation(q, m.act)
    y = O.linear_f32(q, W["proj_out.weight"], W["proj_out.bias"])
    return y.reshape(b, n, m.out_ch)
