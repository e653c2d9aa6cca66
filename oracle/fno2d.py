"""FNO2d inference restated on the oracle's C pieces: what
nflow::InferenceRuntime::Create / Run do for an FNO2d IR
(cpp/src/runtime.cpp:38-48, 94-95), i.e. ir_native::LoadBinary's maps
(cpp/include/neuroflow/ir_loader.h:150-160, 298-322, 556-650), FNO2d's
weight fake-quant (cpp/src/fno.cpp:997-1020 over DequantiseWeight,
:217-289) and FNO2d::Forward (fno.cpp:777-995), in the reference's own
(batch, width, H, W) layout with its permutes.

TEST INFRASTRUCTURE ONLY: the reference results for the device runtime; the product
never imports it.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

from oracle import oracle as O


@dataclass
class Fno2dModel:
    in_ch: int
    out_ch: int
    width: int
    modes_h: int
    modes_w: int
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


def weight_names(n_layers: int) -> List[str]:
    names = ["lift.weight", "lift.bias", "proj_q.weight", "proj_q.bias", "proj_out.weight", "proj_out.bias"]
    for i in range(n_layers):
        names += [f"specs.{i}.weights_real", f"specs.{i}.weights_imag"]
    for i in range(n_layers):
        names += [f"locs.{i}.weight", f"locs.{i}.bias"]
    return names


def from_records(cfg, act_relu: bool, weights: Dict[str, np.ndarray],
                 qrecords: Optional[List[tuple]] = None) -> Fno2dModel:
    """cfg = [in_ch, out_ch, width, modes_h, modes_w, n_layers, pad_factor];
    qrecords None (no NIRQ block) or a list of (kind, name, *payload) in file
    order.  Later records of a name replace earlier ones; per-tensor records
    whose name ends in ".output" are activation qparams; per-token records
    are read but FNO2d has no per-token path."""
    m = Fno2dModel(*[int(c) for c in cfg[:7]], O.ACT_RELU if act_relu else O.ACT_GELU_TANH,
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


def _dequantise_weights(m: Fno2dModel):
    """DequantiseWeight (fno.cpp:217-289): per-channel qparams for 2-D
    weights on axis 0 and 3-D weights on axis 1 (the 4-D spectral weights
    fall through), else the per-tensor qparam of the name."""
    for name in weight_names(m.n_layers):
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


def enable_int8_gemm_fno2d(m: Fno2dModel):
    """The device runtime's FNO2d INT8 opt-in, which has no counterpart in
    the reference: FNO1d's cache (fno.cpp:360-406, an INT8 blob by
    QuantiseWeight2D for each locs.{i} weight with 2-D axis-0 per-channel
    qparams) and its dispatch (LinearDispatchTryInt8, fno.cpp:125-159)."""
    m.int8_enabled = True
    m.int8_cache = {}
    for i in range(m.n_layers):
        name = f"locs.{i}.weight"
        pc = m.per_channel.get(name)
        W = m.weights[name]
        if pc is None or W.ndim != 2 or pc[2] != 0:
            continue
        scales = np.ascontiguousarray(pc[0][:W.shape[0]], np.float32)
        zps = np.ascontiguousarray(pc[1][:W.shape[0]], np.int32)
        Wq, sumw = O.quantise_weight_2d(W, scales, zps)
        m.int8_cache[name] = (Wq, scales, zps, sumw)


def fake_quant(m: Fno2dModel, data: np.ndarray, key: str) -> np.ndarray:
    """The apply_fake_quant helper of FNO2d::Forward (fno.cpp:810-850): the
    log2 "FP8" snap when an FP8 qparam exists for the key (nothing when its
    scale is not positive), else the INT8 per-tensor round trip."""
    if not m.quant_enabled:
        return data
    if key in m.fp8:
        s = m.fp8[key]
        return O.log2_snap(data, s) if s > 0.0 else data
    if key in m.act_tensor:
        s, zp = m.act_tensor[key]
        return O.fake_quant_elementwise(data, s, zp)
    return data


def forward(m: Fno2dModel, x: np.ndarray) -> np.ndarray:
    """FNO2d::Forward (fno.cpp:777-995) on x (batch, H, W, in_ch)."""
    x = np.ascontiguousarray(x, np.float32)
    b, H, W, in_ch = x.shape
    assert in_ch == m.in_ch
    assert H > 0 and (H & (H - 1)) == 0 and W > 0 and (W & (W - 1)) == 0
    w, L = m.width, m.n_layers
    Wt = m.weights
    h = O.linear_f32(x.reshape(b * H * W, in_ch), Wt["lift.weight"], Wt["lift.bias"])
    h = fake_quant(m, h, "lift.output").reshape(b, H, W, w)
    h_perm = np.ascontiguousarray(h.transpose(0, 3, 1, 2))
    pad_h = pad_w = 0
    if m.pad_factor > 1:
        pf = m.pad_factor
        pad_h, pad_w = (pf - H % pf) % pf, (pf - W % pf) % pf
        if pad_h or pad_w:
            padded = np.zeros((b, w, H + pad_h, W + pad_w), np.float32)
            padded[:, :, :H, :W] = h_perm
            h_perm = padded
            H += pad_h
            W += pad_w
    for i in range(L):
        x1 = O.spectral_conv2d(h_perm, Wt[f"specs.{i}.weights_real"], Wt[f"specs.{i}.weights_imag"],
                               m.modes_h, m.modes_w)
        x2_in = np.ascontiguousarray(h_perm.transpose(0, 2, 3, 1)).reshape(b * H * W, w)
        in_key = "lift.output" if i == 0 else f"locs.{i - 1}.output"
        cache_key = f"locs.{i}.weight"
        use_int8 = (m.int8_enabled and in_key not in m.per_token and in_key not in m.fp8
                    and cache_key in m.int8_cache and in_key in m.act_tensor)
        if use_int8:
            Wq, sw, zw, sumw = m.int8_cache[cache_key]
            s_a, zp_a = m.act_tensor[in_key]
            rc, x2_out = O.linear_forward_batched(x2_in, Wq, sw, zw, None, s_a, zp_a, sumw)
            assert rc == 0
            x2_out = (x2_out + Wt[f"locs.{i}.bias"][None, :]).astype(np.float32)
        else:
            x2_out = O.linear_f32(x2_in, Wt[f"locs.{i}.weight"], Wt[f"locs.{i}.bias"])
        x2 = np.ascontiguousarray(x2_out.reshape(b, H, W, w).transpose(0, 3, 1, 2))
        x2 = fake_quant(m, x2, f"locs.{i}.output")
        h_perm = O.apply_activation((x1 + x2).astype(np.float32), m.act)
    if pad_h or pad_w:
        H -= pad_h
        W -= pad_w
        h_perm = np.ascontiguousarray(h_perm[:, :, :H, :W])
    h_back = np.ascontiguousarray(h_perm.transpose(0, 2, 3, 1)).reshape(b * H * W, w)
    q = O.linear_f32(h_back, Wt["proj_q.weight"], Wt["proj_q.bias"])
    q = O.apply_activation(fake_quant(m, q, "proj_q.output"), m.act)
    y = O.linear_f32(q, Wt["proj_out.weight"], Wt["proj_out.bias"])
    y = fake_quant(m, y, "proj_out.output")
    return y.reshape(b, H, W, m.out_ch)
