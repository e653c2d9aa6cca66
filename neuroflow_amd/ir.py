"""NeuroIR binary files (.nneuroir) with their NIRQ quantisation block, read
by libnflow_quant (ir_native::LoadBinary, cpp/include/neuroflow/ir_loader.h:
58-654), and the IR-driven device layers of FNO1d::EnableInt8Gemm
(cpp/src/fno.cpp:325-406) and LinearDispatchTryInt8 (fno.cpp:125-159)."""
from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Dict, List, Optional, Tuple, Union

import numpy as np

from . import _lib
from ._lib import check

OPS = {1: "FNO1d", 2: "FNO2d", 3: "FNO3d", 4: "DeepONet", 5: "TokenMixer", 6: "GraphOp",
       7: "TokenMixer2D", 8: "GraphOp2D"}
QPARAM_KINDS = {0: "per_tensor", 1: "per_channel", 2: "per_token", 3: "fp8_e4m3"}


def _arr(ptr: int, n: int, ctype) -> np.ndarray:
    if n == 0:
        return np.zeros(0, np.dtype(ctype))
    return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ctype)), shape=(n,)).copy()


class IR:
    """An opened IR file: IR(path) or IR(data=bytes)."""

    def __init__(self, path: Union[str, Path, None] = None, data: Optional[bytes] = None):
        self._h = C.c_void_p()
        L = _lib.lib()
        if (path is None) == (data is None):
            raise ValueError("give exactly one of path or data")
        if path is not None:
            check(L.nflow_ir_open(str(path).encode(), C.byref(self._h)), "ir_open")
        else:
            buf = C.create_string_buffer(bytes(data), len(data))
            check(L.nflow_ir_open_memory(buf, len(data), C.byref(self._h)), "ir_open_memory")
        v, op, act, q = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        cfg = (C.c_int32 * 8)()
        check(L.nflow_ir_header(self._h, C.byref(v), C.byref(op), cfg, C.byref(act), C.byref(q)), "ir_header")
        self.version, self.op_code = v.value, op.value
        self.op = OPS[op.value]
        self.config = list(cfg)
        self.activation = "relu" if act.value == 1 else "gelu"
        self.quant_enabled = bool(q.value)

    def weight_names(self) -> List[str]:
        n = C.c_int()
        check(_lib.lib().nflow_ir_num_weights(self._h, C.byref(n)), "ir_num_weights")
        names = []
        for i in range(n.value):
            nm = C.c_char_p()
            check(_lib.lib().nflow_ir_weight_at(self._h, i, C.byref(nm), None, None, None), "ir_weight_at")
            names.append(nm.value.decode())
        return names

    def weight(self, name: str) -> np.ndarray:
        nd = C.c_int()
        dims = (C.c_int64 * 8)()
        data = C.c_void_p()
        check(_lib.lib().nflow_ir_weight(self._h, name.encode(), C.byref(nd), dims, C.byref(data)), "ir_weight")
        shape = tuple(dims[i] for i in range(nd.value))
        return _arr(data.value, int(np.prod(shape, dtype=np.int64)), C.c_float).reshape(shape)

    def qparam_records(self) -> List[Tuple[str, str]]:
        n = C.c_int()
        check(_lib.lib().nflow_ir_num_qparams(self._h, C.byref(n)), "ir_num_qparams")
        out = []
        for i in range(n.value):
            nm, k = C.c_char_p(), C.c_int()
            check(_lib.lib().nflow_ir_qparam_at(self._h, i, C.byref(nm), C.byref(k)), "ir_qparam_at")
            out.append((nm.value.decode(), QPARAM_KINDS[k.value]))
        return out

    def per_tensor(self, name: str) -> Optional[Tuple[float, int]]:
        f, s, z = C.c_int(), C.c_float(), C.c_int32()
        check(_lib.lib().nflow_ir_per_tensor_qparam(self._h, name.encode(), C.byref(f), C.byref(s), C.byref(z)),
              "ir_per_tensor_qparam")
        return (s.value, z.value) if f.value else None

    def per_channel(self, name: str) -> Optional[Tuple[np.ndarray, np.ndarray, int]]:
        f, n, ax, sp, zp = C.c_int(), C.c_int(), C.c_int(), C.c_void_p(), C.c_void_p()
        check(_lib.lib().nflow_ir_per_channel_qparam(self._h, name.encode(), C.byref(f), C.byref(n), C.byref(ax),
                                                     C.byref(sp), C.byref(zp)), "ir_per_channel_qparam")
        if not f.value:
            return None
        return _arr(sp.value, n.value, C.c_float), _arr(zp.value, n.value, C.c_int32), ax.value

    def per_token(self, name: str) -> Optional[Tuple[np.ndarray, np.ndarray, int]]:
        f, n, w, sp, zp = C.c_int(), C.c_int(), C.c_int(), C.c_void_p(), C.c_void_p()
        check(_lib.lib().nflow_ir_per_token_qparam(self._h, name.encode(), C.byref(f), C.byref(n), C.byref(w),
                                                   C.byref(sp), C.byref(zp)), "ir_per_token_qparam")
        if not f.value:
            return None
        return _arr(sp.value, n.value, C.c_float), _arr(zp.value, n.value, C.c_int32), w.value

    def fp8(self, name: str) -> Optional[float]:
        f, s = C.c_int(), C.c_float()
        check(_lib.lib().nflow_ir_fp8_qparam(self._h, name.encode(), C.byref(f), C.byref(s)), "ir_fp8_qparam")
        return s.value if f.value else None

    def layer(self, weight_name: str, bias_name: Optional[str] = None):
        """EnableInt8Gemm for one weight: a device-resident INT8 quant.Layer."""
        from .quant import Layer
        h = C.c_void_p()
        check(_lib.lib().nflow_ir_layer_create(self._h, weight_name.encode(),
                                               None if bias_name is None else bias_name.encode(), C.byref(h)),
              "ir_layer_create")
        return Layer(_handle=h)

    def fno_int8_dispatch(self, layer_index: int) -> Optional[Tuple[float, int]]:
        """(scale_A, zp_A) when locs.{i} would run the INT8 GEMM, else None."""
        use, s, z = C.c_int(), C.c_float(), C.c_int32()
        check(_lib.lib().nflow_ir_fno_int8_dispatch(self._h, layer_index, C.byref(use), C.byref(s), C.byref(z)),
              "ir_fno_int8_dispatch")
        return (s.value, z.value) if use.value else None

    def fno_x2_quant(self, layer_index: int, points: int = 0, device="cuda"):
        """The x2 fake-quant of locs.{i} (fno.cpp:572-648) as a quant.X2Quant,
        per-position arrays uploaded to `device`; None without one, and the
        kind "fp8_log2" for the log2 snap (which the layers reject)."""
        import torch
        from .quant import X2Quant
        q = _lib.X2QuantC()
        check(_lib.lib().nflow_ir_fno_x2_quant(self._h, layer_index, C.byref(q)), "ir_fno_x2_quant")
        if q.kind == _lib.X2_NONE:
            return None
        if q.kind == _lib.X2_PER_TENSOR:
            return X2Quant("per_tensor", scale=q.scale, zero_point=q.zero_point)
        if q.kind == _lib.X2_FP8_LOG2:
            return X2Quant("fp8_log2", scale=q.scale)
        s = torch.from_numpy(_arr(q.scales, q.n_positions, C.c_float)).to(device)
        z = torch.from_numpy(_arr(q.zero_points, q.n_positions, C.c_int32)).to(device)
        return X2Quant("per_position", scales=s, zero_points=z, width=q.width, points=points)

    def close(self) -> None:
        if self._h:
            _lib.lib().nflow_ir_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- writing ----------------------------------------------------------------

_CFG_LEN = {1: 7, 2: 7, 3: 8, 4: 7, 5: 8, 6: 8, 7: 8, 8: 8}


def write_binary(op_code: int, config: List[int], activation: str, weights: Dict[str, np.ndarray],
                 qparams: Optional[List[tuple]] = None, version: int = 3) -> bytes:
    """A NeuroIR binary in the layout ir_native::LoadBinary reads
    (ir_loader.h:1-40, 95-310, 550-650; written by the reference's
    neuroflow/ir/export.py): header, config, activation byte, weight records
    in the given order, and -- when qparams is not None -- the NIRQ block.
    qparams entries: (0, name, scale, zp) per tensor, (1, name, scales, zps,
    axis) per channel, (2, name, scales, zps, width) per token, (3, name,
    scale) FP8."""
    import struct

    cfg = list(config) + [0] * (_CFG_LEN[op_code] - len(config))
    out = [b"NIR0", struct.pack("<HBB", version, op_code, 0), struct.pack(f"<{len(cfg)}i", *cfg),
           struct.pack("<B", 1 if activation == "relu" else 0), b"\x00\x00\x00",
           struct.pack("<I", len(weights))]
    for name, arr in weights.items():
        a = np.ascontiguousarray(arr, np.float32)
        nb = name.encode()
        out += [struct.pack("<B", len(nb)), nb, struct.pack("<B", a.ndim), struct.pack(f"<{a.ndim}i", *a.shape),
                a.tobytes()]
    if qparams is not None:
        out += [b"NIRQ", struct.pack("<BI", 1, len(qparams))]
        for kind, name, *p in qparams:
            nb = name.encode()
            out += [struct.pack("<BB", kind, len(nb)), nb]
            if kind == 0:
                out.append(struct.pack("<fi", p[0], p[1]))
            elif kind in (1, 2):
                scales = np.asarray(p[0], np.float32)
                zps = np.asarray(p[1], np.int32)
                out.append(struct.pack("<IB", scales.size, p[2]) if kind == 1 else
                           struct.pack("<II", scales.size, p[2]))
                out += [scales.tobytes(), zps.tobytes()]
            elif kind == 3:
                out.append(struct.pack("<f", p[0]))
            else:
                raise ValueError(f"unknown qparam kind {kind}")
    return b"".join(out)


# ---- symmetric qparams: the exporter side of the device path -----------------
#
# The reference's calibration writes asymmetric qparams (min/max ranges,
# neuroflow/quant/static_quant.py:480-589), and its INT8 GEMM folds nonzero
# zero points in with formulas that differ between entry points
# (cpp/src/int8_gemm.cpp:386-393, 461-466, 573-575).  The functions below
# write symmetric ones instead -- zero point 0, scale = absmax / 127 (INT8)
# or absmax / 448 (FP8 E4M3) -- in the reference's own qparam dict shape
# (neuroflow/quant/static_quant.py:1120-1139) and NIRQ layout
# (neuroflow/ir/export.py:570-643), so an IR drives EnableInt8Gemm /
# LinearDispatchTryInt8 and the device layers with exact integer products.
# A zero range gives scale 1 with zero point 0, the reference's choice for a
# constant tensor (static_quant.py:508-514).

INT8_QMAX = 127.0
FP8_QMAX = 448.0


def _absmax(x) -> np.float32:
    a = np.asarray(x, np.float32)
    if a.ndim == 0:
        return np.float32(abs(float(a)))
    return np.float32(np.max(np.abs(a))) if a.size else np.float32(0.0)


def _scale(absmax, qmax: float) -> np.ndarray:
    """fl(absmax / qmax) in float32 (1 where absmax is 0 or not finite)."""
    am = np.asarray(absmax, np.float32)
    ok = np.isfinite(am) & (am > 0)
    return np.where(ok, am / np.float32(qmax), np.float32(1.0)).astype(np.float32)


def symmetric_per_channel(W: np.ndarray, channel_axis: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """Per-channel symmetric INT8 weight qparams: scales[c] = absmax of slice c
    along `channel_axis` / 127 (float32), zero points 0."""
    w = np.moveaxis(np.asarray(W, np.float32), channel_axis, 0)
    am = np.max(np.abs(w.reshape(w.shape[0], -1)), axis=1) if w.size else np.zeros(w.shape[0], np.float32)
    return _scale(am, INT8_QMAX), np.zeros(w.shape[0], np.int32)


def symmetric_per_tensor(x) -> Tuple[float, int]:
    """Per-tensor symmetric INT8 activation qparam from a calibration tensor
    (or its absmax): (absmax / 127, 0)."""
    return float(_scale(_absmax(x), INT8_QMAX)), 0


def symmetric_per_token(absmax_per_token, width: int) -> Tuple[np.ndarray, np.ndarray, int]:
    """Static per-token symmetric INT8 qparams (one scale per token position,
    NIRQ kind 2): (absmax[t] / 127, zeros, width)."""
    am = np.asarray(absmax_per_token, np.float32).reshape(-1)
    return _scale(am, INT8_QMAX), np.zeros(am.size, np.int32), int(width)


def fp8_per_tensor(x) -> float:
    """Per-tensor FP8 E4M3 activation scale: absmax / 448."""
    return float(_scale(_absmax(x), FP8_QMAX))


def symmetric_quant(weights: Dict[str, np.ndarray], weight_names: List[str],
                    activations: Optional[Dict[str, object]] = None,
                    per_token: Optional[Dict[str, Tuple[np.ndarray, int]]] = None,
                    fp8_activations: Optional[Dict[str, object]] = None) -> dict:
    """The `quant` dict of neuroflow/quant/static_quant.py:1120-1139
    ({"enabled": True, "qparams": {name: entry}}) with symmetric entries:
    per-channel (axis 0) for each name in weight_names, per-tensor INT8 for
    each activation (a calibration tensor or its absmax), static per-token
    INT8 for each (absmax per token, width) in per_token, FP8 E4M3 for each
    fp8 activation."""
    qp: Dict[str, dict] = {}
    for name in weight_names:
        s, z = symmetric_per_channel(weights[name], 0)
        qp[name] = {"per_channel": True, "channel_axis": 0, "scales": s, "zero_points": z}
    for name, x in (activations or {}).items():
        s, z = symmetric_per_tensor(x)
        qp[name] = {"scale": s, "zero_point": z}
    for name, (am, width) in (per_token or {}).items():
        s, z, w = symmetric_per_token(am, width)
        qp[name] = {"per_token": True, "scales": s, "zero_points": z, "width": w}
    for name, x in (fp8_activations or {}).items():
        qp[name] = {"format": "fp8_e4m3", "scale": fp8_per_tensor(x)}
    return {"enabled": True, "qparams": qp}


def _qparam_tuples(quant: dict) -> List[tuple]:
    """The records of a `quant` dict in write_binary's form, in the dict's
    order, choosing the kind as neuroflow/ir/export.py:612-643 does
    (per_token, then per_channel, then the FP8 format, else per tensor)."""
    out = []
    for name, q in quant.get("qparams", {}).items():
        if q.get("per_token", False):
            out.append((2, name, q["scales"], q["zero_points"], int(q.get("width", 0))))
        elif q.get("per_channel", False):
            out.append((1, name, q["scales"], q["zero_points"], int(q.get("channel_axis", 0))))
        elif q.get("format") == "fp8_e4m3":
            out.append((3, name, float(q["scale"])))
        else:
            out.append((0, name, float(q["scale"]), int(q["zero_point"])))
    return out


def export_symmetric(data: bytes, activations: Optional[Dict[str, object]] = None,
                     per_token: Optional[Dict[str, Tuple[np.ndarray, int]]] = None,
                     fp8_activations: Optional[Dict[str, object]] = None,
                     weight_names: Optional[List[str]] = None) -> bytes:
    """A NeuroIR binary whose NIRQ block holds symmetric qparams: the file's
    header and weights unchanged, any earlier NIRQ block replaced.
    weight_names defaults to every 2-D "*.weight" tensor of the file (the
    Linear weights EnableInt8Gemm looks up: lift, locs.{i}, proj_q,
    proj_out for FNO1d, fno.cpp:360-406)."""
    ir = IR(data=data)
    try:
        names = ir.weight_names()
        weights = {n: ir.weight(n) for n in names}
        op_code, version, config, act = ir.op_code, ir.version, ir.config, ir.activation
    finally:
        ir.close()
    if weight_names is None:
        weight_names = [n for n in names if n.endswith(".weight") and weights[n].ndim == 2]
    quant = symmetric_quant(weights, weight_names, activations, per_token, fp8_activations)
    return write_binary(op_code, config[:_CFG_LEN[op_code]], act, weights, _qparam_tuples(quant), version)
