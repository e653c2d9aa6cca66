"""Builds NeuroIR binary files for the tests, from the layout that
neuroflow/ir/export.py:export_to_binary writes and ir_native::LoadBinary
reads (cpp/include/neuroflow/ir_loader.h:1-40, 550-650): header, config,
activation byte, weight records, optional NIRQ block."""
from __future__ import annotations

import struct
from typing import Dict, List, Sequence, Tuple

import numpy as np

CFG_LEN = {1: 7, 2: 7, 3: 8, 4: 7, 5: 8, 6: 8, 7: 8, 8: 8}


def header(op_code: int, config: Sequence[int], act: int = 0, version: int = 3, n_weights: int = 0) -> bytes:
    cfg = list(config) + [0] * (CFG_LEN.get(op_code, 7) - len(config))
    return (b"NIR0" + struct.pack("<HBB", version, op_code, 0) + struct.pack(f"<{len(cfg)}i", *cfg)
            + struct.pack("<B", act) + b"\x00\x00\x00" + struct.pack("<I", n_weights))


def weight_record(name: str, arr: np.ndarray) -> bytes:
    a = np.ascontiguousarray(arr, np.float32)
    nb = name.encode()
    return (struct.pack("<B", len(nb)) + nb + struct.pack("<B", a.ndim) + struct.pack(f"<{a.ndim}i", *a.shape)
            + a.tobytes())


def qparam_record(kind: int, name: str, *payload) -> bytes:
    nb = name.encode()
    out = struct.pack("<BB", kind, len(nb)) + nb
    if kind == 0:
        scale, zp = payload
        out += struct.pack("<fi", scale, zp)
    elif kind == 1:
        scales, zps, axis = payload
        out += struct.pack("<IB", len(scales), axis)
        out += np.asarray(scales, np.float32).tobytes() + np.asarray(zps, np.int32).tobytes()
    elif kind == 2:
        scales, zps, width = payload
        out += struct.pack("<II", len(scales), width)
        out += np.asarray(scales, np.float32).tobytes() + np.asarray(zps, np.int32).tobytes()
    elif kind == 3:
        (scale,) = payload
        out += struct.pack("<f", scale)
    else:
        raise ValueError(kind)
    return out


def nirq(records: List[bytes], flag: int = 1) -> bytes:
    return b"NIRQ" + struct.pack("<BI", flag, len(records)) + b"".join(records)


def fno1d_weights(rng: np.random.Generator, in_ch: int, out_ch: int, width: int, modes: int,
                  n_layers: int) -> Dict[str, np.ndarray]:
    """The FNO1d weight sequence LoadBinary reads (ir_loader.h:283-305)."""
    f = lambda *s: rng.uniform(-0.5, 0.5, s).astype(np.float32)
    w = {"lift.weight": f(width, in_ch), "lift.bias": f(width)}
    for i in range(n_layers):
        w[f"specs.{i}.weights_real"] = f(width, width, modes)
        w[f"specs.{i}.weights_imag"] = f(width, width, modes)
        w[f"locs.{i}.weight"] = f(width, width)
        w[f"locs.{i}.bias"] = f(width)
    w["proj_q.weight"] = f(width, width)
    w["proj_q.bias"] = f(width)
    w["proj_out.weight"] = f(out_ch, width)
    w["proj_out.bias"] = f(out_ch)
    return w


def fno1d_file(weights: Dict[str, np.ndarray], cfg: Sequence[int], qrecords: List[bytes] | None = None,
               act: int = 0, version: int = 3) -> bytes:
    out = header(1, cfg, act, version, len(weights))
    out += b"".join(weight_record(k, v) for k, v in weights.items())
    if qrecords is not None:
        out += nirq(qrecords)
    return out


def fno2d_weights(rng: np.random.Generator, in_ch: int, out_ch: int, width: int, modes_h: int, modes_w: int,
                  n_layers: int) -> Dict[str, np.ndarray]:
    """The FNO2d weight sequence LoadBinary reads (ir_loader.h:298-322)."""
    f = lambda *s: rng.uniform(-0.5, 0.5, s).astype(np.float32)
    w = {"lift.weight": f(width, in_ch), "lift.bias": f(width)}
    for i in range(n_layers):
        w[f"specs.{i}.weights_real"] = f(width, width, modes_h, modes_w)
        w[f"specs.{i}.weights_imag"] = f(width, width, modes_h, modes_w)
        w[f"locs.{i}.weight"] = f(width, width)
        w[f"locs.{i}.bias"] = f(width)
    w["proj_q.weight"] = f(width, width)
    w["proj_q.bias"] = f(width)
    w["proj_out.weight"] = f(out_ch, width)
    w["proj_out.bias"] = f(out_ch)
    return w


def fno2d_file(weights: Dict[str, np.ndarray], cfg: Sequence[int], qrecords: List[bytes] | None = None,
               act: int = 0, version: int = 3) -> bytes:
    out = header(2, cfg, act, version, len(weights))
    out += b"".join(weight_record(k, v) for k, v in weights.items())
    if qrecords is not None:
        out += nirq(qrecords)
    return out


def symmetric_per_channel(W: np.ndarray, qmax: float = 127.0) -> Tuple[np.ndarray, np.ndarray]:
    s = np.abs(W).max(axis=1).astype(np.float32) / np.float32(qmax)
    s[s == 0] = 1.0
    return s, np.zeros(W.shape[0], np.int32)
