"""The NeuroIR binary + NIRQ reader of libnflow_quant (host code, no GPU):
header, weight records and every qparam kind against the writer, the error
statuses of ir_native::LoadBinary (cpp/include/neuroflow/ir_loader.h:58-654),
and -- where oracle/_ref is built -- record-for-record agreement with the
reference's own reader on whole files and on every truncation of one."""
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from neuroflow_amd import _lib
from neuroflow_amd.ir import IR
from tests import nir_format as F

REF_DUMP = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "ref_ir_dump"


def _fno1d(seed=0, n_layers=2, width=8, quant=True, extra_records=()):
    rng = np.random.default_rng(seed)
    w = F.fno1d_weights(rng, 2, 1, width, 3, n_layers)
    cfg = [2, 1, width, 3, n_layers, 1, 0]
    recs = None
    if quant:
        recs = [F.qparam_record(0, "lift.output", 0.02, 3), F.qparam_record(0, "lift.weight", 0.01, 0)]
        for i in range(n_layers):
            s, z = F.symmetric_per_channel(w[f"locs.{i}.weight"])
            z = z + (np.arange(width) % 3 - 1).astype(np.int32) * (i % 2)
            recs.append(F.qparam_record(1, f"locs.{i}.weight", s, z, 0))
            recs.append(F.qparam_record(0, f"locs.{i}.output", 0.05 + i, -2 * i))
        recs.append(F.qparam_record(2, "proj_q.output", rng.uniform(0.01, 0.1, 5).astype(np.float32),
                                    np.arange(5, dtype=np.int32) - 2, width))
        recs.append(F.qparam_record(3, "proj_out.output", 0.125))
        recs += list(extra_records)
    return F.fno1d_file(w, cfg, recs), w


def _status(data: bytes) -> int:
    import ctypes as C
    h = C.c_void_p()
    buf = C.create_string_buffer(data, len(data))
    rc = _lib.lib().nflow_ir_open_memory(buf, len(data), C.byref(h))
    if rc == 0:
        _lib.lib().nflow_ir_close(h)
    return rc


def test_header_weights_and_qparams_round_trip():
    data, w = _fno1d()
    ir = IR(data=data)
    assert (ir.version, ir.op, ir.activation, ir.quant_enabled) == (3, "FNO1d", "gelu", True)
    assert ir.config[:7] == [2, 1, 8, 3, 2, 1, 0]
    assert ir.weight_names() == list(w)
    for k, v in w.items():
        got = ir.weight(k)
        assert got.shape == v.shape and np.array_equal(got.view(np.uint32), v.view(np.uint32))
    assert ir.per_tensor("lift.output") == (np.float32(0.02), 3)
    assert ir.per_tensor("lift.weight") == (np.float32(0.01), 0)
    s, z, ax = ir.per_channel("locs.1.weight")
    s_ref, _ = F.symmetric_per_channel(w["locs.1.weight"])
    assert ax == 0 and np.array_equal(s, s_ref) and np.array_equal(z, (np.arange(8) % 3 - 1))
    sc, zp, width = ir.per_token("proj_q.output")
    assert width == 8 and sc.shape == (5,) and np.array_equal(zp, np.arange(5) - 2)
    assert ir.fp8("proj_out.output") == 0.125
    assert ir.per_tensor("nope.output") is None and ir.per_channel("lift.weight") is None
    kinds = dict(ir.qparam_records())
    assert kinds["proj_q.output"] == "per_token" and kinds["locs.0.weight"] == "per_channel"
    ir.close()


def test_file_open_and_no_quant_block(tmp_path):
    data, _ = _fno1d(quant=False)
    p = tmp_path / "m.nneuroir"
    p.write_bytes(data + b"trailing bytes that are not a NIRQ block")
    with IR(p) as ir:
        assert not ir.quant_enabled and ir.op == "FNO1d"
    with pytest.raises(_lib.NflowError) as e:
        IR(tmp_path / "missing.nneuroir")
    assert e.value.code == _lib.FILE_NOT_FOUND


@pytest.mark.parametrize("mutate,code", [
    (lambda d: b"NIR1" + d[4:], 3),                                   # bad magic
    (lambda d: d[:4] + struct.pack("<H", 4) + d[6:], 3),               # version 4
    (lambda d: d[:4] + struct.pack("<H", 0) + d[6:], 3),               # version 0
    (lambda d: d[:6] + bytes([9]) + d[7:], 5),                         # unknown op code
    (lambda d: d[:6] + bytes([0]) + d[7:], 5),
])
def test_header_errors(mutate, code):
    data, _ = _fno1d(quant=False)
    assert _status(mutate(data)) == code


def test_nirq_errors():
    data, _ = _fno1d(quant=False)
    assert _status(data + F.nirq([], flag=0)) == 3                       # quant_flag != 1
    assert _status(data + F.nirq([], flag=1)) == 0
    bad = F.qparam_record(0, "x.output", 1.0, 0)
    bad = bytes([7]) + bad[1:]                                           # unknown kind
    assert _status(data + F.nirq([bad])) == 3


def test_last_record_of_a_name_wins():
    data, _ = _fno1d(extra_records=[F.qparam_record(0, "lift.output", 0.5, -7)])
    with IR(data=data) as ir:
        assert ir.per_tensor("lift.output") == (0.5, -7)
        assert [r for r in ir.qparam_records() if r[0] == "lift.output"] == [("lift.output", "per_tensor")] * 2


def test_every_truncation_is_a_parse_error_or_ok_before_the_block():
    data, _ = _fno1d(n_layers=1, width=4)
    core = F.fno1d_file(F.fno1d_weights(np.random.default_rng(0), 2, 1, 4, 3, 1), [2, 1, 4, 3, 1, 1, 0])
    for cut in range(len(data)):
        rc = _status(data[:cut])
        # A file cut inside the weights fails; one cut anywhere before the
        # 4-byte "NIRQ" magic is complete reads as a model without quantisation.
        if cut < len(core):
            assert rc == 3, cut
        elif cut < len(core) + 4:
            assert rc == 0, cut
        else:
            assert rc == 3, cut
    assert _status(data) == 0


def test_fno_int8_dispatch_rule():
    """LinearDispatchTryInt8 (fno.cpp:125-159, 529-536): INT8 for locs.{i} iff
    its input key has a per-tensor qparam and no per-token / FP8 qparam, and
    locs.{i}.weight has axis-0 per-channel qparams on a 2-D weight."""
    rng = np.random.default_rng(3)
    w = F.fno1d_weights(rng, 2, 1, 8, 3, 4)
    s, z = F.symmetric_per_channel(w["locs.0.weight"])
    recs = [F.qparam_record(0, "lift.output", 0.02, 1),
            F.qparam_record(1, "locs.0.weight", s, z, 0),
            F.qparam_record(1, "locs.1.weight", s, z, 0),           # input locs.0.output has no qparam
            F.qparam_record(0, "locs.1.output", 0.03, 0),
            F.qparam_record(1, "locs.2.weight", s, z, 0),
            F.qparam_record(2, "locs.1.output", s, z, 8),            # per-token input -> FP32
            F.qparam_record(0, "locs.2.output", 0.04, 0),
            F.qparam_record(1, "locs.3.weight", s, z, 1)]            # channel axis 1 -> not cached
    with IR(data=F.fno1d_file(w, [2, 1, 8, 3, 4, 1, 0], recs)) as ir:
        assert ir.fno_int8_dispatch(0) == (np.float32(0.02), 1)
        assert ir.fno_int8_dispatch(1) is None
        assert ir.fno_int8_dispatch(2) is None
        assert ir.fno_int8_dispatch(3) is None
        assert ir.fno_int8_dispatch(7) is None
    recs_fp8 = recs[:2] + [F.qparam_record(3, "lift.output", 0.5)]
    with IR(data=F.fno1d_file(w, [2, 1, 8, 3, 4, 1, 0], recs_fp8)) as ir:
        assert ir.fno_int8_dispatch(0) is None


# ---- against the reference's own reader (oracle/_ref, built from the sources) ----

def _our_dump(data: bytes) -> str:
    import ctypes as C
    rc = _status(data)
    lines = [f"status {rc}"]
    if rc != 0:
        return "\n".join(lines)
    ir = IR(data=data)
    lines.append(f"op {ir.op} activation {ir.activation} quant {int(ir.quant_enabled)}")
    lines.append("cfg " + " ".join(str(c) for c in ir.config[:6]))
    for name in ir.weight_names():
        a = ir.weight(name)
        h = 1469598103934665603
        for b in a.tobytes():
            h = ((h ^ b) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
        lines.append(f"weight {name} {a.ndim} " + " ".join(str(d) for d in a.shape) + f" {h:016x}")
    names = sorted({n for n, _ in ir.qparam_records()})
    bits = lambda f: f"{np.float32(f).view(np.uint32):08x}"
    for n in names:
        q = ir.per_tensor(n)
        if q is not None and n.endswith(".output"):
            lines.append(f"act_pt {n} {bits(q[0])} {q[1]}")
    for n in names:
        q = ir.per_tensor(n)
        if q is not None and not n.endswith(".output"):
            lines.append(f"w_pt {n} {bits(q[0])} {q[1]}")
    for n in names:
        q = ir.per_channel(n)
        if q is not None:
            lines.append(f"pc {n} {q[2]} {len(q[0])}" + "".join(f" {bits(s)}" for s in q[0])
                         + "".join(f" {z}" for z in q[1]))
    for n in names:
        q = ir.per_token(n)
        if q is not None:
            lines.append(f"pt {n} {q[2]} {len(q[0])}" + "".join(f" {bits(s)}" for s in q[0])
                         + "".join(f" {z}" for z in q[1]))
    for n in names:
        q = ir.fp8(n)
        if q is not None:
            lines.append(f"fp8 {n} {bits(q)}")
    ir.close()
    return "\n".join(lines)


def _ref_dump(data: bytes, tmp_path: Path) -> str:
    p = tmp_path / "f.nneuroir"
    p.write_bytes(data)
    out = subprocess.run([str(REF_DUMP), str(p)], capture_output=True, text=True, check=True).stdout
    return out.strip()


needs_ref = pytest.mark.skipif(not REF_DUMP.exists(), reason="oracle/_ref/ref_ir_dump not built")


@needs_ref
@pytest.mark.parametrize("seed,n_layers,width,act", [(0, 1, 4, 0), (1, 2, 8, 1), (2, 4, 16, 0)])
def test_reader_matches_reference_loader(tmp_path, seed, n_layers, width, act):
    rng = np.random.default_rng(seed)
    w = F.fno1d_weights(rng, 3, 2, width, 5, n_layers)
    recs = [F.qparam_record(0, "lift.output", float(rng.uniform(0.01, 1)), int(rng.integers(-9, 9)))]
    for i in range(n_layers):
        s, z = F.symmetric_per_channel(w[f"locs.{i}.weight"])
        recs.append(F.qparam_record(1, f"locs.{i}.weight", s, z + i, i % 2))
        recs.append(F.qparam_record(0, f"locs.{i}.output", float(rng.uniform(0.01, 1)), i))
        recs.append(F.qparam_record(0, f"locs.{i}.weight", 0.25, 0))
    recs.append(F.qparam_record(2, "proj_q.output", rng.uniform(0.01, 1, 7).astype(np.float32),
                                rng.integers(-5, 5, 7).astype(np.int32), width))
    recs.append(F.qparam_record(3, "proj_out.output", 0.375))
    recs.append(F.qparam_record(0, "lift.output", 0.5, 1))           # duplicate: last wins
    data = F.fno1d_file(w, [3, 2, width, 5, n_layers, 2, 0], recs, act=act, version=1 + seed % 3)
    assert _our_dump(data) == _ref_dump(data, tmp_path)


@needs_ref
def test_status_matches_reference_on_every_truncation(tmp_path):
    data, _ = _fno1d(n_layers=1, width=4)
    for cut in list(range(0, 64)) + list(range(64, len(data), 7)) + [len(data) - 1, len(data)]:
        assert _our_dump(data[:cut]).splitlines()[0] == _ref_dump(data[:cut], tmp_path).splitlines()[0], cut


@needs_ref
@pytest.mark.parametrize("mutate", [
    lambda d: b"NIR1" + d[4:],
    lambda d: d[:4] + struct.pack("<H", 4) + d[6:],
    lambda d: d[:6] + bytes([9]) + d[7:],
    lambda d: d + F.nirq([], flag=2),
    lambda d: d + F.nirq([bytes([5]) + F.qparam_record(0, "a.output", 1.0, 0)[1:]]),
    lambda d: d + b"NIRQ",
])
def test_errors_match_reference(tmp_path, mutate):
    data, _ = _fno1d(quant=False)
    bad = mutate(data)
    assert _our_dump(bad) == _ref_dump(bad, tmp_path)


# ---- the symmetric exporter (neuroflow_amd.ir.export_symmetric) -------------

def _sym_scale(a) -> np.float32:
    """fl32(a / 127) for a float32 a, through a float64 quotient: rounding a
    double quotient to float32 is the correctly rounded float32 quotient
    (53 >= 2 * 24 + 2); 1 for a zero range."""
    a = np.float32(a)
    return np.float32(1.0) if a == 0 else np.float32(np.float64(a) / 127.0)


def _exported(seed=3, n_layers=2, width=8):
    from neuroflow_amd import ir as IRM
    rng = np.random.default_rng(seed)
    w = F.fno1d_weights(rng, 2, 1, width, 3, n_layers)
    w["locs.0.weight"][2, :] = 0.0                      # a zero channel -> scale 1
    plain = F.fno1d_file(w, [2, 1, width, 3, n_layers, 1, 0], None)
    calib = rng.standard_normal((4, 16, width)).astype(np.float32) * 3
    acts = {"lift.output": calib, "locs.0.output": 2.5, "locs.1.output": 0.0}
    per_token = {"proj_q.output": (np.abs(rng.standard_normal(16 * width)).astype(np.float32), width)}
    fp8 = {"proj_out.output": 10.0}
    out = IRM.export_symmetric(plain, activations=acts, per_token=per_token, fp8_activations=fp8)
    return out, plain, w, calib, per_token


def test_export_symmetric_records_and_closed_form():
    out, plain, w, calib, per_token = _exported()
    ir, ir0 = IR(data=out), IR(data=plain)
    assert (ir.version, ir.op, ir.config, ir.activation) == (ir0.version, ir0.op, ir0.config, ir0.activation)
    assert ir.quant_enabled and not ir0.quant_enabled
    assert ir.weight_names() == ir0.weight_names()
    for n in ir.weight_names():
        assert np.array_equal(ir.weight(n).view(np.uint32), ir0.weight(n).view(np.uint32))
    two_d = [n for n, v in w.items() if v.ndim == 2 and n.endswith(".weight")]
    assert sorted(two_d) == sorted(n for n, k in ir.qparam_records() if k == "per_channel")
    for n in two_d:
        s, z, ax = ir.per_channel(n)
        want = [_sym_scale(np.abs(row).max()) for row in w[n]]
        assert ax == 0 and np.array_equal(s.view(np.uint32), np.asarray(want, np.float32).view(np.uint32)), n
        assert not z.any()
    assert ir.per_channel("locs.0.weight")[0][2] == 1.0
    assert ir.per_tensor("lift.output") == (_sym_scale(np.abs(calib).max()), 0)
    assert ir.per_tensor("locs.0.output") == (_sym_scale(2.5), 0)
    assert ir.per_tensor("locs.1.output") == (1.0, 0)
    sc, zp, width = ir.per_token("proj_q.output")
    am, wd = per_token["proj_q.output"]
    assert width == wd and not zp.any()
    assert np.array_equal(sc.view(np.uint32), np.asarray([_sym_scale(a) for a in am], np.float32).view(np.uint32))
    assert ir.fp8("proj_out.output") == np.float32(np.float64(np.float32(10.0)) / 448.0)
    ir.close()
    ir0.close()


def test_export_symmetric_replaces_an_earlier_block():
    from neuroflow_amd import ir as IRM
    data, w = _fno1d(quant=True)
    out = IRM.export_symmetric(data, activations={"lift.output": 1.0})
    with IR(data=out) as ir:
        assert ir.per_tensor("lift.output") == (_sym_scale(1.0), 0)
        assert ir.per_tensor("locs.0.output") is None and ir.fp8("proj_out.output") is None
        assert not ir.per_channel("locs.1.weight")[1].any()


def test_export_symmetric_codes_reach_127():
    """QuantiseWeight2D (fno.cpp:340-356, the library's host restatement) on
    the exported qparams: codes within [-127, 127], +-127 exactly where a
    channel's absmax is, and the host's per-channel scales agree."""
    from neuroflow_amd import quant as Q
    out, _, w, _, _ = _exported(seed=5, width=16)
    with IR(data=out) as ir:
        for n in ("lift.weight", "locs.1.weight", "proj_q.weight"):
            s, z, _ = ir.per_channel(n)
            q, _ = Q.quantise_weight_2d(w[n], s, z)
            nz = np.abs(w[n]).max(axis=1) > 0
            assert np.abs(q).max() <= 127
            assert np.array_equal(np.abs(q).max(axis=1)[nz], np.full(nz.sum(), 127))
            assert np.array_equal(Q.per_channel_scales(w[n], 127.0)[nz], s[nz])


@needs_ref
def test_export_symmetric_matches_reference_loader(tmp_path):
    out, _, _, _, _ = _exported(seed=7, n_layers=3, width=12)
    assert _our_dump(out) == _ref_dump(out, tmp_path)
