"""The C-ABI library (no GPU needed): it loads, exports every entry point
include/nflow_quant.h declares, the ctypes table matches the header, status
codes equal nflow::StatusCode, and the host-side weight-blob builders match
the oracle bit for bit."""
import re
from pathlib import Path

import numpy as np
import pytest

from neuroflow_amd import _lib
from neuroflow_amd import quant as Q
from neuroflow_amd import workloads as WL
from oracle import oracle as O

INCLUDE = Path(__file__).resolve().parents[1] / "include"
HEADER = INCLUDE / "nflow_quant.h"


def declared_functions():
    names = set()
    for h in sorted(INCLUDE.glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = text.split("#ifdef __cplusplus\n}")[0]     # the C-ABI part (C++ wrappers follow it)
        names |= set(re.findall(r"\b(nflow_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_expected_surface():
    names = declared_functions()
    assert len(names) >= 20
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_functions():
        assert hasattr(L, name), name


def test_abi_version_and_status_values():
    assert _lib.lib().nflow_quant_abi_version() == 3
    text = HEADER.read_text()
    # nflow::StatusCode, cpp/include/neuroflow/tensor.h:29-37
    for name, val in [("NFLOW_OK", 0), ("NFLOW_INVALID_ARG", 1), ("NFLOW_FILE_NOT_FOUND", 2),
                      ("NFLOW_PARSE_ERROR", 3), ("NFLOW_SHAPE_MISMATCH", 4),
                      ("NFLOW_UNSUPPORTED_OP", 5), ("NFLOW_INTERNAL", 99)]:
        assert re.search(rf"\b{name}\s*=\s*{val}\b", text), name


def test_host_weight_quantise_matches_oracle():
    W = WL.uniform(40, (96, 200), -0.3, 0.3)
    W[3] = 0.0
    W[4, 5] = np.nan
    s = Q.per_channel_scales(W, 127.0)
    s_ref = O.per_channel_scales(W, 127.0)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    zps = np.round(WL.uniform(41, (96,), -9, 9)).astype(np.int32)
    q, sw = Q.quantise_weight_2d(W, s_ref, zps)
    q_ref, sw_ref = O.quantise_weight_2d(W, s_ref, zps)
    assert np.array_equal(q, q_ref) and np.array_equal(sw, sw_ref)


def test_host_fp8_weight_blob_matches_oracle():
    W = WL.uniform(42, (64, 128), -0.2, 0.2)
    W[0] = 0.0
    W[1, :3] = [1e-9, -1e-9, 0.5]
    q, s = Q.fp8_quantise_weight(W)
    q_ref, s_ref = O.quantise_weight_fp8(W)
    assert np.array_equal(q, q_ref) and np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))


def test_host_entry_points_reject_bad_arguments():
    with pytest.raises(_lib.NflowError) as ei:
        Q.per_channel_scales(np.zeros((0, 4), np.float32), 127.0)
    assert ei.value.code == _lib.INVALID_ARG
    assert b"bad dims" in _lib.lib().nflow_last_error()


def test_layer_handles_reject_bad_arguments():
    """Argument checks of the layer-handle entry points run before any device
    call (null pointers, dims, format), returning InvalidArg as the
    reference's checks do (int8_gemm.cpp:203-208)."""
    import ctypes as C
    L = _lib.lib()
    h = C.c_void_p(1234)
    W = np.ones((4, 8), np.float32)
    wp = W.ctypes.data_as(C.c_void_p)
    assert L.nflow_layer_create(None, None, 4, 8, 0, C.byref(h)) == _lib.INVALID_ARG
    assert h.value is None                     # the handle is cleared on failure
    assert L.nflow_layer_create(wp, None, 0, 8, 0, C.byref(h)) == _lib.INVALID_ARG
    assert L.nflow_layer_create(wp, None, 4, -1, 0, C.byref(h)) == _lib.INVALID_ARG
    assert L.nflow_layer_create(wp, None, 4, 8, 7, C.byref(h)) == _lib.INVALID_ARG
    assert b"format" in L.nflow_last_error()
    assert L.nflow_layer_create(wp, None, 4, 8, 0, None) == _lib.INVALID_ARG
    assert L.nflow_layer_create_int8(None, None, None, None, None, 4, 8, C.byref(h)) == _lib.INVALID_ARG
    assert L.nflow_layer_forward(None, 10, None, None, None, 0, None) == _lib.INVALID_ARG
    assert L.nflow_layer_shape(None, None, None, None) == _lib.INVALID_ARG
    assert L.nflow_layer_destroy(None) == _lib.OK


def test_noalloc_rejects_a_workspace_beyond_its_scratch_on_the_host():
    """nflow_int8_linear_forward_per_token_noalloc checks the split path's
    workspace (codes + scales + sums) against its static scratch before any
    device call: a shape that needs more returns InvalidArg with the sizes.
    (Dummy, never dereferenced pointers: nothing reaches the device.)"""
    import ctypes as C
    L = _lib.lib()
    cap = 72 << 20
    K = N = 1024
    M = cap // K + 1                        # the codes alone exceed the scratch
    dummy = 1 << 20                         # 16-byte aligned, never dereferenced
    p = _lib.Int8LinearParamsC(C.c_void_p(dummy), C.c_void_p(dummy), C.c_void_p(dummy), None, K, N, 1.0, 0, None)
    rc = L.nflow_int8_linear_forward_per_token_noalloc(C.byref(p), M, dummy, dummy, None, 1, None)
    assert rc == _lib.INVALID_ARG
    msg = L.nflow_last_error().decode()
    assert "noalloc" in msg and str(cap) in msg and "scratch" in msg
    # The scales count too when scale_A_out is not given: M * K just under
    # the cap, plus 4M scales and 4M row sums (zero points), is over it.
    M2 = (cap - 16) // (K + 8) + 1
    assert M2 * K <= cap - 16
    rc = L.nflow_int8_linear_forward_per_token_noalloc(C.byref(p), M2, dummy, dummy, None, 1, None)
    assert rc == _lib.INVALID_ARG
