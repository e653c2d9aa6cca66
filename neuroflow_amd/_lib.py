"""ctypes binding of libnflow_quant.so (include/nflow_quant.h, include/nflow_runtime.h).

The library is loaded from neuroflow_amd/lib/ (built in-tree by
`python -m neuroflow_amd.build`).  There is no fallback: if the library is
missing or lacks a symbol, loading raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import os

# The in-tree build; NFLOW_QUANT_LIB may name another build of the same sources.
LIB_PATH = Path(os.environ.get("NFLOW_QUANT_LIB") or
               Path(__file__).resolve().parent / "lib" / "libnflow_quant.so")

# nflow::StatusCode (cpp/include/neuroflow/tensor.h:29-37).
OK, INVALID_ARG, FILE_NOT_FOUND, PARSE_ERROR, SHAPE_MISMATCH, UNSUPPORTED_OP, INTERNAL = (
    0, 1, 2, 3, 4, 5, 99)
STATUS_NAMES = {0: "Ok", 1: "InvalidArg", 2: "FileNotFound", 3: "ParseError",
                4: "ShapeMismatch", 5: "UnsupportedOp", 99: "Internal"}

ACT_NONE, ACT_RELU, ACT_GELU_TANH = 0, 1, 2
FORMAT_INT8, FORMAT_FP8_E4M3 = 0, 1


class Int8LinearParamsC(C.Structure):
    """nflow_int8_linear_params (device pointers)."""

    _fields_ = [
        ("W_int8", C.c_void_p),
        ("scale_W", C.c_void_p),
        ("zp_W", C.c_void_p),
        ("bias", C.c_void_p),
        ("in_features", C.c_int),
        ("out_features", C.c_int),
        ("scale_A", C.c_float),
        ("zp_A", C.c_int32),
        ("sum_W_per_row", C.c_void_p),
    ]


class Fp8LinearParamsC(C.Structure):
    """nflow_fp8_linear_params (device pointers)."""

    _fields_ = [
        ("W_e4m3", C.c_void_p),
        ("scale_W", C.c_void_p),
        ("bias", C.c_void_p),
        ("in_features", C.c_int),
        ("out_features", C.c_int),
    ]


class X2QuantC(C.Structure):
    """nflow_x2_quant (include/nflow_quant.h)."""
    _fields_ = [
        ("kind", C.c_int),
        ("scale", C.c_float),
        ("zero_point", C.c_int32),
        ("scales", C.c_void_p),
        ("zero_points", C.c_void_p),
        ("n_positions", C.c_int64),
        ("width", C.c_int32),
        ("points", C.c_int32),
    ]


X2_NONE, X2_PER_TENSOR, X2_PER_POSITION, X2_FP8_LOG2 = 0, 1, 2, 3

_vp, _i64, _i32, _f32 = C.c_void_p, C.c_int64, C.c_int, C.c_float
_P8 = C.POINTER(Int8LinearParamsC)
_PF8 = C.POINTER(Fp8LinearParamsC)

# name -> argtypes; every function returns int (status) unless listed in _RESTYPES.
SIGNATURES = {
    "nflow_quant_abi_version": [],
    "nflow_last_error": [],
    "nflow_debug_set_kernel_path": [C.c_char_p, _i32, C.POINTER(C.c_int)],
    "nflow_int8_quantise_activation": [_vp, _vp, _i64, _i32, _f32, C.c_int32, _vp],
    "nflow_int8_precompute_sum_w": [_vp, _vp, _i32, _i32, _vp, _vp],
    "nflow_int8_linear_forward": [_P8, _vp, _vp, _vp],
    "nflow_int8_linear_forward_rows": [_P8, _i64, _vp, _vp, _vp],
    "nflow_int8_linear_forward_batched": [_P8, _i64, _vp, _vp, _vp],
    "nflow_int8_quantise_per_token": [_vp, _i64, _i32, _vp, _vp, _vp, _vp],
    "nflow_int8_linear_forward_per_token": [_P8, _i64, _vp, _vp, _vp, _i32, _vp],
    "nflow_int8_linear_forward_per_token_noalloc": [_P8, _i64, _vp, _vp, _vp, _i32, _vp],
    "nflow_int8_fno_layer_per_token": [_P8, _i64, _vp, _vp, _vp, _vp, _i32, _vp],
    "nflow_int8_fno_layer_per_token_x2q": [_P8, _i64, _vp, _vp, _vp, _vp, _i32, C.POINTER(X2QuantC), _vp],
    "nflow_int8_gemm_i32": [_vp, _vp, _i64, _i32, _i32, _vp, _vp],
    "nflow_int8_linear_forward_quantised": [_P8, _i64, _vp, _vp, _vp, _i32, _vp],
    "nflow_int8_linear_forward_codes": [_P8, _i64, _vp, _vp, _vp, _vp, _i32, _vp],
    "nflow_int8_mlp_forward_per_token": [_P8, C.POINTER(C.c_int), _i32, _i64, _vp, _vp, _vp],
    "nflow_debug_chain_faults": [_vp, C.POINTER(C.c_uint32)],
    "nflow_release_stream_workspace": [_vp],
    "nflow_fp8_e4m3_to_bits": [_vp, _vp, _i64, _vp],
    "nflow_fp8_e4m3_from_bits": [_vp, _vp, _i64, _vp],
    "nflow_fp8_e4m3_fake_quant": [_vp, _f32, _vp, _i64, _vp],
    "nflow_fp8_quantise_per_token": [_vp, _i64, _i32, _vp, _vp, _vp],
    "nflow_fp8_linear_forward_per_token": [_PF8, _i64, _vp, _vp, _vp, _i32, _vp],
    "nflow_fp8_fno_layer_per_token": [_PF8, _i64, _vp, _vp, _vp, _vp, _i32, _vp],
    "nflow_fp8_fno_layer_per_token_x2q": [_PF8, _i64, _vp, _vp, _vp, _vp, _i32, C.POINTER(X2QuantC), _vp],
    "nflow_fp8_gemm_f32": [_vp, _vp, _i64, _i32, _i32, _vp, _vp],
    "nflow_fp8_linear_forward_quantised": [_PF8, _i64, _vp, _vp, _vp, _i32, _vp],
    "nflow_host_quantise_weight_2d": [_vp, _i32, _i32, _vp, _vp, _vp, _vp],
    "nflow_host_per_channel_scales": [_vp, _i32, _i32, _f32, _vp],
    "nflow_host_fp8_quantise_weight": [_vp, _i32, _i32, _vp, _vp],
    "nflow_layer_create": [_vp, _vp, _i32, _i32, _i32, C.POINTER(_vp)],
    "nflow_layer_create_int8": [_vp, _vp, _vp, _vp, _vp, _i32, _i32, C.POINTER(_vp)],
    "nflow_layer_forward": [_vp, _i64, _vp, _vp, _vp, _i32, _vp],
    "nflow_layer_forward_residual": [_vp, _i64, _vp, _vp, _vp, _vp, _i32, _vp],
    "nflow_layer_forward_fno": [_vp, _i64, _vp, _vp, _vp, _vp, _i32, C.POINTER(X2QuantC), _vp],
    "nflow_layer_forward_per_tensor": [_vp, _i64, _vp, _vp, _f32, C.c_int32, _vp],
    "nflow_layer_shape": [_vp, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_i32)],
    "nflow_layer_destroy": [_vp],
    "nflow_ir_open": [C.c_char_p, C.POINTER(_vp)],
    "nflow_ir_open_memory": [_vp, C.c_size_t, C.POINTER(_vp)],
    "nflow_ir_close": [_vp],
    "nflow_ir_header": [_vp, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(C.c_int32), C.POINTER(_i32),
                        C.POINTER(_i32)],
    "nflow_ir_num_weights": [_vp, C.POINTER(_i32)],
    "nflow_ir_weight_at": [_vp, _i32, C.POINTER(C.c_char_p), C.POINTER(_i32), C.POINTER(C.c_int64),
                           C.POINTER(_vp)],
    "nflow_ir_weight": [_vp, C.c_char_p, C.POINTER(_i32), C.POINTER(C.c_int64), C.POINTER(_vp)],
    "nflow_ir_num_qparams": [_vp, C.POINTER(_i32)],
    "nflow_ir_qparam_at": [_vp, _i32, C.POINTER(C.c_char_p), C.POINTER(_i32)],
    "nflow_ir_per_tensor_qparam": [_vp, C.c_char_p, C.POINTER(_i32), C.POINTER(C.c_float),
                                   C.POINTER(C.c_int32)],
    "nflow_ir_per_channel_qparam": [_vp, C.c_char_p, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_i32),
                                    C.POINTER(_vp), C.POINTER(_vp)],
    "nflow_ir_per_token_qparam": [_vp, C.c_char_p, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_i32),
                                  C.POINTER(_vp), C.POINTER(_vp)],
    "nflow_ir_fp8_qparam": [_vp, C.c_char_p, C.POINTER(_i32), C.POINTER(C.c_float)],
    "nflow_ir_layer_create": [_vp, C.c_char_p, C.c_char_p, C.POINTER(_vp)],
    "nflow_ir_fno_int8_dispatch": [_vp, _i32, C.POINTER(_i32), C.POINTER(C.c_float), C.POINTER(C.c_int32)],
    "nflow_ir_fno_x2_quant": [_vp, _i32, C.POINTER(X2QuantC)],
    # include/nflow_runtime.h
    "nflow_runtime_create": [C.c_char_p, C.POINTER(_vp)],
    "nflow_runtime_create_memory": [_vp, C.c_size_t, C.POINTER(_vp)],
    "nflow_runtime_destroy": [_vp],
    "nflow_runtime_op": [_vp],
    "nflow_runtime_config": [_vp, C.POINTER(C.c_int32), C.POINTER(_i32), C.POINTER(_i32)],
    "nflow_runtime_enable_int8_gemm": [_vp],
    "nflow_runtime_enable_int8_gemm_fno2d": [_vp],
    "nflow_runtime_is_int8_gemm_enabled": [_vp, C.POINTER(_i32)],
    "nflow_runtime_layer_dispatch": [_vp, _i32, C.POINTER(_i32)],
    "nflow_runtime_run": [_vp, _vp, C.POINTER(C.c_int64), _i32, _vp, C.POINTER(C.c_int64), _i32],
    "nflow_runtime_run_device": [_vp, _vp, C.POINTER(C.c_int64), _i32, _vp, C.POINTER(C.c_int64), _i32, _vp],
}
_RESTYPES = {"nflow_last_error": C.c_char_p, "nflow_runtime_op": C.c_char_p}

_lib = None


class NflowError(RuntimeError):
    """A non-OK status from libnflow_quant (the pybind module raises
    RuntimeError for a failed Status, pybind_module.cpp:189-191)."""

    def __init__(self, code: int, what: str, msg: str):
        super().__init__(f"{what} failed ({STATUS_NAMES.get(code, code)}): {msg}")
        self.code = code


def lib():
    """Load libnflow_quant.so once; raise if it is absent or incomplete."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m neuroflow_amd.build` "
                "(there is no CPU fallback)")
        L = C.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)  # AttributeError if a symbol is missing
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, C.c_int)
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != OK:
        msg = lib().nflow_last_error().decode(errors="replace")
        raise NflowError(rc, what, msg)
