"""ctypes front-end to the oracle (liboracle.so) and to the reference build
(oracle/_ref/libnflow_ref_*.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, and there only as the reference results / the CPU baseline.
The product never imports this module.

All arrays are numpy, C-contiguous, host memory.
"""
from __future__ import annotations

import ctypes as C
import os
import platform
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ACT_NONE, ACT_RELU, ACT_GELU_TANH = 0, 1, 2


class LinearParams(C.Structure):
    """Host-pointer mirror of int8_gemm.h:45-65 (Int8LinearParams)."""

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


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def make_params(W_q, scale_W, zp_W, bias=None, scale_A=1.0, zp_A=0, sum_W=None):
    """Build a LinearParams; the returned tuple keeps the arrays alive."""
    W_q = np.ascontiguousarray(W_q, dtype=np.int8)
    scale_W = np.ascontiguousarray(scale_W, dtype=np.float32)
    zp_W = np.ascontiguousarray(zp_W, dtype=np.int32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    sum_W = None if sum_W is None else np.ascontiguousarray(sum_W, dtype=np.int32)
    p = LinearParams(_ptr(W_q), _ptr(scale_W), _ptr(zp_W), _ptr(bias),
                     W_q.shape[1], W_q.shape[0], float(scale_A), int(zp_A), _ptr(sum_W))
    return p, (W_q, scale_W, zp_W, bias, sum_W)


def _load(path: Path):
    if not path.exists():
        raise FileNotFoundError(f"{path} not built (run `make -C oracle`)")
    return C.CDLL(str(path))


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load(HERE / "liboracle.so")
        L = _lib
        vp, i64, i32, f32, sz = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_size_t
        L.orc_quantise_one.restype = C.c_int8
        L.orc_quantise_one.argtypes = [f32, f32, C.c_int32]
        L.orc_quantise_activation.argtypes = [vp, vp, i64, i32, f32, C.c_int32]
        L.orc_per_token_scales.argtypes = [vp, i64, i32, f32, vp]
        L.orc_quantise_per_token_i8.argtypes = [vp, i64, i32, vp, vp, vp]
        L.orc_quantise_weight_2d.argtypes = [vp, i32, i32, vp, vp, vp, vp]
        L.orc_per_channel_scales.argtypes = [vp, i32, i32, f32, vp]
        L.orc_precompute_sum_w.argtypes = [vp, vp, i32, i32, vp]
        L.orc_gemm_i8_i32.argtypes = [vp, vp, i64, i32, i32, vp]
        L.orc_linear_forward_batched.argtypes = [C.POINTER(LinearParams), i64, vp, vp]
        L.orc_linear_forward.argtypes = [C.POINTER(LinearParams), vp, vp]
        L.orc_apply_activation.argtypes = [vp, i64, i32]
        L.orc_x2_fake_quant.argtypes = [vp, vp, i64, i32, C.c_float, C.c_int32, vp, vp, i32]
        L.orc_layer_per_token_i8.argtypes = [C.POINTER(LinearParams), i64, vp, vp, i32, vp]
        L.orc_e4m3_encode.restype = C.c_uint8
        L.orc_e4m3_encode.argtypes = [f32]
        L.orc_e4m3_decode.restype = C.c_float
        L.orc_e4m3_decode.argtypes = [C.c_uint8]
        L.orc_e4m3_encode_array.argtypes = [vp, vp, sz]
        L.orc_e4m3_decode_array.argtypes = [vp, vp, sz]
        L.orc_fp8_fake_quant.argtypes = [vp, f32, vp, sz]
        L.orc_e4m3_encode_bits_range.argtypes = [C.c_uint32, C.c_uint32, vp]
        L.orc_e4m3_encode_bits_stride.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, vp]
        L.orc_fp8_quantise_one.restype = C.c_uint8
        L.orc_fp8_quantise_one.argtypes = [f32, f32]
        L.orc_quantise_per_token_fp8.argtypes = [vp, i64, i32, vp, vp]
        L.orc_quantise_weight_fp8.argtypes = [vp, i32, i32, vp, vp]
        L.orc_gemm_fp8_exact.argtypes = [vp, vp, i64, i32, i32, vp]
        L.orc_layer_fp8_composed.argtypes = [vp, vp, vp, i64, i32, i32, i32, vp, vp, vp]
        L.orc_layer_fp8_exact.argtypes = [vp, vp, vp, vp, vp, i64, i32, i32, i32, vp]
        L.orc_cfft.argtypes = [vp, i32, i32]
        L.orc_rfft.argtypes = [vp, i32, vp]
        L.orc_irfft.argtypes = [vp, i32, vp]
        L.orc_spectral_conv1d.argtypes = [vp, i32, i32, i32, i32, vp, vp, vp]
        L.orc_rfft2.argtypes = [vp, i32, i32, vp]
        L.orc_irfft2.argtypes = [vp, i32, i32, vp]
        L.orc_spectral_conv2d.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp]
        L.orc_linear_f32.argtypes = [vp, vp, vp, i64, i32, i32, vp]
        L.orc_fake_quant_arr.argtypes = [vp, vp, vp, vp, i64]
        L.orc_log2_snap_one.restype = f32
        L.orc_log2_snap_one.argtypes = [f32, f32]
        L.orc_log2_snap.argtypes = [vp, f32, vp, i64]
        L.orc_log2_snap_exponent.restype = i32
        L.orc_log2_snap_exponent.argtypes = [f32]
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- INT8 -------------------------------------------------------------------

def quantise_activation(A, scale_A, zp_A=0):
    A = _f32(A)
    out = np.empty(A.shape, dtype=np.int8)
    K = A.shape[-1] if A.ndim else 1
    lib().orc_quantise_activation(_ptr(A), _ptr(out), A.size // max(K, 1), K, scale_A, zp_A)
    return out


def per_token_scales(A, qmax):
    A = _f32(A)
    s = np.empty(A.shape[0], dtype=np.float32)
    lib().orc_per_token_scales(_ptr(A), A.shape[0], A.shape[1], qmax, _ptr(s))
    return s


def quantise_per_token_i8(A):
    A = _f32(A)
    M, K = A.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    sa = np.empty(M, np.int32)
    lib().orc_quantise_per_token_i8(_ptr(A), M, K, _ptr(q), _ptr(s), _ptr(sa))
    return q, s, sa


def per_channel_scales(W, qmax):
    W = _f32(W)
    s = np.empty(W.shape[0], np.float32)
    lib().orc_per_channel_scales(_ptr(W), W.shape[0], W.shape[1], qmax, _ptr(s))
    return s


def quantise_weight_2d(W, scales, zps=None):
    W = _f32(W)
    N, K = W.shape
    scales = _f32(scales)
    zps = np.zeros(N, np.int32) if zps is None else np.ascontiguousarray(zps, np.int32)
    q = np.empty((N, K), np.int8)
    sw = np.empty(N, np.int32)
    lib().orc_quantise_weight_2d(_ptr(W), N, K, _ptr(scales), _ptr(zps), _ptr(q), _ptr(sw))
    return q, sw


def precompute_sum_w(W_q, zp_W):
    W_q = np.ascontiguousarray(W_q, np.int8)
    zp_W = np.ascontiguousarray(zp_W, np.int32)
    out = np.empty(W_q.shape[0], np.int32)
    lib().orc_precompute_sum_w(_ptr(W_q), _ptr(zp_W), W_q.shape[1], W_q.shape[0], _ptr(out))
    return out


def gemm_i8_i32(A_q, W_q):
    A_q = np.ascontiguousarray(A_q, np.int8)
    W_q = np.ascontiguousarray(W_q, np.int8)
    M, K = A_q.shape
    N = W_q.shape[0]
    out = np.empty((M, N), np.int32)
    lib().orc_gemm_i8_i32(_ptr(A_q), _ptr(W_q), M, N, K, _ptr(out))
    return out


def linear_forward_batched(A, W_q, scale_W, zp_W, bias=None, scale_A=1.0, zp_A=0, sum_W=None):
    A = _f32(A)
    p, keep = make_params(W_q, scale_W, zp_W, bias, scale_A, zp_A, sum_W)
    M = A.shape[0]
    out = np.empty((M, p.out_features), np.float32)
    rc = lib().orc_linear_forward_batched(C.byref(p), M, _ptr(A), _ptr(out))
    del keep
    return rc, out


def linear_forward_rows(A, W_q, scale_W, zp_W, bias=None, scale_A=1.0, zp_A=0, sum_W=None):
    """LinearForward called once per row of A with the same parameters."""
    A = _f32(A)
    p, keep = make_params(W_q, scale_W, zp_W, bias, scale_A, zp_A, sum_W)
    M, K = A.shape
    out = np.empty((M, p.out_features), np.float32)
    L = lib()
    for m in range(M):
        rc = L.orc_linear_forward(C.byref(p), _ptr(A[m]), out[m].ctypes.data_as(C.c_void_p))
        if rc:
            return rc, out
    del keep
    return 0, out


def apply_activation(y, act):
    y = np.array(y, dtype=np.float32, copy=True, order="C")
    lib().orc_apply_activation(_ptr(y), y.size, act)
    return y


def x2_fake_quant(x2, scale=1.0, zp=0, scales=None, zps=None, points=0):
    """fno.cpp:572-648 on token-major x2 (M, N): per tensor, or per position
    (scales / zps of N * points entries, the reference's indexing)."""
    x2 = _f32(x2)
    out = np.empty_like(x2)
    sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
    zz = None if zps is None else np.ascontiguousarray(zps, np.int32)
    rc = lib().orc_x2_fake_quant(_ptr(x2), _ptr(out), x2.shape[0], x2.shape[1], float(scale), int(zp),
                                 None if sc is None else _ptr(sc), None if zz is None else _ptr(zz), int(points))
    if rc != 0:
        raise ValueError(f"orc_x2_fake_quant failed ({rc})")
    return out


def layer_per_token_i8(A, W_q, scale_W, zp_W=None, bias=None, sum_W=None, act=ACT_GELU_TANH):
    """Per-token INT8 layer: LinearForward per row with scale_A=absmax/127."""
    A = _f32(A)
    N = W_q.shape[0]
    zp_W = np.zeros(N, np.int32) if zp_W is None else zp_W
    p, keep = make_params(W_q, scale_W, zp_W, bias, 1.0, 0, sum_W)
    M = A.shape[0]
    out = np.empty((M, N), np.float32)
    sa = np.empty(M, np.float32)
    rc = lib().orc_layer_per_token_i8(C.byref(p), M, _ptr(A), _ptr(out), act, _ptr(sa))
    assert rc == 0, rc
    del keep
    return out, sa


# ---- FNO1d forward pieces -----------------------------------------------------

def rfft(x):
    """fft.cpp:72-84 on a 1-D float32 array of power-of-two length."""
    x = _f32(x)
    out = np.empty(2 * (x.size // 2 + 1), np.float32)
    lib().orc_rfft(_ptr(x), x.size, _ptr(out))
    return out


def irfft(xc, n):
    """fft.cpp:86-100: n/2 + 1 interleaved bins -> n reals."""
    xc = _f32(xc)
    assert xc.size == 2 * (n // 2 + 1)
    out = np.empty(n, np.float32)
    lib().orc_irfft(_ptr(xc), n, _ptr(out))
    return out


def spectral_conv1d(h, w_real, w_imag, modes):
    """fno.cpp:164-207: h (b, w, n) -> (b, w, n)."""
    h = _f32(h)
    b, w, n = h.shape
    wr, wi = _f32(w_real), _f32(w_imag)
    assert wr.shape == (w, w, modes) and wi.shape == wr.shape
    out = np.empty_like(h)
    lib().orc_spectral_conv1d(_ptr(h), b, w, n, modes, _ptr(wr), _ptr(wi), _ptr(out))
    return out


def rfft2(x):
    """fft.cpp:101-124 on an (H, W) float32 plane: (H, W/2 + 1, 2) bins."""
    x = _f32(x)
    H, W = x.shape
    out = np.empty((H, W // 2 + 1, 2), np.float32)
    lib().orc_rfft2(_ptr(x), H, W, _ptr(out))
    return out


def irfft2(xc, H, W):
    """fft.cpp:126-148: (H, W/2 + 1, 2) bins -> (H, W) reals."""
    xc = _f32(xc)
    assert xc.shape == (H, W // 2 + 1, 2)
    out = np.empty((H, W), np.float32)
    lib().orc_irfft2(_ptr(xc), H, W, _ptr(out))
    return out


def spectral_conv2d(h, w_real, w_imag, mh, mw):
    """fno.cpp:717-771: h (b, w, H, W) -> (b, w, H, W)."""
    h = _f32(h)
    b, w, H, W = h.shape
    wr, wi = _f32(w_real), _f32(w_imag)
    assert wr.shape == (w, w, mh, mw) and wi.shape == wr.shape
    out = np.empty_like(h)
    lib().orc_spectral_conv2d(_ptr(h), b, w, H, W, mh, mw, _ptr(wr), _ptr(wi), _ptr(out))
    return out


def linear_f32(x, W, b=None):
    """fno.cpp:69-79: x (rows, k) -> (rows, n), bias first, sequential over k."""
    x = _f32(x)
    W = _f32(W)
    bb = None if b is None else _f32(b)
    rows, k = x.shape
    n = W.shape[0]
    assert W.shape[1] == k
    y = np.empty((rows, n), np.float32)
    lib().orc_linear_f32(_ptr(x), _ptr(W), None if bb is None else _ptr(bb), rows, k, n, _ptr(y))
    return y


def fake_quant_elementwise(x, scales, zps):
    """The INT8 fake-quant round trip with per-element (broadcast) scales / zero points."""
    x = _f32(x)
    s = np.ascontiguousarray(np.broadcast_to(np.asarray(scales, np.float32), x.shape))
    z = np.ascontiguousarray(np.broadcast_to(np.asarray(zps, np.int32), x.shape))
    out = np.empty_like(x)
    lib().orc_fake_quant_arr(_ptr(x), _ptr(s), _ptr(z), _ptr(out), x.size)
    return out


def log2_snap(x, scale):
    """fno.cpp:579-606 (the log2 "FP8" snap of x2, per-tensor scale)."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_log2_snap(_ptr(x), float(scale), _ptr(out), x.size)
    return out


# ---- FP8 --------------------------------------------------------------------

def e4m3_encode(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint8)
    lib().orc_e4m3_encode_array(_ptr(x), _ptr(out), x.size)
    return out


def e4m3_decode(b):
    b = np.ascontiguousarray(b, np.uint8)
    out = np.empty(b.shape, np.float32)
    lib().orc_e4m3_decode_array(_ptr(b), _ptr(out), b.size)
    return out


def fp8_fake_quant(x, scale):
    x = _f32(x)
    out = np.empty(x.shape, np.float32)
    lib().orc_fp8_fake_quant(_ptr(x), scale, _ptr(out), x.size)
    return out


def e4m3_encode_bits_range(start, count):
    out = np.empty(count, np.uint8)
    lib().orc_e4m3_encode_bits_range(start, count, _ptr(out))
    return out


def e4m3_encode_bits_stride(start, stride, count):
    out = np.empty(count, np.uint8)
    lib().orc_e4m3_encode_bits_stride(start, stride, count, _ptr(out))
    return out


def quantise_per_token_fp8(A):
    A = _f32(A)
    M, K = A.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty(M, np.float32)
    lib().orc_quantise_per_token_fp8(_ptr(A), M, K, _ptr(q), _ptr(s))
    return q, s


def quantise_weight_fp8(W):
    W = _f32(W)
    N, K = W.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N, np.float32)
    lib().orc_quantise_weight_fp8(_ptr(W), N, K, _ptr(q), _ptr(s))
    return q, s


def gemm_fp8_exact(A_q, W_q):
    A_q = np.ascontiguousarray(A_q, np.uint8)
    W_q = np.ascontiguousarray(W_q, np.uint8)
    M, K = A_q.shape
    N = W_q.shape[0]
    out = np.empty((M, N), np.float64)
    lib().orc_gemm_fp8_exact(_ptr(A_q), _ptr(W_q), M, N, K, _ptr(out))
    return out


def layer_fp8_composed(A, W, bias=None, act=ACT_GELU_TANH):
    A, W = _f32(A), _f32(W)
    M, K = A.shape
    N = W.shape[0]
    bias = None if bias is None else _f32(bias)
    out = np.empty((M, N), np.float32)
    sa = np.empty(M, np.float32)
    sw = np.empty(N, np.float32)
    lib().orc_layer_fp8_composed(_ptr(A), _ptr(W), _ptr(bias), M, N, K, act, _ptr(out),
                                 _ptr(sa), _ptr(sw))
    return out, sa, sw


def layer_fp8_exact(A_q, scale_A, W_q, scale_W, bias=None, act=ACT_GELU_TANH):
    A_q = np.ascontiguousarray(A_q, np.uint8)
    W_q = np.ascontiguousarray(W_q, np.uint8)
    M, K = A_q.shape
    N = W_q.shape[0]
    bias = None if bias is None else _f32(bias)
    out = np.empty((M, N), np.float32)
    lib().orc_layer_fp8_exact(_ptr(A_q), _ptr(_f32(scale_A)), _ptr(W_q), _ptr(_f32(scale_W)),
                              _ptr(bias), M, N, K, act, _ptr(out))
    return out


# ---- reference build (oracle/_ref) -----------------------------------------

def host_cpu_flags() -> set:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def host_cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def ref_variant() -> str | None:
    """'vnni' if this host can run the reference's AVX-512 VNNI build (the
    build its CMakeLists selects), 'avx2' if only AVX2, else None."""
    f = host_cpu_flags()
    if {"avx512_vnni", "avx512f", "avx512bw", "avx512dq"} <= f:
        return "vnni"
    if {"avx2", "fma"} <= f:
        return "avx2"
    return None


_ref = {}


def ref(variant: str | None = None):
    """Load oracle/_ref/libnflow_ref_<variant>.so (the reference's own code)."""
    variant = variant or ref_variant()
    if variant is None:
        raise RuntimeError("host CPU lacks AVX2; the reference build cannot run here")
    if variant not in _ref:
        L = _load(HERE / "_ref" / f"libnflow_ref_{variant}.so")
        vp, i32, f32, sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
        L.ref_linear_forward.argtypes = [C.POINTER(LinearParams), vp, vp]
        L.ref_linear_forward_batched.argtypes = [C.POINTER(LinearParams), i32, vp, vp]
        L.ref_quantise_activation.argtypes = [vp, vp, i32, i32, f32, C.c_int32]
        L.ref_precompute_sum_w.argtypes = [vp, vp, i32, i32, vp]
        L.ref_e4m3_encode_array.argtypes = [vp, vp, sz]
        L.ref_e4m3_decode_array.argtypes = [vp, vp, sz]
        L.ref_fp8_fake_quant.argtypes = [vp, f32, vp, sz]
        L.ref_e4m3_encode_bits_range.argtypes = [C.c_uint32, C.c_uint32, vp]
        L.ref_time_per_token_layer.restype = C.c_double
        L.ref_time_per_token_layer.argtypes = [C.POINTER(LinearParams), C.c_int64, vp, vp,
                                               i32, i32, i32]
        L.ref_time_batched_layer.restype = C.c_double
        L.ref_time_batched_layer.argtypes = [C.POINTER(LinearParams), C.c_int64, vp, vp, i32, i32]
        L.ref_time_fp8_layer.restype = C.c_double
        L.ref_time_fp8_layer.argtypes = [vp, vp, vp, C.c_int64, i32, i32, vp, i32, i32, i32]
        _ref[variant] = L
    return _ref[variant]


def ref_available(variant: str | None = None) -> bool:
    variant = variant or ref_variant()
    return variant is not None and (HERE / "_ref" / f"libnflow_ref_{variant}.so").exists()


def ref_quantise_activation(A, scale_A, zp_A=0, variant=None):
    A = _f32(A)
    out = np.empty(A.shape, np.int8)
    K = A.shape[-1]
    ref(variant).ref_quantise_activation(_ptr(A), _ptr(out), A.size // K, K, scale_A, zp_A)
    return out


def ref_linear_forward_rows(A, W_q, scale_W, zp_W, bias=None, scale_A=1.0, zp_A=0, sum_W=None,
                            scale_A_rows=None, variant=None):
    A = _f32(A)
    p, keep = make_params(W_q, scale_W, zp_W, bias, scale_A, zp_A, sum_W)
    M = A.shape[0]
    out = np.empty((M, p.out_features), np.float32)
    L = ref(variant)
    for m in range(M):
        if scale_A_rows is not None:
            p.scale_A = float(scale_A_rows[m])
        rc = L.ref_linear_forward(C.byref(p), _ptr(A[m]), out[m].ctypes.data_as(C.c_void_p))
        if rc:
            return rc, out
    del keep
    return 0, out


def ref_linear_forward_batched(A, W_q, scale_W, zp_W, bias=None, scale_A=1.0, zp_A=0,
                               sum_W=None, variant=None):
    A = _f32(A)
    p, keep = make_params(W_q, scale_W, zp_W, bias, scale_A, zp_A, sum_W)
    M = A.shape[0]
    out = np.empty((M, p.out_features), np.float32)
    rc = ref(variant).ref_linear_forward_batched(C.byref(p), M, _ptr(A), _ptr(out))
    del keep
    return rc, out


def ref_precompute_sum_w(W_q, zp_W, variant=None):
    W_q = np.ascontiguousarray(W_q, np.int8)
    zp_W = np.ascontiguousarray(zp_W, np.int32)
    out = np.empty(W_q.shape[0], np.int32)
    ok = ref(variant).ref_precompute_sum_w(_ptr(W_q), _ptr(zp_W), W_q.shape[1], W_q.shape[0],
                                          _ptr(out))
    return out if ok else None


def ref_e4m3_encode(x, variant=None):
    x = _f32(x)
    out = np.empty(x.shape, np.uint8)
    ref(variant).ref_e4m3_encode_array(_ptr(x), _ptr(out), x.size)
    return out


def ref_e4m3_decode(b, variant=None):
    b = np.ascontiguousarray(b, np.uint8)
    out = np.empty(b.shape, np.float32)
    ref(variant).ref_e4m3_decode_array(_ptr(b), _ptr(out), b.size)
    return out


def ref_fp8_fake_quant(x, scale, variant=None):
    x = _f32(x)
    out = np.empty(x.shape, np.float32)
    ref(variant).ref_fp8_fake_quant(_ptr(x), scale, _ptr(out), x.size)
    return out


def ref_e4m3_encode_bits_range(start, count, variant=None):
    out = np.empty(count, np.uint8)
    ref(variant).ref_e4m3_encode_bits_range(start, count, _ptr(out))
    return out


def ref_time_per_token_layer(A, W_q, scale_W, bias, sum_W, threads, reps=3, act_gelu=True,
                             variant=None):
    """Median seconds for the reference per-token layer over all rows of A."""
    A = _f32(A)
    N = W_q.shape[0]
    p, keep = make_params(W_q, scale_W, np.zeros(N, np.int32), bias, 1.0, 0, sum_W)
    out = np.empty((A.shape[0], N), np.float32)
    t = ref(variant).ref_time_per_token_layer(C.byref(p), A.shape[0], _ptr(A), _ptr(out),
                                              int(act_gelu), threads, reps)
    del keep
    return t, out


def ref_time_batched_layer(A, W_q, scale_W, bias, sum_W, scale_A, threads, reps=3, variant=None):
    """Median seconds for the reference LinearForwardBatched (one per-tensor
    scale_A, zp_A = 0) over all rows of A, rows split across threads."""
    A = _f32(A)
    N = W_q.shape[0]
    p, keep = make_params(W_q, scale_W, np.zeros(N, np.int32), bias, scale_A, 0, sum_W)
    out = np.empty((A.shape[0], N), np.float32)
    t = ref(variant).ref_time_batched_layer(C.byref(p), A.shape[0], _ptr(A), _ptr(out), threads, reps)
    del keep
    return t, out


def ref_time_fp8_layer(A, W, bias, threads, reps=3, act_gelu=True, variant=None):
    """Median seconds for the reference's FP8 composition (per-row
    fp8_e4m3_per_tensor_fake_quant + the fp32 Linear loop + GELU) over all
    rows of A, rows split across threads."""
    A, W = _f32(A), _f32(W)
    M, K = A.shape
    N = W.shape[0]
    b = None if bias is None else _f32(bias)
    out = np.empty((M, N), np.float32)
    t = ref(variant).ref_time_fp8_layer(_ptr(A), _ptr(W), _ptr(b), M, K, N, _ptr(out), int(act_gelu),
                                        threads, reps)
    return t, out


def usable_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1
