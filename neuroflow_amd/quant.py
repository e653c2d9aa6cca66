"""Host-side mirror of NeuroFlow's `nflow-quant` API on the MI355X kernels.

The functions keep the reference's names and argument meaning
(cpp/include/neuroflow/int8_gemm.h:45-118, cpp/include/neuroflow/fp8_e4m3.h,
cpp/include/neuroflow/fp8_e4m3_pybind.h:24-66) and call libnflow_quant.so
through its C-ABI.  Tensors are torch CUDA tensors (device memory and the
current stream come from torch; the arithmetic is the HIP kernels').  A failed
status raises NflowError (a RuntimeError), as the pybind module turns a
failed Status into RuntimeError (pybind_module.cpp:189-191).
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import ACT_GELU_TANH, ACT_NONE, ACT_RELU, Fp8LinearParamsC, Int8LinearParamsC, check

_ACTS = {None: ACT_NONE, "none": ACT_NONE, "relu": ACT_RELU, "gelu": ACT_GELU_TANH,
         "gelu_tanh": ACT_GELU_TANH, ACT_NONE: ACT_NONE, ACT_RELU: ACT_RELU,
         ACT_GELU_TANH: ACT_GELU_TANH}


def _act(a) -> int:
    if a not in _ACTS:
        raise ValueError(f"unknown activation {a!r}")
    return _ACTS[a]


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: Optional[torch.Tensor], dtype: torch.dtype, name: str) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


@dataclass
class Int8LinearParams:
    """int8_gemm::Int8LinearParams (int8_gemm.h:45-65) with device tensors."""

    W_int8: torch.Tensor                     # (out, in) int8
    scale_W: torch.Tensor                    # (out,) float32
    zp_W: torch.Tensor                       # (out,) int32
    bias: Optional[torch.Tensor] = None      # (out,) float32
    scale_A: float = 1.0
    zp_A: int = 0
    sum_W_per_row: Optional[torch.Tensor] = None  # (out,) int32

    @property
    def in_features(self) -> int:
        return int(self.W_int8.shape[1])

    @property
    def out_features(self) -> int:
        return int(self.W_int8.shape[0])

    def c_struct(self) -> Int8LinearParamsC:
        _dev(self.W_int8, torch.int8, "W_int8")
        _dev(self.scale_W, torch.float32, "scale_W")
        _dev(self.zp_W, torch.int32, "zp_W")
        _dev(self.bias, torch.float32, "bias")
        _dev(self.sum_W_per_row, torch.int32, "sum_W_per_row")
        return Int8LinearParamsC(_p(self.W_int8), _p(self.scale_W), _p(self.zp_W),
                                 _p(self.bias), self.in_features, self.out_features,
                                 float(self.scale_A), int(self.zp_A), _p(self.sum_W_per_row))


@dataclass
class Fp8LinearParams:
    """FP8 E4M3 layer: per-channel symmetric weight bytes + scales."""

    W_e4m3: torch.Tensor                  # (out, in) uint8
    scale_W: torch.Tensor                 # (out,) float32
    bias: Optional[torch.Tensor] = None   # (out,) float32

    @property
    def in_features(self) -> int:
        return int(self.W_e4m3.shape[1])

    @property
    def out_features(self) -> int:
        return int(self.W_e4m3.shape[0])

    def c_struct(self) -> Fp8LinearParamsC:
        _dev(self.W_e4m3, torch.uint8, "W_e4m3")
        _dev(self.scale_W, torch.float32, "scale_W")
        _dev(self.bias, torch.float32, "bias")
        return Fp8LinearParamsC(_p(self.W_e4m3), _p(self.scale_W), _p(self.bias),
                                self.in_features, self.out_features)


def _rows(A: torch.Tensor, K: int, name: str = "A") -> int:
    if A.shape[-1] != K:
        raise ValueError(f"{name} last dim {A.shape[-1]} != in_features {K}")
    return A.numel() // K if K else 0


# ---- int8_gemm namespace ----------------------------------------------------

def quantise_activation(A: torch.Tensor, scale_A: float, zp_A: int = 0) -> torch.Tensor:
    """int8_gemm::QuantiseActivation (int8_gemm.cpp:507-520)."""
    _dev(A, torch.float32, "A")
    out = torch.empty(A.shape, dtype=torch.int8, device=A.device)
    K = A.shape[-1] if A.dim() else 1
    check(_lib.lib().nflow_int8_quantise_activation(_p(A), _p(out), A.numel() // max(K, 1), K,
                                                    float(scale_A), int(zp_A), _stream()),
          "QuantiseActivation")
    return out


def precompute_sum_w(W_int8: torch.Tensor, zp_W: torch.Tensor) -> torch.Tensor:
    """int8_gemm::PrecomputeSumW (int8_gemm.cpp:479-496)."""
    _dev(W_int8, torch.int8, "W_int8")
    _dev(zp_W, torch.int32, "zp_W")
    out = torch.empty(W_int8.shape[0], dtype=torch.int32, device=W_int8.device)
    check(_lib.lib().nflow_int8_precompute_sum_w(_p(W_int8), _p(zp_W), W_int8.shape[1],
                                                 W_int8.shape[0], _p(out), _stream()),
          "PrecomputeSumW")
    return out


def linear_forward(p: Int8LinearParams, A: torch.Tensor) -> torch.Tensor:
    """int8_gemm::LinearForward (int8_gemm.cpp:201-470, VNNI build) applied to
    every row of A (a single row when A is 1-D)."""
    _dev(A, torch.float32, "A")
    ps = p.c_struct()
    M = _rows(A, p.in_features)
    C_ = torch.empty(*A.shape[:-1], p.out_features, dtype=torch.float32, device=A.device)
    L = _lib.lib()
    if A.dim() == 1:
        rc = L.nflow_int8_linear_forward(C.byref(ps), _p(A), _p(C_), _stream())
    else:
        rc = L.nflow_int8_linear_forward_rows(C.byref(ps), M, _p(A), _p(C_), _stream())
    check(rc, "Int8Linear")
    return C_


def linear_forward_batched(p: Int8LinearParams, A: torch.Tensor) -> torch.Tensor:
    """int8_gemm::LinearForwardBatched (int8_gemm.cpp:530-580)."""
    _dev(A, torch.float32, "A")
    ps = p.c_struct()
    M = _rows(A, p.in_features)
    C_ = torch.empty(*A.shape[:-1], p.out_features, dtype=torch.float32, device=A.device)
    check(_lib.lib().nflow_int8_linear_forward_batched(C.byref(ps), M, _p(A), _p(C_), _stream()),
          "LinearForwardBatched")
    return C_


# ---- per-token INT8 ---------------------------------------------------------

def quantise_per_token(A: torch.Tensor):
    """(codes int8, scale_A float32, sum_a int32) with scale = absmax/127."""
    _dev(A, torch.float32, "A")
    K = A.shape[-1]
    M = A.numel() // K
    q = torch.empty(A.shape, dtype=torch.int8, device=A.device)
    s = torch.empty(M, dtype=torch.float32, device=A.device)
    sa = torch.empty(M, dtype=torch.int32, device=A.device)
    check(_lib.lib().nflow_int8_quantise_per_token(_p(A), M, K, _p(q), _p(s), _p(sa), _stream()),
          "quantise_per_token")
    return q, s, sa


def linear_forward_per_token(p: Int8LinearParams, A: torch.Tensor, activation="gelu",
                             out: Optional[torch.Tensor] = None, return_scales: bool = False):
    """Fused per-token INT8 layer (quantise -> MFMA GEMM -> dequant + bias + act)."""
    _dev(A, torch.float32, "A")
    ps = p.c_struct()
    M = _rows(A, p.in_features)
    if out is None:
        out = torch.empty(*A.shape[:-1], p.out_features, dtype=torch.float32, device=A.device)
    else:
        _dev(out, torch.float32, "out")
    s = torch.empty(M, dtype=torch.float32, device=A.device) if return_scales else None
    check(_lib.lib().nflow_int8_linear_forward_per_token(C.byref(ps), M, _p(A), _p(out), _p(s),
                                                         _act(activation), _stream()),
          "linear_forward_per_token")
    return (out, s) if return_scales else out


def gemm_i32(A_q: torch.Tensor, W_q: torch.Tensor) -> torch.Tensor:
    _dev(A_q, torch.int8, "A_q")
    _dev(W_q, torch.int8, "W_q")
    K = A_q.shape[-1]
    M = A_q.numel() // K
    N = W_q.shape[0]
    out = torch.empty(*A_q.shape[:-1], N, dtype=torch.int32, device=A_q.device)
    check(_lib.lib().nflow_int8_gemm_i32(_p(A_q), _p(W_q), M, N, K, _p(out), _stream()), "gemm_i32")
    return out


def linear_forward_quantised(p: Int8LinearParams, A_q: torch.Tensor, scale_A: torch.Tensor,
                             activation="gelu", out: Optional[torch.Tensor] = None) -> torch.Tensor:
    _dev(A_q, torch.int8, "A_q")
    _dev(scale_A, torch.float32, "scale_A")
    ps = p.c_struct()
    M = _rows(A_q, p.in_features, "A_q")
    if out is None:
        out = torch.empty(*A_q.shape[:-1], p.out_features, dtype=torch.float32, device=A_q.device)
    check(_lib.lib().nflow_int8_linear_forward_quantised(C.byref(ps), M, _p(A_q), _p(scale_A),
                                                         _p(out), _act(activation), _stream()),
          "linear_forward_quantised")
    return out


def linear_forward_codes(p: Int8LinearParams, A_q: torch.Tensor, scale_A: torch.Tensor, activation="relu",
                         out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
    """linear_forward_quantised followed by the per-token quantise of its
    output, in one step: (C_q int8 (M, out_features), scale_C float32 (M,)),
    the next layer's input codes and row scales (nflow_int8_linear_forward_codes)."""
    _dev(A_q, torch.int8, "A_q")
    _dev(scale_A, torch.float32, "scale_A")
    ps = p.c_struct()
    M = _rows(A_q, p.in_features, "A_q")
    if out is None:
        out = (torch.empty(*A_q.shape[:-1], p.out_features, dtype=torch.int8, device=A_q.device),
               torch.empty(M, dtype=torch.float32, device=A_q.device))
    C_q, scale_C = out
    check(_lib.lib().nflow_int8_linear_forward_codes(C.byref(ps), M, _p(A_q), _p(scale_A), _p(C_q),
                                                     _p(scale_C), _act(activation), _stream()),
          "linear_forward_codes")
    return C_q, scale_C


def mlp_forward_per_token(layers: Sequence[Int8LinearParams], x: torch.Tensor, activations: Sequence,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """A chain of per-token INT8 layers (DeepONet's branch / trunk MLPs,
    fno.cpp:1318-1341, 1364-1386): nflow_int8_mlp_forward_per_token."""
    _dev(x, torch.float32, "x")
    if len(layers) != len(activations):
        raise ValueError("one activation per layer")
    arr = (Int8LinearParamsC * len(layers))(*[L.c_struct() for L in layers])
    acts = (C.c_int * len(layers))(*[_act(a) for a in activations])
    M = _rows(x, layers[0].in_features, "x")
    if out is None:
        out = torch.empty(*x.shape[:-1], layers[-1].out_features, dtype=torch.float32, device=x.device)
    check(_lib.lib().nflow_int8_mlp_forward_per_token(arr, acts, len(layers), M, _p(x), _p(out), _stream()),
          "mlp_forward_per_token")
    return out


def chain_faults() -> int:
    """Timed-out row-maxima waits of the 8-bit-output kernel on the current
    stream since the last call (synchronises the stream)."""
    n = C.c_uint32(0)
    check(_lib.lib().nflow_debug_chain_faults(_stream(), C.byref(n)), "debug_chain_faults")
    return int(n.value)


# ---- FP8 E4M3 -----------------------------------------------------------------

def _to_device(x, dtype):
    if isinstance(x, torch.Tensor):
        return x, False
    arr = np.ascontiguousarray(x, dtype={torch.float32: np.float32, torch.uint8: np.uint8}[dtype])
    return torch.from_numpy(arr).cuda(), True


def fp8_e4m3_to_bits(x):
    """fp32_array_to_e4m3_bits (fp8_e4m3.h:286-290); neuroflow_cpp.fp8_e4m3_to_bits.
    numpy in -> numpy out, CUDA tensor in -> CUDA tensor out."""
    t, was_np = _to_device(x, torch.float32)
    t = _dev(t.contiguous(), torch.float32, "in")
    out = torch.empty(t.shape, dtype=torch.uint8, device=t.device)
    check(_lib.lib().nflow_fp8_e4m3_to_bits(_p(t), _p(out), t.numel(), _stream()),
          "fp8_e4m3_to_bits")
    return out.cpu().numpy() if was_np else out


def fp8_e4m3_from_bits(b):
    """e4m3_bits_to_fp32_array (fp8_e4m3.h:295-299); neuroflow_cpp.fp8_e4m3_from_bits."""
    t, was_np = _to_device(b, torch.uint8)
    t = _dev(t.contiguous(), torch.uint8, "in")
    out = torch.empty(t.shape, dtype=torch.float32, device=t.device)
    check(_lib.lib().nflow_fp8_e4m3_from_bits(_p(t), _p(out), t.numel(), _stream()),
          "fp8_e4m3_from_bits")
    return out.cpu().numpy() if was_np else out


def fp8_e4m3_fake_quant(x, scale: float):
    """fp8_e4m3_per_tensor_fake_quant (fp8_e4m3.h:312-334); neuroflow_cpp.fp8_e4m3_fake_quant."""
    t, was_np = _to_device(x, torch.float32)
    t = _dev(t.contiguous(), torch.float32, "in")
    out = torch.empty_like(t)
    check(_lib.lib().nflow_fp8_e4m3_fake_quant(_p(t), float(scale), _p(out), t.numel(), _stream()),
          "fp8_e4m3_fake_quant")
    return out.cpu().numpy() if was_np else out


def fp8_quantise_per_token(A: torch.Tensor):
    _dev(A, torch.float32, "A")
    K = A.shape[-1]
    M = A.numel() // K
    q = torch.empty(A.shape, dtype=torch.uint8, device=A.device)
    s = torch.empty(M, dtype=torch.float32, device=A.device)
    check(_lib.lib().nflow_fp8_quantise_per_token(_p(A), M, K, _p(q), _p(s), _stream()),
          "fp8_quantise_per_token")
    return q, s


def fp8_linear_forward_per_token(p: Fp8LinearParams, A: torch.Tensor, activation="gelu",
                                 out: Optional[torch.Tensor] = None, return_scales: bool = False):
    _dev(A, torch.float32, "A")
    ps = p.c_struct()
    M = _rows(A, p.in_features)
    if out is None:
        out = torch.empty(*A.shape[:-1], p.out_features, dtype=torch.float32, device=A.device)
    s = torch.empty(M, dtype=torch.float32, device=A.device) if return_scales else None
    check(_lib.lib().nflow_fp8_linear_forward_per_token(C.byref(ps), M, _p(A), _p(out), _p(s),
                                                        _act(activation), _stream()),
          "fp8_linear_forward_per_token")
    return (out, s) if return_scales else out


@dataclass
class X2Quant:
    """The FNO layer's static INT8 fake-quant of x2 (fno.cpp:572-648),
    nflow_x2_quant: "per_tensor" with (scale, zero_point), or "per_position"
    with device arrays scales / zero_points of at least out_features * points
    entries, indexed column * points + row % points (the reference's flat
    (width, points) offset)."""

    kind: str                                  # "per_tensor" | "per_position"
    scale: float = 1.0
    zero_point: int = 0
    scales: Optional[torch.Tensor] = None      # (n_positions,) float32, device
    zero_points: Optional[torch.Tensor] = None  # (n_positions,) int32, device
    width: int = 0
    points: int = 0

    def c_struct(self) -> "_lib.X2QuantC":
        kinds = {"none": _lib.X2_NONE, "per_tensor": _lib.X2_PER_TENSOR,
                 "per_position": _lib.X2_PER_POSITION, "fp8_log2": _lib.X2_FP8_LOG2}
        _dev(self.scales, torch.float32, "scales")
        _dev(self.zero_points, torch.int32, "zero_points")
        n = 0 if self.scales is None else self.scales.numel()
        return _lib.X2QuantC(kinds[self.kind], float(self.scale), int(self.zero_point), _p(self.scales),
                             _p(self.zero_points), n, int(self.width), int(self.points))


def _fno(fn_name, p, h, x1, activation, out, return_scales, what, x2_quant=None):
    _dev(h, torch.float32, "h")
    _dev(x1, torch.float32, "x1")
    ps = p.c_struct()
    M = _rows(h, p.in_features)
    if x1 is not None and (x1.shape[-1] != p.out_features or x1.numel() != M * p.out_features):
        raise ValueError("x1 must be (M, out_features)")
    if out is None:
        out = torch.empty(*h.shape[:-1], p.out_features, dtype=torch.float32, device=h.device)
    s = torch.empty(M, dtype=torch.float32, device=h.device) if return_scales else None
    if x2_quant is None:
        if x1 is None:
            raise ValueError("x1 is required without x2_quant")
        check(getattr(_lib.lib(), fn_name)(C.byref(ps), M, _p(h), _p(x1), _p(out), _p(s), _act(activation),
                                           _stream()), what)
    else:
        xq = x2_quant.c_struct()
        check(getattr(_lib.lib(), fn_name + "_x2q")(C.byref(ps), M, _p(h), _p(x1), _p(out), _p(s),
                                                    _act(activation), C.byref(xq), _stream()), what)
    return (out, s) if return_scales else out


def fno_layer_per_token(p: Int8LinearParams, h: torch.Tensor, x1: Optional[torch.Tensor], activation="gelu",
                        out: Optional[torch.Tensor] = None, return_scales: bool = False,
                        x2_quant: Optional[X2Quant] = None):
    """The FNO local-linear layer act(x1 + fq(W q(h) + b)) with per-token INT8
    (fno.cpp:515-557, 572-654); x1 is the spectral branch, (M, out_features),
    and fq the optional x2 fake-quant."""
    return _fno("nflow_int8_fno_layer_per_token", p, h, x1, activation, out, return_scales, "fno_layer",
                x2_quant)


def fp8_fno_layer_per_token(p: Fp8LinearParams, h: torch.Tensor, x1: Optional[torch.Tensor], activation="gelu",
                            out: Optional[torch.Tensor] = None, return_scales: bool = False,
                            x2_quant: Optional[X2Quant] = None):
    """fno_layer_per_token on the FP8 E4M3 path."""
    return _fno("nflow_fp8_fno_layer_per_token", p, h, x1, activation, out, return_scales, "fp8_fno_layer",
                x2_quant)


def fp8_gemm_f32(A_q: torch.Tensor, W_q: torch.Tensor) -> torch.Tensor:
    _dev(A_q, torch.uint8, "A_q")
    _dev(W_q, torch.uint8, "W_q")
    K = A_q.shape[-1]
    M = A_q.numel() // K
    N = W_q.shape[0]
    out = torch.empty(*A_q.shape[:-1], N, dtype=torch.float32, device=A_q.device)
    check(_lib.lib().nflow_fp8_gemm_f32(_p(A_q), _p(W_q), M, N, K, _p(out), _stream()),
          "fp8_gemm_f32")
    return out


def fp8_linear_forward_quantised(p: Fp8LinearParams, A_q: torch.Tensor, scale_A: torch.Tensor,
                                 activation="gelu") -> torch.Tensor:
    _dev(A_q, torch.uint8, "A_q")
    _dev(scale_A, torch.float32, "scale_A")
    ps = p.c_struct()
    M = _rows(A_q, p.in_features, "A_q")
    out = torch.empty(*A_q.shape[:-1], p.out_features, dtype=torch.float32, device=A_q.device)
    check(_lib.lib().nflow_fp8_linear_forward_quantised(C.byref(ps), M, _p(A_q), _p(scale_A),
                                                        _p(out), _act(activation), _stream()),
          "fp8_linear_forward_quantised")
    return out


# ---- one-time weight blobs (host, numpy) -----------------------------------------

def _np_ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def per_channel_scales(W: np.ndarray, qmax: float) -> np.ndarray:
    W = np.ascontiguousarray(W, np.float32)
    s = np.empty(W.shape[0], np.float32)
    check(_lib.lib().nflow_host_per_channel_scales(_np_ptr(W), W.shape[0], W.shape[1],
                                                   float(qmax), _np_ptr(s)), "per_channel_scales")
    return s


def quantise_weight_2d(W: np.ndarray, scales: np.ndarray, zero_points: Optional[np.ndarray] = None):
    """fno::QuantiseWeight2D (fno.cpp:325-358) -> (W_q int8, sum_W int32)."""
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    scales = np.ascontiguousarray(scales, np.float32)
    zps = (np.zeros(N, np.int32) if zero_points is None
           else np.ascontiguousarray(zero_points, np.int32))
    q = np.empty((N, K), np.int8)
    sw = np.empty(N, np.int32)
    check(_lib.lib().nflow_host_quantise_weight_2d(_np_ptr(W), N, K, _np_ptr(scales), _np_ptr(zps),
                                                   _np_ptr(q), _np_ptr(sw)), "QuantiseWeight2D")
    return q, sw


def fp8_quantise_weight(W: np.ndarray):
    """Per-channel FP8 E4M3 weight blob -> (W_e4m3 uint8, scales float32)."""
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N, np.float32)
    check(_lib.lib().nflow_host_fp8_quantise_weight(_np_ptr(W), N, K, _np_ptr(q), _np_ptr(s)),
          "fp8_quantise_weight")
    return q, s


# ---- layers: weights uploaded once, per-token activations per call ----------------

class Int8Linear:
    """A per-channel symmetric INT8 linear layer resident on the device.

    Built once from fp32 weights (scales = absmax/127 per output channel,
    codes by QuantiseWeight2D with zero points 0), as EnableInt8Gemm builds
    its Int8GemmLayer cache (fno.cpp:325-406); every call runs the fused
    per-token kernel."""

    def __init__(self, W: np.ndarray, bias: Optional[np.ndarray] = None, device="cuda"):
        W = np.ascontiguousarray(W, np.float32)
        scales = per_channel_scales(W, 127.0)
        q, sum_w = quantise_weight_2d(W, scales)
        dev = torch.device(device)
        self.params = Int8LinearParams(
            W_int8=torch.from_numpy(q).to(dev),
            scale_W=torch.from_numpy(scales).to(dev),
            zp_W=torch.zeros(W.shape[0], dtype=torch.int32, device=dev),
            bias=None if bias is None else torch.from_numpy(np.ascontiguousarray(bias, np.float32)).to(dev),
            sum_W_per_row=torch.from_numpy(sum_w).to(dev))
        self.W_q, self.scale_W, self.sum_W = q, scales, sum_w
        # The per-token calls pass neither the zero points (all 0) nor sum_W
        # (each row's code sum): the same outputs bit for bit, without the
        # kernels' integer-epilogue terms.
        assert np.array_equal(sum_w, q.sum(axis=1, dtype=np.int64))
        self.token_params = dataclasses.replace(self.params, zp_W=None, sum_W_per_row=None)

    def __call__(self, x: torch.Tensor, activation="gelu", out=None) -> torch.Tensor:
        return linear_forward_per_token(self.token_params, x, activation, out=out)

    def launcher(self, activation="gelu"):
        """A prepared call for a hot loop: `run(x_ptr, out_ptr, M, stream)`
        with raw device pointers, the C struct built once.  The caller keeps
        x / out alive and shaped (M, in_features) / (M, out_features)."""
        ps = self.token_params.c_struct()
        fn = _lib.lib().nflow_int8_linear_forward_per_token
        ref = C.byref(ps)
        act = _act(activation)

        def run(x_ptr: int, out_ptr: int, M: int, stream: int) -> None:
            rc = fn(ref, M, x_ptr, out_ptr, None, act, stream)
            if rc:
                check(rc, "linear_forward_per_token")

        run.params = ps  # keep the struct alive with the closure
        return run


class Fp8Linear:
    """A per-channel symmetric FP8 E4M3 linear layer resident on the device."""

    def __init__(self, W: np.ndarray, bias: Optional[np.ndarray] = None, device="cuda"):
        q, scales = fp8_quantise_weight(W)
        dev = torch.device(device)
        self.params = Fp8LinearParams(
            W_e4m3=torch.from_numpy(q).to(dev), scale_W=torch.from_numpy(scales).to(dev),
            bias=None if bias is None else torch.from_numpy(np.ascontiguousarray(bias, np.float32)).to(dev))
        self.W_q, self.scale_W = q, scales

    def __call__(self, x: torch.Tensor, activation="gelu", out=None) -> torch.Tensor:
        return fp8_linear_forward_per_token(self.params, x, activation, out=out)

    def launcher(self, activation="gelu"):
        """Prepared hot-loop call, as Int8Linear.launcher."""
        ps = self.params.c_struct()
        fn = _lib.lib().nflow_fp8_linear_forward_per_token
        ref = C.byref(ps)
        act = _act(activation)

        def run(x_ptr: int, out_ptr: int, M: int, stream: int) -> None:
            rc = fn(ref, M, x_ptr, out_ptr, None, act, stream)
            if rc:
                check(rc, "fp8_linear_forward_per_token")

        run.params = ps
        return run


# ---- device-resident layer handles (nflow_layer) -----------------------------

_FORMATS = {"int8": _lib.FORMAT_INT8, "fp8": _lib.FORMAT_FP8_E4M3}


class Layer:
    """A `nflow_layer` handle: the library quantises the weights, uploads the
    blob once to the current device and owns it (the Int8GemmLayer cache of
    EnableInt8Gemm, fno.cpp:325-406); calls run the fused per-token kernel.

    Layer(W, bias, fmt="int8"|"fp8") builds from fp32 weights;
    Layer.from_int8_blob(W_q, scale_W, zp_W, bias, sum_W) from an existing
    INT8 blob (the per-channel qparams of an IR file)."""

    def __init__(self, W: Optional[np.ndarray] = None, bias: Optional[np.ndarray] = None,
                 fmt: str = "int8", _handle=None):
        self._h = C.c_void_p()
        if _handle is not None:
            self._h = _handle
        else:
            if fmt not in _FORMATS:
                raise ValueError(f"unknown format {fmt!r}")
            W = np.ascontiguousarray(W, np.float32)
            b = None if bias is None else np.ascontiguousarray(bias, np.float32)
            check(_lib.lib().nflow_layer_create(_np_ptr(W), None if b is None else _np_ptr(b),
                                                W.shape[0], W.shape[1], _FORMATS[fmt],
                                                C.byref(self._h)), "layer_create")
        n, k, f = C.c_int(), C.c_int(), C.c_int()
        check(_lib.lib().nflow_layer_shape(self._h, C.byref(n), C.byref(k), C.byref(f)), "layer_shape")
        self.out_features, self.in_features = n.value, k.value
        self.fmt = "int8" if f.value == _lib.FORMAT_INT8 else "fp8"

    @classmethod
    def from_int8_blob(cls, W_q, scale_W, zp_W, bias=None, sum_W=None) -> "Layer":
        W_q = np.ascontiguousarray(W_q, np.int8)
        arrs = [np.ascontiguousarray(scale_W, np.float32), np.ascontiguousarray(zp_W, np.int32),
                None if bias is None else np.ascontiguousarray(bias, np.float32),
                None if sum_W is None else np.ascontiguousarray(sum_W, np.int32)]
        h = C.c_void_p()
        check(_lib.lib().nflow_layer_create_int8(
            _np_ptr(W_q), *[None if a is None else _np_ptr(a) for a in arrs],
            W_q.shape[0], W_q.shape[1], C.byref(h)), "layer_create_int8")
        return cls(_handle=h)

    def __call__(self, x: torch.Tensor, activation="gelu", out: Optional[torch.Tensor] = None,
                 return_scales: bool = False, residual: Optional[torch.Tensor] = None,
                 x2_quant: Optional[X2Quant] = None):
        """act(W q(x) + b), or with `residual` x1 the FNO form act(x1 + (W q(x) + b));
        x2_quant adds the FNO layer's fake-quant of W q(x) + b."""
        _dev(x, torch.float32, "x")
        if x.shape[-1] != self.in_features:
            raise ValueError(f"x has {x.shape[-1]} features, the layer takes {self.in_features}")
        M = x.numel() // self.in_features
        if out is None:
            out = torch.empty(*x.shape[:-1], self.out_features, dtype=torch.float32, device=x.device)
        s = torch.empty(M, dtype=torch.float32, device=x.device) if return_scales else None
        sp = None if s is None else s.data_ptr()
        if x2_quant is not None:
            if residual is not None:
                _dev(residual, torch.float32, "residual")
                if residual.numel() != M * self.out_features:
                    raise ValueError("residual must be (M, out_features)")
            xq = x2_quant.c_struct()
            check(_lib.lib().nflow_layer_forward_fno(self._h, M, x.data_ptr(), _p(residual), out.data_ptr(), sp,
                                                     _act(activation), C.byref(xq), _stream()),
                  "layer_forward_fno")
        elif residual is None:
            check(_lib.lib().nflow_layer_forward(self._h, M, x.data_ptr(), out.data_ptr(), sp,
                                                 _act(activation), _stream()), "layer_forward")
        else:
            _dev(residual, torch.float32, "residual")
            if residual.numel() != M * self.out_features:
                raise ValueError("residual must be (M, out_features)")
            check(_lib.lib().nflow_layer_forward_residual(self._h, M, x.data_ptr(), residual.data_ptr(),
                                                          out.data_ptr(), sp, _act(activation), _stream()),
                  "layer_forward_residual")
        return (out, s) if return_scales else out

    def forward_per_tensor(self, x: torch.Tensor, scale_A: float, zp_A: int = 0,
                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The IR-driven per-tensor INT8 layer: LinearForwardBatched with the
        handle's blob, then + bias (fno.cpp:135-156, 541-549)."""
        _dev(x, torch.float32, "x")
        if x.shape[-1] != self.in_features:
            raise ValueError(f"x has {x.shape[-1]} features, the layer takes {self.in_features}")
        M = x.numel() // self.in_features
        if out is None:
            out = torch.empty(*x.shape[:-1], self.out_features, dtype=torch.float32, device=x.device)
        check(_lib.lib().nflow_layer_forward_per_tensor(self._h, M, x.data_ptr(), out.data_ptr(),
                                                        float(scale_A), int(zp_A), _stream()),
              "layer_forward_per_tensor")
        return out

    def close(self) -> None:
        if self._h:
            _lib.lib().nflow_layer_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
