"""Seeded synthetic inputs for the quantised-GEMM workloads.

Generator: SplitMix64 counter streams.  Stream `sid` yields
x_i = mix64(mix64(sid * G) + (i + 1) * G), G = 0x9E3779B97F4A7C15; uniforms are
u = (x >> 40) * 2^-24 in [0, 1); normals are Box-Muller in float64 over pairs
of uniforms, cast to float32.  Stream ids are `config * 100 + tensor`.
The same bytes are produced on any host, so the oracle and the GPU always see
identical inputs.  (The reference's own generators -- torch.manual_seed,
np.random.default_rng, std::mt19937 in bench_int8_gemm.cpp:65 -- do not cover
these workloads.)

Workloads (rows x K -> N, per layer):
  C1 standalone INT8     32768 x 64 -> 64, N(0,1) activations, GELU
  C2 FNO1d INT8 stack    262144 x 64 -> 64, 4 layers, batch 256 x 1024 points
  C3 FNO2d FP8 stack     1048576 x 64 -> 64, 4 layers, batch 16 x 256 x 256
  C4 TokenMixer INT8     32768 x 256 -> 768 (qkv) and -> 256 (proj), 6 blocks, each
                         layer on its own LayerNorm(N(0,1)) input (attention omitted)
  C5 DeepONet INT8       4096 / 65536 x 1024 -> 1024 (ReLU), trunk head -> 256
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

_G = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_u64(sid: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        seed = _mix(np.array([sid], dtype=np.uint64) * _G)[0]
        idx = np.arange(1, n + 1, dtype=np.uint64)
        return _mix(seed + idx * _G)


def uniform(sid: int, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    u = (stream_u64(sid, n) >> np.uint64(40)).astype(np.float64) * 2.0 ** -24
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal(sid: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    x = stream_u64(sid, 2 * n) >> np.uint64(40)
    u1 = x[0::2].astype(np.float64) * 2.0 ** -24
    u2 = x[1::2].astype(np.float64) * 2.0 ** -24
    z = np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * math.pi * u2)
    return z.astype(np.float32).reshape(shape)


def kaiming_uniform(sid: int, n_out: int, n_in: int) -> np.ndarray:
    """nn.Linear's default init U(+-1/sqrt(fan_in)) (neuroflow/nn/fno.py:108-112)."""
    b = 1.0 / math.sqrt(n_in)
    return uniform(sid, (n_out, n_in), -b, b)


def sinusoid_fields(sid: int, batch: int, n_points: int, n_terms: int) -> np.ndarray:
    """u_b(x) = sum_j A_j sin(2 pi k_j x + phi_j), x = i / n_points;
    A ~ U(0,1), k uniform on 1..16, phi ~ U(0, 2 pi).  Returns (batch, n_points)."""
    amp = uniform(sid, (batch, n_terms)).astype(np.float64)
    k = np.floor(uniform(sid + 1, (batch, n_terms)).astype(np.float64) * 16.0) + 1.0
    phi = uniform(sid + 2, (batch, n_terms)).astype(np.float64) * 2.0 * math.pi
    x = np.arange(n_points, dtype=np.float64) / n_points
    out = np.zeros((batch, n_points), np.float64)
    for j in range(n_terms):
        out += amp[:, j:j + 1] * np.sin(2.0 * math.pi * k[:, j:j + 1] * x[None, :] + phi[:, j:j + 1])
    return out.astype(np.float32)


def layer_norm(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """LayerNorm with gamma = 1, beta = 0 over the last axis (fno.cpp:1418-1438)."""
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=-1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(axis=-1, keepdims=True)
    return ((x64 - mu) / np.sqrt(var + eps)).astype(np.float32)


@dataclass
class Layer:
    W: np.ndarray                 # (N, K) fp32
    bias: Optional[np.ndarray]    # (N,) fp32
    act: str                      # "gelu" / "relu" / "none"
    fmt: str = "int8"             # "int8" / "fp8"
    src: Optional[int] = None     # input: inputs[src]; None = the previous layer's output
                                  # (inputs[0] for the first layer)


@dataclass
class Workload:
    name: str
    x: np.ndarray                 # (M, K) fp32, the first layer's input (inputs[0])
    layers: List[Layer] = field(default_factory=list)
    samples: int = 1              # samples per pass (for samples/s)
    extra: List[np.ndarray] = field(default_factory=list)   # inputs[1:]

    @property
    def M(self) -> int:
        return self.x.shape[0]

    @property
    def inputs(self) -> List[np.ndarray]:
        return [self.x] + list(self.extra)

    def source(self, l: int):
        """Where layer l reads its input: ("input", k) for inputs[k], or
        ("layer", j) for layer j's output."""
        src = self.layers[l].src
        if src is not None:
            return ("input", src)
        return ("layer", l - 1) if l > 0 else ("input", 0)

    def bytes_per_layer(self, l: int) -> int:
        """Algorithmic HBM bytes of one fused layer: 4MK + 4MN + NK*b_w + 8N."""
        L = self.layers[l]
        N, K = L.W.shape
        return 4 * self.M * K + 4 * self.M * N + N * K + 8 * N

    def ops_per_layer(self, l: int) -> int:
        N, K = self.layers[l].W.shape
        return 2 * self.M * N * K


def c1_standalone(M: int = 32768, K: int = 64, N: int = 64) -> Workload:
    x = normal(100, (M, K))
    W = uniform(101, (N, K), -0.125, 0.125)
    b = uniform(102, (N,), -0.1, 0.1)
    return Workload("C1 standalone INT8 GEMM", x, [Layer(W, b, "gelu")], samples=M // 1024)


def fno1d_lifted(batch: int, n_points: int, width: int, sid: int) -> np.ndarray:
    """Seeded FNO1d input: sums of 8 sinusoids lifted by a 1 -> width fp32
    linear layer (W, b ~ U(-1, 1)); token-major (batch * n_points, width)."""
    u = sinusoid_fields(sid, batch, n_points, 8)
    w_lift = uniform(sid + 3, (width,), -1.0, 1.0).astype(np.float64)
    b_lift = uniform(sid + 4, (width,), -1.0, 1.0).astype(np.float64)
    h = u.reshape(-1, 1).astype(np.float64) * w_lift[None, :] + b_lift[None, :]
    return h.astype(np.float32)


def c2_fno1d(batch: int = 256, n_points: int = 1024, width: int = 64, n_layers: int = 4) -> Workload:
    x = fno1d_lifted(batch, n_points, width, 200)
    layers = [Layer(uniform(210 + l, (width, width), -0.125, 0.125),
                    uniform(220 + l, (width,), -0.125, 0.125), "gelu") for l in range(n_layers)]
    return Workload(f"C2 FNO1d INT8 local-linear stack (batch {batch} x {n_points} points, "
                    f"width {width}, {n_layers} layers)", x, layers, samples=batch)


def c3_fno2d(batch: int = 16, grid: int = 256, width: int = 64, n_layers: int = 4) -> Workload:
    M = batch * grid * grid
    x = 2.0 * normal(300, (M, width))
    mask = uniform(301, (M, width)) < 0.01
    x = np.where(mask, x * 20.0, x).astype(np.float32)
    layers = [Layer(uniform(310 + l, (width, width), -0.125, 0.125),
                    uniform(320 + l, (width,), -0.125, 0.125), "gelu", "fp8")
              for l in range(n_layers)]
    return Workload(f"C3 FNO2d FP8 local-linear stack (batch {batch} x {grid}x{grid}, "
                    f"width {width}, {n_layers} layers)", x, layers, samples=batch)


def c4_tokenmixer(tokens: int = 4096, batch: int = 8, d: int = 256, blocks: int = 6) -> Workload:
    """6 blocks of qkv (d -> 3d) and proj (d -> d), both with bias and no
    activation.  Each layer reads its own LayerNorm(N(0,1)) input: the
    attention between qkv and proj and the residual stream are omitted, so
    block b's qkv reads inputs[2b] and its proj inputs[2b + 1]."""
    M = tokens * batch
    ins, layers = [], []
    for b in range(blocks):
        sid = 400 + 10 * b
        ins.append(layer_norm(normal(sid, (M, d))))
        ins.append(layer_norm(normal(sid + 5, (M, d))))
        layers.append(Layer(kaiming_uniform(sid + 1, 3 * d, d), uniform(sid + 2, (3 * d,), -1 / 16, 1 / 16),
                            "none", src=2 * b))
        layers.append(Layer(kaiming_uniform(sid + 3, d, d), uniform(sid + 4, (d,), -1 / 16, 1 / 16),
                            "none", src=2 * b + 1))
    return Workload(f"C4 TokenMixer INT8 blocks (M={M}, d={d}, {blocks} blocks)", ins[0], layers,
                    samples=batch, extra=ins[1:])


def c5_deeponet_trunk(n_query: int = 65536, width: int = 1024, p: int = 256) -> Workload:
    """Trunk MLP body: the fp32 2 -> width input layer is applied on the host
    (K = 2 is not an MFMA shape), then 3 x (width -> width, ReLU) and
    width -> p."""
    xy = uniform(520, (n_query, 2))
    W0 = kaiming_uniform(521, width, 2).astype(np.float64)
    b0 = uniform(522, (width,), -0.5, 0.5).astype(np.float64)
    h = np.maximum(xy.astype(np.float64) @ W0.T + b0, 0.0).astype(np.float32)
    layers = [Layer(kaiming_uniform(530 + l, width, width),
                    uniform(535 + l, (width,), -1 / 32, 1 / 32), "relu") for l in range(3)]
    layers.append(Layer(kaiming_uniform(540, p, width), uniform(541, (p,), -1 / 32, 1 / 32), "none"))
    return Workload(f"C5 DeepONet trunk INT8 MLP ({n_query} queries, width {width})", h, layers,
                    samples=n_query)


def c5_deeponet_branch(n_samples: int = 4096, sensors: int = 1024, width: int = 1024) -> Workload:
    u = sinusoid_fields(500, n_samples, sensors, 32)
    layers = [Layer(kaiming_uniform(510 + l, width, sensors if l == 0 else width),
                    uniform(515 + l, (width,), -1 / 32, 1 / 32), "relu") for l in range(4)]
    return Workload(f"C5 DeepONet branch INT8 MLP ({n_samples} samples, width {width})", u, layers,
                    samples=n_samples)


@dataclass
class Fno1dModel:
    name: str
    ir: bytes                     # NeuroIR binary with its NIRQ block
    x: np.ndarray                 # (batch, n_points, 1) fp32
    config: List[int]             # [in_ch, out_ch, width, modes, n_layers, pad_factor]
    weights: dict = field(default_factory=dict)   # name -> fp32 array, as written into ir
    qparams: list = field(default_factory=list)   # the NIRQ records, as written into ir


def fno1d_model(batch: int = 256, n_points: int = 1024, width: int = 64, modes: int = 16,
                n_layers: int = 4) -> Fno1dModel:
    """C2's FNO1d as a whole model (the input fields of C2, width 64, modes
    16, 4 layers, GELU): lift 1 -> width, the spectral + local-linear layers,
    proj_q width -> width, proj_out width -> 1.  Weights seeded as the
    reference's PyTorch modules initialise them (nn.Linear's U(+-1/sqrt(fan_in));
    spectral weights (1 / width^2) N(0, 1), neuroflow/nn/fno.py:51-56).  The
    NIRQ block is what calibration exports: per-channel symmetric INT8
    qparams for every Linear / spectral weight and per-tensor symmetric
    activation qparams (absmax / 127 over the first two samples, from a
    float64 pass of the same forward) for lift.output and locs.{i}.output."""
    from .ir import write_binary

    w = width
    rng_id = 600
    weights = {"lift.weight": uniform(rng_id, (w, 1), -1.0, 1.0), "lift.bias": uniform(rng_id + 1, (w,), -1.0, 1.0)}
    for i in range(n_layers):
        sc = 1.0 / (w * w)
        weights[f"specs.{i}.weights_real"] = (sc * normal(rng_id + 10 + 4 * i, (w, w, modes))).astype(np.float32)
        weights[f"specs.{i}.weights_imag"] = (sc * normal(rng_id + 11 + 4 * i, (w, w, modes))).astype(np.float32)
        weights[f"locs.{i}.weight"] = kaiming_uniform(rng_id + 12 + 4 * i, w, w)
        b = 1.0 / math.sqrt(w)
        weights[f"locs.{i}.bias"] = uniform(rng_id + 13 + 4 * i, (w,), -b, b)
    b = 1.0 / math.sqrt(w)
    weights["proj_q.weight"] = kaiming_uniform(rng_id + 90, w, w)
    weights["proj_q.bias"] = uniform(rng_id + 91, (w,), -b, b)
    weights["proj_out.weight"] = kaiming_uniform(rng_id + 92, 1, w)
    weights["proj_out.bias"] = uniform(rng_id + 93, (1,), -b, b)
    x = sinusoid_fields(200, batch, n_points, 8)[:, :, None].astype(np.float32)

    # Calibration pass (float64, two samples): absmax of each activation.
    def gelu(z):
        return 0.5 * z * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (z + 0.044715 * z ** 3)))

    h = x[:2].astype(np.float64) @ weights["lift.weight"].T.astype(np.float64) + weights["lift.bias"]
    amax = {"lift.output": float(np.abs(h).max())}
    for i in range(n_layers):
        spec = np.fft.rfft(h, axis=1)[:, :modes, :]                       # (b, modes, w_in)
        wc = weights[f"specs.{i}.weights_real"] + 1j * weights[f"specs.{i}.weights_imag"]
        mixed = np.einsum("bmi,iom->bmo", spec, wc)
        full = np.zeros((h.shape[0], n_points // 2 + 1, w), np.complex128)
        full[:, :modes, :] = mixed
        x1 = np.fft.irfft(full, n=n_points, axis=1)
        x2 = h @ weights[f"locs.{i}.weight"].T.astype(np.float64) + weights[f"locs.{i}.bias"]
        amax[f"locs.{i}.output"] = float(np.abs(x2).max())
        h = gelu(x1 + x2)
    q = []
    for name, t in weights.items():
        if t.ndim == 2:
            s = np.abs(t).max(axis=1).astype(np.float32) / np.float32(127.0)
            s[s == 0] = 1.0
            q.append((1, name, s, np.zeros(t.shape[0], np.int32), 0))
        elif t.ndim == 3:
            s = np.abs(t).max(axis=(0, 2)).astype(np.float32) / np.float32(127.0)
            s[s == 0] = 1.0
            q.append((1, name, s, np.zeros(t.shape[1], np.int32), 1))
    for key, a in amax.items():
        q.append((0, key, float(np.float32(a) / np.float32(127.0)), 0))
    cfg = [1, 1, w, modes, n_layers, 1]
    ir = write_binary(1, cfg + [0], "gelu", weights, q)
    return Fno1dModel(f"FNO1d model, C2 configuration (batch {batch} x {n_points} points, width {w}, "
                      f"modes {modes}, {n_layers} layers, INT8 local-linear layers, GELU)", ir, x, cfg, weights, q)


def sinusoid_fields_2d(sid: int, batch: int, h: int, w: int, n_terms: int) -> np.ndarray:
    """u_b(x, y) = sum_j A_j sin(2 pi (kx_j x + ky_j y) + phi_j) on the
    (h, w) grid x = i / h, y = j / w; A ~ U(0,1), kx, ky uniform on 1..16,
    phi ~ U(0, 2 pi).  Returns (batch, h, w)."""
    amp = uniform(sid, (batch, n_terms)).astype(np.float64)
    kx = np.floor(uniform(sid + 1, (batch, n_terms)).astype(np.float64) * 16.0) + 1.0
    ky = np.floor(uniform(sid + 2, (batch, n_terms)).astype(np.float64) * 16.0) + 1.0
    phi = uniform(sid + 3, (batch, n_terms)).astype(np.float64) * 2.0 * math.pi
    xs = (np.arange(h, dtype=np.float64) / h)[:, None]
    ys = (np.arange(w, dtype=np.float64) / w)[None, :]
    out = np.zeros((batch, h, w), np.float64)
    for j in range(n_terms):
        arg = 2.0 * math.pi * (kx[:, j, None, None] * xs + ky[:, j, None, None] * ys) + phi[:, j, None, None]
        out += amp[:, j, None, None] * np.sin(arg)
    return out.astype(np.float32)


def fno2d_model(batch: int = 16, grid: int = 256, width: int = 64, modes: int = 12,
                n_layers: int = 4) -> Fno1dModel:
    """C3's FNO2d as a whole model (batch 16 x 256 x 256 grid, width 64,
    modes 12 x 12, 4 layers, GELU) with the runtime's FP8 semantics: the
    NIRQ block carries FP8 E4M3 activation qparams (scale absmax / 448 over
    the first sample, from a float64 pass of the same forward) for
    lift.output, every locs.{i}.output and proj_q.output, which FNO2d::Forward
    applies as its log2 snap (fno.cpp:810-829).  Weights seeded as the
    reference's PyTorch modules initialise them."""
    from .ir import write_binary

    w, m = width, modes
    rng_id = 700
    weights = {"lift.weight": uniform(rng_id, (w, 1), -1.0, 1.0), "lift.bias": uniform(rng_id + 1, (w,), -1.0, 1.0)}
    for i in range(n_layers):
        sc = 1.0 / (w * w)
        weights[f"specs.{i}.weights_real"] = (sc * normal(rng_id + 10 + 4 * i, (w, w, m, m))).astype(np.float32)
        weights[f"specs.{i}.weights_imag"] = (sc * normal(rng_id + 11 + 4 * i, (w, w, m, m))).astype(np.float32)
        weights[f"locs.{i}.weight"] = kaiming_uniform(rng_id + 12 + 4 * i, w, w)
        b = 1.0 / math.sqrt(w)
        weights[f"locs.{i}.bias"] = uniform(rng_id + 13 + 4 * i, (w,), -b, b)
    b = 1.0 / math.sqrt(w)
    weights["proj_q.weight"] = kaiming_uniform(rng_id + 90, w, w)
    weights["proj_q.bias"] = uniform(rng_id + 91, (w,), -b, b)
    weights["proj_out.weight"] = kaiming_uniform(rng_id + 92, 1, w)
    weights["proj_out.bias"] = uniform(rng_id + 93, (1,), -b, b)
    x = sinusoid_fields_2d(210, batch, grid, grid, 8)[..., None].astype(np.float32)

    # Calibration pass (float64, one sample, channel-last): absmax of each activation.
    def gelu(z):
        return 0.5 * z * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (z + 0.044715 * z ** 3)))

    h = x[:1].astype(np.float64) @ weights["lift.weight"].T.astype(np.float64) + weights["lift.bias"]
    amax = {"lift.output": float(np.abs(h).max())}
    for i in range(n_layers):
        spec = np.fft.rfft2(h, axes=(1, 2))[:, :m, :m, :]                 # (b, m, m, w_in)
        wc = weights[f"specs.{i}.weights_real"] + 1j * weights[f"specs.{i}.weights_imag"]
        mixed = np.einsum("bxyi,ioxy->bxyo", spec, wc)
        full = np.zeros((h.shape[0], grid, grid // 2 + 1, w), np.complex128)
        full[:, :m, :m, :] = mixed
        x1 = np.fft.irfft2(full, s=(grid, grid), axes=(1, 2))
        x2 = h @ weights[f"locs.{i}.weight"].T.astype(np.float64) + weights[f"locs.{i}.bias"]
        amax[f"locs.{i}.output"] = float(np.abs(x2).max())
        h = gelu(x1 + x2)
    amax["proj_q.output"] = float(np.abs(h @ weights["proj_q.weight"].T.astype(np.float64)
                                         + weights["proj_q.bias"]).max())
    q = [(3, key, float(np.float32(a) / np.float32(448.0))) for key, a in amax.items()]
    cfg = [1, 1, w, m, m, n_layers, 1]
    ir = write_binary(2, cfg, "gelu", weights, q)
    return Fno1dModel(f"FNO2d model, C3 configuration (batch {batch} x {grid}x{grid} grid, width {w}, "
                      f"modes {m}x{m}, {n_layers} layers, FP8 activation snap, GELU)", ir, x, cfg, weights, q)


WORKLOADS = {
    "c1": c1_standalone,
    "c2": c2_fno1d,
    "c3": c3_fno2d,
    "c4": c4_tokenmixer,
    "c5_trunk": c5_deeponet_trunk,
    "c5_branch": c5_deeponet_branch,
}
