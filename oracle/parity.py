"""Sampled-row parity of a workload's layer outputs against the oracle.

Test infrastructure, like the rest of oracle/: used by tests/ and by
bench.py's check leg, never by the product.

Every output row of a per-token layer depends only on its input row (the
scale is the row's own absmax), so the oracle run on a sample of input rows
checks exactly those rows of a full-size launch.  The samples are chosen to
cover the kernels' work units:

  K = N = 64 (one 16-row tile per wave and step of the persistent loop):
      one row in every 16-row tile (so every tile of every wave, whatever the
      grid), the first 1024 rows and the last 4096 rows whole (the first
      tiles of the first waves, the last tiles of the last waves, the partial
      tail);
  wider layers (row tiles of 64-256 rows, every column computed per row):
      every 97th row, the first and the last 256 rows.

The bar, for INT8 (reference-exact codes and int32 accumulators): per-row
scales bit-exact; outputs bit-exact for no activation and ReLU, within
1e-5 relative / 1e-6 absolute for GELU (the device evaluates the tanh form
through exp2).  For FP8 (the reference's E4M3 codec, exact products, fp32
accumulation): scales bit-exact, outputs within 1e-5 / 1e-6 of the
exact-product oracle.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O

RTOL, ATOL = 1e-5, 1e-6
ACT_CODE = {"none": O.ACT_NONE, "relu": O.ACT_RELU, "gelu": O.ACT_GELU_TANH}


def sample_rows(M: int, K: int, N: int) -> np.ndarray:
    """Sorted unique row indices to check for an (M, K) -> (M, N) layer."""
    if K == 64 and N == 64:
        t = np.arange((M + 15) // 16, dtype=np.int64)
        one_per_tile = np.minimum(16 * t + (7 * t) % 16, M - 1)
        parts = [one_per_tile, np.arange(min(M, 1024)), np.arange(max(0, M - 4096), M)]
    else:
        parts = [np.arange(0, M, 97), np.arange(min(M, 256)), np.arange(max(0, M - 256), M)]
    return np.unique(np.concatenate(parts)).astype(np.int64)


def layer_ref(fmt: str, W_q, scale_W, sum_W, bias, x_rows: np.ndarray, act: str):
    """(outputs, per-row scales) of the oracle for a per-channel symmetric
    layer (zero points 0) on the given input rows."""
    code = ACT_CODE[act]
    if fmt == "int8":
        return O.layer_per_token_i8(x_rows, W_q, scale_W, None, bias, sum_W, code)
    qa, sa = O.quantise_per_token_fp8(x_rows)
    return O.layer_fp8_exact(qa, sa, W_q, scale_W, bias, code), sa


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def compare(got: np.ndarray, want: np.ndarray, fmt: str, act: str) -> dict:
    """Checks `got` against `want` at the bar of the format / activation.
    Returns {"ok", "exact", "rows", "bit_exact_frac", "max_abs", "max_rel"}."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    same = _bits(got) == _bits(want)
    exact = fmt == "int8" and act != "gelu"
    if exact:
        ok = bool(same.all())
    else:
        ok = bool(np.allclose(got, want, rtol=RTOL, atol=ATOL))
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    rel = diff / np.maximum(np.abs(want.astype(np.float64)), 1e-30)
    return {"ok": ok, "exact": exact, "rows": int(got.shape[0]),
            "bit_exact_frac": float(same.mean()) if same.size else 1.0,
            "max_abs": float(diff.max()) if diff.size else 0.0,
            "max_rel": float(rel[diff > ATOL].max()) if (diff > ATOL).any() else 0.0}
