"""Exhaustive device checks of the runtime kernels' GELU and log2-snap forms
(tests/native/gelu_device_check.hip, built by __graft_entry__.build()):

* gelu_fast, the GELU the kernels run (fno.cpp:41-46 with glibc's tanhf; its
  two common-path divisions as a reciprocal step), equals gelu_ref, the
  IEEE-division form that tests/test_gelu_exact.py checks against glibc on
  all 2^32 inputs, on every one of the 2^32 float inputs;
* the snap exponent from the binade and one table compare equals the count
  of table steps (fno.cpp:579-606) on every float in [2^-6, FLT_MAX], for
  the nominal step table and for tables moved 500 ulps either way."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

LIB = Path(__file__).resolve().parent / "native" / "libgelu_device_check.so"

pytestmark = pytest.mark.gpu


def _table(shift):
    steps = []
    for j in range(15):
        e = j - 5
        steps.append(2.0 ** (e - 1 + 1 / 16) if e <= 0 else 2.0 ** (e - 1 / 16))
    bits = np.array(steps, np.float32).view(np.uint32).astype(np.int64) + shift
    return bits.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("shift", [0, -500, 500])
def test_gelu_and_snap_exhaustive(shift):
    import torch

    assert torch.cuda.is_available()
    assert LIB.exists(), f"{LIB} is not built (run __graft_entry__.build())"
    lib = ctypes.CDLL(str(LIB))
    thr = np.ascontiguousarray(_table(shift))
    counts = (ctypes.c_ulonglong * 3)()
    first = (ctypes.c_uint32 * 3)()
    rc = lib.nfq_check_gelu_snap(thr.ctypes.data_as(ctypes.c_void_p), counts, first)
    assert rc == 0, f"HIP error {rc}"
    refine = lib.nfq_gelu_refine()
    print(f"gelu_fast<0>: {counts[0]} differ (first {first[0]:#010x}); "
          f"gelu_fast<1>: {counts[1]} differ (first {first[1]:#010x}); snap: {counts[2]} differ")
    assert counts[refine] == 0, f"gelu_fast<{refine}> differs on {counts[refine]} inputs, first {first[refine]:#010x}"
    assert counts[2] == 0, f"snap exponent differs on {counts[2]} inputs, first {first[2]:#010x}"
