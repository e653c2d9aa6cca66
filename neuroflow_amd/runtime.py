"""The FNO1d inference runtime on the GPU (include/nflow_runtime.h) from
Python: the pybind11 module `neuroflow_cpp`, built into neuroflow_amd/lib/
next to libnflow_quant.so, with the reference module's surface
(cpp/bindings/pybind_module.cpp:58-238): InferenceRuntime(path) with op(),
enable_int8_gemm(), is_int8_gemm_enabled(), run(x, y) -- plus run_device()
on device pointers -- infer_arrays, infer, infer_deeponet_arrays and the FP8
E4M3 codec functions.

    from neuroflow_amd.runtime import load
    neuroflow_cpp = load()
    rt = neuroflow_cpp.InferenceRuntime("model.nneuroir")

A caller that imports `neuroflow_cpp` directly puts neuroflow_amd/lib on
sys.path (LIB_DIR below).
"""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"


def load():
    """Import neuroflow_cpp from the in-tree build; raises ImportError if it is not built."""
    if str(LIB_DIR) not in sys.path:
        sys.path.insert(0, str(LIB_DIR))
    return importlib.import_module("neuroflow_cpp")
