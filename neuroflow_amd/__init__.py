"""neuroflow_amd -- NeuroFlow's quantised inference GEMM on AMD MI355X (gfx950).

The compute lives in libnflow_quant.so (hand-written HIP kernels behind the
C-ABI of include/nflow_quant.h); this package is its Python front-end:

  quant      the nflow-quant API (int8_gemm::*, the FP8 E4M3 codec) on
             torch CUDA tensors, plus Int8Linear / Fp8Linear layers
  workloads  the seeded synthetic inputs of the benchmark configurations
  build      in-tree build of libnflow_quant.so
"""
from ._lib import NflowError, lib  # noqa: F401

__all__ = ["NflowError", "lib"]
