"""Build libnflow_quant.so (the gfx950 kernels + C-ABI) in-tree, and the
pybind11 module neuroflow_cpp on top of it.

    python -m neuroflow_amd.build

Compiles neuroflow_amd/csrc/*.hip and *.cpp with hipcc for gfx950 and links
neuroflow_amd/lib/libnflow_quant.so; then compiles
neuroflow_amd/bindings/neuroflow_cpp.cpp (host code only) into
neuroflow_amd/lib/neuroflow_cpp<ext>, which loads the library from its own
directory.  Flags:
  -ffp-contract=off   float expressions round in the written order (the
                      dequantise step must match the reference bit for bit);
  -target-feature -packed-fp32-ops   no packed fp32 VALU instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libnflow_quant.so"
ARCH = os.environ.get("NFLOW_OFFLOAD_ARCH", "gfx950")

COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
          "-I", str(PKG.parent / "include")] + os.environ.get("NFLOW_EXTRA_FLAGS", "").split()
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *COMMON]
    if src.suffix == ".hip":
        cmd += DEVICE + ["-x", "hip"]
    cmd += ["-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build_bindings(verbose: bool = True) -> Path:
    """neuroflow_cpp: g++ against pybind11 and the Python headers, linked to
    libnflow_quant.so with an $ORIGIN rpath."""
    import sysconfig

    import pybind11

    out = LIB_DIR / ("neuroflow_cpp" + sysconfig.get_config_var("EXT_SUFFIX"))
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    tmp = out.with_name(out.name + ".tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC", "-D__HIP_PLATFORM_AMD__",
           "-I", str(PKG.parent / "include"), "-I", pybind11.get_include(), "-I", sysconfig.get_paths()["include"],
           "-I", str(rocm / "include"), str(PKG / "bindings" / "neuroflow_cpp.cpp"), "-o", str(tmp),
           "-L", str(LIB_DIR), "-lnflow_quant", "-Wl,-rpath,$ORIGIN", "-L", str(rocm / "lib"), "-lamdhip64",
           "-Wl,-rpath," + str(rocm / "lib")]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"bindings build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


def build(verbose: bool = True, lib: Path = LIB) -> Path:
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    obj_dir = PKG / "_build" / lib.stem
    obj_dir.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objs = [obj_dir / (s.name + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    lib.parent.mkdir(parents=True, exist_ok=True)
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    if len(sys.argv) > 1:
        build(lib=Path(sys.argv[1]).resolve())
    else:
        build()
        build_bindings()
    sys.exit(0)
