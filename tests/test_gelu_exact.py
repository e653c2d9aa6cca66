"""The device GELU (neuroflow_amd/csrc/gelu_exact.h, compiled here for the
host with the library's -ffp-contract=off) against glibc, the libm of the
reference's tanhf (fno.cpp:41-46): tanhf_fdlibm and its straight-line form
tanhf_fdlibm_select equal to glibc tanhf, and gelu_ref equal to the
reference build's expression with glibc tanhf, on
every third float bit pattern (all 2^32 with NFLOW_GELU_STRIDE=1).  The
same run checks the log2 snap's exponent from the binade (snap.h) against
the reference's int(std::round(std::log2(a) * 8) / 8) under glibc
(fno.cpp:579-606) on those floats from 2^-6 to FLT_MAX, with the step table
located from that formula."""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_gelu_exact_matches_glibc(tmp_path):
    exe = tmp_path / "gelu_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I", str(ROOT / "neuroflow_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "gelu_exact_check.cpp"), "-o", str(exe), "-lm", "-lpthread"],
                   check=True)
    out = subprocess.run([str(exe), os.environ.get("NFLOW_GELU_STRIDE", "3")], capture_output=True, text=True,
                         check=True, timeout=600).stdout.split()
    got = dict(zip(out[0::2], out[1::2]))
    assert got == {"tanh_mismatches": "0", "select_mismatches": "0", "gelu_mismatches": "0", "c_ok": "1",
                   "snap_steps": "15", "snap_binned": "1", "snap_mismatches": "0"}, out
