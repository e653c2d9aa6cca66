"""Write tests/golden/ref_int8_vectors.npz from the reference's own code.

Runs NeuroFlow's int8_gemm::QuantiseActivation / LinearForward /
LinearForwardBatched / PrecomputeSumW and fp32_to_e4m3_bits, compiled from
the reference sources into oracle/_ref by `make -C oracle ref`, on small
seeded inputs, and stores inputs and outputs.  The fixture is data only; the
tests compare the oracle (and, on the GPU, the HIP kernels) against it.

    python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from neuroflow_amd import workloads as WL  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "ref_int8_vectors.npz"


def main() -> None:
    assert O.ref_variant() == "vnni", "fixtures come from the reference's VNNI build"
    d = {}
    # QuantiseActivation: ties, specials, zero points.
    A = WL.normal(900, (8, 40)) * 4.0
    A[0, :12] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, np.nan, np.inf, -np.inf, 3e9, -3e9, 0.0]
    d["qa_A"] = A
    cases = [(0.05, 0), (0.05, 3), (0.03, -7), (0.0, 0), (1.0, 100), (0.5, -128)]
    d["qa_cases"] = np.array(cases, dtype=np.float64)
    for i, (s, zp) in enumerate(cases):
        d[f"qa_out_{i}"] = O.ref_quantise_activation(A, np.float32(s), int(zp))

    # LinearForward / LinearForwardBatched with asymmetric weights, K in
    # {64, 100 (VNNI tail), 4100 (scalar path)}.
    for K, N, M in ((64, 24, 6), (100, 24, 6), (4100, 6, 2)):
        W = WL.uniform(901 + K, (N, K), -0.125, 0.125)
        s = O.per_channel_scales(W, 127.0)
        zps = np.round(WL.uniform(902 + K, (N,), -6, 6)).astype(np.int32)
        q, sw = O.quantise_weight_2d(W, s, zps)
        b = WL.uniform(903 + K, (N,), -0.1, 0.1)
        X = WL.normal(904 + K, (M, K))
        d[f"lf{K}_Wq"], d[f"lf{K}_sW"], d[f"lf{K}_zpW"], d[f"lf{K}_b"], d[f"lf{K}_X"] = q, s, zps, b, X
        d[f"lf{K}_sumW_ref"] = O.ref_precompute_sum_w(q, zps)
        for zpa in (0, 5):
            for use_sum in (0, 1):
                sumW = d[f"lf{K}_sumW_ref"] if use_sum else None
                rc, out = O.ref_linear_forward_rows(X, q, s, zps, b, 0.02, zpa, sumW)
                assert rc == 0
                d[f"lf{K}_rows_zp{zpa}_sum{use_sum}"] = out
                rc, out = O.ref_linear_forward_batched(X, q, s, zps, b, 0.02, zpa, sumW)
                assert rc == 0
                d[f"lf{K}_batched_zp{zpa}_sum{use_sum}"] = out

    # Per-token calling pattern: LinearForward per row with scale = absmax/127.
    K, N, M = 64, 64, 16
    X = WL.normal(950, (M, K))
    W = WL.uniform(951, (N, K), -0.125, 0.125)
    s = O.per_channel_scales(W, 127.0)
    q, sw = O.quantise_weight_2d(W, s)
    b = WL.uniform(952, (N,), -0.1, 0.1)
    sa = O.per_token_scales(X, 127.0)
    rc, out = O.ref_linear_forward_rows(X, q, s, np.zeros(N, np.int32), b, 1.0, 0, sw,
                                        scale_A_rows=sa)
    assert rc == 0
    d.update(pt_X=X, pt_Wq=q, pt_sW=s, pt_b=b, pt_sumW=sw, pt_sA=sa, pt_out=out)

    # FP8 codec bytes for a spread of values.
    x = np.concatenate([(WL.uniform(960, (4096,)) - 0.5) * 1000.0,
                        (WL.uniform(961, (1024,)) - 0.5) * 0.05,
                        np.array([464.0, 470.0, 479.9, 480.0, 0.0146, 0.0147, 7.5 * 2 ** -9],
                                 np.float32)]).astype(np.float32)
    d["fp8_x"] = x
    d["fp8_bytes"] = O.ref_e4m3_encode(x)
    d["fp8_fq_2p5"] = O.ref_fp8_fake_quant(x, 2.5)
    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
