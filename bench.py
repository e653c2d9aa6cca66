"""Benchmark of the MI355X quantised-GEMM path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2]

A step is one pass of the hot path over one batch of synthetic input: for the
default workload (FNO1d INT8 local-linear stack: batch 256 x 1024 grid points,
width 64, 4 layers, so each layer is M=262144, K=N=64) that is 4 chained fused
layers h <- GELU((s_w * s_a) * (W_q q(h)) + b), each one launch of the
per-token quantise -> INT8 MFMA -> dequant + bias + GELU kernel.

Inputs are resident in HBM before timing.  Steps rotate over enough input /
output buffer sets (> 1 GB in total) that a step's input is not resident in
the 256 MB last-level cache.  W untimed warm-up steps run first; then exactly
K steps are timed with events on the launch stream, bracketed by
torch.cuda.synchronize().  One JSON line is printed.

Roofline: the dominant kernel is the fused layer; its algorithmic bytes per
launch are 4MK + 4MN + NK*b_w + 8N and its duration is the timed region
divided by the number of launches.  The CPU baseline is the reference's own
INT8 kernel (int8_gemm::LinearForward, AVX-512 VNNI build from oracle/_ref)
called once per row with that row's scale, plus the tanh GELU, on the host's
cores, over a bounded sample of the same rows; the line also carries
LinearForwardBatched (the FNO1d runtime's path) and, for FP8, the reference
codec's fake-quant + fp32 loop.

Parity: the outputs of the last timed step (every layer, on the input it
read) are compared with the oracle on sampled rows (oracle/parity.py).

By default every other configuration (C1, C3, C4, C5 trunk / branch) is
measured the same way after the headline one and reported under "configs",
each with its kernel time, roofline fraction, parity and a CPU figure.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "quantised GEMM TOPS & HBM GB/s (% roofline) + FNO layer samples/s, 1 MI355X"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_PEAK_TOPS = {"int8": 5000.0, "fp8": 5000.0}   # dense, TOPS


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c2",
                    choices=["c1", "c2", "c3", "c4", "c5_trunk", "c5_branch", "fno1d", "fno2d"])
    ap.add_argument("--sets", type=int, default=0, help="buffer sets to rotate (0 = auto)")
    ap.add_argument("--prewarm-ms", type=float, default=100.0,
                    help="before the warm-up steps, repeat the workload's steps for this much wall "
                         "time so that the timed steps run at the clocks a sustained load settles at "
                         "(0 = off); reported as \"prewarm\"")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="measure only --workload (by default every other configuration is measured "
                         "too and reported under \"configs\")")
    ap.add_argument("--graph", action="store_true",
                    help="replay each step as a HIP graph (K = 64 workloads)")
    ap.add_argument("--no-check", dest="check", action="store_false",
                    help="skip the oracle parity of the timed step's outputs")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also time a plain streaming kernel over the layer's bytes "
                         "(torch.neg: read M*N*4, write M*N*4): the achievable-bandwidth "
                         "reference and the kernel whose FETCH_SIZE / WRITE_SIZE calibrate "
                         "the counters")
    return ap.parse_args()


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` on `workload` from its committed
    rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE per dispatch, each
    scaled by what the counter reads for a plain streaming kernel of known
    size), or None when no summary exists for that pair."""
    f = ROOT / "profiles" / f"{kernel.split('::')[-1]}_{workload}_counters.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def time_gemm_only(wl, layers, sets, stream, reps):
    """Average duration of the tiled GEMM kernel alone (codes in, fused
    epilogue out) for layer 0, on per-token codes prepared outside the timed
    region; launches go through the C entry point with a prebuilt struct so
    that Python overhead stays off the GPU's critical path.  The layer's
    weights are per-channel symmetric (zero points 0, sum_W equal to the
    codes' own sums), so the struct leaves zp_W and sum_W out, as the
    layer's own per-token calls do: the same GEMM kernel as in the layer,
    with identical outputs.  Back to back, the 1024-wide trunk GEMMs reach
    the chip's power limit after ~1.5 ms (86-90 us per launch, then ~108
    us), so this average sits a little above the same kernel's duration in
    the layer chain, where a quantise launch separates them (a median of
    ~84 us in the kernel trace); the time of an event recorded between the
    two launches of a layer is taken before the quantise has finished, so
    events cannot bracket the GEMM inside the chain."""
    import ctypes as C

    import torch
    from neuroflow_amd import _lib
    from neuroflow_amd import quant as Q
    obj, _, L = layers[0]
    M, N = wl.M, L.W.shape[0]
    kind, k = wl.source(0)
    codes = [Q.quantise_per_token(s_["in"][k]) for s_ in sets]
    outs = [torch.empty(M, N, dtype=torch.float32, device=sets[0]["in"][0].device) for _ in sets]
    assert not obj.params.zp_W.any().item()
    ps = obj.token_params.c_struct()
    fn = _lib.lib().nflow_int8_linear_forward_quantised
    act = {"none": 0, "relu": 1, "gelu": 2}[L.act]
    sptr = stream.cuda_stream

    def launch(i):
        q, sc, _ = codes[i % len(codes)]
        _lib.check(fn(C.byref(ps), M, q.data_ptr(), sc.data_ptr(), outs[i % len(outs)].data_ptr(), act,
                      sptr), "linear_forward_quantised")

    for i in range(3):
        launch(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    K = L.W.shape[1]
    gemm_bytes = M * K + 4 * M + 4 * M * N + N * K + 8 * N
    return us, gemm_bytes, 2 * M * N * K


def chained(wl):
    """Whether the workload's step is one per-token layer chain (each layer
    reading the previous one's output): the DeepONet MLPs, run through
    nflow_int8_mlp_forward_per_token, whose hidden activations stay int8
    codes + row scales."""
    return all(L.fmt == "int8" and L.src is None for L in wl.layers) and wl.name.startswith("C5")


def chain_fused(wl):
    """Whether the library takes the 8-bit-output kernel for the chain: its
    condition in nflow_int8_mlp_forward_per_token (K = 1024 hidden layers,
    rows enough for two 128 x 256 tiles per CU)."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return (chained(wl) and all(L.W.shape[1] == 1024 for L in wl.layers)
            and all(L.W.shape[0] == 1024 for L in wl.layers[:-1]) and (wl.M + 127) // 128 * 4 >= 2 * cus)


def time_codes_only(wl, layers, stream, reps):
    """Average duration of the 8-bit-output kernel alone (layer 0: codes and
    row scales in, the next layer's codes and row scales out), on per-token
    codes of the workload's input prepared outside the timed region, over 4
    rotating buffer sets."""
    import ctypes as C

    import torch
    from neuroflow_amd import _lib
    from neuroflow_amd import quant as Q
    obj, _, L = layers[0]
    M, N, K = wl.M, L.W.shape[0], L.W.shape[1]
    x = torch.from_numpy(wl.x).to("cuda")
    q0, s0, _ = Q.quantise_per_token(x)
    del x
    ins = [(q0, s0)] + [(q0.clone(), s0.clone()) for _ in range(3)]
    outs = [(torch.empty(M, N, dtype=torch.int8, device="cuda"), torch.empty(M, device="cuda")) for _ in ins]
    ps = obj.token_params.c_struct()
    fn = _lib.lib().nflow_int8_linear_forward_codes
    act = {"none": 0, "relu": 1, "gelu": 2}[L.act]
    sptr = stream.cuda_stream

    def launch(i):
        (q, sc), (cq, cs) = ins[i % 4], outs[i % 4]
        _lib.check(fn(C.byref(ps), M, q.data_ptr(), sc.data_ptr(), cq.data_ptr(), cs.data_ptr(), act, sptr),
                   "linear_forward_codes")

    for i in range(3):
        launch(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    return us, M * K + M * N + 8 * M + N * K + 8 * N, 2 * M * N * K


def build_layers(wl, dev):
    from neuroflow_amd import quant as Q
    layers = []
    for L in wl.layers:
        obj = (Q.Fp8Linear if L.fmt == "fp8" else Q.Int8Linear)(L.W, L.bias, device=dev)
        layers.append((obj, obj.launcher(L.act), L))
    return layers


def _cpu_rows(K, N, ops_log2):
    """Rows of a K x N layer holding about 2^ops_log2 multiply-adds."""
    return max(256, (1 << ops_log2) // (K * N))


def cpu_baseline(wl, layers, legs=("token",), budget_log2=32):
    """The reference kernel on the host cores over a bounded sample of the
    workload's layer-0 rows (about 2^budget_log2 multiply-adds on all cores,
    a quarter of that on one), scaled to samples/s of the whole step (the
    step's layers weighted by their multiply-adds).

    Legs (the reference has no batched per-token entry point and no FP8 GEMM):
      token    int8_gemm::LinearForward once per row with scale_A = absmax/127
               (int8_gemm.cpp:201-470), + tanh GELU -- the per-token path;
      batched  int8_gemm::LinearForwardBatched with one per-tensor scale
               (int8_gemm.cpp:530-580) -- what FNO1d's runtime runs;
      fp8      per-row fp8_e4m3_per_tensor_fake_quant (fp8_e4m3.h:312-334) +
               the fp32 Linear loop (fno.cpp:68-79) + GELU.
    """
    import numpy as np
    from oracle import oracle as O

    L0 = wl.layers[0]
    obj = layers[0][0]
    N, K = L0.W.shape
    cores = O.usable_cores()
    variant = O.ref_variant()
    if variant is None or not O.ref_available(variant):
        raise RuntimeError("oracle/_ref (the reference build) is not available on this host")
    step_row_layers = sum(wl.M * wl.layers[l].W.shape[0] * wl.layers[l].W.shape[1]
                          for l in range(len(wl.layers))) / (K * N)   # layer-0-equivalent rows per step
    to_samples = wl.samples / step_row_layers
    x0 = wl.inputs[wl.source(0)[1]]
    nN = min(wl.M, _cpu_rows(K, N, budget_log2))
    n1 = min(wl.M, _cpu_rows(K, N, budget_log2 - 2))
    gelu = L0.act == "gelu"
    out = {"unit": "samples/s", "cores": cores, "kind": "reference", "host": O.host_cpu_model(),
           "legs": {}}
    for leg in legs:
        rates = {}
        for threads, n in ((1, n1), (cores, nN)):
            if leg == "token":
                t, _ = O.ref_time_per_token_layer(x0[:n], obj.W_q, obj.scale_W, L0.bias, obj.sum_W,
                                                  threads=threads, reps=3, act_gelu=gelu, variant=variant)
            elif leg == "batched":
                s_a = float(np.float32(np.abs(x0[:n]).max()) / np.float32(127.0))
                t, _ = O.ref_time_batched_layer(x0[:n], obj.W_q, obj.scale_W, L0.bias, obj.sum_W, s_a,
                                                threads=threads, reps=3, variant=variant)
            else:
                t, _ = O.ref_time_fp8_layer(x0[:n], L0.W, L0.bias, threads=threads, reps=3, act_gelu=gelu,
                                            variant=variant)
            rates[threads] = n / t
        desc = {"token": "int8_gemm::LinearForward once per row with scale_A = absmax/127 "
                         "(the per-token path)" + (" + tanh GELU" if gelu else ""),
                "batched": "int8_gemm::LinearForwardBatched, one per-tensor scale (FNO1d's runtime "
                           "path; no GELU)",
                "fp8": "per-row fp8_e4m3_per_tensor_fake_quant + fp32 Linear loop"
                       + (" + tanh GELU" if gelu else "") + " (the reference has no FP8 GEMM)"}[leg]
        out["legs"][leg] = {"value": rates[cores] * to_samples, "value_1core": rates[1] * to_samples,
                            "rows_per_s": rates[cores], "rows_per_s_1core": rates[1],
                            "sample": f"{desc}: layer 0 (K={K}, N={N}), {nN} rows x 3 reps on {cores} threads, "
                                      f"{n1} rows x 3 reps on 1 thread, median"}
    first = out["legs"][legs[0]]
    out.update({"value": first["value"], "value_1core": first["value_1core"],
                "sample": first["sample"] + f"; {variant.upper()} build of the reference sources; host "
                                            f"{out['host']}"})
    return out


def _kernel_of(wl):
    N0, K0 = wl.layers[0].W.shape
    if chain_fused(wl):
        return "nfq::k_chain_wide"    # 8-bit-output layers after one per-token quantise launch
    if K0 == 64 and N0 == 64:
        return "nfq::k_rows64"
    if (wl.layers[0].fmt == "int8" and all(l.W.shape[1] in (128, 256, 512) and l.W.shape[0] % 64 == 0
                                           for l in wl.layers)):
        return "nfq::k_token_gemm"    # the whole per-token layer in one launch
    if K0 in (512, 1024) and N0 % 4 == 0 and wl.layers[0].fmt == "int8":
        return "nfq::k_gemm_wide"     # persistent GEMM after a per-token quantise launch
    if K0 % 64 == 0 and K0 >= 128 and wl.layers[0].fmt == "int8":
        return "nfq::k_gemm_pipe"     # after a per-token quantise launch
    return "nfq::k_rows"


def check_timed_step(wl, layers, bufs):
    """Oracle parity of every layer output of one timed step (sampled rows;
    layer l is checked on the input it read in that step)."""
    import torch
    from oracle import parity as P

    res = []
    for l, (obj, _, L) in enumerate(layers):
        kind, k = wl.source(l)
        x = bufs["in"][k] if kind == "input" else bufs["out"][k]
        y = bufs["out"][l]
        N, K = L.W.shape
        rows = P.sample_rows(wl.M, K, N)
        idx = torch.from_numpy(rows).to(x.device)
        x_rows = x.index_select(0, idx).cpu().numpy()
        got = y.index_select(0, idx).cpu().numpy()
        want, _ = P.layer_ref(L.fmt, obj.W_q, obj.scale_W, getattr(obj, "sum_W", None), L.bias, x_rows, L.act)
        r = P.compare(got, want, L.fmt, L.act)
        res.append(r)
    return {"ok": all(r["ok"] for r in res), "layers": len(res), "rows_per_layer": [r["rows"] for r in res],
            "bit_exact_frac_min": round(min(r["bit_exact_frac"] for r in res), 6),
            "max_abs_diff": max(r["max_abs"] for r in res),
            "bar": "INT8: bit-exact without GELU, 1e-5 rel / 1e-6 abs with GELU; FP8: 1e-5 / 1e-6 of the "
                   "exact-product oracle"}


def check_chain_step(wl, layers, bufs):
    """Oracle parity of a chained step's output (sampled rows): the oracle's
    per-token layers applied in sequence to the step's input rows."""
    import torch
    from oracle import parity as P

    x = bufs["in"][0]
    y = bufs["out"][-1]
    N, K = wl.layers[0].W.shape
    rows = P.sample_rows(wl.M, K, N)
    idx = torch.from_numpy(rows).to(x.device)
    h = x.index_select(0, idx).cpu().numpy()
    for obj, _, L in layers:
        h, _ = P.layer_ref(L.fmt, obj.W_q, obj.scale_W, getattr(obj, "sum_W", None), L.bias, h, L.act)
    got = y.index_select(0, idx).cpu().numpy()
    r = P.compare(got, h, wl.layers[-1].fmt, "gelu" if any(L.act == "gelu" for L in wl.layers) else "none")
    return {"ok": r["ok"], "layers": len(layers), "rows_per_layer": [r["rows"]] * len(layers),
            "bit_exact_frac_min": round(r["bit_exact_frac"], 6), "max_abs_diff": r["max_abs"],
            "checked": "the chain's output against the oracle's per-token layers in sequence",
            "bar": "INT8: bit-exact without GELU, 1e-5 rel / 1e-6 abs with GELU; FP8: 1e-5 / 1e-6 of the "
                   "exact-product oracle"}


def bench_workload(name, args, steps, warmup, cpu_legs=None, copy_calib=False, graph=False):
    """Times `steps` steps of workload `name` (after `warmup`) and returns its
    measurement record."""
    import torch
    from neuroflow_amd import workloads as WL

    dev = torch.device("cuda:0")
    t_gen = time.perf_counter()
    wl = WL.WORKLOADS[name]()
    t_gen = time.perf_counter() - t_gen
    layers = build_layers(wl, dev)
    M = wl.M
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream

    # Buffer sets (the inputs and one output per layer), rotated across steps
    # so that a step's input is not resident in the 256 MB last-level cache.
    # A chained workload (one call per step) keeps only the last output.
    chain = chained(wl)
    out_layers = wl.layers[-1:] if chain else wl.layers
    set_bytes = sum(x.nbytes for x in wl.inputs) + sum(4 * M * L.W.shape[0] for L in out_layers)
    # At least 1.1 GB of sets, so that no step's input is still in the
    # 256 MB last-level cache from an earlier step (C1's 16.8 MB sets: 66).
    n_sets = args.sets or max(2, min(96, -(-1_100_000_000 // set_bytes)))
    host_in = [torch.from_numpy(x) for x in wl.inputs]
    sets = []
    for _ in range(n_sets):
        sets.append({"in": [h.to(dev) for h in host_in],
                     "out": [torch.empty(M, L.W.shape[0], dtype=torch.float32, device=dev) for L in out_layers]})
    torch.cuda.synchronize()
    srcs = [wl.source(l) for l in range(len(layers))]

    if chain:
        import ctypes as C
        from neuroflow_amd import _lib
        from neuroflow_amd._lib import Int8LinearParamsC
        chain_ps = (Int8LinearParamsC * len(layers))(*[obj.token_params.c_struct() for obj, _, _ in layers])
        chain_acts = (C.c_int * len(layers))(*[{"none": 0, "relu": 1, "gelu": 2}[L.act] for _, _, L in layers])
        chain_fn = _lib.lib().nflow_int8_mlp_forward_per_token

        def step(i, sp=sptr):
            b = sets[i % n_sets]
            _lib.check(chain_fn(chain_ps, chain_acts, len(layers), M, b["in"][0].data_ptr(),
                                b["out"][-1].data_ptr(), sp), "mlp_forward_per_token")
    else:
        def step(i, sp=sptr):
            b = sets[i % n_sets]
            for l, (_, run, _) in enumerate(layers):
                kind, k = srcs[l]
                src = b["in"][k] if kind == "input" else b["out"][k]
                run(src.data_ptr(), b["out"][l].data_ptr(), M, sp)

    # Device pre-warm: the same steps for at least `args.prewarm_ms` of wall
    # time, in batches that double in size (a synchronize after each), ahead of
    # the `warmup` steps.  The GPU and its memory start a run at idle clocks:
    # at C2, 5-10 warm-up steps leave the timed layers at 25-26 us, against
    # 23.5 us after 50 ms of load.
    pw_steps, pw_t0, batch = 0, time.perf_counter(), 4
    while args.prewarm_ms > 0 and (time.perf_counter() - pw_t0) * 1e3 < args.prewarm_ms:
        for _ in range(batch):
            step(pw_steps)
            pw_steps += 1
        torch.cuda.synchronize()
        batch = min(2 * batch, 4096)
    pw_ms = (time.perf_counter() - pw_t0) * 1e3 if pw_steps else 0.0

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()

    # HIP graphs: one per buffer set, each the step's launches, replayed in
    # the same rotation (the K = 64 path allocates nothing, so it captures).
    graphs = None
    if graph and all(L.W.shape[1] == 64 for L in wl.layers):
        graphs = []
        for k in range(n_sets):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(k, torch.cuda.current_stream().cuda_stream)
            graphs.append(g)
        torch.cuda.synchronize()
        # Every replay equals the eager step: eager set 0, replay it twice
        # with eager work between, compare the last output bit for bit.
        last = sets[0]["out"][-1]
        step(0)
        torch.cuda.synchronize()
        want = last.clone()
        for _ in range(2):
            last.fill_(float("nan"))
            graphs[0].replay()
            torch.cuda.synchronize()
            if not torch.equal(last.view(torch.int32), want.view(torch.int32)):
                raise RuntimeError("bench.py: a graph replay differs from the eager step")
            step(1 % n_sets)
            torch.cuda.synchronize()
        for i in range(warmup):
            graphs[i % n_sets].replay()
        torch.cuda.synchronize()

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for i in range(steps):
        if graphs is not None:
            graphs[i % n_sets].replay()
        else:
            step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    ms_per_step = ms / steps
    launches = steps * len(layers)
    kernel_us = ms * 1e3 / launches

    # Parity of the timed step: the last timed step wrote set (steps - 1) % n_sets.
    parity = None
    if args.check:
        bufs = sets[(steps - 1) % n_sets]
        parity = check_chain_step(wl, layers, bufs) if chain else check_timed_step(wl, layers, bufs)

    bytes_step = sum(wl.bytes_per_layer(l) for l in range(len(layers)))
    ops_step = sum(wl.ops_per_layer(l) for l in range(len(layers)))
    gbs = bytes_step / (ms_per_step * 1e-3) / 1e9
    tops = ops_step / (ms_per_step * 1e-3) / 1e12
    fmt = wl.layers[0].fmt
    ai = ops_step / bytes_step
    bound = "hbm" if ai < MFMA_PEAK_TOPS[fmt] * 1e12 / (HBM_PEAK_GBS * 1e9) else "mfma"
    if name.startswith("c5"):
        bound = "mfma"
    if bound == "hbm":
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}
    else:
        roof = {"bound": "mfma", "achieved": round(tops, 2), "peak": MFMA_PEAK_TOPS[fmt],
                "unit": "TFLOP/s" if fmt == "fp8" else "TOPS",
                "frac": round(tops / MFMA_PEAK_TOPS[fmt], 4), "traffic": None}
    kernel = _kernel_of(wl)
    roof.update({"kernel": kernel,
                 "kernel_avg_us": round(kernel_us, 3),
                 "bytes_per_launch": bytes_step // len(layers),
                 "ops_per_launch": ops_step // len(layers),
                 "tops": round(tops, 2), "gbs": round(gbs, 1)})
    if kernel == "nfq::k_chain_wide":
        # The hidden layers are one launch each (codes in, codes out) after
        # the first layer's quantise; the roofline is that kernel's own,
        # timed alone on layer 0's shape.
        g_us, g_bytes, g_ops = time_codes_only(wl, layers, stream, max(20, steps))
        g_gbs, g_tops = g_bytes / (g_us * 1e-6) / 1e9, g_ops / (g_us * 1e-6) / 1e12
        roof.update({"layer_avg_us": round(kernel_us, 3), "kernel_avg_us": round(g_us, 3),
                     "bytes_per_launch": g_bytes, "ops_per_launch": g_ops,
                     "tops": round(g_tops, 2), "gbs": round(g_gbs, 1),
                     "achieved": round(g_tops, 2), "frac": round(g_tops / MFMA_PEAK_TOPS[fmt], 4),
                     "layer_level_tops": round(tops, 2),
                     "layer_level_frac": round(tops / MFMA_PEAK_TOPS[fmt], 4)})
    elif kernel in ("nfq::k_gemm_pipe", "nfq::k_gemm_wide"):
        # The layer is two launches (quantise, then the GEMM); the roofline
        # is the GEMM kernel's own, timed alone on layer 0's shape.
        g_us, g_bytes, g_ops = time_gemm_only(wl, layers, sets, stream, max(20, steps))
        g_gbs, g_tops = g_bytes / (g_us * 1e-6) / 1e9, g_ops / (g_us * 1e-6) / 1e12
        roof.update({"layer_avg_us": round(kernel_us, 3), "kernel_avg_us": round(g_us, 3),
                     "bytes_per_launch": g_bytes, "ops_per_launch": g_ops,
                     "tops": round(g_tops, 2), "gbs": round(g_gbs, 1)})
        if bound == "hbm":
            roof.update({"achieved": round(g_gbs, 1), "frac": round(g_gbs / HBM_PEAK_GBS, 4)})
        else:
            roof.update({"achieved": round(g_tops, 2), "frac": round(g_tops / MFMA_PEAK_TOPS[fmt], 4)})
    roof["traffic"] = measured_traffic(kernel, name)
    if kernel == "nfq::k_rows64" and len(layers) > 1 and not chain and graphs is None:
        # A step's first layer reads a cold input (the sets rotate over more
        # than the last-level cache); the later ones read their
        # predecessor's output, partly still in that cache.  The same steps
        # again, over the same rotation, with an event after every layer
        # split each step into its layers.  Each event leaves a gap before
        # the next launch (C2: the four layers so timed sum to ~14 us more
        # than the step), so the excess over the step's own time
        # (ms_per_step) is taken off every layer in equal parts; the kernel
        # trace's per-launch durations are the direct measurement.
        nl = len(layers)
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(nl + 1)] for _ in range(steps)]
        torch.cuda.synchronize()
        for i in range(steps):
            b = sets[i % n_sets]
            evs[i][0].record(stream)
            for l, (_, run, _) in enumerate(layers):
                kind, k = srcs[l]
                src = b["in"][k] if kind == "input" else b["out"][k]
                run(src.data_ptr(), b["out"][l].data_ptr(), M, sptr)
                evs[i][l + 1].record(stream)
        torch.cuda.synchronize()
        per = [[evs[i][l].elapsed_time(evs[i][l + 1]) * 1e3 for i in range(steps)] for l in range(nl)]
        gap_us = max(0.0, (sum(sum(x) for x in per) / steps - ms_per_step * 1e3) / nl)
        cold_us = sum(per[0]) / steps - gap_us
        chain_us = sum(sum(x) for x in per[1:]) / (steps * (nl - 1)) - gap_us
        b0 = wl.bytes_per_layer(0)
        roof.update({"cold_first_layer_us": round(cold_us, 3),
                     "cold_first_layer_frac": round(b0 / (cold_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "chained_layers_avg_us": round(chain_us, 3),
                     "chained_layers_frac": round(b0 / (chain_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "layer_split_steps": steps, "layer_split_event_gap_us": round(gap_us, 3)})

    copy = None
    if copy_calib:
        L0 = wl.layers[0]
        srcs_c = [s_["in"][0] for s_ in sets]
        dsts = [s_["out"][0] for s_ in sets]
        n_out = min(M * min(L0.W.shape), dsts[0].numel())   # within both the input and the output
        # torch.neg is one elementwise kernel that reads and writes each
        # float once (a same-dtype copy_ would go to the runtime's blit).
        for i in range(3):
            torch.neg(srcs_c[i % n_sets].view(-1)[:n_out], out=dsts[i % n_sets].view(-1)[:n_out])
        torch.cuda.synchronize()
        reps = max(20, steps)
        ev0.record(stream)
        for i in range(reps):
            torch.neg(srcs_c[i % n_sets].view(-1)[:n_out], out=dsts[i % n_sets].view(-1)[:n_out])
        ev1.record(stream)
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3 / reps
        cbytes = 8 * n_out
        copy = {"kernel": "torch.neg (float32 elementwise)", "bytes_per_launch": cbytes,
                "avg_us": round(us, 3), "gbs": round(cbytes / (us * 1e-6) / 1e9, 1),
                "frac_of_peak": round(cbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}

    cpu = None
    if cpu_legs:
        try:
            cpu = cpu_baseline(wl, layers, cpu_legs)
        except Exception as e:  # reported, not fatal: the GPU figure stands alone
            cpu = {"error": f"{type(e).__name__}: {e}"}

    rec = {"wl": wl, "n_sets": n_sets, "graphs": graphs is not None,
           "prewarm": {"steps": pw_steps, "ms": round(pw_ms, 1)}, "ms_per_step": ms_per_step,
           "value": wl.samples / (ms_per_step * 1e-3), "roofline": roof, "parity": parity, "cpu": cpu,
           "copy": copy, "gen_s": t_gen}
    del sets, layers
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return rec


def ref_runtime_baseline(model, threads_all, b_all=16, b_one=16, reps=3):
    """The reference runtime itself (InferenceRuntime with EnableInt8Gemm,
    oracle/_ref/ref_fno_run built from its sources) on the host cores over a
    bounded sample of the same batch: b_all samples over all threads, b_one
    on one thread."""
    import subprocess
    import tempfile

    import numpy as np
    from oracle import oracle as O

    exe = ROOT / "oracle" / "_ref" / "ref_fno_run"
    if not exe.exists():
        raise FileNotFoundError(f"{exe} not built")
    grid = "x".join(str(d) for d in model.x.shape[1:-1])
    ci, co = model.x.shape[-1], model.config[1]
    with tempfile.TemporaryDirectory() as d:
        ir, xf = Path(d) / "m.nneuroir", Path(d) / "x.f32"
        ir.write_bytes(model.ir)
        np.ascontiguousarray(model.x[:max(b_all, b_one)]).tofile(xf)
        rates = {}
        for threads, b_s in ((1, b_one), (threads_all, b_all)):
            out = subprocess.run([str(exe), str(ir), str(xf), str(b_s), grid, str(ci), str(co), "-", "int8",
                                  str(reps), str(threads)], capture_output=True, text=True, check=True).stdout
            us = float(out.split("us_per_run")[1].split()[0])
            rates[threads] = b_s / (us * 1e-6)
    return {"value": rates[threads_all], "unit": "samples/s", "cores": threads_all, "kind": "reference",
            "sample": (f"InferenceRuntime::Run with EnableInt8Gemm (the reference runtime built from its "
                       f"sources: runtime.cpp, fno.cpp, fft.cpp, int8_gemm.cpp VNNI) on {b_all} of the "
                       f"batch's samples split over {threads_all} threads with one runtime each, and on "
                       f"{b_one} samples on 1 thread, median of {reps} runs; host {O.host_cpu_model()}"),
            "value_1core": rates[1]}


def bench_fno1d_model(args):
    """The whole FNO1d model through the device runtime: one step = one
    InferenceRuntime run (lift, 4 x [input fake-quant, spectral convolution,
    INT8 local-linear layer, act(x1 + x2)], proj_q, proj_out) over the batch,
    with its input already in HBM."""
    from neuroflow_amd import workloads as WL
    from oracle import fno1d as OF

    def oracle_forward(model, x):
        m = OF.from_records(model.config, False, model.weights, model.qparams)
        OF.enable_int8_gemm(m)
        return OF.forward(m, x)

    bench_runtime_model(args, WL.fno1d_model(), oracle_forward, "int8", 16, 16)


def bench_fno2d_model(args):
    """The whole FNO2d model through the device runtime: one step = one
    InferenceRuntime run (lift, 4 x [row / column FFTs, 12 x 12 mode mix,
    inverse FFTs, local linear, FP8 snap of x2, act(x1 + x2)], proj_q,
    proj_out) over the batch, with its input already in HBM."""
    from neuroflow_amd import workloads as WL
    from oracle import fno2d as OF2

    def oracle_forward(model, x):
        return OF2.forward(OF2.from_records(model.config, False, model.weights, model.qparams), x)

    bench_runtime_model(args, WL.fno2d_model(), oracle_forward, "fp32", 16, 1, 1)


def bench_runtime_model(args, model, oracle_forward, dtype, cpu_b_all, cpu_b_one, cpu_reps=3):
    import ctypes as C

    import numpy as np
    import torch
    from neuroflow_amd import _lib

    L = _lib.lib()
    dev = torch.device("cuda:0")
    h = C.c_void_p()
    buf = C.create_string_buffer(model.ir, len(model.ir))
    _lib.check(L.nflow_runtime_create_memory(buf, len(model.ir), C.byref(h)), "runtime_create")
    _lib.check(L.nflow_runtime_enable_int8_gemm(h), "runtime_enable_int8_gemm")
    b = model.x.shape[0]
    co = model.config[1]
    ys_shape = list(model.x.shape[:-1]) + [co]
    nd = model.x.ndim
    xsh = (C.c_int64 * nd)(*model.x.shape)
    ysh = (C.c_int64 * nd)(*ys_shape)
    n_sets = 4
    xs = [torch.from_numpy(model.x).to(dev) for _ in range(n_sets)]
    ys = [torch.empty(*ys_shape, dtype=torch.float32, device=dev) for _ in range(n_sets)]
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream
    fn = L.nflow_runtime_run_device

    def step(i):
        _lib.check(fn(h, xs[i % n_sets].data_ptr(), xsh, nd, ys[i % n_sets].data_ptr(), ysh, nd, sptr),
                   "runtime_run_device")

    for i in range(max(1, args.warmup)):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps

    parity = None
    if args.check:
        b2 = 2 if nd == 3 else 1
        want = oracle_forward(model, model.x[:b2])
        y2 = torch.empty(b2, *ys_shape[1:], dtype=torch.float32, device=dev)
        _lib.check(fn(h, xs[0].data_ptr(), (C.c_int64 * nd)(b2, *model.x.shape[1:]), nd, y2.data_ptr(),
                      (C.c_int64 * nd)(b2, *ys_shape[1:]), nd, sptr), "runtime_run_device")
        torch.cuda.synchronize()
        parity = bool(np.array_equal(y2.cpu().numpy().view(np.uint32), want.view(np.uint32)))

    cpu = None
    if not args.no_cpu_baseline:
        try:
            from oracle import oracle as O
            cpu = ref_runtime_baseline(model, O.usable_cores(), cpu_b_all, cpu_b_one, cpu_reps)
        except Exception as e:  # reported, not fatal
            cpu = {"error": f"{type(e).__name__}: {e}"}
    L.nflow_runtime_destroy(h)
    out = {
        "metric": METRIC,
        "value": round(b / (ms_per_step * 1e-3), 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded SplitMix64 input fields, seeded PyTorch-style initial weights)",
        "config": {"workload": model.name, "batch": b, "grid": list(model.x.shape[1:-1]), "config": model.config,
                   "parallelism": "single GPU"},
        "roofline": None,
        "cpu_baseline": cpu,
        "parity_vs_oracle": parity,
    }
    print(json.dumps(out))


def _config_entry(name, rec):
    wl, roof = rec["wl"], rec["roofline"]
    e = {"workload": wl.name, "rows": wl.M, "layers": len(wl.layers),
         "ms_per_step": round(rec["ms_per_step"], 5), "samples_per_s": round(rec["value"], 2),
         "dtype": wl.layers[0].fmt, "prewarm": rec["prewarm"]}
    e.update({k: roof[k] for k in ("bound", "kernel", "kernel_avg_us", "achieved", "unit", "frac", "tops", "gbs",
                                   "bytes_per_launch", "ops_per_launch", "traffic")})
    for k in ("layer_avg_us", "layer_level_tops", "layer_level_frac", "cold_first_layer_us", "cold_first_layer_frac",
              "chained_layers_avg_us", "chained_layers_frac", "layer_split_event_gap_us"):
        if k in roof:
            e[k] = roof[k]
    e["buffer_sets"] = rec["n_sets"]
    if rec["copy"] is not None:
        e["copy_calibration"] = rec["copy"]
    e["parity_vs_oracle"] = rec["parity"]
    if rec["cpu"] is not None:
        e["cpu_baseline"] = rec["cpu"]
    return e


CONFIGS = ["c1", "c2", "c3", "c4", "c5_trunk", "c5_branch"]


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported (the layers shard "
              "along rows with no collective: each GPU would run its own rows' share)",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "fno1d":
        bench_fno1d_model(args)
        return
    if args.workload == "fno2d":
        bench_fno2d_model(args)
        return

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    head = args.workload
    legs = None
    if not args.no_cpu_baseline:
        legs = ("fp8",) if head == "c3" else ("token", "batched")
    print(f"bench.py: {head} ({args.steps} steps, {args.warmup} warm-up)", file=sys.stderr, flush=True)
    # The K = 64 layers are reported beside a same-size streaming copy over
    # the same buffer rotation.
    k64 = ("c1", "c2", "c3")
    rec = bench_workload(head, args, args.steps, args.warmup, cpu_legs=legs, copy_calib=args.copy_calib or head in k64,
                         graph=args.graph)
    wl, roof = rec["wl"], rec["roofline"]

    configs = {}
    if not args.no_configs:
        # Every other workload configuration, measured the same way (fewer
        # steps), with its parity and a CPU figure of its own.
        for name in CONFIGS:
            if name == head:
                continue
            print(f"bench.py: {name}", file=sys.stderr, flush=True)
            c_legs = None if args.no_cpu_baseline else (("fp8",) if name == "c3" else ("token",))
            r = bench_workload(name, args, max(5, min(args.steps, 20)), max(2, min(args.warmup, 5)),
                               cpu_legs=c_legs, copy_calib=name in k64)
            configs[name] = _config_entry(name, r)

    out = {
        "metric": METRIC,
        "value": round(rec["value"], 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm": rec["prewarm"],
        "ms_per_step": round(rec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.layers[0].fmt,
        "data": "synthetic (seeded SplitMix64 inputs, seeded Kaiming-uniform weights)",
        "config": {
            "workload": wl.name,
            "rows": wl.M,
            "layers": [list(L.W.shape[::-1]) for L in wl.layers],
            "samples_per_step": wl.samples,
            "buffer_sets": rec["n_sets"],
            "launch": "hip graph per step" if rec["graphs"] else "stream",
            "parallelism": "single GPU",
        },
        "roofline": roof,
        "cpu_baseline": rec["cpu"],
        "parity_vs_oracle": None if rec["parity"] is None else rec["parity"]["ok"],
        "parity_detail": rec["parity"],
    }
    if rec["copy"] is not None:
        out["copy_calibration"] = rec["copy"]
    if configs:
        out["configs"] = configs
    print(json.dumps(out))


if __name__ == "__main__":
    main()
