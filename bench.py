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
cores, over a bounded sample of the same rows.
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
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="replay each step as a HIP graph (K = 64 workloads)")
    ap.add_argument("--check", action="store_true", default=True)
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
    codes' own sums), so the struct leaves zp_W and sum_W out: the GEMM then
    needs no byte sums and runs the same LDS-DMA kernel as the layer, with
    identical outputs."""
    import ctypes as C
    import torch
    from neuroflow_amd import _lib
    from neuroflow_amd import quant as Q
    obj, _, L = layers[0]
    M, N = wl.M, L.W.shape[0]
    codes = [Q.quantise_per_token(s_[0]) for s_ in sets]
    outs = [torch.empty(M, N, dtype=torch.float32, device=sets[0][0].device) for _ in sets]
    import dataclasses
    assert not obj.params.zp_W.any().item()
    ps = dataclasses.replace(obj.params, zp_W=None, sum_W_per_row=None).c_struct()
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


def build_layers(wl, dev):
    from neuroflow_amd import quant as Q
    layers = []
    for L in wl.layers:
        obj = (Q.Fp8Linear if L.fmt == "fp8" else Q.Int8Linear)(L.W, L.bias, device=dev)
        layers.append((obj, obj.launcher(L.act), L))
    return layers


def cpu_baseline(wl, layers, args):
    """Reference kernel on the host cores over a bounded sample of rows."""
    import numpy as np
    from oracle import oracle as O

    L0 = wl.layers[0]
    obj = layers[0][0]
    cores = O.usable_cores()
    M_all = wl.M
    total_rows = M_all * len(wl.layers)          # rows of one step
    variant = O.ref_variant()
    if L0.fmt == "int8" and variant is not None and O.ref_available(variant):
        gelu = L0.act == "gelu"
        n1 = min(M_all, 16384)
        t1, _ = O.ref_time_per_token_layer(wl.x[:n1], obj.W_q, obj.scale_W, L0.bias, obj.sum_W,
                                           threads=1, reps=3, act_gelu=gelu, variant=variant)
        nN = min(M_all, 262144)
        tN, _ = O.ref_time_per_token_layer(wl.x[:nN], obj.W_q, obj.scale_W, L0.bias, obj.sum_W,
                                           threads=cores, reps=3, act_gelu=gelu, variant=variant)
        rows_s_1, rows_s_N = n1 / t1, nN / tN
        kind = "reference"
        sample = (f"int8_gemm::LinearForward ({variant.upper()} build of the reference "
                  f"sources) once per row with scale_A = absmax/127 + tanh GELU, layer 0 "
                  f"(K={L0.W.shape[1]}, N={L0.W.shape[0]}): {nN} rows x 3 reps on {cores} "
                  f"threads, {n1} rows x 3 reps on 1 thread; host {O.host_cpu_model()}")
    else:
        # FP8 (no reference kernel exists): the reference's fake-quant + FP32
        # Linear composition, restated in the oracle, on one thread.
        n1 = min(M_all, 4096)
        t0 = time.perf_counter()
        O.layer_fp8_composed(wl.x[:n1], L0.W, L0.bias, O.ACT_GELU_TANH)
        t1 = time.perf_counter() - t0
        rows_s_1 = rows_s_N = n1 / t1
        cores = 1
        kind = "port"
        sample = (f"FP8 E4M3 fake-quant (fp8_e4m3.h:312-334) + FP32 Linear loop (fno.cpp:68-79), "
                  f"restated in oracle/, {n1} rows of layer 0 on 1 thread (the reference has "
                  f"no FP8 GEMM); host {O.host_cpu_model()}")
    to_unit = wl.samples / total_rows          # samples per row-layer
    return {
        "value": rows_s_N * to_unit,
        "unit": "samples/s",
        "cores": cores,
        "kind": kind,
        "sample": sample,
        "value_1core": rows_s_1 * to_unit,
        "layer_rows_per_s": rows_s_N,
    }


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


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one MI355X; --gpus {args.gpus} is not supported "
              "(the path shards along rows with no collective; see the design notes)",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "fno1d":
        bench_fno1d_model(args)
        return
    if args.workload == "fno2d":
        bench_fno2d_model(args)
        return

    import numpy as np
    import torch
    from neuroflow_amd import workloads as WL

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    wl = WL.WORKLOADS[args.workload]()
    layers = build_layers(wl, dev)
    M = wl.M
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream

    # Buffer sets: input x and one output per layer, rotated across steps.
    widths = [wl.x.shape[1]] + [L.W.shape[0] for L in wl.layers]
    set_bytes = sum(4 * M * w for w in widths)
    n_sets = args.sets or max(2, min(8, -(-1_100_000_000 // set_bytes)))
    x0 = torch.from_numpy(wl.x).to(dev)
    sets = []
    for _ in range(n_sets):
        bufs = [x0.clone()] + [torch.empty(M, w, dtype=torch.float32, device=dev) for w in widths[1:]]
        sets.append(bufs)
    torch.cuda.synchronize()

    def step(i, sp=sptr):
        bufs = sets[i % n_sets]
        for l, (_, run, L) in enumerate(layers):
            src = bufs[l] if wl.chained else bufs[0]
            run(src.data_ptr(), bufs[l + 1].data_ptr(), M, sp)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # HIP graphs: one per buffer set, each the step's launches, replayed in
    # the same rotation (the K = 64 path allocates nothing, so it captures).
    graphs = None
    if args.graph and all(L.W.shape[1] == 64 for L in wl.layers):
        graphs = []
        for k in range(n_sets):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(k, torch.cuda.current_stream().cuda_stream)
            graphs.append(g)
        torch.cuda.synchronize()
        # Every replay equals the eager step: eager set 0, replay it twice
        # with eager work between, compare the last output bit for bit.
        last = sets[0][-1]
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
        for i in range(args.warmup):
            graphs[i % n_sets].replay()
        torch.cuda.synchronize()

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for i in range(args.steps):
        if graphs is not None:
            graphs[i % n_sets].replay()
        else:
            step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    ms_per_step = ms / args.steps
    launches = args.steps * len(layers)
    kernel_us = ms * 1e3 / launches

    # Dominant kernel: the most common layer shape (all layers share one shape
    # in c1-c3; for c4/c5 the bytes/ops are averaged over the step's launches).
    bytes_step = sum(wl.bytes_per_layer(l) for l in range(len(layers)))
    ops_step = sum(wl.ops_per_layer(l) for l in range(len(layers)))
    gbs = bytes_step / (ms_per_step * 1e-3) / 1e9
    tops = ops_step / (ms_per_step * 1e-3) / 1e12
    fmt = wl.layers[0].fmt
    ai = ops_step / bytes_step
    bound = "hbm" if ai < MFMA_PEAK_TOPS[fmt] * 1e12 / (HBM_PEAK_GBS * 1e9) else "mfma"
    if args.workload.startswith("c5"):
        bound = "mfma"
    if bound == "hbm":
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}
    else:
        roof = {"bound": "mfma", "achieved": round(tops, 2), "peak": MFMA_PEAK_TOPS[fmt],
                "unit": "TFLOP/s" if fmt == "fp8" else "TOPS",
                "frac": round(tops / MFMA_PEAK_TOPS[fmt], 4), "traffic": None}
    N0, K0 = wl.layers[0].W.shape
    if K0 == 64 and N0 == 64:
        kernel = "nfq::k_rows64"
    elif (wl.layers[0].fmt == "int8" and all(l.W.shape[1] in (128, 256, 512) and l.W.shape[0] % 64 == 0
                                             for l in wl.layers)):
        kernel = "nfq::k_token_gemm"    # the whole per-token layer in one launch
    elif K0 % 64 == 0 and K0 >= 128 and wl.layers[0].fmt == "int8":
        kernel = "nfq::k_gemm_pipe"     # after a per-token quantise launch
    else:
        kernel = "nfq::k_rows"
    roof.update({"kernel": kernel,
                 "kernel_avg_us": round(kernel_us, 3),
                 "bytes_per_launch": bytes_step // len(layers),
                 "ops_per_launch": ops_step // len(layers),
                 "tops": round(tops, 2), "gbs": round(gbs, 1)})
    if kernel == "nfq::k_gemm_pipe":
        # The layer is two launches (quantise, then the GEMM); the roofline
        # is the GEMM kernel's own, timed alone on layer 0's shape.
        g_us, g_bytes, g_ops = time_gemm_only(wl, layers, sets, stream, max(20, args.steps))
        g_gbs, g_tops = g_bytes / (g_us * 1e-6) / 1e9, g_ops / (g_us * 1e-6) / 1e12
        roof.update({"layer_avg_us": round(kernel_us, 3), "kernel_avg_us": round(g_us, 3),
                     "bytes_per_launch": g_bytes, "ops_per_launch": g_ops,
                     "tops": round(g_tops, 2), "gbs": round(g_gbs, 1)})
        if bound == "hbm":
            roof.update({"achieved": round(g_gbs, 1), "frac": round(g_gbs / HBM_PEAK_GBS, 4)})
        else:
            roof.update({"achieved": round(g_tops, 2), "frac": round(g_tops / MFMA_PEAK_TOPS[fmt], 4)})
    roof["traffic"] = measured_traffic(kernel, args.workload)

    parity = None
    if args.check:
        from oracle import oracle as O
        # Re-run layer 0 on the first rows and compare with the oracle.
        n = min(M, 512)
        L0 = wl.layers[0]
        obj = layers[0][0]
        y = obj(torch.from_numpy(wl.x[:n]).to(dev), L0.act).cpu().numpy()
        act = {"none": 0, "relu": 1, "gelu": 2}[L0.act]
        if L0.fmt == "int8":
            ref, _ = O.layer_per_token_i8(wl.x[:n], obj.W_q, obj.scale_W, None, L0.bias, obj.sum_W, act)
        else:
            qa, sa = O.quantise_per_token_fp8(wl.x[:n])
            ref = O.layer_fp8_exact(qa, sa, obj.W_q, obj.scale_W, L0.bias, act)
        parity = bool(np.allclose(y, ref, rtol=1e-5, atol=1e-6))

    copy = None
    if args.copy_calib:
        L0 = wl.layers[0]
        n_out = M * min(L0.W.shape)          # within both the input and the output
        srcs = [s_[0] for s_ in sets]
        dsts = [s_[1] for s_ in sets]
        # torch.neg is one elementwise kernel that reads and writes each
        # float once (a same-dtype copy_ would go to the runtime's blit).
        for i in range(3):
            torch.neg(srcs[i % n_sets].view(-1)[:n_out], out=dsts[i % n_sets].view(-1)[:n_out])
        torch.cuda.synchronize()
        reps = max(20, args.steps)
        ev0.record(stream)
        for i in range(reps):
            torch.neg(srcs[i % n_sets].view(-1)[:n_out], out=dsts[i % n_sets].view(-1)[:n_out])
        ev1.record(stream)
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3 / reps
        cbytes = 8 * n_out
        copy = {"kernel": "torch.neg (float32 elementwise)", "bytes_per_launch": cbytes,
                "avg_us": round(us, 3), "gbs": round(cbytes / (us * 1e-6) / 1e9, 1),
                "frac_of_peak": round(cbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(wl, layers, args)
        except Exception as e:  # reported, not fatal: the GPU figure stands alone
            cpu = {"error": f"{type(e).__name__}: {e}"}

    value = wl.samples / (ms_per_step * 1e-3)
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": fmt,
        "data": "synthetic (seeded SplitMix64 inputs, seeded Kaiming-uniform weights)",
        "config": {
            "workload": wl.name,
            "rows": M,
            "layers": [list(L.W.shape[::-1]) for L in wl.layers],
            "samples_per_step": wl.samples,
            "buffer_sets": n_sets,
            "launch": "hip graph per step" if graphs is not None else "stream",
            "parallelism": "single GPU",
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "parity_vs_oracle": parity,
    }
    if copy is not None:
        out["copy_calibration"] = copy
    print(json.dumps(out))


if __name__ == "__main__":
    main()
