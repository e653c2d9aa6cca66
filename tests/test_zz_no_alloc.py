"""nflow_int8_linear_forward_per_token_noalloc against
nflow_int8_linear_forward_per_token, through the C-ABI: the same bits
(outputs and per-row scales) on two calls in a row, the second with a
smaller input, for

  - shapes that keep their workspace in the static scratch: K = 1024 / 2048
    (per-token quantise -> tiled GEMM; with zero points and a caller's sum_W
    every region -- codes, scales, row sums, weight-row sums -- is used),
    K = 1000 (quantise -> the row-tile kernel on codes), the C5 trunk and
    branch shapes;
  - shapes that need none (K = N = 64 and K = 256: one launch each).

The first wide case is also held to the oracle on sampled rows."""
import ctypes as C

import numpy as np
import pytest
import torch

from neuroflow_amd import _lib
from neuroflow_amd import quant as Q
from neuroflow_amd import workloads as WL
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _layer(N, K, sid, zp, sum_off):
    W = WL.uniform(sid, (N, K), -0.125, 0.125)
    s = O.per_channel_scales(W, 127.0)
    zps = (WL.uniform(sid + 1, (N,), -6, 6).astype(np.int32) if zp else np.zeros(N, np.int32))
    q, sw = O.quantise_weight_2d(W, s, zps)
    b = WL.uniform(sid + 2, (N,), -0.1, 0.1)
    sum_w = None if sum_off is None else (sw + sum_off).astype(np.int32)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    p = Q.Int8LinearParams(cu(q), cu(s), cu(zps), cu(b), sum_W_per_row=None if sum_w is None else cu(sum_w))
    return p, (q, s, zps, b, sum_w)


def _run(name, p, x, act, with_scales):
    M, N = x.shape[0], p.out_features
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device=x.device)
    sc = torch.full((M,), float("nan"), dtype=torch.float32, device=x.device) if with_scales else None
    ps = p.c_struct()
    rc = getattr(_lib.lib(), name)(C.byref(ps), M, x.data_ptr(), out.data_ptr(),
                                   None if sc is None else sc.data_ptr(), act,
                                   torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, name)
    return out, sc


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


# (M, K, N, zero points, sum_W offset or None, scales out, activation code)
PAIRS = [
    ((6000, 1024, 1024, True, 3, False, 2), (700, 1024, 512, False, 0, True, 1)),
    ((65536, 1024, 1024, False, None, False, 1), (4096, 1024, 1024, False, None, True, 1)),
    ((3000, 2048, 256, True, None, True, 0), (10, 2048, 256, True, None, False, 2)),
    ((500, 1000, 100, True, 0, False, 2), (37, 1000, 100, False, None, True, 0)),
    ((262144, 64, 64, False, None, True, 2), (1000, 64, 64, False, None, False, 2)),
    ((32768, 256, 768, False, None, False, 0), (100, 256, 256, True, 1, True, 1)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_equals_the_allocating_entry_point(gpu, first, second):
    for i, (M, K, N, zp, sum_off, with_scales, act) in enumerate((first, second)):
        print(f"noalloc case {i}: M={M} K={K} N={N} zp={zp} sum_off={sum_off} scales={with_scales} "
              f"act={act}", flush=True)
        p, host = _layer(N, K, 900 + K + i, zp, sum_off)
        A = WL.normal(950 + K + i, (M, K))
        x = torch.from_numpy(A).cuda()
        y_na, s_na = _run("nflow_int8_linear_forward_per_token_noalloc", p, x, act, with_scales)
        y_ref, s_ref = _run("nflow_int8_linear_forward_per_token", p, x, act, True)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(y_na), _bits(y_ref)), f"case {i}: outputs differ"
        if with_scales:
            assert np.array_equal(_bits(s_na), _bits(s_ref)), f"case {i}: scales differ"
        if i == 0 and K == 1024 and zp:
            q, s, zps, b, sum_w = host
            rows = np.unique(np.concatenate([np.arange(0, M, 97), [M - 1]]))
            want, _ = O.layer_per_token_i8(A[rows], q, s, zps, b, sum_w, act)
            got = y_na.cpu().numpy()[rows]
            if act == 2:
                np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
            else:
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_rejects_a_workspace_beyond_its_scratch(gpu):
    """A shape whose codes and scales exceed the static scratch returns
    NFLOW_INVALID_ARG before any launch, and leaves the output untouched."""
    M, K, N = 80000, 1024, 64          # 80000 * 1024 + 4 * 80000 bytes > 72 MiB
    p, _ = _layer(N, K, 990, False, None)
    x = torch.zeros(M, K, dtype=torch.float32, device="cuda")
    out = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    ps = p.c_struct()
    rc = _lib.lib().nflow_int8_linear_forward_per_token_noalloc(C.byref(ps), M, x.data_ptr(), out.data_ptr(),
                                                                None, 1, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == _lib.INVALID_ARG
    assert b"scratch" in _lib.lib().nflow_last_error()
    assert bool((out == 7.0).all())


def test_noalloc_under_graph_capture(gpu):
    """A K = 1024 call (quantise into the static scratch, then the tiled
    GEMM) captured into a HIP graph: every replay, with eager work between
    replays, equals the eager call bit for bit."""
    M, K, N = 3000, 1024, 512
    p, _ = _layer(N, K, 991, True, 2)
    x = torch.from_numpy(WL.normal(992, (M, K))).cuda()
    ps = p.c_struct()
    fn = _lib.lib().nflow_int8_linear_forward_per_token_noalloc
    want = torch.empty(M, N, dtype=torch.float32, device="cuda")
    _lib.check(fn(C.byref(ps), M, x.data_ptr(), want.data_ptr(), None, 2, torch.cuda.current_stream().cuda_stream),
               "noalloc eager")
    torch.cuda.synchronize()
    got = torch.empty(M, N, dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.check(fn(C.byref(ps), M, x.data_ptr(), got.data_ptr(), None, 2,
                      torch.cuda.current_stream().cuda_stream), "noalloc captured")
    other = torch.from_numpy(WL.normal(993, (500, K))).cuda()
    scratch_out = torch.empty(500, N, dtype=torch.float32, device="cuda")
    for r in range(3):
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(got), _bits(want)), f"replay {r}"
        # Eager work on the same scratch between replays.
        _lib.check(fn(C.byref(ps), 500, other.data_ptr(), scratch_out.data_ptr(), None, 1,
                      torch.cuda.current_stream().cuda_stream), "noalloc between replays")
        torch.cuda.synchronize()


def test_noalloc_host_threads_share_one_stream(gpu):
    """Four host threads issue no-allocation calls on one stream through the
    C entry point (ctypes releases the GIL, so the calls overlap on the
    host): each keeps its codes in the one static scratch, so one call's
    quantise and product must not be split by another call's launches."""
    import threading

    K, N = 1024, 256
    p, _ = _layer(N, K, 994, False, None)
    ps = p.c_struct()
    fn = _lib.lib().nflow_int8_linear_forward_per_token_noalloc
    stream = torch.cuda.Stream()
    xs = [torch.from_numpy(WL.normal(995 + i, (3000 + 700 * i, K))).cuda() for i in range(4)]
    want = []
    for x in xs:
        w = torch.empty(x.shape[0], N, dtype=torch.float32, device="cuda")
        _lib.check(fn(C.byref(ps), x.shape[0], x.data_ptr(), w.data_ptr(), None, 1, stream.cuda_stream), "alone")
        torch.cuda.synchronize()
        want.append(w)
    outs = [[torch.empty(x.shape[0], N, dtype=torch.float32, device="cuda") for _ in range(6)] for x in xs]
    errors = []

    def worker(i):
        try:
            for r in range(6):
                _lib.check(fn(C.byref(ps), xs[i].shape[0], xs[i].data_ptr(), outs[i][r].data_ptr(), None, 1,
                              stream.cuda_stream), "noalloc thread")
        except Exception as e:  # reported below
            errors.append(e)

    torch.cuda.synchronize()
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors
    for i in range(4):
        for r in range(6):
            assert np.array_equal(_bits(outs[i][r]), _bits(want[i])), f"thread {i} call {r}"
