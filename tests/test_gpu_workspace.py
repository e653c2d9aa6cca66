"""GPU tests of the split per-token path's workspace, which is kept per
(device, stream) and reused by the next call on that stream: calls whose
workspace grows and shrinks in one stream, two streams running the split
path at once, and host threads sharing one stream.  Every output must equal,
bit for bit, the same call made alone with the device idle before and after
it (and the oracle on sampled rows)."""
import ctypes
import threading

import numpy as np
import pytest
import torch

from neuroflow_amd import _lib
from neuroflow_amd import quant as Q
from neuroflow_amd import workloads as WL
from oracle import oracle as O

pytestmark = pytest.mark.gpu

K, N = 1024, 256     # a 1024-wide layer: quantise launch + persistent GEMM through the workspace


def _layer(sid):
    W = WL.uniform(sid, (N, K), -0.125, 0.125)
    b = WL.uniform(sid + 1, (N,), -0.1, 0.1)
    return Q.Int8Linear(W, b), W, b


def _alone(lay, x):
    """The call with the device idle before and after it."""
    torch.cuda.synchronize()
    out = lay(x, "relu")
    torch.cuda.synchronize()
    return out.clone()


def _bits(t):
    return t.view(torch.int32)


def test_workspace_grows_and_shrinks_on_one_stream(gpu):
    """Calls on one stream with no synchronisation between them, sized so the
    workspace grows twice (the old buffer freed in stream order while earlier
    calls may still run) and is then reused by smaller calls."""
    lay, _, b = _layer(700)
    sizes = [100, 5000, 300, 20000, 1, 3000, 20000, 64]
    xs = [torch.from_numpy(WL.normal(710 + i, (m, K))).cuda() for i, m in enumerate(sizes)]
    want = [_alone(lay, x) for x in xs]
    torch.cuda.synchronize()
    for _ in range(2):
        outs = [lay(x, "relu") for x in xs]
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(_bits(o), _bits(w))
    # The oracle on sampled rows of the largest call.
    A = xs[4].cpu().numpy()
    rows = np.unique(np.concatenate([np.arange(0, A.shape[0], 97), [A.shape[0] - 1]]))
    ref, _ = O.layer_per_token_i8(A[rows], lay.W_q, lay.scale_W, np.zeros(N, np.int32), b, lay.sum_W, 1)
    got = want[4].cpu().numpy()[rows]
    assert np.array_equal(got.view(np.uint32), np.asarray(ref, np.float32).view(np.uint32))


def test_two_streams_run_the_split_path_at_once(gpu):
    """Two streams, each with its own workspace, interleaving calls with no
    synchronisation; a shared buffer would show as outputs of one stream
    computed from the other's codes."""
    lay, _, _ = _layer(720)
    xa = [torch.from_numpy(WL.normal(730 + i, (12000, K))).cuda() for i in range(3)]
    xb = [torch.from_numpy(WL.normal(740 + i, (9000, K))).cuda() for i in range(3)]
    wa = [_alone(lay, x) for x in xa]
    wb = [_alone(lay, x) for x in xb]
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    oa, ob = [], []
    for rep in range(3):
        for i in range(3):
            with torch.cuda.stream(sa):
                oa.append(lay(xa[i], "relu"))
            with torch.cuda.stream(sb):
                ob.append(lay(xb[i], "relu"))
    torch.cuda.synchronize()
    for k, o in enumerate(oa):
        assert torch.equal(_bits(o), _bits(wa[k % 3]))
    for k, o in enumerate(ob):
        assert torch.equal(_bits(o), _bits(wb[k % 3]))


def test_host_threads_share_one_stream(gpu):
    """Four host threads issue calls on one stream through the C entry point
    (ctypes releases the GIL, so the calls overlap on the host): one call's
    quantise and product must not be split by another call's launches."""
    lay, _, _ = _layer(750)
    stream = torch.cuda.Stream()
    xs = [torch.from_numpy(WL.normal(760 + i, (6000 + 500 * i, K))).cuda() for i in range(4)]
    want = [_alone(lay, x) for x in xs]
    outs = [[torch.empty(x.shape[0], N, device="cuda") for _ in range(6)] for x in xs]
    run = lay.launcher("relu")
    errors = []

    def worker(i):
        try:
            for r in range(6):
                run(xs[i].data_ptr(), outs[i][r].data_ptr(), xs[i].shape[0], stream.cuda_stream)
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
            assert torch.equal(_bits(outs[i][r]), _bits(want[i]))
