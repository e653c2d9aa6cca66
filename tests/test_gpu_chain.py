"""GPU parity of the 8-bit-output layer (nflow_int8_linear_forward_codes) and
the per-token layer chain (nflow_int8_mlp_forward_per_token): codes and row
scales bit-equal to the fp32 layer followed by the per-token quantise (on
the device and in the oracle), whole chains bit-equal to the layer-by-layer
chain and, with ReLU / no activation, to the oracle's per-token layers
(LinearForward per row with scale_A = absmax / 127, int8_gemm.cpp:201-470,
507-520)."""
import numpy as np
import pytest
import torch

from neuroflow_amd import quant as Q
from neuroflow_amd import workloads as WL
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ACT = {"none": O.ACT_NONE, "relu": O.ACT_RELU, "gelu": O.ACT_GELU_TANH}


def _cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _layer(N, K, sid, bias_lo=-1 / 32, bias_hi=1 / 32):
    """Per-channel symmetric INT8 layer (zp_W and sum_W left out, as the
    per-token calls pass them), and its oracle-side arrays."""
    W = WL.kaiming_uniform(sid, N, K)
    s = O.per_channel_scales(W, 127.0)
    q, _ = O.quantise_weight_2d(W, s)
    b = WL.uniform(sid + 1, (N,), bias_lo, bias_hi)
    p = Q.Int8LinearParams(W_int8=_cu(q), scale_W=_cu(s), zp_W=None, bias=_cu(b), sum_W_per_row=None)
    return p, (q, s, b)


def _no_faults():
    assert Q.chain_faults() == 0


@pytest.mark.parametrize("M,N,act", [(1000, 1024, "relu"), (4096, 1024, "relu"), (128, 256, "none"),
                                     (333, 512, "gelu"), (20000, 1024, "relu"), (40000, 512, "none"),
                                     (1, 1024, "relu"), (16513, 1024, "gelu")])
def test_codes_layer_equals_layer_then_quantise(gpu, M, N, act):
    K = 1024
    x = WL.normal(7000 + M, (M, K)) * 2.0
    x[0] = 0.0                                   # an all-zero input row
    q_in, s_in, _ = O.quantise_per_token_i8(x)
    p, (wq, ws, b) = _layer(N, K, 7100 + N)
    cq, cs = Q.linear_forward_codes(p, _cu(q_in), _cu(s_in), act)
    # The device's own two steps: fp32 output, then the per-token quantise.
    y = Q.linear_forward_quantised(p, _cu(q_in), _cu(s_in), act)
    q2, s2, _ = Q.quantise_per_token(y)
    assert np.array_equal(_host(cq), _host(q2))
    assert np.array_equal(_bits(_host(cs)), _bits(_host(s2)))
    if act != "gelu":
        # The oracle on a sample of rows: its per-token layer quantises x
        # itself (the same codes), then the next layer's per-token quantise.
        rows = np.unique(np.r_[0, min(1, M - 1), M - 1, np.linspace(0, M - 1, 64).astype(int)])
        y_ref, s_ref = O.layer_per_token_i8(x[rows], wq, ws, bias=b, act=ACT[act])
        assert np.array_equal(_bits(s_ref), _bits(s_in[rows]))
        q_ref, sc_ref, _ = O.quantise_per_token_i8(y_ref)
        assert np.array_equal(_host(cq)[rows], q_ref)
        assert np.array_equal(_bits(_host(cs)[rows]), _bits(sc_ref))
    _no_faults()


def test_codes_layer_all_zero_rows_and_ties(gpu):
    # A bias far below the products zeroes every ReLU output: scale 1, codes 0.
    M, K, N = 700, 1024, 1024
    x = WL.normal(7300, (M, K))
    q_in, s_in, _ = O.quantise_per_token_i8(x)
    p, _ = _layer(N, K, 7310, bias_lo=-1e6, bias_hi=-1e5)
    cq, cs = Q.linear_forward_codes(p, _cu(q_in), _cu(s_in), "relu")
    assert not _host(cq).any()
    assert np.all(_host(cs) == 1.0)
    # Quotients on k + 0.5: input codes 1 in column 0 only, scale 1, no
    # bias or activation, so y[m][n] = scale_W[n] * W_q[n][0], all exact:
    # y0 = 127 / 128 is the row max (scale 1 / 128), y1 = 5 / 256 and
    # y2 = -5 / 256 give quotients +-2.5, which round half away from zero to
    # +-3 (half to even would give +-2).
    Wq = np.zeros((N, K), np.int8)
    Wq[0, 0], Wq[1, 0], Wq[2, 0] = 127, 5, -5
    sw = np.full(N, 2.0 ** -7, np.float32)
    sw[1] = sw[2] = 2.0 ** -8
    qa = np.zeros((M, K), np.int8)
    qa[:, 0] = 1
    sa = np.ones(M, np.float32)
    pt = Q.Int8LinearParams(W_int8=_cu(Wq), scale_W=_cu(sw), zp_W=None, bias=None, sum_W_per_row=None)
    cq, cs = Q.linear_forward_codes(pt, _cu(qa), _cu(sa), "none")
    y = Q.linear_forward_quantised(pt, _cu(qa), _cu(sa), "none")
    q2, s2, _ = Q.quantise_per_token(y)
    assert np.array_equal(_host(cq), _host(q2))
    assert np.array_equal(_bits(_host(cs)), _bits(_host(s2)))
    want = np.zeros(N, np.int8)
    want[:3] = [127, 3, -3]
    assert np.array_equal(_host(cq), np.broadcast_to(want, (M, N)))
    assert np.all(_host(cs) == 2.0 ** -7)
    _no_faults()


@pytest.mark.parametrize("M,special,act", [(300, "nan", "relu"), (300, "nan", "none"), (300, "inf", "relu"),
                                           (300, "-inf", "none"), (20000, "nan", "relu"), (20000, "inf", "none")])
def test_codes_layer_nan_and_inf_outputs(gpu, M, special, act):
    # One column's bias NaN or +-Inf, so every row holds a NaN or an infinite
    # output: the absmax skips NaN (the reference's `a > m`), an infinite
    # absmax gives an infinite scale, and those values' codes take the exact
    # path.  Codes and scales as the fp32 layer followed by the per-token
    # quantise, on the device and in the oracle.
    K, N = 1024, 1024
    x = WL.normal(7400 + M, (M, K))
    q_in, s_in, _ = O.quantise_per_token_i8(x)
    W = WL.kaiming_uniform(7410, N, K)
    s = O.per_channel_scales(W, 127.0)
    wq, _ = O.quantise_weight_2d(W, s)
    b = WL.uniform(7411, (N,), -1 / 32, 1 / 32)
    b[5] = float(special)
    p = Q.Int8LinearParams(W_int8=_cu(wq), scale_W=_cu(s), zp_W=None, bias=_cu(b), sum_W_per_row=None)
    cq, cs = Q.linear_forward_codes(p, _cu(q_in), _cu(s_in), act)
    y = Q.linear_forward_quantised(p, _cu(q_in), _cu(s_in), act)
    q2, s2, _ = Q.quantise_per_token(y)
    assert np.array_equal(_host(cq), _host(q2))
    assert np.array_equal(_bits(_host(cs)), _bits(_host(s2)))
    rows = np.unique(np.r_[0, M - 1, np.linspace(0, M - 1, 32).astype(int)])
    y_ref, _ = O.layer_per_token_i8(x[rows], wq, s, bias=b, act=ACT[act])
    q_ref, sc_ref, _ = O.quantise_per_token_i8(y_ref)
    assert np.array_equal(_host(cq)[rows], q_ref)
    assert np.array_equal(_bits(_host(cs)[rows]), _bits(sc_ref))
    _no_faults()


@pytest.mark.parametrize("M,N", [(1, 1024), (100, 512), (129, 1024), (1000, 256), (4097, 1024), (33000, 1024)])
def test_codes_layer_writes_only_its_rows(gpu, M, N):
    """Outputs as views at the start of larger buffers (256 more rows, so a
    stray write of a partial row tile stays inside them): every element past
    row M keeps its sentinel, and the rows equal a plain call's."""
    K = 1024
    x = WL.normal(7200 + M, (M, K))
    q_in, s_in, _ = O.quantise_per_token_i8(x)
    p, _ = _layer(N, K, 7210 + N)
    big_q = torch.full((M + 256, N), 90, dtype=torch.int8, device="cuda")
    big_s = torch.full((M + 256,), -7.0, dtype=torch.float32, device="cuda")
    cq, cs = Q.linear_forward_codes(p, _cu(q_in), _cu(s_in), "relu", out=(big_q[:M], big_s[:M]))
    assert bool((big_q[M:] == 90).all()), "codes written past row M"
    assert bool((big_s[M:] == -7.0).all()), "row scales written past row M"
    cq2, cs2 = Q.linear_forward_codes(p, _cu(q_in), _cu(s_in), "relu")
    assert np.array_equal(_host(cq), _host(cq2))
    assert np.array_equal(_bits(_host(cs)), _bits(_host(cs2)))
    # A fused chain's fp32 output likewise.
    ps = [_layer(1024, K, 7230)[0], _layer(256, 1024, 7240)[0]]
    xin = _cu(x)
    big_y = torch.full((M + 256, 256), -3.0, dtype=torch.float32, device="cuda")
    y = Q.mlp_forward_per_token(ps, xin, ["relu", "none"], out=big_y[:M])
    assert bool((big_y[M:] == -3.0).all()), "chain output written past row M"
    assert np.array_equal(_bits(_host(y)), _bits(_host(_layer_by_layer(ps, ["relu", "none"], xin))))
    _no_faults()


def _chain_params(wl):
    ps, ref = [], []
    for l, L in enumerate(wl.layers):
        N, K = L.W.shape
        s = O.per_channel_scales(L.W, 127.0)
        q, _ = O.quantise_weight_2d(L.W, s)
        ps.append(Q.Int8LinearParams(W_int8=_cu(q), scale_W=_cu(s), zp_W=None, bias=_cu(L.bias),
                                     sum_W_per_row=None))
        ref.append((q, s, L.bias, L.act))
    return ps, ref


def _layer_by_layer(ps, acts, x):
    h = x
    for p, a in zip(ps, acts):
        h = Q.linear_forward_per_token(p, h, a)
    return h


def _oracle_chain(ref, x):
    h = x
    for q, s, b, a in ref:
        h, _ = O.layer_per_token_i8(h, q, s, bias=b, act=ACT[a])
    return h


@pytest.mark.parametrize("which", ["trunk", "branch"])
def test_mlp_chain_full_size_c5(gpu, which):
    """The DeepONet MLPs at their full sizes (trunk 65536 x 1024 through
    3 x (1024 -> 1024, ReLU) and 1024 -> 256; branch 4096 x 1024 through
    4 x (1024 -> 1024, ReLU)): the fused chain equals the layer-by-layer
    chain on every row, and the oracle on a sample of rows."""
    wl = WL.c5_deeponet_trunk() if which == "trunk" else WL.c5_deeponet_branch()
    ps, ref = _chain_params(wl)
    acts = [L.act for L in wl.layers]
    x = _cu(wl.x)
    y = Q.mlp_forward_per_token(ps, x, acts)
    y_l = _layer_by_layer(ps, acts, x)
    assert np.array_equal(_bits(_host(y)), _bits(_host(y_l)))
    rows = np.unique(np.r_[0, wl.M - 1, np.linspace(0, wl.M - 1, 200).astype(int)])
    y_ref = _oracle_chain(ref, wl.x[rows])
    assert np.array_equal(_bits(_host(y)[rows]), _bits(y_ref))
    _no_faults()


@pytest.mark.parametrize("M", [1, 127, 129, 1000, 5000, 33333])
def test_mlp_chain_ragged_rows_and_repeats(gpu, M):
    """Partial row tiles, both tile widths, and back-to-back calls of
    different sizes on one stream (each launch's published row maxima carry
    a new epoch: an earlier call's must never read as fresh)."""
    ps, ref, acts = [], [], ["relu", "gelu", "relu", "none"]
    for l in range(4):
        N = 1024 if l < 3 else 384
        p, r = _layer(N, 1024, 7400 + 10 * l)
        ps.append(p)
        ref.append(r + (acts[l],))
    for rep in range(2):
        x = WL.normal(7500 + M + rep, (M, 1024))
        xs = _cu(x)
        y = Q.mlp_forward_per_token(ps, xs, acts)
        y_l = _layer_by_layer(ps, acts, xs)
        assert np.array_equal(_bits(_host(y)), _bits(_host(y_l))), f"repeat {rep}"
        # A smaller call in between leaves stale words past its rows.
        small = WL.normal(7600 + rep, (max(1, M // 3), 1024))
        ys = Q.mlp_forward_per_token(ps, _cu(small), acts)
        assert np.array_equal(_bits(_host(ys)), _bits(_host(_layer_by_layer(ps, acts, _cu(small)))))
    _no_faults()


def test_mlp_chain_relu_oracle_small(gpu):
    M = 300
    ps, ref, acts = [], [], ["relu", "relu", "none"]
    for l in range(3):
        N = 1024 if l < 2 else 256
        p, r = _layer(N, 1024, 7700 + 10 * l)
        ps.append(p)
        ref.append(r + (acts[l],))
    x = WL.normal(7800, (M, 1024)) * 5.0
    x[3] = 0.0
    y = Q.mlp_forward_per_token(ps, _cu(x), acts)
    assert np.array_equal(_bits(_host(y)), _bits(_oracle_chain(ref, x)))
    _no_faults()


def test_mlp_chain_unfused_layers(gpu):
    """Layers the fused kernel does not take (asymmetric weights, widths
    other than 1024) run layer by layer, with the same results."""
    M, K = 500, 512
    W1 = WL.kaiming_uniform(7900, 768, K)
    s1 = O.per_channel_scales(W1, 127.0)
    zp1 = WL.uniform(7901, (768,), -5, 5).astype(np.int32)
    q1, sw1 = O.quantise_weight_2d(W1, s1, zp1)
    b1 = WL.uniform(7902, (768,), -0.05, 0.05)
    p1 = Q.Int8LinearParams(W_int8=_cu(q1), scale_W=_cu(s1), zp_W=_cu(zp1), bias=_cu(b1), sum_W_per_row=None)
    p2, _ = _layer(100, 768, 7910)
    x = _cu(WL.normal(7920, (M, K)))
    y = Q.mlp_forward_per_token([p1, p2], x, ["gelu", "none"])
    y_l = _layer_by_layer([p1, p2], ["gelu", "none"], x)
    assert np.array_equal(_bits(_host(y)), _bits(_host(y_l)))
    # The single 8-bit-output layer on such a layer takes its fallback.
    q_in, s_in, _ = Q.quantise_per_token(x)
    cq, cs = Q.linear_forward_codes(p1, q_in, s_in, "gelu")
    q2, s2, _ = Q.quantise_per_token(Q.linear_forward_quantised(p1, q_in, s_in, "gelu"))
    assert np.array_equal(_host(cq), _host(q2))
    assert np.array_equal(_bits(_host(cs)), _bits(_host(s2)))


def test_mlp_chain_rejects_bad_chains(gpu):
    p1, _ = _layer(1024, 1024, 8000)
    p2, _ = _layer(256, 512, 8010)
    x = _cu(WL.normal(8020, (10, 1024)))
    with pytest.raises(Exception, match="ShapeMismatch|in_features"):
        Q.mlp_forward_per_token([p1, p2], x, ["relu", "none"])


@pytest.mark.skip(reason="faulted the GPU (illegal memory access) on its first replay when the chain entry points "
                         "took a layer-by-layer route inside the capture, allocating their buffers in the graph; the "
                         "cause was not found in the library, which now refuses capture in these entry points "
                         "(test_chain_entry_points_refuse_graph_capture)")
def test_chain_entry_points_under_graph_capture(gpu):
    """Captured into a HIP graph, both chain entry points take the
    layer-by-layer route (no row-maxima words or launch epochs recorded in
    the graph): every replay, with new input values and eager fused calls on
    the stream between replays, equals the eager call bit for bit."""
    M = 20000
    ps, acts = [], ["relu", "relu", "relu", "none"]
    for l in range(4):
        p, _ = _layer(1024 if l < 3 else 256, 1024, 8100 + 10 * l)
        ps.append(p)
    x = torch.empty(M, 1024, dtype=torch.float32, device="cuda")
    y = torch.empty(M, 256, dtype=torch.float32, device="cuda")
    q_in = torch.empty(M, 1024, dtype=torch.int8, device="cuda")
    s_in = torch.empty(M, dtype=torch.float32, device="cuda")
    cq = torch.empty(M, 1024, dtype=torch.int8, device="cuda")
    cs = torch.empty(M, dtype=torch.float32, device="cuda")
    x.copy_(_cu(WL.normal(8150, (M, 1024))))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        Q.mlp_forward_per_token(ps, x, acts, out=y)
        Q.linear_forward_codes(ps[0], q_in, s_in, "relu", out=(cq, cs))
    for r in range(3):
        xr = _cu(WL.normal(8160 + r, (M, 1024)) * (1.0 + r))
        qr, sr, _ = Q.quantise_per_token(xr)
        x.copy_(xr)
        q_in.copy_(qr)
        s_in.copy_(sr)
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want_y = Q.mlp_forward_per_token(ps, xr, acts)              # eager, fused
        want_q, want_s = Q.linear_forward_codes(ps[0], qr, sr, "relu")
        assert np.array_equal(_bits(_host(y)), _bits(_host(want_y))), f"replay {r}"
        assert np.array_equal(_host(cq), _host(want_q)), f"replay {r}"
        assert np.array_equal(_bits(_host(cs)), _bits(_host(want_s))), f"replay {r}"
    _no_faults()


def test_chain_entry_points_refuse_graph_capture(gpu):
    """On a stream being captured into a graph both chain entry points
    return NFLOW_UNSUPPORTED_OP before allocating or launching anything (the
    capture ends empty), and the stream works as before afterwards."""
    import ctypes as C
    from neuroflow_amd import _lib
    M = 256
    p, _ = _layer(1024, 1024, 8200)
    ps = (_lib.Int8LinearParamsC * 2)(p.c_struct(), p.c_struct())
    acts = (C.c_int * 2)(1, 1)
    x = _cu(WL.normal(8210, (M, 1024)))
    y = torch.empty(M, 1024, dtype=torch.float32, device="cuda")
    qa, sa, _ = Q.quantise_per_token(x)
    cq = torch.empty(M, 1024, dtype=torch.int8, device="cuda")
    cs = torch.empty(M, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    L = _lib.lib()
    rcs = []
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sp = torch.cuda.current_stream().cuda_stream
        rcs.append(L.nflow_int8_mlp_forward_per_token(ps, acts, 2, M, x.data_ptr(), y.data_ptr(), sp))
        rcs.append(L.nflow_int8_linear_forward_codes(C.byref(p.c_struct()), M, qa.data_ptr(), sa.data_ptr(),
                                                     cq.data_ptr(), cs.data_ptr(), 1, sp))
    assert rcs == [_lib.UNSUPPORTED_OP, _lib.UNSUPPORTED_OP]
    # Eager afterwards: the same results as layer by layer.
    y2 = Q.mlp_forward_per_token([p, p], x, ["relu", "relu"])
    assert np.array_equal(_bits(_host(y2)), _bits(_host(_layer_by_layer([p, p], ["relu", "relu"], x))))
    _no_faults()
