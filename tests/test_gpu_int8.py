"""GPU parity of the INT8 path against the oracle (bit-exact codes, int32
accumulators and dequantised outputs; GELU within 1e-5 rel / 1e-6 abs)."""
import contextlib
import ctypes
import functools
from pathlib import Path

import numpy as np
import pytest
import torch

from neuroflow_amd import _lib
from neuroflow_amd import quant as Q
from neuroflow_amd import workloads as WL
from oracle import oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6   # floating-point tolerance for the fp32 outputs


def _cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def _weights(N, K, sid, zp=False):
    W = WL.uniform(sid, (N, K), -0.125, 0.125)
    s = O.per_channel_scales(W, 127.0)
    zps = (WL.uniform(sid + 1, (N,), -6, 6).astype(np.int32) if zp else np.zeros(N, np.int32))
    q, sw = O.quantise_weight_2d(W, s, zps)
    b = WL.uniform(sid + 2, (N,), -0.1, 0.1)
    return W, q, s, zps, sw, b


@pytest.mark.parametrize("M,K", [(1, 64), (37, 64), (1000, 64), (513, 256), (77, 100), (64, 1024),
                                 (33, 4), (31, 512), (66, 1024), (20001, 256), (3, 2048)])
def test_quantise_per_token_codes_bit_exact(gpu, M, K):
    A = WL.normal(11, (M, K)) * 3.0
    A[0, 0] = 0.0
    if M > 2:
        A[1] = 0.0                      # an all-zero row -> scale 1
        A[2, : min(K, 8)] = np.array([1.5, -2.5, 0.5, -0.5, 127.0, -127.0, 2.5, 3.5][: min(K, 8)])
    q, s, sa = Q.quantise_per_token(_cu(A))
    q_ref, s_ref, sa_ref = O.quantise_per_token_i8(A)
    assert _bits_equal(_host(s), s_ref)
    assert np.array_equal(_host(q), q_ref)
    assert np.array_equal(_host(sa), sa_ref)


def test_quantise_per_token_ties_and_specials(gpu):
    # Rows whose quotients land exactly on k + 0.5 (absmax 127 -> scale 1).
    K = 64
    A = np.zeros((4, K), np.float32)
    A[:, 0] = 127.0
    A[0, 1:] = np.arange(1, K, dtype=np.float32) * 0.5 - 16.0
    A[1, 1:] = -(np.arange(1, K, dtype=np.float32) * 0.5)
    A[2, 1:5] = [np.nan, 3.5, -3.5, 1e-30]
    A[3, 0] = np.inf
    A[3, 1:4] = [1.0, -np.inf, 0.0]
    q, s, _ = Q.quantise_per_token(_cu(A))
    q_ref, s_ref, _ = O.quantise_per_token_i8(A)
    assert _bits_equal(_host(s), s_ref)
    assert np.array_equal(_host(q), q_ref)


@pytest.mark.parametrize("K", [256, 512, 1024, 2048])
def test_quantise_per_token_special_rows_wide(gpu, K):
    """The register-resident quantise (K = 256 KV) on exact ties, zero, NaN,
    signalling NaN, infinite and subnormal rows: codes, scales and sums."""
    A = (WL.normal(42, (9, K)) * 3.0).astype(np.float32)
    A[0, 0] = 127.0
    A[0, 1:] = (np.arange(1, K, dtype=np.float32) % 200 - 100.0) * 0.5   # k + 0.5 ties
    A[1] = 0.0
    A[2] = np.nan
    A[3, 9] = np.nan
    A.view(np.uint32)[4, 3] = 0x7F800001
    A[5, 2] = np.inf
    A[6] = 1e-40
    A[7, :] *= 3e-37 / np.abs(A[7]).max()
    q, s, sa = Q.quantise_per_token(_cu(A))
    q_ref, s_ref, sa_ref = O.quantise_per_token_i8(A)
    assert _bits_equal(_host(s), s_ref)
    assert np.array_equal(_host(q), q_ref)
    assert np.array_equal(_host(sa), sa_ref)


@pytest.mark.parametrize("scale,zp", [(0.05, 0), (0.05, 3), (0.03, -7), (0.0, 0), (1.0, 100)])
def test_quantise_activation_bit_exact(gpu, scale, zp):
    A = WL.normal(12, (300, 96)) * 4.0
    A[0, :6] = [np.nan, np.inf, -np.inf, 3e9, -3e9, 0.5]
    got = _host(Q.quantise_activation(_cu(A), scale, zp))
    assert np.array_equal(got, O.quantise_activation(A, scale, zp))


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (100, 64, 64), (1000, 48, 64), (257, 768, 256),
                                   (33, 256, 1024), (50, 20, 100), (64, 1024, 1024)])
def test_gemm_i32_bit_exact(gpu, M, N, K):
    A = WL.uniform(13, (M, K), -128, 128).astype(np.int64).clip(-128, 127).astype(np.int8)
    W = WL.uniform(14, (N, K), -128, 128).astype(np.int64).clip(-128, 127).astype(np.int8)
    A[0, :] = -128
    W[0, :] = -128
    got = _host(Q.gemm_i32(_cu(A), _cu(W)))
    assert np.array_equal(got, O.gemm_i8_i32(A, W))


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (1000, 64, 64), (513, 768, 256), (300, 256, 256),
                                   (40, 64, 100), (16, 64, 4)])
@pytest.mark.parametrize("act", ["none", "relu", "gelu"])
def test_per_token_layer(gpu, M, N, K, act):
    A = WL.normal(15, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 16)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), sum_W_per_row=_cu(sw))
    out, sa = Q.linear_forward_per_token(p, _cu(A), act, return_scales=True)
    ref, sa_ref = O.layer_per_token_i8(A, q, s, zps, b, sw, {"none": 0, "relu": 1, "gelu": 2}[act])
    out = _host(out)
    assert _bits_equal(_host(sa), sa_ref)
    if act == "gelu":
        np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)
    else:
        assert _bits_equal(out, ref)        # dequant + bias (+ relu) is bit-exact


@pytest.mark.parametrize("M", [200, 140000])
def test_symmetric_weights_with_a_mismatched_sum_w(gpu, M):
    """Zero weight zero points, zp_A = 0 and a caller's sum_W that is not the
    weights' byte sums, at K = N = 64 (the K = 64 kernel, static deal and tile
    queue): the batched formula uses sum_W only times zp_A, the per-row (VNNI)
    formula adds 128 (byte sum - sum_W), and the per-token layer (no zero
    points at all) takes the same term.  Each equals the oracle bit for bit,
    so the kernel's choice of which integer terms to form follows the
    formula, not the weights."""
    N = K = 64
    A = WL.normal(21, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 22)          # zps: zeros
    sumW = (sw + (np.arange(N, dtype=np.int32) % 9) - 4).astype(np.int32)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), scale_A=0.02, zp_A=0, sum_W_per_row=_cu(sumW))
    rows = np.unique(np.concatenate([np.arange(0, M, max(1, M // 300)), [M - 1]]))
    rc, ref_b = O.linear_forward_batched(A[rows], q, s, zps, b, 0.02, 0, sumW)
    assert rc == 0
    assert _bits_equal(_host(Q.linear_forward_batched(p, _cu(A)))[rows], ref_b)
    rc, ref_r = O.linear_forward_rows(A[rows], q, s, zps, b, 0.02, 0, sumW)
    assert rc == 0
    assert _bits_equal(_host(Q.linear_forward(p, _cu(A)))[rows], ref_r)
    pt = Q.Int8LinearParams(_cu(q), _cu(s), None, _cu(b), sum_W_per_row=_cu(sumW))
    out = _host(Q.linear_forward_per_token(pt, _cu(A), "relu"))
    ref_t, _ = O.layer_per_token_i8(A[rows], q, s, None, b, sumW, 1)
    assert _bits_equal(out[rows], ref_t)


@pytest.mark.parametrize("M,N,K", [(200, 64, 64), (100, 768, 256), (30, 64, 100)])
@pytest.mark.parametrize("zp_a", [0, 5])
@pytest.mark.parametrize("with_sum", [False, True])
def test_linear_forward_matches_reference_formulas(gpu, M, N, K, zp_a, with_sum):
    """LinearForward (per row) and LinearForwardBatched, asymmetric weights."""
    A = WL.normal(17, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 18, zp=True)
    sumW = sw if with_sum else None
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), scale_A=0.02, zp_A=zp_a,
                           sum_W_per_row=None if sumW is None else _cu(sumW))
    rc, ref_rows = O.linear_forward_rows(A, q, s, zps, b, 0.02, zp_a, sumW)
    assert rc == 0
    assert _bits_equal(_host(Q.linear_forward(p, _cu(A))), ref_rows)
    assert _bits_equal(_host(Q.linear_forward(p, _cu(A[0]))), ref_rows[0])
    rc, ref_b = O.linear_forward_batched(A, q, s, zps, b, 0.02, zp_a, sumW)
    assert rc == 0
    assert _bits_equal(_host(Q.linear_forward_batched(p, _cu(A))), ref_b)


@pytest.mark.parametrize("zp_a", [0, 5])
@pytest.mark.parametrize("with_sum", [False, True])
def test_linear_forward_scalar_formula_k4100_reference_vectors(gpu, zp_a, with_sum):
    """Above K = 4096 the reference turns its SIMD path off (int8_gemm.cpp:218)
    and LinearForward takes the scalar loop with its own zero-point
    correction (:436-466); LinearForwardBatched keeps its formula
    (:530-580).  The reference build's own outputs at K = 4100, asymmetric
    weights, zp_A 0 / 5, with and without sum_W."""
    fix = np.load(Path(__file__).resolve().parent / "golden" / "ref_int8_vectors.npz")
    q, s, zps, b, X = (fix[f"lf4100_{n}"] for n in ("Wq", "sW", "zpW", "b", "X"))
    sumW = fix["lf4100_sumW_ref"] if with_sum else None
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), scale_A=0.02, zp_A=zp_a,
                           sum_W_per_row=None if sumW is None else _cu(sumW))
    tag = f"zp{zp_a}_sum{int(with_sum)}"
    assert _bits_equal(_host(Q.linear_forward(p, _cu(X))), fix[f"lf4100_rows_{tag}"])
    assert _bits_equal(_host(Q.linear_forward(p, _cu(X[1]))), fix[f"lf4100_rows_{tag}"][1])
    assert _bits_equal(_host(Q.linear_forward_batched(p, _cu(X))), fix[f"lf4100_batched_{tag}"])


@pytest.mark.parametrize("M,N,K", [(50, 64, 4100), (37, 30, 8192), (3, 5, 4097)])
@pytest.mark.parametrize("zp_a", [0, 5])
@pytest.mark.parametrize("with_sum", [False, True])
def test_linear_forward_scalar_formula_random(gpu, M, N, K, zp_a, with_sum):
    """The K > 4096 formulas on random asymmetric layers against the oracle
    (pinned to the reference build by the K = 4100 vectors above)."""
    A = WL.normal(19, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 20, zp=True)
    sumW = (sw + (np.arange(N, dtype=np.int32) % 7) - 3).astype(np.int32) if with_sum else None
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), scale_A=0.02, zp_A=zp_a,
                           sum_W_per_row=None if sumW is None else _cu(sumW))
    rc, ref_rows = O.linear_forward_rows(A, q, s, zps, b, 0.02, zp_a, sumW)
    assert rc == 0
    assert _bits_equal(_host(Q.linear_forward(p, _cu(A))), ref_rows)
    rc, ref_b = O.linear_forward_batched(A, q, s, zps, b, 0.02, zp_a, sumW)
    assert rc == 0
    assert _bits_equal(_host(Q.linear_forward_batched(p, _cu(A))), ref_b)


# The fixed-scale K = N = 64 kernel (k_rows64 FIXED, what LinearForwardBatched
# and LinearForward run at the FNO local-linear shape): sizes with one tile per
# wave (1000), several (262144) and the doubled grid with a partial last tile
# (1048581); scales in the reciprocal fast path, at powers of two (exact ties
# k + 0.5), zero (every quotient inf / NaN), below and above its range.
FIXED_SCALES = [(0.02, 0), (0.02, 5), (0.25, -3), (0.0, 0), (1e-38, 2), (3e36, 4), (1e30, 3)]


@functools.lru_cache(maxsize=4)
def _fixed_input(M):
    return WL.normal(70, (M, 64)) * 3.0


@pytest.mark.parametrize("M", [1, 1000, 262144, 1048581])
@pytest.mark.parametrize("scale,zp_a", FIXED_SCALES)
@pytest.mark.parametrize("form", ["batched", "rows"])
def test_fixed_scale_k64_kernel(gpu, M, scale, zp_a, form):
    N = K = 64
    A = _fixed_input(M).copy()
    if M >= 16:
        A[1, :] = (np.arange(K, dtype=np.float32) - 32.0 + 0.5) * 0.25    # ties when scale = 0.25
        A[2, :8] = [np.nan, np.inf, -np.inf, 3e9, -3e9, 1e-40, -0.0, 1e38]
        A[3, :] = 0.0
        A[M // 2, :] = (np.arange(K, dtype=np.float32) + 0.5) * 0.02      # near-ties at 0.02
    _, q, s, zps, sw, b = _weights(N, K, 71, zp=True)
    sumW = sw if form == "batched" else None
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), scale_A=scale, zp_A=zp_a,
                           sum_W_per_row=None if sumW is None else _cu(sumW))
    x = _cu(A)
    run = Q.linear_forward_batched if form == "batched" else Q.linear_forward
    got = _host(run(p, x))
    rows = np.arange(M) if M <= 4096 else np.unique(np.concatenate(
        [np.arange(1024), np.arange(M - 4096, M), np.arange(0, M, 61), [M // 2]]))
    oracle = O.linear_forward_batched if form == "batched" else O.linear_forward_rows
    rc, want = oracle(A[rows], q, s, zps, b, scale, zp_a, sumW)
    assert rc == 0
    fin = ~np.isnan(want)
    assert np.array_equal(np.isnan(got[rows]), ~fin)
    assert _bits_equal(got[rows][fin], want[fin])
    if M <= 262144:
        with _env(NFLOW_NO_ROWS64="1"):
            generic = _host(run(p, x))
        keep = ~np.isnan(generic)
        assert np.array_equal(np.isnan(got), ~keep)
        assert _bits_equal(got[keep], generic[keep])


def test_quantised_entry_matches_fused(gpu):
    M, N, K = 4096, 1024, 1024
    A = np.maximum(WL.normal(19, (M, K)), 0)
    W = WL.kaiming_uniform(20, N, K)
    layer = Q.Int8Linear(W, WL.uniform(21, (N,), -0.03, 0.03))
    Aq, sa, _ = Q.quantise_per_token(_cu(A))
    y1 = _host(Q.linear_forward_quantised(layer.params, Aq, sa, "relu"))
    y2 = _host(layer(_cu(A), "relu"))
    assert _bits_equal(y1, y2)
    ref, _ = O.layer_per_token_i8(A[:64], layer.W_q, layer.scale_W, None,
                                  WL.uniform(21, (N,), -0.03, 0.03), layer.sum_W, 1)
    assert _bits_equal(y1[:64], ref)


@pytest.mark.parametrize("zp_none", [False, True])
@pytest.mark.parametrize("sum_mode", ["none", "own", "off"])
def test_quantised_entry_param_forms(gpu, zp_none, sum_mode):
    """linear_forward_quantised with and without zp_W / sum_W (the GEMM picks
    its kernel from them; a sum_W off the weights' own sums enters the
    formula verbatim)."""
    M, N, K = 3000, 512, 320
    A = WL.normal(24, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 25)
    sumW = {"none": None, "own": sw, "off": (sw + 3).astype(np.int32)}[sum_mode]
    p = Q.Int8LinearParams(_cu(q), _cu(s), None if zp_none else _cu(zps), _cu(b),
                           sum_W_per_row=None if sumW is None else _cu(sumW))
    Aq, sa, _ = Q.quantise_per_token(_cu(A))
    y = _host(Q.linear_forward_quantised(p, Aq, sa, "none"))
    rows = np.unique(np.concatenate([np.arange(0, M, 29), [M - 1]]))
    ref, _ = O.layer_per_token_i8(A[rows], q, s, zps, b, sumW, 0)
    assert _bits_equal(y[rows], ref)


def test_precompute_sum_w(gpu):
    _, q, s, zps, sw, b = _weights(300, 200, 22, zp=True)
    got = _host(Q.precompute_sum_w(_cu(q), _cu(zps)))
    assert np.array_equal(got, O.precompute_sum_w(q, zps))


def test_status_codes(gpu):
    from neuroflow_amd._lib import NflowError
    _, q, s, zps, sw, b = _weights(64, 64, 23)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b))
    x = torch.zeros(0, 64, device="cuda")
    assert Q.linear_forward_batched(p, x).shape == (0, 64)        # bsz <= 0 -> Ok, no work
    with pytest.raises(ValueError):
        Q.linear_forward_per_token(p, torch.zeros(4, 32, device="cuda"))
    with pytest.raises(ValueError):
        Q.linear_forward_per_token(p, torch.zeros(4, 64, device="cuda"), activation="swish")
    import ctypes
    from neuroflow_amd import _lib
    ps = p.c_struct()
    ps.W_int8 = None
    rc = _lib.lib().nflow_int8_linear_forward(ctypes.byref(ps), None, None, None)
    assert rc == _lib.INVALID_ARG
    assert b"null" in _lib.lib().nflow_last_error()
    with pytest.raises(NflowError) as ei:
        _lib.check(rc, "Int8Linear")
    assert ei.value.code == _lib.INVALID_ARG


@pytest.mark.parametrize("act", ["none", "gelu"])
def test_fused_k64_layer_special_rows(gpu, act):
    """The K = N = 64 fused layer on rows that exercise its exact slow path
    (quotients on k + 0.5), zero rows, NaN / Inf and tiny values."""
    M, K, N = 67, 64, 64
    A = WL.normal(50, (M, K))
    A[1] = 0.0
    A[2, 0] = 127.0
    A[2, 1:] = (np.arange(1, K, dtype=np.float32) - 32.0) * 0.5      # k + 0.5 ties
    A[3, 0] = -127.0
    A[3, 1:] = (np.arange(1, K, dtype=np.float32) * 0.5)
    A[4, 5] = np.nan
    A[5, 7] = np.inf
    A[6] = 1e-30
    A[7, :3] = [1e30, -1e30, 2.5]
    A[8] = np.nan                                   # every element NaN: scale 1
    A[9, :4] = np.nan                               # one lane's whole chunk NaN
    A.view(np.uint32)[10, 3] = 0x7F800001          # signalling NaN
    A[11] = -0.0
    A[12] = 1e-40                                   # subnormal absmax
    A[13, :] *= 3e-37 / np.abs(A[13]).max()         # normal absmax, subnormal scale
    A[14] = -np.inf
    _, q, s, zps, sw, b = _weights(N, K, 51)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), sum_W_per_row=_cu(sw))
    out, sa = Q.linear_forward_per_token(p, _cu(A), act, return_scales=True)
    ref, sa_ref = O.layer_per_token_i8(A, q, s, zps, b, sw, {"none": 0, "gelu": 2}[act])
    out = _host(out)
    assert _bits_equal(_host(sa), sa_ref)
    if act == "none":
        finite = np.isfinite(ref)
        assert _bits_equal(out[finite], ref[finite])
        assert np.array_equal(np.isnan(out), np.isnan(ref))
    else:
        np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)


def test_fused_k64_layer_asymmetric_weights(gpu):
    """Zero points in the K = N = 64 fused layer reproduce LinearForward's formula."""
    M, K, N = 300, 64, 64
    A = WL.normal(52, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 53, zp=True)
    for sumW in (None, sw):
        p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b),
                               sum_W_per_row=None if sumW is None else _cu(sumW))
        out = _host(Q.linear_forward_per_token(p, _cu(A), "none"))
        ref, _ = O.layer_per_token_i8(A, q, s, zps, b, sumW, 0)
        assert _bits_equal(out, ref)


# ---- the tiled GEMM (K a multiple of 64, K >= 128): every tile shape ----------

# (M, N, K) choosing the 256x256, 128x256 and 128x128 block tiles on 256 CUs.
GEMM_SHAPES = [(16384, 1024, 256), (8192, 1024, 128), (2000, 200, 192), (1, 64, 128), (500, 256, 320)]
# Tile shapes forced through NFLOW_GEMM_TILE: "TM TN", a block tile of 32 TM x 32 TN outputs
# (None: the launcher's choice).
GEMM_TILES = [None, "22", "24", "44", "48", "88"]


@contextlib.contextmanager
def _env(**kv):
    """Kernel-selection overrides through nflow_debug_set_kernel_path
    (NFLOW_NO_TOKEN_GEMM="1" -> "no_token_gemm" = 1, NFLOW_GEMM_TILE="22" ->
    "gemm_tile" = 22; None -> 0), restored afterwards."""
    L = _lib.lib()
    old = {}
    try:
        for k, v in kv.items():
            name = k[len("NFLOW_"):].lower().encode()
            prev = ctypes.c_int(0)
            _lib.check(L.nflow_debug_set_kernel_path(name, int(v) if v is not None else 0, ctypes.byref(prev)),
                       "debug_set_kernel_path")
            old[name] = prev.value
        yield
    finally:
        for name, v in old.items():
            _lib.check(L.nflow_debug_set_kernel_path(name, v, None), "debug_set_kernel_path")


@pytest.mark.parametrize("tile", GEMM_TILES)
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_i32_tile_shapes(gpu, M, N, K, tile):
    """int32 accumulators of every tile shape, bit-exact; the float64 product
    is exact here (|sum| <= K * 128^2 < 2^24)."""
    A = WL.uniform(30, (M, K), -128, 128).astype(np.int64).clip(-128, 127).astype(np.int8)
    W = WL.uniform(31, (N, K), -128, 128).astype(np.int64).clip(-128, 127).astype(np.int8)
    A[-1, :] = -128
    W[-1, :] = -128
    with _env(NFLOW_GEMM_TILE=tile):
        got = _host(Q.gemm_i32(_cu(A), _cu(W)))
    want = (A.astype(np.float64) @ W.astype(np.float64).T).astype(np.int64)
    assert np.array_equal(got, want)


# The per-token layer's paths: "tiled" forces quantise + tiled GEMM where the
# one-pass kernel (K = 128 / 256 / 512, N % 64 = 0) would take the shape.
PATHS = {"auto": {}, "tiled": {"NFLOW_NO_TOKEN_GEMM": "1"}, "tiled22": {"NFLOW_NO_TOKEN_GEMM": "1",
                                                                       "NFLOW_GEMM_TILE": "22"},
         "pipe": {"NFLOW_NO_TOKEN_GEMM": "1", "NFLOW_NO_WIDE": "1"}}


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES[:3])
@pytest.mark.parametrize("act", ["none", "gelu"])
def test_gemm_per_token_layer_tile_shapes(gpu, M, N, K, act, path):
    """The per-token layer through quantise + tiled GEMM (or the one-pass
    kernel), on sampled rows (each output row depends only on its input row)."""
    A = WL.normal(32, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 33)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), sum_W_per_row=_cu(sw))
    with _env(**PATHS[path]):
        out, sa = Q.linear_forward_per_token(p, _cu(A), act, return_scales=True)
    out, sa = _host(out), _host(sa)
    rows = np.unique(np.concatenate([np.arange(0, M, 97), [M - 1]]))
    ref, sa_ref = O.layer_per_token_i8(A[rows], q, s, zps, b, sw, {"none": 0, "gelu": 2}[act])
    assert _bits_equal(sa[rows], sa_ref)
    if act == "gelu":
        np.testing.assert_allclose(out[rows], ref, rtol=RTOL, atol=ATOL)
    else:
        assert _bits_equal(out[rows], ref)


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("M,N,K", [(300, 256, 256), (70, 512, 1024), (9000, 1024, 128),
                                   (16384, 1024, 256), (8192, 1024, 128)])
@pytest.mark.parametrize("with_sum", [False, True])
def test_gemm_layer_asymmetric_weights(gpu, M, N, K, with_sum, path):
    """Zero points through the tiled GEMM: the row code sums and weight sums it
    accumulates feed LinearForward's formula (int8_gemm.cpp:386-393, 461-467)."""
    A = WL.normal(34, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 35, zp=True)
    sumW = sw if with_sum else None
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b),
                           sum_W_per_row=None if sumW is None else _cu(sumW))
    with _env(**PATHS[path]):
        out = _host(Q.linear_forward_per_token(p, _cu(A), "none"))
    rows = np.unique(np.concatenate([np.arange(0, M, 13), [M - 1]]))
    ref, _ = O.layer_per_token_i8(A[rows], q, s, zps, b, sumW, 0)
    assert _bits_equal(out[rows], ref)


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("M,N,K", [(300, 256, 256), (16384, 1024, 320), (64, 1024, 1024)])
def test_gemm_layer_given_sum_w_not_matching(gpu, M, N, K, path):
    """A caller-given sum_W_per_row that is not the weights' byte sum enters
    the row-VNNI formula verbatim (int8_gemm.cpp:386-393): the tiled GEMM must
    then form each column's own byte sum to reproduce it."""
    A = WL.normal(36, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 37)
    sw_bad = (sw + np.arange(N, dtype=np.int32) % 11 - 5).astype(np.int32)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), sum_W_per_row=_cu(sw_bad))
    with _env(**PATHS[path]):
        out = _host(Q.linear_forward_per_token(p, _cu(A), "relu"))
    rows = np.unique(np.concatenate([np.arange(0, M, 17), [M - 1]]))
    ref, _ = O.layer_per_token_i8(A[rows], q, s, zps, b, sw_bad, 1)
    assert _bits_equal(out[rows], ref)


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (63, 192, 128), (65, 64, 256), (1000, 768, 256),
                                   (130, 256, 512), (64, 1024, 512), (33000, 128, 512)])
@pytest.mark.parametrize("form", ["sym", "zp", "zp_sum_off"])
@pytest.mark.parametrize("act", ["none", "relu", "gelu"])
def test_token_gemm_layer(gpu, M, N, K, form, act):
    """The one-pass per-token layer for K = 128 / 256 / 512 (quantise into
    LDS, then every column block) against LinearForward per row with the
    row's scale: bit-exact codes' scales and, before GELU, bit-exact outputs;
    with zero points and a caller's sum_W off the weights' own sums; rows with
    exact ties, NaN, +-Inf and all zeros; equal to the split path."""
    A = WL.normal(60 + K, (M, K))
    if M > 8:
        A[0, 1:] = (np.arange(1, K, dtype=np.float32) % 200 - 100.0) * 0.5   # k + 0.5 ties
        A[0, 0] = 127.0
        A[1, :] = 0.0
        A[2, 5], A[2, 9] = np.nan, np.inf
        A[3, 7] = -np.inf
        A[4] = np.nan                                   # every element NaN: scale 1
        A[5] = 1e-40                                    # subnormal absmax
        A[6, :] *= 3e-37 / np.abs(A[6]).max()           # normal absmax, subnormal scale
        A[7, :3] = [1e30, -1e30, 2.5]
    _, q, s, zps, sw, b = _weights(N, K, 61, zp=form != "sym")
    sumW = (sw + 3).astype(np.int32) if form == "zp_sum_off" else sw
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), sum_W_per_row=_cu(sumW))
    out, sa = Q.linear_forward_per_token(p, _cu(A), act, return_scales=True)
    code = {"none": 0, "relu": 1, "gelu": 2}[act]
    # Large M: the oracle on a sample of rows (the specials, every 37th, the last).
    rows = np.arange(M) if M <= 4096 else np.unique(np.concatenate([np.arange(8), np.arange(0, M, 37), [M - 1]]))
    ref, sa_ref = O.layer_per_token_i8(A[rows], q, s, zps, b, sumW, code)
    out = _host(out)
    assert _bits_equal(_host(sa)[rows], sa_ref)
    out_all = out
    out = out[rows]
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    if act == "gelu":
        np.testing.assert_allclose(out[fin], ref[fin], rtol=RTOL, atol=ATOL)
    else:
        assert _bits_equal(out[fin], ref[fin])
    with _env(NFLOW_NO_TOKEN_GEMM="1"):
        split = _host(Q.linear_forward_per_token(p, _cu(A), act))
    keep = ~np.isnan(split)
    assert np.array_equal(np.isnan(out_all), ~keep)
    assert _bits_equal(out_all[keep], split[keep])


# ---- the persistent GEMM (K = 512 / 1024, fused epilogue) --------------------------

# (M, N, K): one partial 128-row tile; N not a multiple of the 128 / 256-column
# tile; C5's branch (128 x 128 tiles, one per CU); a ragged shape; several
# 128 x 256 tiles per CU with a partial last row tile; K = 512; C5's trunk
# (eight 128 x 256 tiles per CU: both accumulator sets, the table parities and
# the load stream across tile boundaries); 258 tiles of 128 x 128 (most
# blocks run one tile, whose first steps wait on the prologue's instruction
# count -- the case where merged prologue stores once broke those waits).
WIDE_SHAPES = [(1, 1024, 1024), (100, 260, 1024), (4096, 1024, 1024), (10000, 1000, 1024),
               (20000, 1024, 1024), (3000, 776, 512), (65536, 1024, 1024), (33000, 128, 512),
               (33000, 128, 1024)]


@pytest.mark.parametrize("M,N,K", WIDE_SHAPES)
@pytest.mark.parametrize("form", ["sym", "zp", "zp_sum_off"])
@pytest.mark.parametrize("act", ["none", "relu", "gelu"])
def test_wide_gemm_layer(gpu, M, N, K, form, act):
    """The per-token layer on the persistent GEMM: sampled rows against the
    oracle (bit-exact without GELU), and every output bit-equal to the
    LDS-DMA tiled GEMM on the same codes (NFLOW_NO_WIDE), which the tests
    above pin separately."""
    A = WL.normal(60, (M, K))
    if M > 3:
        A[1] = 0.0
        A[2, :4] = np.array([np.nan, 1.0, -2.0, 3.0], np.float32)
    _, q, s, zps, sw, b = _weights(N, K, 61, zp=form != "sym")
    sumW = sw if form != "zp_sum_off" else (sw + np.arange(N, dtype=np.int32) % 7 - 3).astype(np.int32)
    p = Q.Int8LinearParams(_cu(q), _cu(s), _cu(zps), _cu(b), sum_W_per_row=_cu(sumW))
    code = {"none": 0, "relu": 1, "gelu": 2}[act]
    with _env(NFLOW_NO_TOKEN_GEMM="1", NFLOW_NO_WIDE="1"):
        ref_pipe = _host(Q.linear_forward_per_token(p, _cu(A), act))
    with _env(NFLOW_NO_TOKEN_GEMM="1"):
        for _ in range(3):   # a missed wait would show as run-to-run differences
            out = _host(Q.linear_forward_per_token(p, _cu(A), act))
            assert _bits_equal(out, ref_pipe)
    step = max(1, M // 400)
    rows = np.unique(np.concatenate([np.arange(0, M, step), np.arange(max(0, M - 130), M)]))
    ref, _ = O.layer_per_token_i8(A[rows], q, s, zps, b, sumW, code)
    if act == "gelu":
        np.testing.assert_allclose(out[rows], ref, rtol=RTOL, atol=ATOL)
    else:
        finite = np.isfinite(ref)
        assert _bits_equal(out[rows][finite], ref[finite])
        assert np.array_equal(np.isnan(out[rows]), np.isnan(ref))


@pytest.mark.parametrize("M,N,K", [(4096, 1024, 1024), (65536, 1024, 1024), (777, 516, 512)])
@pytest.mark.parametrize("with_sum", [False, True])
def test_wide_gemm_quantised_codes(gpu, M, N, K, with_sum):
    """linear_forward_quantised on per-token codes with symmetric weights:
    without zero points and sum_W the persistent GEMM takes its plain
    epilogue; with a caller's sum_W the row-VNNI term needs the weight-row
    byte sums.  Equal to the LDS-DMA tiled GEMM bit for bit, and to the oracle
    on sampled rows."""
    A = WL.normal(62, (M, K))
    _, q, s, zps, sw, b = _weights(N, K, 63)
    qa, sa, _ = Q.quantise_per_token(_cu(A))
    p = Q.Int8LinearParams(_cu(q), _cu(s), None, _cu(b), sum_W_per_row=_cu(sw) if with_sum else None)
    out = _host(Q.linear_forward_quantised(p, qa, sa, "relu"))
    with _env(NFLOW_NO_WIDE="1"):
        ref_pipe = _host(Q.linear_forward_quantised(p, qa, sa, "relu"))
    assert _bits_equal(out, ref_pipe)
    rows = np.unique(np.concatenate([np.arange(0, M, max(1, M // 300)), [M - 1]]))
    ref, _ = O.layer_per_token_i8(A[rows], q, s, zps, b, sw if with_sum else None, 1)
    assert _bits_equal(out[rows], ref)
