"""Row-split decode GEMV (gemv_rows.hip) against the oracle, through the C ABI.

The row-split kernel takes every weight of 4..160 K blocks, one
workgroup per 32-row sub-tile: the model's qkv (5120 -> 6144), o_proj
(4096 -> 5120), gate and up (5120 -> 17408), down (17408 -> 5120) and its
small projections, which the golden cases also cover.  Above 256 sub-tiles
a launch runs several rounds of workgroups.
Here: ragged and maximal shapes of that class, unaligned activations (the
scalar-load staging), every token count class (1, 2, 4 or 8 tokens per
staging layout), batch == n single calls and multi-weight == single calls
bit for bit -- also when one call mixes row-split and stream-K weights --
and the MLP block when all three of its weights are row-split.

Bar: ||y - y_ref||_inf / ||y_ref||_inf <= 1e-5 per token (the decode GEMV
bar); bitwise where results must equal other calls of the same library.
"""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5


def _dev(arr, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr, np.float32)).to(gpu)


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("m,k,n", [(1, 1003, 4100), (4, 1003, 4100), (5, 1000, 4065), (8, 8192, 8192),
                                   (3, 4096, 5120), (8, 5120, 6144), (2, 1024, 7777), (6, 20480, 4100),
                                   (7, 17400, 5000), (1, 1024, 20000), (3, 2048, 9001),
                                   # aligned rows, a last block of 8 columns (k % 16 == 8)
                                   (8, 1032, 4100), (4, 1032, 4100)])
def test_row_split_shapes(q, oracle, wl, gpu, m, k, n):
    W, sc = wl.gen_weight_ragged(7 * n + k + m, n, k)
    X = wl.gen_act(n + m, m, k, outlier_frac=0.01)
    Y = q.mm_fp8_batch(W, sc, X)
    Yr = oracle.mm_batch(W, sc, X)
    for t in range(m):
        assert normwise_rel(Y[t], Yr[t]) <= GEMV_TOL, (m, k, n, t)
    q.release(W)


@pytest.mark.parametrize("m", [1, 4, 8])
def test_row_split_unaligned_activations(q, oracle, wl, gpu, m):
    """Activations 4 bytes past a 16-byte boundary: the staging takes the
    scalar-load path; results are the aligned call's, bit for bit."""
    import torch
    k, n = 4096, 5120
    W, sc = wl.gen_weight(90 + m, n, k)
    X = wl.gen_act(91 + m, m, k)
    w = q.Weight(W, sc)
    big = torch.zeros(m * k + 1, device=gpu)
    big[1:] = _dev(X.reshape(-1), gpu)
    Xu = big[1:].view(m, k)
    assert Xu.data_ptr() % 16 == 4
    Yu = torch.empty((m, n), device=gpu)
    q.matmul(w, Xu, Yu)
    Ya = torch.empty((m, n), device=gpu)
    q.matmul(w, _dev(X, gpu), Ya)
    yu, ya = _host(Yu), _host(Ya)
    assert (yu.view(np.uint32) == ya.view(np.uint32)).all()
    Yr = oracle.mm_batch(W, sc, X)
    for t in range(m):
        assert normwise_rel(yu[t], Yr[t]) <= GEMV_TOL, t
    w.free()


def test_row_split_batch_equals_single_bitwise(q, wl, gpu):
    """qwen35-c/tests/test_batch_mm.c: batch rows are the bits of single
    calls, for a row-split shape with ragged rows and K."""
    W, sc = wl.gen_weight_ragged(77, 4100, 1003)
    X = wl.gen_act(78, 8, 1003, outlier_frac=0.01)
    Yb = q.mm_fp8_batch(W, sc, X)
    for t in range(8):
        assert (q.mm_fp8(W, sc, X[t]).view(np.uint32) == Yb[t].view(np.uint32)).all(), t
    for mm in (2, 5):
        assert (q.mm_fp8_batch(W, sc, X[:mm]).view(np.uint32) == Yb[:mm].view(np.uint32)).all(), mm
    q.release(W)


def test_mixed_multi_equals_single_bitwise(q, wl, gpu):
    """One multi4 call over weights of both decompositions (row-split: 4096
    and 5000 rows; stream-K: 1280 and 48 rows) returns the bits of four
    single calls."""
    K = 1024
    segs = [wl.gen_weight(60 + i, n, K) for i, n in enumerate((4096, 1280, 5000, 48))]
    x = wl.gen_act(65, 1, K)[0]
    outs = q.mm_fp8_multi4([s[0] for s in segs], [s[1] for s in segs], x)
    for (W, sc), y in zip(segs, outs):
        assert (q.mm_fp8(W, sc, x).view(np.uint32) == y.view(np.uint32)).all()
    for W, _ in segs:
        q.release(W)


def test_mixed_matmul_multi_device_api(q, oracle, wl, gpu):
    """q35mm_matmul_multi at m = 3 over a row-split and a stream-K weight."""
    import torch
    K = 2048
    Ws = [wl.gen_weight(70 + i, n, K) for i, n in enumerate((6000, 640))]
    X = wl.gen_act(72, 3, K)
    ws = [q.Weight(*w) for w in Ws]
    Ys = [torch.empty((3, w.rows), device=gpu) for w in ws]
    q.matmul_multi(ws, _dev(X, gpu), Ys)
    for (W, sc), Y, w in zip(Ws, Ys, ws):
        y = _host(Y)
        Yr = oracle.mm_batch(W, sc, X)
        for t in range(3):
            assert normwise_rel(y[t], Yr[t]) <= GEMV_TOL
        Ys1 = torch.empty((3, w.rows), device=gpu)
        q.matmul(w, _dev(X, gpu), Ys1)
        assert (_host(Ys1).view(np.uint32) == y.view(np.uint32)).all()
        w.free()


@pytest.mark.parametrize("m,H,I", [(1, 4096, 8192), (2, 4096, 8192), (3, 4096, 8192), (8, 1024, 4096),
                                   (5, 1536, 4100), (13, 1024, 4096)])
def test_mlp_block_all_row_split(q, oracle, wl, gpu, m, H, I):
    """Gate, up and down all row-split (8+ K blocks; ragged rows at
    I = 4100, two token groups at m = 13): gate and up as the paired launch
    (RMSNorm inside at one token, else its own kernel; SwiGLU inside), the
    residual add in the down GEMV.  Checked against the oracle's block and,
    bit for bit, against the separate calls."""
    import torch
    W = {nm: wl.gen_weight(0x400 + i, *((H, I) if nm == "down" else (I, H)))
         for i, nm in enumerate(("gate", "up", "down"))}
    dw = {nm: q.Weight(*v) for nm, v in W.items()}
    rng = np.random.default_rng(30 + m)
    x = rng.standard_normal((m, H)).astype(np.float32)
    nw = (rng.standard_normal(H) * 0.1).astype(np.float32)
    dnw = _dev(nw, gpu)
    dx = _dev(x, gpu)
    q.mlp(dw["gate"], dw["up"], dw["down"], dnw, dx)
    out = _host(dx)
    r = oracle.mlp(x, nw, W["gate"], W["up"], W["down"])
    y = out.astype(np.float64) - x.astype(np.float64)
    yref = r["y"].astype(np.float64)
    scale = np.abs(yref).max()
    slack = 0.5 * np.spacing(np.abs(out)).astype(np.float64)
    assert (np.abs(y - yref) <= GEMV_TOL * scale + slack).all()
    # the separate device calls
    dx2 = _dev(x, gpu)
    xn = torch.empty_like(dx2)
    g = torch.empty((m, I), device=gpu)
    u = torch.empty_like(g)
    yy = torch.empty_like(dx2)
    q.rmsnorm(dx2, dnw, xn)
    q.matmul_multi([dw["gate"], dw["up"]], xn, [g, u])
    q.swiglu(g, u, g)
    q.matmul(dw["down"], g, yy)
    want = _host(dx2 + yy)
    assert (out.view(np.uint32) == want.view(np.uint32)).all()
    for w in dw.values():
        w.free()
