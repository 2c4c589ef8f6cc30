"""Seeded random shapes through the drop-in q35_mm_fp8_batch (host
pointers), against the oracle.  m, k and n are drawn so that every
dispatch is reached at sizes the oracle finishes in about a second: the
row-split and stream-K GEMVs, token groups of eight (9..63 tokens), the
GEMM's narrow 128 x 512 tiles (64..128 tokens) and its 256 x 256 tiles
above, whole tiles, K slices and 64x64 tails, K and N not multiples of 8
or 128.  A second set sends 2..4 weights of random row counts through one
q35mm_matmul_multi call.

Bars as in test_gpu_parity.py: the GEMV (m < 64) within
||y - y_ref||_inf / ||y_ref||_inf <= 1e-5 per token and a batch equal to its
single-token calls bit for bit; the GEMM within relative L2 5e-3 and max
|Y - Y_ref| 2e-2 on outputs of unit scale (GEMM activations are scaled by
a power of two so that outputs have an RMS of at most 1).
"""
import numpy as np
import pytest

from conftest import normwise_rel, unit_scale_act

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
GEMM_REL_L2 = 5e-3
GEMM_MAX_ABS = 2e-2


def _cases(count=48, seed=20260312):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        band = i % 4
        m = int(rng.integers(*((1, 9), (9, 64), (64, 129), (129, 321))[band]))
        kind = i % 3
        k = int(rng.integers(1, 6000))
        if kind == 0:
            k = max(128, k // 128 * 128)
        elif kind == 1:
            k = max(8, k // 8 * 8)
        n = int(rng.integers(1, 5000))
        n = max(1, min(n, int(4e8 // (m * k))))
        out.append((i, m, k, n))
    return out


@pytest.mark.parametrize("i,m,k,n", _cases())
def test_random_shape(q, oracle, wl, gpu, i, m, k, n):
    gemm = m >= 64
    if gemm or i % 2:
        W, sc = wl.gen_weight(0x5EED00 + i, n, k)
    else:
        W, sc = wl.gen_weight_ragged(0x5EED00 + i, n, k)
    X = wl.gen_act(0x5EED80 + i, m, k, outlier_frac=0.0 if gemm else 0.01)
    if gemm:
        X = unit_scale_act(X, k)
    Y = q.mm_fp8_batch(W, sc, X)
    Yr = oracle.mm_batch(W, sc, X)
    if gemm:
        Yd, Yrd = Y.astype(np.float64), Yr.astype(np.float64)
        rel = np.linalg.norm(Yd - Yrd) / np.linalg.norm(Yrd)
        mx = np.abs(Yd - Yrd).max()
        assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (m, k, n, rel, mx)
    else:
        for t in range(m):
            assert normwise_rel(Y[t], Yr[t]) <= GEMV_TOL, (m, k, n, t)
        for t in (0, m - 1):
            assert (q.mm_fp8(W, sc, X[t]).view(np.uint32) == Y[t].view(np.uint32)).all(), (m, k, n, t)
    q.release(W)


def _multi_cases(count=16, seed=20260313):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        band = i % 4
        m = int(rng.integers(*((1, 9), (9, 64), (64, 129), (129, 257))[band]))
        k = int(rng.integers(1, 4000))
        if i % 2:
            k = max(8, k // 8 * 8)
        nseg = int(rng.integers(2, 5))
        rows = [int(rng.integers(1, 3000)) for _ in range(nseg)]
        cap = int(3e8 // (m * k))
        rows = [max(1, min(r, cap // nseg)) for r in rows]
        out.append((i, m, k, tuple(rows)))
    return out


@pytest.mark.parametrize("i,m,k,rows", _multi_cases())
def test_random_multi(q, oracle, wl, gpu, i, m, k, rows):
    """q35mm_matmul_multi over 2..4 weights of random row counts sharing K:
    each segment within its bar of the oracle; on the GEMV the bits of a
    single q35mm_matmul of that weight."""
    import torch
    gemm = m >= 64
    Ws = [wl.gen_weight(0x3E6000 + 8 * i + s, r, k) for s, r in enumerate(rows)]
    X = wl.gen_act(0x3E6100 + i, m, k)
    if gemm:
        X = unit_scale_act(X, k)
    ws = [q.Weight(W, sc) for W, sc in Ws]
    dX = torch.from_numpy(X).to(gpu)
    Ys = [torch.empty((m, r), dtype=torch.float32, device=gpu) for r in rows]
    q.matmul_multi(ws, dX, Ys)
    torch.cuda.synchronize()
    for (W, sc), w, Y in zip(Ws, ws, Ys):
        y = Y.cpu().numpy()
        yr = oracle.mm_batch(W, sc, X)
        if gemm:
            yd, yrd = y.astype(np.float64), yr.astype(np.float64)
            rel = np.linalg.norm(yd - yrd) / np.linalg.norm(yrd)
            mx = np.abs(yd - yrd).max()
            assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (m, k, W.shape, rel, mx)
        else:
            for t in range(m):
                assert normwise_rel(y[t], yr[t]) <= GEMV_TOL, (m, k, W.shape, t)
            single = torch.empty_like(Y)
            q.matmul(w, dX, single)
            torch.cuda.synchronize()
            assert (single.cpu().numpy().view(np.uint32) == y.view(np.uint32)).all(), (m, k, W.shape)
    for w in ws:
        w.free()
