"""q35mm_matmul_noalloc (the allocation-free variant of q35mm_matmul) against
q35mm_matmul, through the C ABI: same kernels on the library's fixed device
scratch instead of its own allocations, so the outputs must be the same
bits.  Each case makes two calls in a row, the second with a smaller input,
on the decode GEMV that uses scratch (stream-K: K beyond the row-split
kernel's 160 blocks), on the row-split GEMV (no scratch) and on the prefill
GEMM (bf16 activations and, for few tiles, K-slice partials in scratch);
a GEMM of at most 128 tokens whose narrow-tile partials exceed the scratch
runs on 256 x 256 tiles (within the GEMM bars of q35mm_matmul's results);
a GEMM whose activations exceed the scratch is refused; a HIP graph of
stream-K calls replays with the eager bits.
"""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5


def _dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu)


def _both(q, w, X, m, gpu):
    import torch
    Ya = torch.full((m, w.rows), float("nan"), device=gpu)
    Yb = torch.full((m, w.rows), float("nan"), device=gpu)
    q.matmul(w, X, Ya, m=m)
    q.matmul_noalloc(w, X, Yb, m=m)
    torch.cuda.synchronize()
    return Ya.cpu().numpy(), Yb.cpu().numpy()


@pytest.mark.parametrize("rows,k,ms", [(1500, 168 * 128, (5, 2)),     # stream-K GEMV
                                       (5120, 5120, (3, 1)),          # row-split GEMV
                                       (700, 2048, (300, 96)),        # GEMM: 64x64 tail tiles, then narrow tiles in K slices
                                       (4352, 768, (64, 64))])        # GEMM: 9 narrow tiles x 3 K slices
def test_noalloc_equals_matmul(q, oracle, wl, gpu, rows, k, ms):
    q.init()
    W, sc = wl.gen_weight(rows + k, rows, k)
    w = q.Weight(W, sc)
    X = wl.gen_act(rows * 3 + k, ms[0], k)
    for i, m in enumerate(ms):
        Xm = X[:m] if i else X
        if i and ms[1] == ms[0]:
            Xm = wl.gen_act(rows + 7, m, k)     # same size, other data: nothing carried over
        ya, yb = _both(q, w, _dev(Xm, gpu), m, gpu)
        assert (ya.view(np.uint32) == yb.view(np.uint32)).all(), (rows, k, m)
        assert q.debug_counters(noalloc=True)[0] == 0   # the shared counters are back at zero
        if m < 64:
            yr = oracle.mm_batch(W, sc, Xm)
            for t in range(m):
                assert normwise_rel(yb[t], yr[t]) <= GEMV_TOL
    w.free()


def test_noalloc_narrow_partials_beyond_scratch(q, oracle, wl, gpu):
    """64 tokens x 34816 rows: q35mm_matmul cuts its 68 narrow tiles into
    3 K slices (51 MB of partials), more than the fixed scratch holds, so the
    allocation-free call runs the 256 x 256 tiles instead: no error, results
    within the GEMM bars of the oracle (384 sampled columns) and of
    q35mm_matmul's."""
    import torch
    q.init()
    m, k, n = 64, 5120, 34816
    W, sc = wl.gen_weight(21, n, k)
    w = q.Weight(W, sc)
    X = wl.gen_act(22, m, k, bf16=True)
    ya, yb = _both(q, w, _dev(X, gpu), m, gpu)
    assert np.isfinite(yb).all()
    idx = np.sort(np.random.default_rng(23).choice(n, 384, replace=False)).astype(np.uint32)
    idx[:2] = [0, n - 1]
    yr = oracle.mm_rows(W, sc, X, idx)
    for y in (ya, yb):
        d = y[:, idx] - yr
        rel = np.sqrt((d.astype(np.float64) ** 2).sum() / (yr.astype(np.float64) ** 2).sum())
        assert rel <= 5e-3 and np.abs(d).max() <= 2e-2, rel
    d = (ya - yb).astype(np.float64)
    assert np.sqrt((d ** 2).sum() / (ya.astype(np.float64) ** 2).sum()) <= 5e-3
    w.free()


def test_noalloc_refuses_oversized_gemm(q, wl, gpu):
    """512 tokens x 17408 columns of bf16 activations (17.8 MB) exceed the
    16 MiB scratch: a clear error, nothing launched, the library still works."""
    import torch
    q.init()
    W, sc = wl.gen_weight(5, 256, 17408)
    w = q.Weight(W, sc)
    X = torch.zeros((512, 17408), device=gpu)
    Y = torch.zeros((512, 256), device=gpu)
    with pytest.raises(q.Q35mmError) as e:
        q.matmul_noalloc(w, X, Y)
    assert e.value.code == -1 and "no-alloc scratch" in str(e.value)
    x = _dev(wl.gen_act(6, 1, 17408), gpu)
    ya, yb = _both(q, w, x, 1, gpu)
    assert (ya.view(np.uint32) == yb.view(np.uint32)).all()
    w.free()


def test_noalloc_in_a_graph(q, wl, gpu):
    """Stream-K GEMV calls captured into a HIP graph and replayed three
    times, with eager work of the library in between: every replay gives the
    eager bits (the arrival counters are back at zero after each launch)."""
    import torch
    q.init()
    k = 168 * 128
    W, sc = wl.gen_weight(11, 1500, k)
    w = q.Weight(W, sc)
    X = _dev(wl.gen_act(12, 4, k), gpu)
    want = torch.empty((4, 1500), device=gpu)
    q.matmul(w, X, want)
    Y = torch.empty((4, 1500), device=gpu)
    q.matmul_noalloc(w, X, Y)            # warm
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            q.matmul_noalloc(w, X, Y)
    torch.cuda.synchronize()
    other = torch.empty((2, 1500), device=gpu)
    for r in range(3):
        Y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert (Y.cpu().numpy().view(np.uint32) == want.cpu().numpy().view(np.uint32)).all(), r
        q.matmul_noalloc(w, X[:2], other)   # eager use of the same scratch between replays
        torch.cuda.synchronize()
        assert q.debug_counters(noalloc=True)[0] == 0
    del g
    w.free()
