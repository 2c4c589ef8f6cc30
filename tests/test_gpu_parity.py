"""GPU parity of libq35mm.so against the CPU oracle (the reference's
arithmetic, pinned in test_oracle.py), through the C ABI.

Bars (written in each test):
  - dequant and e4m3 -> bf16 conversion: bit-exact;
  - decode GEMV (fp32 path, m < 64 by default): ||y - y_ref||_inf / ||y_ref||_inf <= 1e-5;
  - prefill GEMM (bf16 MFMA path): ||Y - Y_ref||_2 / ||Y_ref||_2 <= 5e-3 and
    max |Y - Y_ref| <= 2e-2 on outputs of unit scale (fp32 activations of the
    larger K are scaled by a power of two so that the outputs' RMS is at
    most 1).
"""
import numpy as np
import pytest

from conftest import fixture_names, goldens, load_fixture, normwise_rel, unit_scale_act

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
GEMM_REL_L2 = 5e-3
GEMM_MAX_ABS = 2e-2


def _inputs(wl, case):
    if case["kind"] == "ragged":
        W, sc = wl.gen_weight_ragged(case["seed"], case["n"], case["k"])
    else:
        W, sc = wl.gen_weight(case["seed"], case["n"], case["k"])
    X = wl.gen_act(case["seed"] + 0x100, case["m"], case["k"], **case["act"])
    return W, sc, X


def _all_codes_matrix(rows=256, cols=384, seed=0):
    """Every e4m3 code in every lane position class, NaN codes included."""
    rng = np.random.default_rng(seed)
    W = rng.integers(0, 256, size=(rows, cols), dtype=np.uint8)
    W[:, :256] = (np.arange(256)[None, :] + np.arange(rows)[:, None]) % 256
    return W


def _torch_dev(arr, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr)).to(gpu)


# ------------------------------------------------------------- conversions
def test_decode_bf16_exhaustive_bit_exact(q, oracle, gpu):
    import torch
    W = _all_codes_matrix()
    sc = np.full((2, 3), 0x3F80, np.uint16)
    w = q.Weight(W, sc)
    out = torch.empty(W.shape, dtype=torch.int16, device=gpu)
    q.decode_bf16(w, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    lut = oracle.lut()
    want = (lut.view(np.uint32) >> 16).astype(np.uint16)[W]
    nan = (W == 0x7F) | (W == 0xFF)
    assert (got[~nan] == want[~nan]).all()
    assert ((got[nan] & 0x7F80) == 0x7F80).all() and ((got[nan] & 0x7F) != 0).all()


@pytest.mark.parametrize("shape", [(256, 384), (129, 129), (3, 5), (300, 4700)])
def test_dequant_f32_bit_exact(q, oracle, wl, gpu, shape):
    import torch
    rows, cols = shape
    W = _all_codes_matrix(rows, cols, seed=rows) if cols >= 256 else \
        np.random.default_rng(rows).integers(0, 256, size=shape, dtype=np.uint8)
    rng = np.random.default_rng(cols)
    sc = wl.bf16_rne((10.0 ** rng.uniform(-6, 3, size=((rows + 127) // 128, (cols + 127) // 128)))
                     .astype(np.float32))
    w = q.Weight(W, sc)
    out = torch.empty(shape, dtype=torch.float32, device=gpu)
    q.dequant_f32(w, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = oracle.dequant(W, sc)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    assert (got[~nan].view(np.uint32) == want[~nan].view(np.uint32)).all()


def test_dequant_f32_scale_mode_bit_exact(q, oracle, gpu):
    import torch
    rng = np.random.default_rng(5)
    W = rng.integers(0, 0x7F, size=(200, 300), dtype=np.uint8)
    sc = rng.uniform(1e-5, 3.0, size=(2, 3)).astype(np.float32)   # not bf16-representable
    w = q.Weight(W, sc)
    out = torch.empty((200, 300), dtype=torch.float32, device=gpu)
    q.dequant_f32(w, out)
    torch.cuda.synchronize()
    assert (out.cpu().numpy().view(np.uint32) == oracle.dequant(W, sc).view(np.uint32)).all()


# ------------------------------------------------------------ decode GEMV
@pytest.mark.parametrize("name", fixture_names(fp8=True))
def test_gemv_reference_fixtures(q, oracle, gpu, name):
    """The reference's own test_mm check (tol 5e-4 vs f64 yref) and the fp32
    bar against the oracle."""
    c, W, sc, x, yref = load_fixture(name)
    y = q.mm_fp8(W, sc, x)
    tol = c["tol"]
    assert (np.abs(y.astype(np.float64) - yref) <= tol + tol * np.abs(yref)).all()
    assert normwise_rel(y, oracle.mm(W, sc, x)) <= GEMV_TOL


GEMV_CASES = [c["name"] for c in goldens()["cases"] if c["m"] < 64]


@pytest.mark.parametrize("name", GEMV_CASES)
def test_gemv_golden_cases(q, oracle, wl, gpu, name):
    case = next(c for c in goldens()["cases"] if c["name"] == name)
    W, sc, X = _inputs(wl, case)
    Y = q.mm_fp8_batch(W, sc, X)
    Yr = oracle.mm_batch(W, sc, X)
    assert f"{oracle.fnv64(Yr):016x}" == case["fnv_y_ref"]   # oracle == compiled reference
    for t in range(X.shape[0]):
        assert normwise_rel(Y[t], Yr[t]) <= GEMV_TOL, (name, t)
    q.release(W)


def test_gemv_batch_equals_single_bitwise(q, wl, gpu):
    """qwen35-c/src/q35_mm.c:155-157: batch results are the bits of n single
    calls (and tests/test_batch_mm.c), here for the GPU path."""
    W, sc = wl.gen_weight(41, 6144, 5120)
    X = wl.gen_act(42, 8, 5120)
    Yb = q.mm_fp8_batch(W, sc, X)
    for t in range(8):
        assert (q.mm_fp8(W, sc, X[t]).view(np.uint32) == Yb[t].view(np.uint32)).all()
    Y5 = q.mm_fp8_batch(W, sc, X[:5])
    assert (Y5.view(np.uint32) == Yb[:5].view(np.uint32)).all()
    q.release(W)


def test_gemv_multi4_equals_single_bitwise(q, wl, gpu):
    """multi4 rows equal single-call rows (qwen35-c/src/q35_mm.c:176-198), with
    the DeltaNet segment shapes (qkv, z, a, b) of qwen35-c/src/q35_deltanet.c:325-329
    at a smaller K."""
    K = 1024
    segs = [wl.gen_weight(50 + i, n, K) for i, n in enumerate((1280, 768, 48, 48))]
    x = wl.gen_act(55, 1, K)[0]
    outs = q.mm_fp8_multi4([s[0] for s in segs], [s[1] for s in segs], x)
    for (W, sc), y in zip(segs, outs):
        assert (q.mm_fp8(W, sc, x).view(np.uint32) == y.view(np.uint32)).all()
    outs2 = q.mm_fp8_multi4([segs[0][0], None, segs[2][0], None], [segs[0][1], None, segs[2][1], None], x)
    assert outs2[1] is None and (outs2[0].view(np.uint32) == outs[0].view(np.uint32)).all()
    for W, _ in segs:
        q.release(W)


def test_gemv_full_size_properties(q, wl, gpu):
    """Size-independent laws at a full decode shape.
    Exact: doubling x doubles y (power-of-two scaling commutes with every
    rounding); permuting rows inside every 128-row group (same blocks, same
    scales) permutes y; repeated calls give the same bits.
    To tolerance only: flipping every sign bit negates y -- the matrix core's
    internal accumulation is not odd-symmetric, so a few outputs move by a
    few ulps (measured: 51 of 17408, <= 8 ulps)."""
    W, sc = wl.gen_weight(61, 17408, 5120)
    x = wl.gen_act(62, 1, 5120)[0]
    y = q.mm_fp8(W, sc, x)
    assert (q.mm_fp8(W, sc, x).view(np.uint32) == y.view(np.uint32)).all()
    assert (q.mm_fp8(W, sc, 2 * x).view(np.uint32) == (2 * y).view(np.uint32)).all()
    perm = np.random.default_rng(63).permutation(128)
    Wp = np.ascontiguousarray(W.reshape(-1, 128, W.shape[1])[:, perm].reshape(W.shape))
    yp = q.mm_fp8(Wp, sc, x)
    assert (yp.view(np.uint32) == y.reshape(-1, 128)[:, perm].reshape(-1).view(np.uint32)).all()
    Wn = W ^ np.uint8(0x80)
    assert normwise_rel(q.mm_fp8(Wn, sc, x), -y) <= 1e-6
    for a in (W, Wp, Wn):
        q.release(a)


def test_gemv_edge_shapes(q, oracle, wl, gpu):
    for (m, k, n) in [(1, 1, 1), (2, 127, 129), (3, 128, 128), (8, 257, 3000), (1, 4700, 48),
                      (5, 17408, 200), (1, 40, 70000), (2, 17408, 48), (8, 65536, 200)]:
        W, sc = wl.gen_weight_ragged(m * 1000 + k + n, n, k)
        X = wl.gen_act(k + n, m, k, outlier_frac=0.01)
        Y = q.mm_fp8_batch(W, sc, X)
        Yr = oracle.mm_batch(W, sc, X)
        for t in range(m):
            assert normwise_rel(Y[t], Yr[t]) <= GEMV_TOL, (m, k, n, t)
        q.release(W)


@pytest.mark.parametrize("k", [5120, 168 * 128 + 40])
def test_gemv_nonfinite_activations(q, oracle, wl, gpu, k):
    """Activations holding +-inf and finite values beyond bf16's range
    (+-3.4e38, which round to infinity in bf16), in some tokens of a batch:
    each output is NaN, +inf or -inf exactly where the reference's fmaf
    chain (qwen35-c/src/q35_mm.c:110-111,135-137) makes it so, and the
    finite outputs meet the GEMV bar.  K = 5120 runs the row-split GEMV,
    168 blocks (+40 columns) the stream-K one."""
    n, m = 700, 5
    W, sc = wl.gen_weight(0x51E50900 + k, n, k)
    X = wl.gen_act(0x51E50901 + k, m, k)
    rng = np.random.default_rng(k)
    # token 0: one +inf; token 1: +inf and -inf; token 2: two huge finite
    # values of both signs; token 3: huge values and one -inf; token 4 plain
    X[0, rng.integers(k)] = np.inf
    X[1, 7] = np.inf
    X[1, k - 3] = -np.inf
    X[2, 100] = np.float32(3.4e38)
    X[2, k // 2] = np.float32(-3.39e38)
    X[3, 5] = np.float32(-3.4028235e38)
    X[3, k - 1] = -np.inf
    Y = q.mm_fp8_batch(W, sc, X)
    Yr = oracle.mm_batch(W, sc, X)
    assert np.array_equal(np.isnan(Y), np.isnan(Yr))
    assert np.array_equal(np.isposinf(Y), np.isposinf(Yr))
    assert np.array_equal(np.isneginf(Y), np.isneginf(Yr))
    assert np.isinf(Yr[0]).any() and np.isnan(Yr[1]).any() and np.isfinite(Yr[2]).all()
    for t in range(m):
        fin = np.isfinite(Yr[t])
        if fin.any():
            assert normwise_rel(Y[t][fin], Yr[t][fin]) <= GEMV_TOL, t
    # the plain token is unaffected by its neighbours
    Y4 = q.mm_fp8_batch(W, sc, np.ascontiguousarray(X[4:5]))
    assert np.array_equal(Y4[0], Y[4])
    q.release(W)


def test_zero_sizes(q):
    y = q.mm_fp8(np.zeros((4, 0), np.uint8), np.zeros((1, 0), np.uint16), np.zeros(0, np.float32))
    assert (y == 0).all()


# ------------------------------------------------------------ prefill GEMM
def _gemm_check(Y, Yr):
    """Relative L2 error and max |Y - Y_ref| (absolute: the callers feed
    activations that keep the outputs' RMS at most 1, unit_scale_act, or
    bf16-representable ones, whose error is far below the bar)."""
    Y = Y.astype(np.float64)
    Yr = Yr.astype(np.float64)
    rel = np.linalg.norm(Y - Yr) / np.linalg.norm(Yr)
    mx = np.abs(Y - Yr).max()
    return rel, mx


@pytest.mark.parametrize("name", ["prefill_m512_5120x256", "prefill_m512_17408x128"])
def test_gemm_golden_cases(q, oracle, wl, gpu, name):
    case = next(c for c in goldens()["cases"] if c["name"] == name)
    W, sc, X = _inputs(wl, case)
    Y = q.mm_fp8_batch(W, sc, X)          # n = 512 >= 64 -> bf16 GEMM
    Yr = oracle.mm_batch(W, sc, X)
    rel, mx = _gemm_check(Y, Yr)
    assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (rel, mx)
    q.release(W)


@pytest.mark.parametrize("k,n", [(5120, 34816), (17408, 5120), (5120, 17408)])
def test_gemm_full_prefill_shapes_sampled(q, oracle, wl, gpu, k, n):
    """Full M=512 prefill shapes on the GPU, checked on 384 sampled output
    columns against the oracle: gate and up fused (256 whole tiles + a 64x64
    tail), down (every tile in K slices), gate alone (136 whole tiles)."""
    import torch
    W, sc = wl.gen_weight(0x51E50002 + k, n, k)
    X = wl.gen_act(0x51E50102 + k, 512, k, bf16=True)
    w = q.Weight(W, sc)
    dX = _torch_dev(X, gpu)
    dY = torch.empty((512, n), dtype=torch.float32, device=gpu)
    q.gemm(w, dX, dY)
    torch.cuda.synchronize()
    Y = dY.cpu().numpy()
    idx = np.sort(np.random.default_rng(k).choice(n, 384, replace=False)).astype(np.uint32)
    idx[:2] = [0, n - 1]
    Yr = oracle.mm_rows(W, sc, X, idx)
    rel, mx = _gemm_check(Y[:, idx], Yr)
    assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (rel, mx)


@pytest.mark.parametrize("m,k,n", [(64, 256, 384), (100, 4700, 3000), (37, 4736, 3000), (129, 129, 129),
                                   (300, 1000, 700), (64, 17408, 64), (513, 640, 300), (100, 512, 33000),
                                   (200, 256, 384), (160, 4700, 3000), (129, 17408, 64), (200, 512, 33000),
                                   (128, 4736, 3000), (65, 17408, 5120), (67, 5120, 4100), (258, 17408, 640)])
def test_gemm_ragged(q, oracle, wl, gpu, m, k, n):
    """Ragged m, k, n.  Above 128 tokens (256 x 256 tiles), with at most one
    tile per 16 CUs every tile runs as 64x64 tiles: partial token and weight
    rows, K not a multiple of 128, a K range longer than eight wavefronts'
    share (17408), a third token tile holding one row (513); 200 x 33000
    has 129 whole tiles, the last holding 232 of its 256 rows.  Up to 128
    tokens the same shapes run the narrow 128 x 512 tiles, their partial
    round cut into K slices (37 tokens: the GEMV).  The slices skip the
    float4s of padding token rows: 65 and 67 tokens end inside a float4,
    and 258 x 17408 x 640 slices a second token tile of two rows."""
    import torch
    W, sc = wl.gen_weight(m + k + n, n, k)
    X = unit_scale_act(wl.gen_act(m * k, m, k), k)
    w = q.Weight(W, sc)
    dX = _torch_dev(X, gpu)
    dY = torch.empty((m, n), dtype=torch.float32, device=gpu)
    q.gemm(w, dX, dY)
    torch.cuda.synchronize()
    rel, mx = _gemm_check(dY.cpu().numpy(), oracle.mm_batch(W, sc, X))
    assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (rel, mx)


@pytest.mark.parametrize("m", [64, 128, 300])
def test_gemm_multi_segment(q, oracle, wl, gpu, m):
    """q35mm_matmul_multi on the GEMM path: three weights sharing K run as one
    launch over all their tiles (row counts 640, 3000 and 5000: odd row
    groups, ragged last tiles).  Each output within the GEMM bars of the
    oracle."""
    import torch
    k = 1000
    Ws = [wl.gen_weight(95 + i, n, k) for i, n in enumerate((640, 3000, 5000))]
    X = wl.gen_act(98, m, k)
    ws = [q.Weight(*w) for w in Ws]
    Ys = [torch.empty((m, w.rows), dtype=torch.float32, device=gpu) for w in ws]
    q.matmul_multi(ws, _torch_dev(X, gpu), Ys)
    torch.cuda.synchronize()
    for (W, sc), Y in zip(Ws, Ys):
        rel, mx = _gemm_check(Y.cpu().numpy(), oracle.mm_batch(W, sc, X))
        assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (W.shape, rel, mx)
    for w in ws:
        w.free()


@pytest.mark.parametrize("m,k,n", [(64, 1000, 3000), (200, 1000, 3000), (200, 1000, 1000), (300, 256, 16640),
                                   (100, 256, 70000)])
def test_gemm_multi_two_weights_of_one_shape(q, oracle, wl, gpu, m, k, n):
    """Two weights of one shape (the MLP's gate and up) on the GEMM path run
    as paired tiles, each holding the same rows of both weights: narrow tiles
    cut along K (64 tokens), 256 x 256 tiles cut along K (200 x 3000), only
    64x64 tiles (200 x 1000), whole tiles with padding tokens and a fused
    64x64 tail (300 x 16640), whole narrow tiles then a round cut along K
    (100 x 70000).  Each output within the GEMM bars of the oracle."""
    import torch
    Ws = [wl.gen_weight(0x9A1 + i + n, n, k) for i in range(2)]
    X = wl.gen_act(0x9A3 + m, m, k)
    ws = [q.Weight(*w) for w in Ws]
    Ys = [torch.empty((m, n), dtype=torch.float32, device=gpu) for _ in ws]
    q.matmul_multi(ws, _torch_dev(X, gpu), Ys)
    torch.cuda.synchronize()
    for (W, sc), Y in zip(Ws, Ys):
        rel, mx = _gemm_check(Y.cpu().numpy(), oracle.mm_batch(W, sc, X))
        assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (W.shape, rel, mx)
    for w in ws:
        w.free()


def test_gemm_zero_scale_blocks(q, oracle, wl, gpu):
    """Blocks whose scale is 0 contribute nothing (the reference's
    lut[code] * 0): first K blocks of a row group, blocks in the middle and a
    whole row group, with nonzero codes behind them.  A row group with no
    live block must come out exactly 0."""
    import torch
    m, k, n = 96, 1536, 640
    rng = np.random.default_rng(91)
    W = rng.integers(0, 0x7E, size=(n, k), dtype=np.uint8) | (rng.integers(0, 2, size=(n, k), dtype=np.uint8) << 7)
    sc = np.full((n // 128, k // 128), 0x3980, np.uint16)           # bf16 2^-12: outputs of unit scale
    sc[0, 0] = 0                      # first block of group 0
    sc[1, 5:7] = 0                    # middle blocks of group 1
    sc[2, :] = 0                      # group 2 dead
    sc[3, -1] = 0                     # last block of group 3
    X = wl.gen_act(92, m, k)
    w = q.Weight(W, sc)
    dY = torch.empty((m, n), dtype=torch.float32, device=gpu)
    q.gemm(w, _torch_dev(X, gpu), dY)
    torch.cuda.synchronize()
    Y = dY.cpu().numpy()
    Yr = oracle.mm_batch(W, sc, X)
    rel, mx = _gemm_check(Y, Yr)
    assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (rel, mx)
    assert (Y[:, 256:384] == 0).all()


@pytest.mark.parametrize("pair", [False, True])
def test_gemm_whole_rounds_then_k_slices(q, oracle, wl, gpu, pair):
    """A long prompt (1200 tokens): whole rounds of 256 x 256 tiles, then a
    last partial round of 24 tiles cut along K, in one launch -- one weight
    of 14336 rows, or (paired tiles) two of 7168.  Checked on 384 sampled
    output columns of each weight against the oracle."""
    import torch
    m, k = 1200, 1024
    shapes = [7168, 7168] if pair else [14336]
    Ws = [wl.gen_weight(0x9C0 + i, n, k) for i, n in enumerate(shapes)]
    X = wl.gen_act(0x9C8, m, k, bf16=True)
    ws = [q.Weight(*w) for w in Ws]
    Ys = [torch.empty((m, n), dtype=torch.float32, device=gpu) for n in shapes]
    dX = _torch_dev(X, gpu)
    if pair:
        q.matmul_multi(ws, dX, Ys)
    else:
        q.gemm(ws[0], dX, Ys[0])
    torch.cuda.synchronize()
    for i, ((W, sc), Y) in enumerate(zip(Ws, Ys)):
        n = W.shape[0]
        idx = np.sort(np.random.default_rng(n + i).choice(n, 384, replace=False)).astype(np.uint32)
        idx[:2] = [0, n - 1]
        rel, mx = _gemm_check(Y.cpu().numpy()[:, idx], oracle.mm_rows(W, sc, X, idx))
        assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (i, rel, mx)
    for w in ws:
        w.free()


@pytest.mark.parametrize("m", [96, 200])
def test_gemm_paired_zero_scale_blocks(q, oracle, wl, gpu, m):
    """Paired tiles of two weights whose zero-scale blocks differ (each
    weight's block scales tracked on their own): narrow tiles cut along K
    (96 tokens) and 64x64 tiles only (200).  Within the GEMM bars of the
    oracle; a row group with no live block exactly 0 in its own weight
    only."""
    import torch
    k, n = 1536, 640
    rng = np.random.default_rng(95)
    Ws, scs = [], []
    for i in range(2):
        W = rng.integers(0, 0x7E, size=(n, k), dtype=np.uint8) | (rng.integers(0, 2, size=(n, k), dtype=np.uint8) << 7)
        sc = np.full((n // 128, k // 128), 0x3980, np.uint16)       # bf16 2^-12: outputs of unit scale
        Ws.append(W)
        scs.append(sc)
    scs[0][0, 0] = 0                  # first block of group 0, weight 0 only
    scs[1][1, 5:7] = 0                # middle blocks of group 1, weight 1 only
    scs[0][2, :] = 0                  # group 2 dead in weight 0, live in weight 1
    scs[1][3, -1] = 0                 # last block of group 3, weight 1 only
    X = wl.gen_act(96, m, k)
    ws = [q.Weight(W, sc) for W, sc in zip(Ws, scs)]
    Ys = [torch.empty((m, n), dtype=torch.float32, device=gpu) for _ in ws]
    q.matmul_multi(ws, _torch_dev(X, gpu), Ys)
    torch.cuda.synchronize()
    for W, sc, dY in zip(Ws, scs, Ys):
        rel, mx = _gemm_check(dY.cpu().numpy(), oracle.mm_batch(W, sc, X))
        assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (rel, mx)
    assert (Ys[0].cpu().numpy()[:, 256:384] == 0).all()
    assert (Ys[1].cpu().numpy()[:, 256:384] != 0).any()
    for w in ws:
        w.free()


@pytest.mark.parametrize("m", [64, 200])
def test_gemm_k_beyond_one_slice_table(q, oracle, wl, gpu, m):
    """K of 1025 blocks: more than one workgroup's LDS scale table (1024
    blocks per row group for 256 x 256 tiles, 512 for the narrow tiles of
    m <= 128), so every tile is cut into K slices and summed by the
    reduction kernel."""
    import torch
    k, n = 1025 * 128, 256
    W, sc = wl.gen_weight(93, n, k)
    X = wl.gen_act(94, m, k, bf16=True)
    w = q.Weight(W, sc)
    dY = torch.empty((m, n), dtype=torch.float32, device=gpu)
    q.gemm(w, _torch_dev(X, gpu), dY)
    torch.cuda.synchronize()
    rel, mx = _gemm_check(dY.cpu().numpy(), oracle.mm_batch(W, sc, X))
    assert rel <= GEMM_REL_L2 and mx <= GEMM_MAX_ABS, (rel, mx)


def test_gemm_bf16_exact_inputs_near_exact(q, oracle, wl, gpu):
    """With bf16-representable activations the only rounding left in the GEMM
    is fp32 accumulation, so it agrees with the oracle far inside the bar."""
    import torch
    W, sc = wl.gen_weight(71, 512, 2048)
    X = wl.gen_act(72, 256, 2048, bf16=True)
    w = q.Weight(W, sc)
    dY = torch.empty((256, 512), dtype=torch.float32, device=gpu)
    q.gemm(w, _torch_dev(X, gpu), dY)
    torch.cuda.synchronize()
    Y = dY.cpu().numpy()
    Yr = oracle.mm_batch(W, sc, X)
    assert normwise_rel(Y, Yr) <= 1e-5


# ------------------------------------------------------------- device API
def test_device_api_matches_host_abi(q, wl, gpu):
    import torch
    W, sc = wl.gen_weight(81, 3000, 4736)
    X = wl.gen_act(82, 6, 4736)
    Yh = q.mm_fp8_batch(W, sc, X)
    w = q.Weight(W, sc)
    dY = torch.empty((6, 3000), dtype=torch.float32, device=gpu)
    q.matmul(w, _torch_dev(X, gpu), dY)
    torch.cuda.synchronize()
    assert (dY.cpu().numpy().view(np.uint32) == Yh.view(np.uint32)).all()
    # multi on device pointers == per-segment results
    W2, sc2 = wl.gen_weight(83, 500, 4736)
    w2 = q.Weight(W2, sc2)
    dY1 = torch.empty((6, 3000), dtype=torch.float32, device=gpu)
    dY2 = torch.empty((6, 500), dtype=torch.float32, device=gpu)
    q.matmul_multi([w, w2], _torch_dev(X, gpu), [dY1, dY2])
    torch.cuda.synchronize()
    assert (dY1.cpu().numpy().view(np.uint32) == Yh.view(np.uint32)).all()
    assert (dY2.cpu().numpy().view(np.uint32) == q.mm_fp8_batch(W2, sc2, X).view(np.uint32)).all()
    q.release(W)
    q.release(W2)


def test_registry_detects_reused_pointer(q, oracle, wl, gpu):
    q.release_all()
    W, sc = wl.gen_weight(91, 256, 512)
    x = wl.gen_act(92, 1, 512)[0]
    y1 = q.mm_fp8(W, sc, x)
    assert q.resident_count() == 1
    y1b = q.mm_fp8(W, sc, x)
    assert q.resident_count() == 1 and (y1.view(np.uint32) == y1b.view(np.uint32)).all()
    # new contents behind the same pointers must be picked up
    W2, sc2 = wl.gen_weight(93, 256, 512)
    W[...] = W2
    sc[...] = sc2
    y2 = q.mm_fp8(W, sc, x)
    assert normwise_rel(y2, oracle.mm(W2, sc2, x)) <= GEMV_TOL
    q.release(W)
    assert q.resident_count() == 0


def test_registry_reused_pointers_multi4_and_bf16(q, oracle, wl, gpu):
    """The fingerprint of a found pointer is checked while the device runs
    the call; a mismatch repeats the call on a fresh upload.  multi4 with
    one of two weights replaced in place (the other unchanged), a batch
    call, and the BF16 matvec: every result is the new contents'."""
    q.release_all()
    W1, s1 = wl.gen_weight(94, 300, 1024)
    W2, s2 = wl.gen_weight(95, 200, 1024)
    x = wl.gen_act(96, 1, 1024)[0]
    X = wl.gen_act(97, 5, 1024)
    for _ in range(2):
        q.mm_fp8_multi4([W1, W2], [s1, s2], x)
    N2, n2 = wl.gen_weight(98, 200, 1024)
    W2[...] = N2
    s2[...] = n2
    ya, yb = q.mm_fp8_multi4([W1, W2], [s1, s2], x)[:2]
    assert normwise_rel(ya, oracle.mm(W1, s1, x)) <= GEMV_TOL
    assert normwise_rel(yb, oracle.mm(N2, n2, x)) <= GEMV_TOL
    N1, n1 = wl.gen_weight(99, 300, 1024)
    W1[...] = N1
    s1[...] = n1
    Y = q.mm_fp8_batch(W1, s1, X)
    Yr = oracle.mm_batch(N1, n1, X)
    for t in range(5):
        assert normwise_rel(Y[t], Yr[t]) <= GEMV_TOL
    assert q.resident_count() == 2
    B = (wl.gen_act(100, 96, 256) * np.float32(0.05)).view(np.uint32)
    Wb = (B >> 16).astype(np.uint16)
    xb = wl.gen_act(101, 1, 256)[0]
    q.mm_bf16(Wb, xb)
    Wb[...] = (Wb.astype(np.uint32) ^ 0x8000).astype(np.uint16)   # every sign flipped
    yb2 = q.mm_bf16(Wb, xb)
    assert (yb2.view(np.uint32) == oracle.mm_bf16(Wb, xb).view(np.uint32)).all()
    q.release_all()
    assert q.resident_count() == 0


# ------------------------------------------------------------- BF16 matvec
# The BF16 matvec keeps the reference's summation order (eight fmaf chains,
# ordered final sum), so it is compared bit for bit.
def test_bf16_reference_fixture(q, oracle, gpu):
    c, W, _, x, yref = load_fixture("mid_bf16")
    y = q.mm_bf16(W, x)
    assert (np.abs(y.astype(np.float64) - yref) <= 5e-4 + 5e-4 * np.abs(yref)).all()
    assert (y.view(np.uint32) == oracle.mm_bf16(W, x).view(np.uint32)).all()
    q.release(W)


@pytest.mark.parametrize("rows,cols", [(2048, 5120), (1000, 77), (333, 5000), (70, 8), (65, 72)])
def test_bf16_gemv_random(q, oracle, wl, gpu, rows, cols):
    """Vector path (cols % 8 == 0: full and partial 64-column tiles, partial
    64-row groups) and the element path (cols = 77), bit for bit."""
    rng = np.random.default_rng(rows + cols)
    W = wl.bf16_rne(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05))
    x = rng.standard_normal(cols, dtype=np.float32)
    y = q.mm_bf16(W, x)
    assert (y.view(np.uint32) == oracle.mm_bf16(W, x).view(np.uint32)).all()
    q.release(W)


def test_bf16_gemv_device_api_lm_head_rows(q, oracle, wl, gpu):
    """Device API on a tall matrix (the lm_head's shape class): 248320 rows
    would need 2.5 GB; 16384 x 5120 covers the same per-row path."""
    import torch
    rows, cols = 16384, 5120
    rng = np.random.default_rng(7)
    W = wl.bf16_rne(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(cols, dtype=np.float32)
    dW = _torch_dev(W.view(np.int16), gpu)
    dx = _torch_dev(x, gpu)
    dy = torch.empty(rows, dtype=torch.float32, device=gpu)
    q.bf16_gemv(dW, dx, dy)
    torch.cuda.synchronize()
    assert (dy.cpu().numpy().view(np.uint32) == oracle.mm_bf16(W, x).view(np.uint32)).all()


def test_host_abi_from_several_threads(q, wl, gpu):
    """The drop-in calls are serialised by the library lock: four host
    threads calling q35_mm_fp8 / q35_mm_fp8_batch / q35_mm_fp8_multi4 at once
    on shared and private weights get the bits of the same calls made one at
    a time."""
    import threading
    Ws = [wl.gen_weight(200 + i, 640 + 128 * i, 1024) for i in range(3)]
    Xs = [wl.gen_act(210 + i, 1 + i, 1024) for i in range(4)]
    want = {}
    for i, X in enumerate(Xs):
        for j, (W, sc) in enumerate(Ws):
            want[(i, j)] = q.mm_fp8_batch(W, sc, X)
    errors = []

    def worker(i):
        try:
            for rep in range(6):
                j = (i + rep) % 3
                W, sc = Ws[j]
                got = q.mm_fp8_batch(W, sc, Xs[i]) if rep % 2 else np.stack(
                    [q.mm_fp8(W, sc, x) for x in Xs[i]])
                if not (got.view(np.uint32) == want[(i, j)].view(np.uint32)).all():
                    errors.append((i, rep, j))
            ys = q.mm_fp8_multi4([Ws[0][0], Ws[1][0]], [Ws[0][1], Ws[1][1]], Xs[i][0])
            for j in range(2):
                if not (ys[j].view(np.uint32) == want[(i, j)][0].view(np.uint32)).all():
                    errors.append((i, "multi4", j))
        except Exception as e:   # surfaced below
            errors.append((i, repr(e)))
    th = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors
    for W, _ in Ws:
        q.release(W)


def _scale_pattern(nb, kb, e_hi, e_lo):
    """bf16 scales alternating 2^e_hi and 2^e_lo along K in every row group."""
    sc = np.empty((nb, kb), np.uint16)
    for j in range(kb):
        e = e_hi if j % 2 == 0 else e_lo
        sc[:, j] = (127 + e) << 7
    return sc


def test_gemm_wide_scale_spread_runs_on_gemv(q, oracle, wl, gpu):
    """Block scales 2^60 and 2^-60 in one row group (bf16-representable):
    the reference's lut*s*x stays finite, while a GEMM accumulator kept in
    the current block's units would overflow.  q35_mm_fp8_batch at 96 tokens
    (the GEMM range) runs such a weight on the GEMV and meets the GEMV bar;
    q35mm_gemm refuses it."""
    import torch
    rng = np.random.default_rng(341)
    W = rng.integers(0, 0x7E, size=(256, 1024), dtype=np.uint8) | (rng.integers(0, 2, size=(256, 1024), dtype=np.uint8) << 7)
    sc = _scale_pattern(2, 8, 60, -60)
    X = wl.gen_act(342, 96, 1024)
    Y = q.mm_fp8_batch(W, sc, X)
    Yr = oracle.mm_batch(W, sc, X)
    assert np.isfinite(Yr).all() and np.isfinite(Y).all()
    for t in range(96):
        assert normwise_rel(Y[t], Yr[t]) <= GEMV_TOL, t
    w = q.Weight(W, sc)
    with pytest.raises(q.Q35mmError):
        q.gemm(w, torch.from_numpy(X).to(gpu), torch.empty((96, 256), device=gpu))
    w.free()
    q.release(W)


def test_gemm_scale_spread_2_pow_40(q, oracle, wl, gpu):
    """Scales 2^20 and 2^-20 alternating along K (a spread of 2^40, inside
    the GEMM's range): the GEMM with bf16-representable activations agrees
    with the oracle far inside its bar."""
    import torch
    rng = np.random.default_rng(343)
    W = rng.integers(0, 0x7E, size=(256, 1024), dtype=np.uint8) | (rng.integers(0, 2, size=(256, 1024), dtype=np.uint8) << 7)
    sc = _scale_pattern(2, 8, 20, -20)
    X = wl.gen_act(344, 96, 1024, bf16=True)
    w = q.Weight(W, sc)
    dY = torch.empty((96, 256), device=gpu)
    q.gemm(w, torch.from_numpy(X).to(gpu), dY)
    torch.cuda.synchronize()
    Y = dY.cpu().numpy().astype(np.float64)
    Yr = oracle.mm_batch(W, sc, X).astype(np.float64)
    assert np.linalg.norm(Y - Yr) / np.linalg.norm(Yr) <= 1e-5
    w.free()
