"""Pins the oracle's restatement of the MLP neighbours (RMSNorm, SiLU,
SwiGLU, residual add; qwen35-c/src/q35_kern.c, q35_model.c:927-939) before
the device kernels are compared with it.

Independent checks: the reference's own fixtures (its NumPy model, with its
test's tolerances), the FNV-1a-32 of the compiled reference's output on
those fixtures (committed, so the check runs without the reference tree),
bitwise equality with the compiled q35_kern.c on seeded and ragged inputs
(both its AVX2 and scalar paths), float64 closed forms, and special values.
"""
import numpy as np
import pytest

from conftest import kern_manifest, load_kern_fixture, within_kern_tol

KERN_CASES = sorted(kern_manifest())


def _run(oracle, c, ins):
    if c["kernel"] == "rmsnorm":
        return oracle.rmsnorm(ins[0], ins[1], c["eps"])
    if c["kernel"] == "silu":
        return oracle.silu(ins[0])
    return oracle.swiglu(ins[0], ins[1])


@pytest.mark.parametrize("name", KERN_CASES)
def test_kern_fixture_within_reference_tolerance(oracle, name):
    c, ins, want = load_kern_fixture(name)
    y = _run(oracle, c, ins)
    assert y.shape == want.shape
    assert within_kern_tol(y, want, c["atol"], c["rtol"])


@pytest.mark.parametrize("name", KERN_CASES)
def test_kern_fixture_bitwise_equals_reference_hash(oracle, name):
    c, ins, _ = load_kern_fixture(name)
    assert "%08x" % oracle.fnv32(_run(oracle, c, ins)) == c["fnv1a_ref"]


@pytest.mark.parametrize("n", [1, 3, 7, 8, 9, 127, 5120, 5123, 17408])
@pytest.mark.parametrize("scalar", [False, True])
def test_kern_bitwise_equals_compiled_reference(oracle, refkern, n, scalar):
    rng = np.random.default_rng(1000 + n)
    x = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 30.0], n)).astype(np.float32)
    w = (rng.standard_normal(n) * 0.1).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    for eps in (1e-6, 1e-5):
        a, b = oracle.rmsnorm(x, w, eps), refkern.rmsnorm(x, w, eps, scalar=scalar)
        assert (a.view(np.uint32) == b.view(np.uint32)).all()
    assert (oracle.silu(x).view(np.uint32) == refkern.silu(x, scalar=scalar).view(np.uint32)).all()
    assert (oracle.swiglu(x, u).view(np.uint32) == refkern.swiglu(x, u, scalar=scalar).view(np.uint32)).all()


def test_rmsnorm_rows_are_independent_calls(oracle):
    rng = np.random.default_rng(5)
    X = rng.standard_normal((6, 333)).astype(np.float32)
    w = rng.standard_normal(333).astype(np.float32)
    Y = oracle.rmsnorm(X, w)
    for r in range(6):
        assert (Y[r].view(np.uint32) == oracle.rmsnorm(X[r], w).view(np.uint32)).all()


def test_rmsnorm_closed_forms(oracle):
    # constant vector: mean(x^2) = c^2 exactly for c a power of two, so
    # y = c / sqrt(c^2 + eps) * (1 + w) in float64 to a few ulps
    n = 4096
    w = np.linspace(-0.5, 0.5, n).astype(np.float32)
    for c in (0.25, 1.0, 8.0):
        y = oracle.rmsnorm(np.full(n, c, np.float32), w, 1e-6)
        want = c / np.sqrt(c * c + 1e-6) * (1.0 + w.astype(np.float64))
        assert np.allclose(y, want, rtol=4e-7, atol=0)
    # w = 0 normalises to unit RMS; a one-hot x gives sqrt(n) at the hot index
    rng = np.random.default_rng(3)
    x = rng.standard_normal(5120).astype(np.float32)
    y = oracle.rmsnorm(x, np.zeros(5120, np.float32), 0.0)
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 1e-6
    e = np.zeros(1024, np.float32)
    e[17] = 3.0
    y = oracle.rmsnorm(e, np.zeros(1024, np.float32), 0.0)
    assert y[17] == np.float32(32.0) and np.count_nonzero(y) == 1


def test_rmsnorm_lane_order_is_the_references(oracle):
    # x[0]^2 = 2^20, every other square 2^-4 = half an ulp of 2^20.  In one
    # running sum each small square is absorbed (ties to even): 2^20.  In the
    # reference's eight lanes, lane 0 absorbs its 7 small squares but lanes
    # 1..7 each sum 8 of them to 0.5 exactly, and the fold adds 3.5:
    # 2^20 + 3.5.  The exact sum is 2^20 + 63/16.  Only the lane order gives
    # 2^20 + 3.5, and the outputs tell the three apart.
    n = 64
    x = np.full(n, 0.25, np.float32)
    x[0] = 1024.0
    y = oracle.rmsnorm(x, np.zeros(n, np.float32), 0.0)

    def y0(total):
        inv = np.float32(1.0) / np.sqrt(np.float32(np.float32(total) / np.float32(n)))
        return np.float32(np.float32(1024.0) * inv)
    assert y[0] == y0(2.0 ** 20 + 3.5)
    assert y0(2.0 ** 20 + 3.5) != y0(2.0 ** 20) and y0(2.0 ** 20 + 3.5) != y0(2.0 ** 20 + 3.9375)


def test_silu_swiglu_special_values(oracle):
    g = np.array([0.0, -0.0, 1.0, -1.0, 30.0, 100.0, -30.0, -100.0, -200.0,
                  np.inf, -np.inf, np.nan], np.float32)
    s = oracle.silu(g)
    assert s[0] == 0 and s[2] == np.float32(1.0 / (1.0 + np.exp(-1.0)))
    assert s[4] == np.float32(30.0) and s[5] == np.float32(100.0)      # sigmoid rounds to 1
    assert s[7] == 0 and np.signbit(s[7]) and s[8] == 0                # exp overflows: -0
    assert s[9] == np.inf and np.isnan(s[10]) and np.isnan(s[11])       # -inf * 0 = NaN
    u = np.full_like(g, 2.0)
    assert (oracle.swiglu(g, u)[:10] == (s * np.float32(2.0))[:10]).all()
    # float64 model away from the special values
    x = np.linspace(-20, 20, 40001).astype(np.float32)
    want = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    got = oracle.silu(x).astype(np.float64)
    assert np.all(np.abs(got - want) <= 3 * np.spacing(np.abs(want).astype(np.float32)).astype(np.float64) + 1e-45)


def test_expf_is_libm(oracle):
    # within one ulp of exp in float64 below the overflow threshold, inf above
    x = np.linspace(-100, 88.7, 10001).astype(np.float32)
    y = oracle.expf(x)
    want = np.exp(x.astype(np.float64))
    assert np.all(np.abs(y - want) <= np.spacing(want.astype(np.float32)) + 1e-44)
    assert (oracle.expf(np.array([88.73, 100.0, np.inf], np.float32)) == np.inf).all()


def test_mlp_composition_order(oracle):
    """The MLP block is rmsnorm -> gate/up -> swiglu -> down -> x + y; a
    closed form on a diagonal down projection checks the wiring."""
    rng = np.random.default_rng(11)
    H, II = 256, 384
    x = rng.standard_normal((2, H)).astype(np.float32)
    nw = (rng.standard_normal(H) * 0.1).astype(np.float32)
    gate = oracle.quantize(rng.standard_normal((II, H)).astype(np.float32) * 0.05)
    up = oracle.quantize(rng.standard_normal((II, H)).astype(np.float32) * 0.05)
    down = oracle.quantize(rng.standard_normal((H, II)).astype(np.float32) * 0.05)
    r = oracle.mlp(x, nw, gate, up, down)
    xn = oracle.rmsnorm(x, nw)
    assert (r["xn"] == xn).all()
    assert (r["gate"] == oracle.mm_batch(gate[0], gate[1], xn)).all()
    assert (r["mid"] == oracle.swiglu(r["gate"], r["up"])).all()
    assert (r["out"] == (x + r["y"]).astype(np.float32)).all()
    # against float64 math on the dequantized weights
    Wg, Wu, Wd = (oracle.dequant(*t).astype(np.float64) for t in (gate, up, down))
    xn64 = xn.astype(np.float64)
    g64, u64 = xn64 @ Wg.T, xn64 @ Wu.T
    mid64 = g64 / (1 + np.exp(-g64)) * u64
    y64 = mid64 @ Wd.T
    assert np.abs(r["y"] - y64).max() <= 1e-5 * np.abs(y64).max()
