"""Pins the CPU oracle (oracle/q35_oracle.c) before it is trusted as the
oracle the HIP path is compared with.

Each part is checked against something independent of the restatement:
  - e4m3 / bf16 decode: torch's float8_e4m3fn / bfloat16 casts, the OCP
    table's defining values, and the reference's compiled LUT;
  - the quantizer: torch's round-to-nearest-even casts, a pure-Python
    nearest-code search on small inputs, and hand-computed blocks;
  - the matmul: the reference's own fixtures (f64 yref with the reference's
    tolerance, and the FNV hashes its test prints), golden hashes of the
    compiled reference on seeded inputs, bitwise equality with the compiled
    reference, exact special cases and the reference's batch/multi4 laws.
"""
import numpy as np
import pytest
import torch

from conftest import fixture_names, goldens, load_fixture


# ---------------------------------------------------------------- decoders
def test_e4m3_table_matches_torch_and_ocp(oracle):
    lut = oracle.lut()
    codes = torch.arange(256, dtype=torch.uint8)
    t = codes.view(torch.float8_e4m3fn).float().numpy()
    nan_codes = {0x7F, 0xFF}
    for c in range(256):
        if c in nan_codes:
            assert np.isnan(lut[c])
        else:
            assert lut[c].view(np.uint32) == np.float32(t[c]).view(np.uint32), hex(c)
    # defining values of the OCP OFP8 E4M3 format
    assert lut[0x38] == 1.0 and lut[0x7E] == 448.0 and lut[0xFE] == -448.0
    assert lut[0x01] == 2.0 ** -9 and lut[0x07] == 7 * 2.0 ** -9 and lut[0x08] == 2.0 ** -6
    assert lut[0x00] == 0.0 and lut[0x80] == 0.0 and np.signbit(lut[0x80])
    # NaN bit patterns of the reference (NAN, and -NAN for the sign bit)
    assert lut[0x7F].view(np.uint32) == 0x7FC00000
    assert lut[0xFF].view(np.uint32) == 0xFFC00000


def test_e4m3_table_bitwise_equals_reference(oracle, ref):
    assert (oracle.lut().view(np.uint32) == ref.lut().view(np.uint32)).all()


def test_bf16_decode_matches_torch(oracle):
    bits = np.arange(0, 65536, 7, dtype=np.uint16)
    t = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).float().numpy()
    got = np.array([oracle.lib.orc_bf16_to_f32(int(b)) for b in bits], np.float32)
    ok = np.isnan(t) & np.isnan(got) | (got.view(np.uint32) == t.view(np.uint32))
    assert ok.all()


# --------------------------------------------------------------- quantizer
def test_f32_to_bf16_is_rne(oracle):
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10,
                        # exact ties: low half 0x8000 with even and odd kept lsb
                        (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x40490000], np.uint32)
                         .view(np.float32))])
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (oracle.f32_to_bf16(v) == want).all()


def _python_nearest_e4m3(v: float) -> int:
    """Independent brute force over the finite codes in exact arithmetic:
    minimal |v| - value, ties to the even code, saturating, sign from v<0."""
    mags = [(m * 2.0 ** -9) if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
            for e in range(16) for m in range(8)][:127]
    a = abs(v)
    best = min(range(127), key=lambda i: (abs(a - mags[i]), i & 1))
    return (0x80 if v < 0 else 0) | best


def test_f32_to_e4m3_against_bruteforce_and_torch(oracle):
    rng = np.random.default_rng(1)
    lut = oracle.lut()
    fin = lut[:127].astype(np.float64)
    mids = ((fin[:-1] + fin[1:]) / 2).astype(np.float32)           # exact ties
    v = np.concatenate([lut[:127], mids, -mids, rng.standard_normal(600).astype(np.float32) * 50,
                        np.array([0.0, 447.9, 448.0, 460.0, 500.0, 1e5, 2.0 ** -10, 3 * 2.0 ** -11],
                                 np.float32)])
    got = oracle.f32_to_e4m3(v)
    want = np.array([_python_nearest_e4m3(float(x)) for x in v], np.uint8)
    assert (got == want).all()
    # torch rounds to nearest even too; it does not saturate, so compare
    # only where |v| <= 448
    inr = np.abs(v) <= 448
    t = torch.from_numpy(v[inr]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    t = np.where(v[inr] == 0, 0, t)          # the reference maps -0.0 to 0x00
    assert (got[inr] == t).all()


def test_f32_to_e4m3_special_values(oracle):
    f = oracle.lib.orc_f32_to_e4m3
    assert f(float("nan")) == 0x7F
    assert f(-0.0) == 0x00 and f(0.0) == 0x00
    assert f(-1e-6) == 0x80          # negative values that round to zero keep the sign
    assert f(1000.0) == 0x7E and f(-1000.0) == 0xFE


def test_quantize_block_recipe_by_hand(oracle):
    # one 2x3 block: amax = 0.7 -> scale = bf16(0.7/448)
    w = np.array([[0.7, -0.35, 0.0], [0.07, 0.001, -0.7]], np.float32)
    q, sc = oracle.quantize(w)
    s32 = np.float32(0.7) / np.float32(448.0)
    sb = int(oracle.f32_to_bf16(np.array([s32]))[0])
    assert sc.shape == (1, 1) and int(sc[0, 0]) == sb
    s = np.float32(oracle.lib.orc_bf16_to_f32(sb))
    want = np.array([[_python_nearest_e4m3(float(np.float32(x) / s)) for x in r] for r in w], np.uint8)
    assert (q == want).all()
    # 0.7/s is within a rounding of 448: the code must be 448 exactly
    assert q[0, 0] == 0x7E and q[1, 2] == 0xFE


def test_quantize_zero_block_and_partial_blocks(oracle):
    w = np.zeros((130, 260), np.float32)
    w[129, 259] = 3.0
    q, sc = oracle.quantize(w)
    assert sc.shape == (2, 3)
    assert (sc[0] == 0).all() and sc[1, 0] == 0 and sc[1, 1] == 0 and sc[1, 2] != 0
    assert q[129, 259] == 0x7E and np.count_nonzero(q) == 1


# ------------------------------------------------------------------ matmul
@pytest.mark.parametrize("name", fixture_names(fp8=True))
def test_mm_reference_fixtures(oracle, name):
    """The reference's test_mm check (qwen35-c/tests/test_mm.c:63-75) plus the
    FNV hash that test prints for the compiled reference."""
    c, W, sc, x, yref = load_fixture(name)
    y = oracle.mm(W, sc, x)
    tol = c["tol"]
    assert (np.abs(y.astype(np.float64) - yref) <= tol + tol * np.abs(yref)).all()
    assert f"{oracle.fnv64_q35test(y):016x}" == c["fnv_q35test"]


def test_mm_bf16_reference_fixture(oracle):
    c, W, _, x, yref = load_fixture("mid_bf16")
    y = oracle.mm_bf16(W, x)
    assert (np.abs(y.astype(np.float64) - yref) <= 5e-4 + 5e-4 * np.abs(yref)).all()
    assert f"{oracle.fnv64_q35test(y):016x}" == c["fnv_q35test"]


def _inputs(wl, case):
    if case["kind"] == "ragged":
        W, sc = wl.gen_weight_ragged(case["seed"], case["n"], case["k"])
    else:
        W, sc = wl.gen_weight(case["seed"], case["n"], case["k"])
    X = wl.gen_act(case["seed"] + 0x100, case["m"], case["k"], **case["act"])
    return W, sc, X


SMALL_GOLDENS = [c["name"] for c in goldens()["cases"] if c["m"] * c["k"] * c["n"] <= 120_000_000]


@pytest.mark.parametrize("name", SMALL_GOLDENS)
def test_mm_matches_reference_golden_hashes(oracle, wl, name):
    case = next(c for c in goldens()["cases"] if c["name"] == name)
    W, sc, X = _inputs(wl, case)
    assert f"{oracle.fnv64(W):016x}" == case["fnv_codes"]
    assert f"{oracle.fnv64(sc):016x}" == case["fnv_scales"]
    assert f"{oracle.fnv64(X):016x}" == case["fnv_x"]
    Y = oracle.mm_batch(W, sc, X)
    assert f"{oracle.fnv64(Y):016x}" == case["fnv_y_ref"]


def test_mm_bitwise_equals_compiled_reference(oracle, ref, wl):
    for seed, (m, k, n) in enumerate([(1, 5120, 640), (3, 129, 257), (7, 4700, 300), (2, 40, 1000)]):
        W, sc = wl.gen_weight_ragged(100 + seed, n, k)
        X = wl.gen_act(200 + seed, m, k, outlier_frac=0.05)
        a = oracle.mm_batch(W, sc, X)
        b = ref.mm_batch(W, sc, X)
        assert (a.view(np.uint32) == b.view(np.uint32)).all()


def test_mm_scalar_reference_build_agrees(oracle, wl):
    from oracle import REF_SCALAR_PATH, RefMM
    if not RefMM.available(REF_SCALAR_PATH):
        pytest.skip("scalar reference build absent")
    r = RefMM(REF_SCALAR_PATH)
    assert r.impl() == "scalar"
    W, sc = wl.gen_weight(9, 300, 777)
    X = wl.gen_act(10, 3, 777)
    assert (oracle.mm_batch(W, sc, X).view(np.uint32) == r.mm_batch(W, sc, X).view(np.uint32)).all()


def test_mm_batch_equals_single_and_multi4(oracle, wl):
    """Reference laws: batch == n x single bitwise (qwen35-c/src/q35_mm.c:155-157,
    tests/test_batch_mm.c), multi4 rows == single rows (q35_mm.c:176-198)."""
    W, sc = wl.gen_weight(11, 700, 1000)
    X = wl.gen_act(12, 5, 1000)
    Y = oracle.mm_batch(W, sc, X)
    for t in range(5):
        assert (Y[t].view(np.uint32) == oracle.mm(W, sc, X[t]).view(np.uint32)).all()
    W2, sc2 = wl.gen_weight(13, 48, 1000)
    outs = [np.empty(700, np.float32), np.empty(48, np.float32)]
    import ctypes as C
    from oracle import _f32p, _u8p, _u16p
    Wp = (_u8p * 4)(W.ctypes.data_as(_u8p), W2.ctypes.data_as(_u8p), None, None)
    Sp = (_u16p * 4)(sc.ctypes.data_as(_u16p), sc2.ctypes.data_as(_u16p), None, None)
    Rs = (C.c_uint32 * 4)(700, 48, 0, 0)
    Yp = (_f32p * 4)(outs[0].ctypes.data_as(_f32p), outs[1].ctypes.data_as(_f32p), None, None)
    x0 = np.ascontiguousarray(X[0])
    oracle.lib.orc_mm_fp8_multi4.argtypes = None
    oracle.lib.orc_mm_fp8_multi4(Wp, Sp, Rs, C.c_uint32(1000), x0.ctypes.data_as(_f32p), Yp)
    assert (outs[0].view(np.uint32) == Y[0].view(np.uint32)).all()
    assert (outs[1].view(np.uint32) == oracle.mm(W2, sc2, X[0]).view(np.uint32)).all()


def test_mm_special_cases(oracle, wl):
    W, sc = wl.gen_weight_ragged(21, 260, 300)
    deq = oracle.dequant(W, sc)
    # one-hot x picks a dequantized column exactly
    for col in (0, 127, 128, 299):
        x = np.zeros(300, np.float32)
        x[col] = 1.0
        assert (oracle.mm(W, sc, x).view(np.uint32) == deq[:, col].view(np.uint32)).all()
    # dequant is the exact product lut[b] * s (e4m3 x bf16 fits in fp32)
    lut = oracle.lut().astype(np.float64)
    s = np.repeat(np.repeat(wl.bf16_to_f32(sc).astype(np.float64), 128, 0), 128, 1)[:260, :300]
    assert (deq.astype(np.float64) == lut[W] * s).all()
    # a zero scale block contributes nothing
    sc0 = sc.copy()
    sc0[:, 1] = 0
    x = wl.gen_act(22, 1, 300)[0]
    x_cut = x.copy()
    x_cut[128:256] = 0
    assert np.array_equal(oracle.mm(W, sc0, x), oracle.mm(W, sc, x_cut))


def test_mm_close_to_exact_math(oracle, wl):
    W, sc = wl.gen_weight(31, 300, 5120)
    X = wl.gen_act(32, 2, 5120)
    y = oracle.mm_batch(W, sc, X).astype(np.float64)
    y64 = oracle.mm_f64(W, sc, X)
    assert np.abs(y - y64).max() / np.abs(y64).max() < 2e-6
