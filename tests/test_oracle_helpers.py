"""Pins for the oracle helpers that the GPU tests compare with besides the
reference-shaped entry points: the row-subset matmul (orc_mm_fp8_rows, the
oracle of the full-size prefill GEMM shapes), the fp32-scale dequant and the
fp32-scale batch matmul.  Each is pinned to something independent of its own
code: the bf16-scale path (itself bit-identical to the compiled reference),
exact rational arithmetic with one explicit rounding per reference operation
(qwen35-c/src/q35_mm.c:88-142: w = lut[b]*s rounded once, acc[c mod 8] =
fmaf(w, x[c], acc), lanes added 0..7), float64 products, and power-of-two
scaling laws.  A C driver runs the batch and row-subset paths under
AddressSanitizer at more than 1024 K blocks."""
import os
import shutil
import subprocess
from fractions import Fraction

import numpy as np
import pytest

from conftest import ROOT


def _f32_round(q: Fraction) -> Fraction:
    """q rounded to the nearest fp32 value, ties to even (normal and
    subnormal range; no overflow in these tests)."""
    if q == 0:
        return Fraction(0)
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1                      # now 2^e <= a < 2^(e+1)
    ulp_e = max(e - 23, -149)
    m = round(a / Fraction(2) ** ulp_e)   # Fraction rounding: half to even
    r = Fraction(m) * Fraction(2) ** ulp_e
    assert r < Fraction(2) ** 128
    return r if q > 0 else -r


def _exact_dot(codes, srow, x, lut):
    """One output of the reference's dot product, every operation rounded
    once to fp32 from its exact value."""
    acc = [Fraction(0)] * 8
    for c in range(len(codes)):
        s = Fraction(float(srow[c // 128]))
        w = _f32_round(Fraction(float(lut[codes[c]])) * s)
        acc[c & 7] = _f32_round(w * Fraction(float(x[c])) + acc[c & 7])
    total = Fraction(0)
    for j in range(8):
        total = _f32_round(total + acc[j])
    return np.float32(float(total))


def _ragged(seed, rows, cols, scale_kind="bf16"):
    rng = np.random.default_rng(seed)
    W = rng.integers(0, 256, size=(rows, cols), dtype=np.uint8)
    W[(W & 0x7F) == 0x7F] -= 1                         # no NaN codes
    nb, kb = (rows + 127) // 128, (cols + 127) // 128
    if scale_kind == "bf16":
        sc = (0x3B00 + rng.integers(0, 0x300, size=(nb, kb))).astype(np.uint16)
    else:   # fp32 scales with full 24-bit significands, one zero block
        sc = (rng.uniform(1e-3, 1e-1, size=(nb, kb))).astype(np.float32)
        sc[0, -1] = 0.0
    return W, sc


def test_rows_equal_batch_columns_bitwise(oracle):
    for rows, cols, n in ((300, 1000, 3), (130, 4700, 2), (1, 129, 1)):
        W, sc = _ragged(rows + cols, rows, cols)
        X = np.random.default_rng(7).standard_normal((n, cols)).astype(np.float32)
        Yb = oracle.mm_batch(W, sc, X)
        idx = np.array(sorted({0, rows - 1, min(127, rows - 1), min(128, rows - 1), rows // 2}) + [0], np.uint32)
        Yr = oracle.mm_rows(W, sc, X, idx)
        assert Yr.shape == (n, idx.size)
        assert (Yr.view(np.uint32) == Yb[:, idx].view(np.uint32)).all()


def test_dequant_f32scale_is_one_rounded_multiply(oracle):
    lut = oracle.lut()
    rng = np.random.default_rng(3)
    scales = np.concatenate([
        rng.uniform(1e-4, 10.0, 200).astype(np.float32),
        np.array([0.0, 1.0, 2.0 ** -126, 2.0 ** -140, 3.0e38 / 448, 1.0000001, 0.33333334], np.float32)])
    W = np.tile(np.arange(256, dtype=np.uint8), (1, 1))          # one row, every code
    for s in scales:
        sc = np.array([[s, s]], np.float32)
        out = oracle.dequant(W, sc)[0]
        want = (lut.astype(np.float64) * np.float64(s)).astype(np.float32)   # exact product, one rounding
        nan = np.isnan(want)
        assert (np.isnan(out) == nan).all()
        assert (out[~nan].view(np.uint32) == want[~nan].view(np.uint32)).all(), s


def test_dequant_f32scale_equals_bf16_path_on_bf16_scales(oracle):
    W, sc16 = _ragged(11, 260, 300)
    sc32 = (sc16.astype(np.uint32) << 16).view(np.float32)
    a = oracle.dequant(W, sc16)
    b = oracle.dequant(W, sc32)
    assert (a.view(np.uint32) == b.view(np.uint32)).all()


def test_batch_f32scale_equals_bf16_path_on_bf16_scales(oracle):
    for rows, cols in ((300, 1000), (129, 4700)):
        W, sc16 = _ragged(rows * 3 + cols, rows, cols)
        sc32 = (sc16.astype(np.uint32) << 16).view(np.float32)
        X = np.random.default_rng(5).standard_normal((3, cols)).astype(np.float32)
        a = oracle.mm_batch(W, sc16, X)
        b = oracle.mm_batch(W, sc32, X)
        assert (a.view(np.uint32) == b.view(np.uint32)).all()


def test_batch_f32scale_power_of_two_scaling(oracle):
    """Multiplying every scale by 2^k multiplies every output by 2^k exactly
    (each rounding commutes with a power-of-two factor away from the
    subnormal and overflow ranges)."""
    W, sc = _ragged(21, 200, 900, scale_kind="f32")
    X = np.random.default_rng(6).standard_normal((2, 900)).astype(np.float32)
    y = oracle.mm_batch(W, sc, X)
    for k in (-7, 5):
        yk = oracle.mm_batch(W, (sc * np.float32(2.0 ** k)).astype(np.float32), X)
        assert (yk.view(np.uint32) == (y * np.float32(2.0 ** k)).view(np.uint32)).all()


def test_batch_f32scale_exact_rational_brute_force(oracle):
    """Tiny ragged shape (a partial row group and a partial K block) with
    fp32 scales that bf16 cannot hold: every output equals the reference's
    operation sequence evaluated in exact arithmetic with one rounding per
    operation."""
    W, sc = _ragged(33, 130, 300, scale_kind="f32")
    X = np.random.default_rng(8).standard_normal((2, 300)).astype(np.float32)
    X[0, 5] = 0.0
    Y = oracle.mm_batch(W, sc, X)
    lut = oracle.lut()
    for r in (0, 1, 127, 128, 129):
        for t in range(2):
            want = _exact_dot(W[r], sc[r // 128], X[t], lut)
            assert Y[t, r].view(np.uint32) == want.view(np.uint32), (r, t)


def test_batch_exact_rational_brute_force_bf16_scales(oracle):
    """The same brute force on the bf16-scale path, which the compiled
    reference pins as well: the emulation itself is right."""
    W, sc16 = _ragged(34, 130, 300)
    sc32 = (sc16.astype(np.uint32) << 16).view(np.float32)
    X = np.random.default_rng(9).standard_normal((1, 300)).astype(np.float32)
    Y = oracle.mm_batch(W, sc16, X)
    lut = oracle.lut()
    for r in (0, 64, 128, 129):
        want = _exact_dot(W[r], sc32[r // 128], X[0], lut)
        assert Y[0, r].view(np.uint32) == want.view(np.uint32), r


def test_batch_and_rows_under_asan_beyond_1024_blocks(tmp_path):
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    exe = str(tmp_path / "oracle_asan")
    build = subprocess.run(
        ["gcc", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer", "-ffp-contract=off", "-fopenmp",
         "-I", os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests", "c", "oracle_asan.c"),
         os.path.join(ROOT, "oracle", "q35_oracle.c"), "-o", exe, "-lm"], capture_output=True, text=True)
    if build.returncode != 0 and "asan" in build.stderr.lower():
        pytest.skip("AddressSanitizer runtime not available")
    assert build.returncode == 0, build.stderr
    for kb in ("1025", "3"):
        res = subprocess.run([exe, kb], capture_output=True, text=True, env={**os.environ, "OMP_NUM_THREADS": "4"})
        assert res.returncode == 0, res.stdout + res.stderr[-2000:]
        assert res.stdout.startswith("ok")
