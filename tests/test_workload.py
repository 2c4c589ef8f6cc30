"""The synthetic generator follows the reference quantizer recipe code for
code (checked against the oracle's exhaustive-search restatement)."""
import numpy as np
import pytest


@pytest.mark.parametrize("shape", [(3, 5), (129, 129), (300, 700), (128, 4736), (200, 4700)])
def test_generator_quantizer_equals_oracle(wl, oracle, shape):
    rng = np.random.default_rng(sum(shape))
    w = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)
    w[0, 0] = -0.0
    a, sa = wl.quantize_fp8(w)
    b, sb = oracle.quantize(w)
    assert (a == b).all() and (sa == sb).all()


def test_ragged_generator_equals_oracle_and_has_edge_codes(wl, oracle):
    seed, n, k = 77, 300, 700
    W, sc = wl.gen_weight_ragged(seed, n, k)
    # regenerate the fp32 weights exactly as the generator does and quantize
    # them with the oracle
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k), dtype=np.float32)
    amax_t = (10.0 ** rng.uniform(-4.0, 2.0, size=((n + 127) // 128, (k + 127) // 128))).astype(np.float32)
    for bi in range(amax_t.shape[0]):
        for bj in range(amax_t.shape[1]):
            blk = w[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            blk *= np.float32(amax_t[bi, bj] / np.float32(np.abs(blk).max()))
    b, sb = oracle.quantize(w)
    assert (W == b).all() and (sc == sb).all()
    codes = set(np.unique(W).tolist())
    assert not ({0x7F, 0xFF} & codes), "no NaN codes"
    assert {0x7E, 0xFE} & codes, "saturation codes present"
    assert {1, 2, 3, 4, 5, 6, 7} & codes, "subnormal codes present"


def test_e4m3_encode_matches_oracle_on_specials(wl, oracle):
    v = np.array([0.0, -0.0, 448.0, 449.0, 464.0, 480.0, 1e6, -1e6, np.inf, -np.inf, np.nan,
                  2.0 ** -10, -2.0 ** -10, 3 * 2.0 ** -10, 1e30, 9.9e29, 2.0 ** 33, -2.0 ** 32], np.float32)
    assert (wl.e4m3_encode(v) == oracle.f32_to_e4m3(v)).all()


def test_gen_weight_deterministic_and_shaped(wl):
    a, sa = wl.gen_weight(5, 300, 260)
    b, sb = wl.gen_weight(5, 300, 260)
    assert a.shape == (300, 260) and sa.shape == (3, 3)
    assert (a == b).all() and (sa == sb).all()
    c, _ = wl.gen_weight(6, 300, 260)
    assert (a != c).any()


def test_gen_act_options(wl):
    x = wl.gen_act(1, 4, 1000, bf16=True)
    assert (wl.bf16_to_f32(wl.bf16_rne(x)).reshape(x.shape) == x).all()
    y = wl.gen_act(2, 50, 1000, outlier_frac=0.01)
    frac = (np.abs(y) > 8).mean()
    assert 0.003 < frac < 0.02


def test_algorithmic_bytes_formula(wl):
    # one 5120x5120 matvec: codes + fp32 scales + x + y
    assert wl.algorithmic_bytes(1, 5120, 5120) == 26_261_760
    assert wl.flops(512, 5120, 34816) == 182_536_110_080
