"""The reference's real decode projections besides the MLP, on the GPU
through the drop-in C ABI, against the oracle.

Shapes (rows x cols of W, K = cols):
  DeltaNet multi4 in_proj_qkv / in_proj_z / in_proj_a / in_proj_b
    (10240, 6144, 48, 48) x 5120   qwen35-c/src/q35_deltanet.c:325-329
  GQA q / k / v  12288 / 1024 / 1024 x 5120   qwen35-c/src/q35_attn.c:273-275
  out_proj / o_proj 5120 x 6144   qwen35-c/src/q35_deltanet.c:360, q35_attn.c:262
and out_proj / o_proj over a prefill's tokens as one batch (63 tokens on the
decode GEMV, 512 on the prefill GEMM) instead of the reference's per-token
calls (qwen35-c/src/q35_deltanet.c:498, qwen35-c/src/q35_attn.c:262,311).
The single-weight M=1 and 63-token cases are golden cases
(tests/golden/ref_hashes.json) that test_gpu_parity.py runs, the oracle's
outputs hash-equal to the compiled reference's.

Bars: decode GEMV ||y - y_ref||_inf / ||y_ref||_inf <= 1e-5 per token; prefill
GEMM ||Y - Y_ref||_2 / ||Y_ref||_2 <= 5e-3 and max |Y - Y_ref| <= 2e-2;
bitwise where results must equal other calls of the library.
"""
import numpy as np
import pytest

from conftest import goldens, normwise_rel

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
GEMM_REL_L2 = 5e-3
GEMM_MAX_ABS = 2e-2


def _case(name):
    return next(c for c in goldens()["cases"] if c["name"] == name)


def _inputs(wl, c):
    W, sc = wl.gen_weight(c["seed"], c["n"], c["k"])
    X = wl.gen_act(c["seed"] + 0x100, c["m"], c["k"], **c["act"])
    return W, sc, X


def test_deltanet_multi4_real_shapes(q, oracle, wl, gpu):
    """One q35_mm_fp8_multi4 over (10240, 6144, 48, 48) x 5120: each segment
    within the GEMV bar of the oracle and bit-identical to its single call;
    the qkv segment's oracle output hash-equal to the compiled reference's."""
    c = _case("model_dn_qkv_m1_5120x10240")
    Wq, sq, X = _inputs(wl, c)
    x = X[0]
    segs = [(Wq, sq)] + [wl.gen_weight(wl.SEED_BASE + 0x40 + i, n, 5120) for i, n in enumerate((6144, 48, 48))]
    outs = q.mm_fp8_multi4([s[0] for s in segs], [s[1] for s in segs], x)
    for i, ((W, sc), y) in enumerate(zip(segs, outs)):
        yr = oracle.mm(W, sc, x)
        if i == 0:
            assert f"{oracle.fnv64(yr[None, :]):016x}" == c["fnv_y_ref"]
        assert normwise_rel(y, yr) <= GEMV_TOL, i
        assert (q.mm_fp8(W, sc, x).view(np.uint32) == y.view(np.uint32)).all(), i
    for W, _ in segs:
        q.release(W)


def test_gqa_qkv_real_shapes_in_call_order(q, oracle, wl, gpu):
    """q, k, v as three q35_mm_fp8 calls on one x, in the reference's order."""
    x = wl.gen_act(wl.SEED_BASE + 0x48, 1, 5120)[0]
    ws = [wl.gen_weight(wl.SEED_BASE + 0x49 + i, n, 5120) for i, n in enumerate((12288, 1024, 1024))]
    for W, sc in ws:
        assert normwise_rel(q.mm_fp8(W, sc, x), oracle.mm(W, sc, x)) <= GEMV_TOL
    for W, _ in ws:
        q.release(W)


def test_gqa_qkv_as_one_multi4_call(q, wl, gpu):
    """q, k, v folded into one q35_mm_fp8_multi4 call (three segments, the
    fourth empty: rows 0, as the reference's multi4 allows): every output the
    bits of its separate q35_mm_fp8 call."""
    x = wl.gen_act(wl.SEED_BASE + 0x48, 1, 5120)[0]
    ws = [wl.gen_weight(wl.SEED_BASE + 0x49 + i, n, 5120) for i, n in enumerate((12288, 1024, 1024))]
    outs = q.mm_fp8_multi4([W for W, _ in ws], [sc for _, sc in ws], x)
    assert outs[3] is None
    for (W, sc), y in zip(ws, outs[:3]):
        assert (q.mm_fp8(W, sc, x).view(np.uint32) == y.view(np.uint32)).all()
    for W, _ in ws:
        q.release(W)


def test_out_proj_63_tokens_equal_single_calls(q, wl, gpu):
    """The straggler batch on the decode GEMV (63 < 64 tokens): every row
    the bits of the per-token call the reference makes."""
    c = _case("straggler_m63_6144x5120")
    W, sc, X = _inputs(wl, c)
    Y = q.mm_fp8_batch(W, sc, X)
    for t in range(X.shape[0]):
        assert (q.mm_fp8(W, sc, X[t]).view(np.uint32) == Y[t].view(np.uint32)).all(), t
    q.release(W)


def test_out_proj_512_tokens_gemm(q, oracle, wl, gpu):
    """The straggler batch on the prefill GEMM (512 tokens, fp32 activations
    rounded to bf16 inside): within the GEMM bars of the oracle, whose
    output is hash-equal to the compiled reference's."""
    c = _case("straggler_m512_6144x5120")
    W, sc, X = _inputs(wl, c)
    Y = q.mm_fp8_batch(W, sc, X)
    Yr = oracle.mm_batch(W, sc, X)
    assert f"{oracle.fnv64(Yr):016x}" == c["fnv_y_ref"]
    d = Y.astype(np.float64) - Yr.astype(np.float64)
    rel = np.linalg.norm(d) / np.linalg.norm(Yr.astype(np.float64))
    assert rel <= GEMM_REL_L2 and np.abs(d).max() <= GEMM_MAX_ABS, (rel, np.abs(d).max())
    q.release(W)


def test_multi4_outputs_beyond_the_direct_path(q, wl, gpu):
    """A q35_mm_fp8_multi4 whose outputs (400000 + 200000 rows: 2.4 MB) are
    too large for the kernels to write straight into pinned memory, so they
    come back over DMA in two chunks, the first ending inside segment 0;
    each segment the bits of its own q35_mm_fp8 call."""
    x = wl.gen_act(wl.SEED_BASE + 0x4A, 1, 128)[0]
    ws = [wl.gen_weight(wl.SEED_BASE + 0x4B + i, n, 128) for i, n in enumerate((400000, 200000))]
    outs = q.mm_fp8_multi4([W for W, _ in ws], [sc for _, sc in ws], x)
    for (W, sc), y in zip(ws, outs[:2]):
        assert (q.mm_fp8(W, sc, x).view(np.uint32) == y.view(np.uint32)).all()
    for W, _ in ws:
        q.release(W)

