"""Seeded synthetic workloads for the FP8 block-dequant matmul.

Weights are sampled in fp32 and quantized per 128x128 block with the
reference's own in-tree recipe (qwen35-c/src/q35_model.c:325-344, helpers
:31-37 and :41-57): scale = bf16_rne(amax / 448), codes = nearest e4m3fn of
w / scale with ties to the even code, saturating at +-448, zero codes for a
zero-scale block.  The quantizer here is vectorised numpy; tests pin it code
for code against the oracle's exhaustive-search restatement.

Named workloads (sizes from the benchmark definition):
  single   M=1, 5120 -> 5120
  decode   M in {1,2,4,8} over one layer's projections
           5120->6144 (qkv), 4096->5120 (o_proj), 5120->17408 (gate, up),
           17408->5120 (down)
  prefill  M=512: 5120->34816 (fused gate+up), 17408->5120 (down),
           activations bf16-representable
  stack    64 layers (48 DeltaNet + 16 GQA) of the decode shapes at M=1
  ragged   M=37, K=4736, N=3000, per-block amax log-uniform in [1e-4, 1e2],
           1% of activations scaled by 100
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x51E50000

DECODE_SHAPES = [  # (name, K, N)
    ("qkv", 5120, 6144),
    ("o_proj", 4096, 5120),
    ("gate", 5120, 17408),
    ("up", 5120, 17408),
    ("down", 17408, 5120),
]
PREFILL_SHAPES = [("gate_up", 5120, 34816), ("down", 17408, 5120)]
SINGLE_SHAPE = ("single", 5120, 5120)

# The reference model's decode calls per layer besides the MLP (K, N):
# a Gated DeltaNet layer makes one q35_mm_fp8_multi4 over in_proj_qkv /
# in_proj_z / in_proj_a / in_proj_b (qwen35-c/src/q35_deltanet.c:325-329)
# and one q35_mm_fp8 for out_proj (:360); a GQA layer three q35_mm_fp8 for
# q / k / v (qwen35-c/src/q35_attn.c:273-275) and one for o_proj (:262).
# Every layer then runs the MLP: one multi4 over gate and up, one call for
# down (qwen35-c/src/q35_model.c:929-937).  Layers 3, 7, ..., 63 are GQA.
MODEL_DELTANET_SHAPES = [("in_proj_qkv", 5120, 10240), ("in_proj_z", 5120, 6144), ("in_proj_a", 5120, 48),
                         ("in_proj_b", 5120, 48), ("out_proj", 6144, 5120)]
MODEL_GQA_SHAPES = [("q_proj", 5120, 12288), ("k_proj", 5120, 1024), ("v_proj", 5120, 1024), ("o_proj", 6144, 5120)]
MODEL_MLP_SHAPES = [("gate_proj", 5120, 17408), ("up_proj", 5120, 17408), ("down_proj", 17408, 5120)]


def model_layer_is_gqa(i: int) -> bool:
    return i % 4 == 3
STACK_LAYERS = 64          # 48 Gated DeltaNet + 16 GQA layers
RAGGED = dict(m=37, k=4736, n=3000)


def bf16_rne(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (qwen35-c/src/q35_model.c:31-37)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return ((u >> 16) & 0xFFFF).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """Nearest e4m3fn code of fp32 values, ties to the even code, saturating
    at 448, with the edge behaviour of the reference's exhaustive search
    (qwen35-c/src/q35_model.c:41-57): NaN -> 0x7F, the sign bit set iff
    v < 0 (so -0.0 -> 0x00).  Magnitudes above 448 go through that search
    itself, fp32 distances and all, so that even absurd inputs (where
    a - 448 rounds in fp32, or infinities) get the reference's code."""
    v = np.ascontiguousarray(v, np.float32)
    a = np.abs(v)
    u = a.view(np.uint32)
    with np.errstate(over="ignore", invalid="ignore"):
        # Normal e4m3 range (|v| >= 2^-6): round the fp32 significand to 3
        # bits, nearest-even on the 20 dropped bits; a carry moves into the
        # exponent field.
        r = (u + (np.uint32(0x7FFFF) + ((u >> 20) & np.uint32(1)))) >> 20
        cn = r.astype(np.int64) - ((127 - 7) << 3)
        # Subnormal range: multiples of 2^-9 (a * 512 is exact).
        small = a < np.float32(2.0 ** -6)
        cs = np.rint(np.where(small, a, 0) * np.float32(512.0)).astype(np.int64)
    code = np.where(small, cs, np.minimum(cn, 0x7E))
    big = np.nonzero((a > np.float32(448.0)) & ~np.isnan(a))
    if big[0].size:
        code[big] = _search_e4m3(a[big])
    out = (code.astype(np.uint8) | ((v < 0).astype(np.uint8) << 7)).astype(np.uint8)
    out[np.isnan(v)] = 0x7F
    return out


def _e4m3_magnitudes() -> np.ndarray:
    """fp32 values of codes 0x00..0x7E (OCP e4m3fn)."""
    c = np.arange(127)
    e, m = c >> 3, c & 7
    return np.where(e == 0, m * 2.0 ** -9, (1 + m / 8.0) * 2.0 ** (e - 7)).astype(np.float32)


def _search_e4m3(a: np.ndarray) -> np.ndarray:
    """The exhaustive nearest-code search on fp32 magnitudes: first strictly
    closer code wins, an exact tie moves to an even code; distances are
    rounded fp32 differences and the initial best distance is 1e30."""
    mags = _e4m3_magnitudes()
    best = np.zeros(a.shape, np.int64)
    best_d = np.full(a.shape, np.float32(1e30), np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for i in range(127):
            d = np.abs(a - mags[i]).astype(np.float32)
            take = (d < best_d) | ((d == best_d) & ((i & 1) == 0) & ((best & 1) == 1))
            best = np.where(take, i, best)
            best_d = np.where(take, d, best_d)
    return best


def _quantize_rows(w: np.ndarray):
    """Quantize rows that form one 128-row block row."""
    n, k = w.shape
    kb = (k + 127) // 128
    pad = np.zeros((n, kb * 128), np.float32)
    pad[:, :k] = np.abs(w)
    amax = pad.reshape(n, kb, 128).max(axis=(0, 2))
    sc_bits = bf16_rne(amax / np.float32(448.0))
    s = bf16_to_f32(sc_bits)
    srow = np.repeat(s, 128)[:k]
    safe = np.where(srow == 0, np.float32(1.0), srow)
    codes = e4m3_encode(w / safe[None, :])
    codes[:, srow == 0] = 0
    return codes, sc_bits


def _parallel_block_rows(n: int, fn):
    """Runs fn(bi) for every 128-row block row on a small thread pool (numpy
    releases the GIL in the bulk operations)."""
    from concurrent.futures import ThreadPoolExecutor
    import os
    nb = (n + 127) // 128
    workers = max(1, min(16, os.cpu_count() or 1, nb))
    with ThreadPoolExecutor(workers) as ex:
        return list(ex.map(fn, range(nb)))


def quantize_fp8(w: np.ndarray):
    """fp32 [N][K] -> (e4m3 codes [N][K] uint8, bf16 scales [NB][KB] uint16)."""
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    nb, kb = (n + 127) // 128, (k + 127) // 128
    codes = np.empty((n, k), np.uint8)
    scales = np.empty((nb, kb), np.uint16)

    def one(bi):
        r0, r1 = bi * 128, min(n, bi * 128 + 128)
        codes[r0:r1], scales[bi] = _quantize_rows(w[r0:r1])

    _parallel_block_rows(n, one)
    return codes, scales


def gen_weight(seed: int, n: int, k: int, std: float = 0.02):
    """W ~ N(0, std^2) fp32, quantized.  Block row bi draws from its own
    stream default_rng([seed, bi]) so block rows can be generated in
    parallel; the result depends only on (seed, n, k, std)."""
    nb, kb = (n + 127) // 128, (k + 127) // 128
    codes = np.empty((n, k), np.uint8)
    scales = np.empty((nb, kb), np.uint16)

    def one(bi):
        r0, r1 = bi * 128, min(n, bi * 128 + 128)
        rng = np.random.default_rng([seed, bi])
        w = rng.standard_normal((r1 - r0, k), dtype=np.float32) * np.float32(std)
        codes[r0:r1], scales[bi] = _quantize_rows(w)

    _parallel_block_rows(n, one)
    return codes, scales


def gen_weight_ragged(seed: int, n: int, k: int):
    """Per-block amax drawn log-uniform in [1e-4, 1e2]: block values are
    N(0,1) rescaled so the block's max |w| equals its drawn amax."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k), dtype=np.float32)
    nb, kb = (n + 127) // 128, (k + 127) // 128
    amax_t = (10.0 ** rng.uniform(-4.0, 2.0, size=(nb, kb))).astype(np.float32)
    for bi in range(nb):
        for bj in range(kb):
            blk = w[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            cur = np.float32(np.abs(blk).max())
            blk *= np.float32(amax_t[bi, bj] / cur)
    return quantize_fp8(w)


def gen_act(seed: int, m: int, k: int, bf16: bool = False, outlier_frac: float = 0.0,
            outlier_scale: float = 100.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32)
    if outlier_frac > 0:
        mask = rng.random((m, k)) < outlier_frac
        x[mask] *= np.float32(outlier_scale)
    if bf16:
        x = bf16_to_f32(bf16_rne(x)).reshape(m, k)
    return x


def algorithmic_bytes(m: int, k: int, n: int) -> int:
    """HBM bytes one matmul must move: e4m3 codes, fp32 block scales, fp32
    activations in and outputs out."""
    nb, kb = (n + 127) // 128, (k + 127) // 128
    return n * k + 4 * nb * kb + 4 * m * k + 4 * m * n


def flops(m: int, k: int, n: int) -> int:
    return 2 * m * n * k
