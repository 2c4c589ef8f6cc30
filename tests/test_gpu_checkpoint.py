"""Checkpoint -> HBM through the C ABI (q35mm_st_load_*, q35mm_quantize_f32),
checked against the oracle on the GPU.

Bars: everything here is integer or exact arithmetic, so bit-exact:
  - F8_E4M3 tensors loaded from a file dequantize to the oracle's
    lut[code] * scale of the same file bytes, and multiply exactly as a
    weight created from the same arrays;
  - BF16 tensors quantized on the device give the oracle quantizer's codes
    and bf16 scales (the reference's bind_ab recipe), code for code;
  - a BF16 lm_head loaded from the file gives the reference-order matvec.
"""
import json
import os
import struct
import time

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

ST = os.path.join(GOLDEN, "st")
ENOTFOUND, ESHAPE = -7, -8


def write_st(path, tensors):
    hdr, off = {}, 0
    for name, dt, shape, data in tensors:
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        off += len(data)
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h)
        for _, _, _, data in tensors:
            f.write(data)
    return path


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _dequant(q, w, rows, cols, gpu):
    import torch
    out = torch.empty((rows, cols), dtype=torch.float32, device=gpu)
    q.dequant_f32(w, out)
    return _host(out)


def _codes(q, w, rows, cols, gpu):
    """e4m3 codes of a resident weight, read back through the exact
    e4m3 -> bf16 conversion (injective on all but the two NaN codes)."""
    import torch
    out = torch.empty((rows, cols), dtype=torch.int16, device=gpu)
    q.decode_bf16(w, out)
    return _host(out).view(np.uint16)


def _same_f32(a, b):
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


def test_model_checkpoint_fp8_weights(q, oracle, gpu):
    ck = q.Checkpoint(os.path.join(ST, "model.safetensors"))
    names = [n for n in ck.names() if ck.info(n)[0] == "F8_E4M3"]
    assert names
    for n in names:
        _, (rows, cols), _ = ck.info(n)
        W = np.frombuffer(ck.read(n), np.uint8).reshape(rows, cols)
        sc = np.frombuffer(ck.read(n + "_scale_inv"), np.uint16).reshape((rows + 127) // 128, (cols + 127) // 128)
        for loader in (ck.load_fp8, ck.load_ab):
            w = loader(n, rows, cols)
            assert _same_f32(_dequant(q, w, rows, cols, gpu), oracle.dequant(W, sc)), n
            w.free()


def test_loaded_weight_multiplies_as_array_weight(q, wl, gpu):
    import torch
    ck = q.Checkpoint(os.path.join(ST, "model.safetensors"))
    n = "model.language_model.layers.0.linear_attn.in_proj_qkv.weight"
    _, (rows, cols), _ = ck.info(n)
    W = np.frombuffer(ck.read(n), np.uint8).reshape(rows, cols)
    sc = np.frombuffer(ck.read(n + "_scale_inv"), np.uint16).reshape(-1, 1)
    a, b = ck.load_fp8(n, rows, cols), q.Weight(W, sc)
    X = torch.from_numpy(wl.gen_act(5, 3, cols)).to(gpu)
    Ya = torch.empty((3, rows), device=gpu)
    Yb = torch.empty_like(Ya)
    q.matmul(a, X, Ya)
    q.matmul(b, X, Yb)
    assert torch.equal(Ya, Yb)


def test_lm_head_bf16_from_file(q, oracle, gpu):
    import torch
    ck = q.Checkpoint(os.path.join(ST, "model.safetensors"))
    _, (rows, cols), _ = ck.info("lm_head.weight")
    W16 = np.frombuffer(ck.read("lm_head.weight"), np.uint16).reshape(rows, cols)
    p = ck.load_bf16("lm_head.weight", rows, cols)
    try:
        x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
        dx = torch.from_numpy(x).to(gpu)
        dy = torch.empty(rows, device=gpu)
        q.lib.q35mm_bf16_gemv(p, rows, cols, q._dptr(dx), q._dptr(dy), q._stream(None))
        assert (_host(dy).view(np.uint32) == oracle.mm_bf16(W16, x).view(np.uint32)).all()
    finally:
        q.free(p)


def _bf16_bits(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("rows,cols", [(48, 5120), (100, 300), (129, 128), (1, 1), (256, 384)])
def test_bind_ab_quantizes_bf16_like_the_reference(q, oracle, gpu, tmp_path, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    w = (rng.standard_normal((rows, cols)) * 10.0 ** rng.uniform(-6, 2, (rows, 1))).astype(np.float32)
    if rows * cols > 64:
        flat = w.reshape(-1)
        flat[:8] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -3e-39, 448.0]
    if rows >= 129:
        w[128:, :] = 0.0                      # a block of zeros: scale 0, zero codes
    bits = _bf16_bits(w)
    wf = (bits.astype(np.uint32) << 16).view(np.float32)
    path = write_st(str(tmp_path / "ab.safetensors"), [("proj.weight", "BF16", (rows, cols), bits.tobytes())])
    ck = q.Checkpoint(path)
    dw = ck.load_ab("proj.weight", rows, cols)
    codes, sc = oracle.quantize(wf)
    lut_bits = (oracle.lut().view(np.uint32) >> 16).astype(np.uint16)
    got = _codes(q, dw, rows, cols, gpu)
    want = lut_bits[codes]
    nan = (codes & 0x7F) == 0x7F
    assert (got[~nan] == want[~nan]).all()
    assert (((got[nan] & 0x7F80) == 0x7F80) & ((got[nan] & 0x7F) != 0)).all()
    assert _same_f32(_dequant(q, dw, rows, cols, gpu), oracle.dequant(codes, sc))


def test_quantize_f32_dense_sweep(q, oracle, gpu):
    """Every 97th float32 in [0, 449.75] (and its negative), 128x128 blocks
    whose amax is exactly 448 (scale 1.0, so codes = nearest e4m3 of the value
    itself), plus every midpoint between adjacent e4m3 magnitudes and its two
    float neighbours: the device codes equal the oracle's exhaustive search."""
    import torch
    top = np.float32(449.75).view(np.uint32)
    vals = np.arange(0, top, 97, dtype=np.uint32).view(np.float32)
    lut = oracle.lut()[:127].astype(np.float64)
    mids = ((lut[:-1] + lut[1:]) / 2).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))])
    vals = np.concatenate([vals, near, -vals[1:], -near]).astype(np.float32)
    per = 128 * 128 - 1
    nblk = (vals.size + per - 1) // per
    buf = np.zeros((nblk, per), np.float32)
    buf.reshape(-1)[: vals.size] = vals
    blocks = np.concatenate([np.full((nblk, 1), 448.0, np.float32), buf], axis=1)     # amax 448 each
    W = blocks.reshape(nblk, 128, 128).transpose(1, 0, 2).reshape(128, nblk * 128).copy()
    rows, cols = W.shape
    dW = torch.from_numpy(W).to(gpu)
    dC = torch.empty((rows, cols), dtype=torch.uint8, device=gpu)
    dS = torch.empty((1, nblk), dtype=torch.int16, device=gpu)
    q.quantize_f32(dW, dC, dS)
    codes, sc = oracle.quantize(W)
    assert (_host(dS).view(np.uint16) == sc).all() and (sc == 0x3F80).all()
    assert (_host(dC) == codes).all()


def test_quantize_f32_ragged_and_special(q, oracle, gpu):
    import torch
    rng = np.random.default_rng(9)
    for rows, cols in ((300, 200), (1, 129), (130, 5)):
        W = (rng.standard_normal((rows, cols)) * 10.0 ** rng.uniform(-30, 30, (rows, 1))).astype(np.float32)
        W.reshape(-1)[:6] = [np.nan, np.inf, -np.inf, -0.0, 1e-45, 3e38]
        dW = torch.from_numpy(W).to(gpu)
        dC = torch.empty((rows, cols), dtype=torch.uint8, device=gpu)
        dS = torch.empty(((rows + 127) // 128, (cols + 127) // 128), dtype=torch.int16, device=gpu)
        q.quantize_f32(dW, dC, dS)
        codes, sc = oracle.quantize(W)
        assert (_host(dS).view(np.uint16) == sc).all()
        assert (_host(dC) == codes).all()


def test_load_errors(q, gpu, tmp_path):
    path = write_st(str(tmp_path / "e.safetensors"), [
        ("a.weight", "F8_E4M3", (4, 8), bytes(32)),
        ("a.weight_scale_inv", "BF16", (1, 1), b"\x80\x3f"),
        ("b.weight", "F8_E4M3", (4, 8), bytes(32)),                     # no scale
        ("c.weight", "F32", (4, 8), bytes(128)),
    ])
    ck = q.Checkpoint(path)
    ck.load_fp8("a.weight", 4, 8).free()
    for fn, name, shape, code in ((ck.load_fp8, "missing", (4, 8), ENOTFOUND),
                                  (ck.load_fp8, "a.weight", (4, 9), ESHAPE),
                                  (ck.load_fp8, "b.weight", (4, 8), ENOTFOUND),
                                  (ck.load_fp8, "c.weight", (4, 8), ESHAPE),
                                  (ck.load_ab, "c.weight", (4, 8), ESHAPE),
                                  (ck.load_ab, "missing", (4, 8), ENOTFOUND)):
        with pytest.raises(q.Q35mmError) as e:
            fn(name, *shape)
        assert getattr(e.value, "code", None) == code, str(e.value)


def test_large_tensor_upload(q, oracle, wl, gpu, tmp_path):
    """One 17408 x 5120 FP8 tensor (89 MB, several upload chunks) from a
    file: sampled rows dequantize exactly."""
    import torch
    rows, cols = 17408, 5120
    W, sc = wl.gen_weight(wl.SEED_BASE + 0x400, rows, cols)
    path = write_st(str(tmp_path / "big.safetensors"), [("big.weight", "F8_E4M3", (rows, cols), W.tobytes()),
                                                         ("big.weight_scale_inv", "BF16", sc.shape, sc.tobytes())])
    ck = q.Checkpoint(path)
    t = time.perf_counter()
    w = ck.load_fp8("big.weight", rows, cols)
    dt = time.perf_counter() - t
    print(f"upload {rows}x{cols}: {W.nbytes / dt / 1e9:.2f} GB/s ({dt * 1e3:.1f} ms)", flush=True)
    out = torch.empty((rows, cols), dtype=torch.float32, device=gpu)
    q.dequant_f32(w, out)
    idx = np.random.default_rng(1).choice(rows, 64, replace=False)
    got = _host(out[torch.from_numpy(idx).to(gpu)])
    want = np.stack([oracle.dequant(W[r:r + 1], sc[r // 128:r // 128 + 1])[0] for r in idx])
    assert _same_f32(got, want)
