"""Concurrency and residency edge cases of libq35mm.so on the GPU.

- Calls on two streams that overlap on the GPU: each stream has its own
  scratch (stream-K split partials and counters, the GEMM's bf16
  activations), so both results equal the oracle's and the single-stream
  bits.
- A q35_mm_fp8_multi4 that passes one weight pointer twice with different
  row counts (the reference reads the same bytes both ways,
  qwen35-c/src/q35_mm.c:176-198).
- The host-pointer residency check: a new tensor behind a reused pointer is
  seen; an in-place edit of a few codes outside the sampled fingerprint is
  not, until q35mm_release(W), or always with Q35MM_VERIFY_WEIGHTS=full.
- The drop-in entry points called from several host threads at once (the
  reference is called from one thread; the library serialises calls behind
  one lock): every result the bits of the same call made alone.
- Graphs: calls captured on a stream the library has not seen, replayed
  with eager calls in between (the GEMM, the MLP block at decode and
  prefill), every replay the eager bits; scratch that grew after a capture
  stays alive for the graph; a capture cannot grow scratch.

Bars: decode GEMV ||y - y_ref||_inf / ||y_ref||_inf <= 1e-5; prefill GEMM
rel-L2 <= 5e-3 and max-abs <= 2e-2; bitwise where results must equal
other calls of the library.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT, normwise_rel

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5


def _dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu)


def test_two_streams_overlap(q, oracle, wl, gpu):
    """Stream-K GEMVs (K of 168 blocks, beyond the row-split kernel) and
    prefill GEMMs queued alternately on two streams, 20 rounds without
    synchronising in between; every output equals the same call made alone."""
    import torch
    k = 168 * 128
    Wa, sa = wl.gen_weight(301, 1500, k)
    Wb, sb = wl.gen_weight(302, 900, k)
    Wg, sg_ = wl.gen_weight(303, 700, 2048)
    wa, wb, wg = q.Weight(Wa, sa), q.Weight(Wb, sb), q.Weight(Wg, sg_)
    xa, xb = _dev(wl.gen_act(304, 3, k), gpu), _dev(wl.gen_act(305, 5, k), gpu)
    Xg1, Xg2 = _dev(wl.gen_act(306, 96, 2048), gpu), _dev(wl.gen_act(307, 160, 2048), gpu)
    ref = {}
    for name, w, x, m, gemm in (("a", wa, xa, 3, False), ("b", wb, xb, 5, False),
                                ("g1", wg, Xg1, 96, True), ("g2", wg, Xg2, 160, True)):
        y = torch.empty((m, w.rows), device=gpu)
        (q.gemm if gemm else q.gemv)(w, x, y)
        torch.cuda.synchronize()
        ref[name] = y.cpu().numpy()
    ya = oracle.mm_batch(Wa, sa, xa.cpu().numpy())
    for t in range(3):
        assert normwise_rel(ref["a"][t], ya[t]) <= GEMV_TOL
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for r in range(20):
        with torch.cuda.stream(s1):
            y1 = torch.empty((3, wa.rows), device=gpu)
            g1 = torch.empty((96, wg.rows), device=gpu)
            q.gemv(wa, xa, y1)
            q.gemm(wg, Xg1, g1)
        with torch.cuda.stream(s2):
            y2 = torch.empty((5, wb.rows), device=gpu)
            g2 = torch.empty((160, wg.rows), device=gpu)
            q.gemv(wb, xb, y2)
            q.gemm(wg, Xg2, g2)
        outs.append((y1, g1, y2, g2))
    torch.cuda.synchronize()
    for y1, g1, y2, g2 in outs:
        for got, name in ((y1, "a"), (g1, "g1"), (y2, "b"), (g2, "g2")):
            assert (got.cpu().numpy().view(np.uint32) == ref[name].view(np.uint32)).all(), name
    # every stream-K launch returned the arrival counters it took to zero
    for st in (s1, s2, torch.cuda.current_stream()):
        nz, words = q.debug_counters(st.cuda_stream)
        assert words > 0 and nz == 0, (nz, words)
    for st in (s1, s2):
        q.stream_release(st.cuda_stream)
        assert q.debug_counters(st.cuda_stream) == (0, 0)
    for w in (wa, wb, wg):
        w.free()


def test_multi4_repeated_pointer_other_rows(q, oracle, wl, gpu):
    """W and its first 128 rows (same pointer) in one multi4 call, twice, and
    then single calls: each segment as its single call, bit for bit."""
    W, sc = wl.gen_weight(311, 384, 1024)
    x = wl.gen_act(312, 1, 1024)[0]
    head = W[:128]
    assert head.ctypes.data == W.ctypes.data
    for _ in range(2):
        y_full, y_head = q.mm_fp8_multi4([W, head], [sc, sc[:1]], x)[:2]
        assert normwise_rel(y_full, oracle.mm(W, sc, x)) <= GEMV_TOL
        assert normwise_rel(y_head, oracle.mm(head, sc[:1], x)) <= GEMV_TOL
    assert (q.mm_fp8(W, sc, x).view(np.uint32) == y_full.view(np.uint32)).all()
    q.release(W)
    assert (q.mm_fp8(head, sc[:1], x).view(np.uint32) == y_head.view(np.uint32)).all()
    q.release(W)


def test_in_place_edit_needs_release(q, oracle, wl, gpu):
    """An edit of a few codes between the fingerprint's sampled windows keeps
    the resident copy (the documented limit); q35mm_release(W) picks it up."""
    W, sc = wl.gen_weight(321, 512, 4096)
    x = wl.gen_act(322, 1, 4096)[0]
    y0 = q.mm_fp8(W, sc, x)
    # row 300, columns 1000..1007: offset 1229800, inside no 256-byte window
    # (windows start every (2097152 - 256) / 15 = 139793 bytes) nor the edges
    off = 300 * 4096 + 1000
    assert all(not (o <= off < o + 256) for o in [(W.size - 256) // 15 * i for i in range(16)])
    W[300, 1000:1008] ^= np.uint8(0x80)
    y_stale = q.mm_fp8(W, sc, x)
    assert (y_stale.view(np.uint32) == y0.view(np.uint32)).all()
    q.release(W)
    y_new = q.mm_fp8(W, sc, x)
    assert normwise_rel(y_new, oracle.mm(W, sc, x)) <= GEMV_TOL
    assert not (y_new.view(np.uint32) == y0.view(np.uint32)).all()
    q.release(W)


def test_host_abi_calls_from_several_threads(q, oracle, wl, gpu):
    """Four host threads calling the drop-in ABI at once, 25 rounds each
    (ctypes releases the interpreter lock around every call): q35_mm_fp8;
    q35_mm_fp8_batch on the GEMV (3 tokens) and on the GEMM (64 tokens);
    q35_mm_fp8_multi4 passing the weight pointer another thread uses;
    q35_mm_bf16.  Every result the bits of the same call made alone."""
    import threading
    rng = np.random.default_rng(0x7EAD)
    W1, s1 = wl.gen_weight(wl.SEED_BASE + 0x60, 2048, 5120)
    W2, s2 = wl.gen_weight(wl.SEED_BASE + 0x61, 1024, 4096)
    W3, s3 = wl.gen_weight(wl.SEED_BASE + 0x62, 48, 5120)
    W16 = (rng.standard_normal((1536, 2048)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    x1 = wl.gen_act(wl.SEED_BASE + 0x63, 1, 5120)[0]
    X3 = wl.gen_act(wl.SEED_BASE + 0x64, 3, 4096)
    X64 = wl.gen_act(wl.SEED_BASE + 0x65, 64, 5120, bf16=True)
    x16 = rng.standard_normal(2048).astype(np.float32)
    jobs = [
        lambda: [q.mm_fp8(W1, s1, x1)],
        lambda: [q.mm_fp8_batch(W2, s2, X3)],
        lambda: q.mm_fp8_multi4([W1, W3], [s1, s3], x1)[:2],
        lambda: [q.mm_fp8_batch(W1, s1, X64), q.mm_bf16(W16, x16)],
    ]
    want = [job() for job in jobs]
    assert normwise_rel(want[0][0], oracle.mm(W1, s1, x1)) <= GEMV_TOL
    assert (want[3][1].view(np.uint32) == oracle.mm_bf16(W16, x16).view(np.uint32)).all()
    errors = []

    def worker(j):
        try:
            for it in range(25):
                for a, b in zip(jobs[j](), want[j]):
                    if not (a.view(np.uint32) == b.view(np.uint32)).all():
                        errors.append((j, it))
                        return
        except Exception as e:   # reported below, in the main thread
            errors.append((j, repr(e)))

    threads = [threading.Thread(target=worker, args=(j,)) for j in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    for W in (W1, W2, W3, W16):
        q.release(W)


def test_verify_weights_full_sees_in_place_edit():
    """With Q35MM_VERIFY_WEIGHTS=full the same edit is seen without a release
    (a fresh process: the setting is read when the library initialises)."""
    code = r"""
import sys, numpy as np
sys.path.insert(0, %r); sys.path.insert(0, %r)
import q35mm as q, workload as wl
from oracle import Oracle
W, sc = wl.gen_weight(321, 512, 4096)
x = wl.gen_act(322, 1, 4096)[0]
y0 = q.mm_fp8(W, sc, x)
W[300, 1000:1008] ^= np.uint8(0x80)
y1 = q.mm_fp8(W, sc, x)
yr = Oracle().mm(W, sc, x)
d = float(np.abs(y1.astype(np.float64) - yr).max() / np.abs(yr).max())
print("changed", int(not (y1.view(np.uint32) == y0.view(np.uint32)).all()), "err", d)
""" % (os.path.join(ROOT, "qwen38-in-c_amd"), os.path.join(ROOT, "oracle"))
    env = dict(os.environ, Q35MM_VERIFY_WEIGHTS="full")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    words = out.stdout.split()
    assert words[0] == "changed" and words[1] == "1" and float(words[3]) <= GEMV_TOL, out.stdout


def test_graph_captured_on_a_fresh_stream(q, wl, gpu):
    """Warm-up calls on one stream, capture on a stream the library has not
    seen (the pattern of torch.cuda.graph's own capture stream): the capture
    cannot allocate, so the stream borrows the warm-up's scratch; each
    replay, with eager calls in between, gives the eager bits."""
    import torch
    W, sc = wl.gen_weight(331, 700, 2048)
    w = q.Weight(W, sc)
    X = _dev(wl.gen_act(332, 96, 2048), gpu)
    want = torch.empty((96, 700), device=gpu)
    q.gemm(w, X, want)                      # warm-up on the current stream
    torch.cuda.synchronize()
    Y = torch.empty_like(want)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            q.gemm(w, X, Y)
    torch.cuda.synchronize()
    other = torch.empty((64, 700), device=gpu)
    for r in range(3):
        Y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert (Y.cpu().numpy().view(np.uint32) == want.cpu().numpy().view(np.uint32)).all(), r
        q.gemm(w, X[:64], other)
        torch.cuda.synchronize()
    del g
    w.free()


@pytest.mark.parametrize("m,H,I", [(1, 640, 1664), (200, 640, 1664), (300, 1024, 16640)])
def test_graph_of_mlp_blocks(q, wl, gpu, m, H, I):
    """q35mm_mlp captured in a graph on a fresh stream after an eager call:
    decode (m = 1: the paired GEMV with the RMSNorm inside, then down) and
    prefill (paired gate+up tiles writing the down GEMM's bf16 activations:
    64x64 tiles only at 200 tokens, whole tiles, padding tokens and a fused
    tail at 300).  Each replay, from the same input with eager MLP calls of
    another size in between, gives the eager bits."""
    import torch
    ws = {}
    for i, nm in enumerate(("gate", "up", "down")):
        rows, cols = (H, I) if nm == "down" else (I, H)
        ws[nm] = q.Weight(*wl.gen_weight(0x7A0 + i + I, rows, cols))
    rng = np.random.default_rng(m)
    x0 = _dev(rng.standard_normal((m, H)).astype(np.float32), gpu)
    nw = _dev((rng.standard_normal(H) * 0.1).astype(np.float32), gpu)
    want = x0.clone()
    q.mlp(ws["gate"], ws["up"], ws["down"], nw, want)        # eager, warms the stream's workspace
    torch.cuda.synchronize()
    X = x0.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            q.mlp(ws["gate"], ws["up"], ws["down"], nw, X)
    torch.cuda.synchronize()
    other = _dev(rng.standard_normal((max(1, m // 2), H)).astype(np.float32), gpu)
    for r in range(3):
        X.copy_(x0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert (X.cpu().numpy().view(np.uint32) == want.cpu().numpy().view(np.uint32)).all(), r
        q.mlp(ws["gate"], ws["up"], ws["down"], nw, other)
        torch.cuda.synchronize()
    del g
    for w in ws.values():
        w.free()


def test_graph_replays_after_its_scratch_grew(q, wl, gpu):
    """A graph captured on a fresh stream keeps the addresses of the scratch
    it borrowed from the warm-up stream.  An eager call with more tokens on
    that stream then needs larger buffers: the set, marked as captured,
    retires its old buffers instead of freeing them, so every replay still
    gives the eager bits (a freed buffer could by then belong to anything,
    another set's counters included).  The counters read zero throughout."""
    import torch
    W, sc = wl.gen_weight(341, 700, 2048)
    w = q.Weight(W, sc)
    cur = torch.cuda.current_stream()
    q.stream_release(cur.cuda_stream)       # start from an empty set on this stream
    X = _dev(wl.gen_act(342, 96, 2048), gpu)
    want = torch.empty((96, 700), device=gpu)
    q.gemm(w, X, want)                      # warm-up: the set holds 96 tokens' worth
    torch.cuda.synchronize()
    Y = torch.empty_like(want)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(cur)
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            q.gemm(w, X, Y)
    torch.cuda.synchronize()
    Xb = _dev(wl.gen_act(343, 512, 2048), gpu)
    big = torch.empty((512, 700), device=gpu)
    for r, m in enumerate((256, 512, 512)):   # the set grows on the first two rounds
        Y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert (Y.cpu().numpy().view(np.uint32) == want.cpu().numpy().view(np.uint32)).all(), r
        q.gemm(w, Xb[:m], big[:m])
        torch.cuda.synchronize()
        assert q.debug_counters(cur.cuda_stream)[0] == 0
    del g
    w.free()


def test_capture_cannot_grow_scratch(q, wl, gpu):
    """A call that would need more scratch than the set a capture borrows
    is refused with a clear error before it launches anything (a capture
    cannot allocate); the same call made once outside capture first then
    captures and replays with the eager bits."""
    import torch
    W, sc = wl.gen_weight(351, 700, 2048)
    w = q.Weight(W, sc)
    cur = torch.cuda.current_stream()
    q.stream_release(cur.cuda_stream)
    X = _dev(wl.gen_act(352, 300, 2048), gpu)
    small = torch.empty((64, 700), device=gpu)
    q.gemm(w, X[:64], small)                # warm-up with fewer tokens than the capture
    torch.cuda.synchronize()
    Y = torch.empty((300, 700), device=gpu)
    s = torch.cuda.Stream()
    s.wait_stream(cur)
    g = torch.cuda.CUDAGraph()
    with pytest.raises(q.Q35mmError, match="captured into a graph"):
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                q.gemm(w, X, Y)
    torch.cuda.synchronize()
    want = torch.empty_like(Y)
    q.gemm(w, X, want)                      # the warm-up the capture needs
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    s2 = torch.cuda.Stream()
    s2.wait_stream(cur)
    with torch.cuda.stream(s2):
        with torch.cuda.graph(g2, stream=s2):
            q.gemm(w, X, Y)
    for r in range(2):
        Y.fill_(float("nan"))
        g2.replay()
        torch.cuda.synchronize()
        assert (Y.cpu().numpy().view(np.uint32) == want.cpu().numpy().view(np.uint32)).all(), r
    del g, g2
    w.free()
