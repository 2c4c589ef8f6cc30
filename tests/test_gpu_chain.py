"""The chained decode launch (q35mm_chain_*): a sequence of decode GEMVs,
each reading what earlier ones wrote, run as one persistent launch.

Every output must have the bits of the same projections called one after
another (q35mm_matmul_multi per step, the row-split GEMV), which the tests
check bit for bit: one decoder layer's projections (qkv-like, o_proj-like,
gate and up as one multi-weight step, down with the residual add) at m = 1,
3 and 8 tokens; three layers in one launch with their activation buffers
reused from layer to layer (the coherence of re-read buffers along the
chain); graph replays with eager work in between; launches queued back to
back (the counters return to zero by themselves); a residual written back
in place into the layer input; 40 seeded random step lists over a pool of
buffers (reads, writes, in-place and cross-buffer residuals in every
order).  One output is also
checked against the oracle (decode bar ||y - y_ref||_inf / ||y_ref||_inf <=
1e-5), so the chain's bits are the reference's arithmetic.
"""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
# K -> N of one layer whose outputs feed the next projection's input:
# qkv-like 5120 -> 4096, o_proj 4096 -> 5120, gate and up 5120 -> 17408,
# down 17408 -> 5120 (the model's shapes but qkv's rows, so they chain)
LAYER = [("q", 5120, 4096), ("o", 4096, 5120), ("g", 5120, 17408), ("u", 5120, 17408), ("d", 17408, 5120)]


def _layer_weights(q, wl, seed):
    out = {}
    for i, (name, k, n) in enumerate(LAYER):
        W, sc = wl.gen_weight(seed + i, n, k)
        out[name] = (q.Weight(W, sc), W, sc)
    return out


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


def _layer_steps(L, x, bufs, resid):
    """q -> o -> (g, u) -> d (+ resid): each step reads the previous output."""
    return [([L["q"][0]], x, [bufs["q"]]),
            ([L["o"][0]], bufs["q"], [bufs["o"]]),
            ([L["g"][0], L["u"][0]], bufs["o"], [bufs["g"], bufs["u"]]),
            ([L["d"][0]], bufs["g"], [bufs["d"]], [resid])]


def _layer_sequential(q, L, x, bufs, resid, m):
    q.matmul(L["q"][0], x, bufs["q"], m=m)
    q.matmul(L["o"][0], bufs["q"], bufs["o"], m=m)
    q.matmul_multi([L["g"][0], L["u"][0]], bufs["o"], [bufs["g"], bufs["u"]], m=m)
    # down with the residual: the library's GEMV adds it in its epilogue
    # only inside the MLP block; the separate call is product then add,
    # the same single rounding as the epilogue's resid + sum
    q.matmul(L["d"][0], bufs["g"], bufs["d"], m=m)
    bufs["d"] += resid


def _bufs(torch, gpu, m):
    return {name: torch.empty((m, n), dtype=torch.float32, device=gpu) for name, _, n in LAYER}


@pytest.mark.parametrize("m", [1, 3, 8])
def test_chain_layer_equals_sequential_calls(q, oracle, wl, gpu, m):
    import torch
    L = _layer_weights(q, wl, 0xC4A1 + m)
    x = torch.from_numpy(wl.gen_act(0xC4B0 + m, m, 5120)).to(gpu)
    resid = torch.from_numpy(wl.gen_act(0xC4C0 + m, m, 5120)).to(gpu)
    want = _bufs(torch, gpu, m)
    _layer_sequential(q, L, x, want, resid, m)
    got = _bufs(torch, gpu, m)
    for b in got.values():
        b.fill_(float("nan"))
    ch = q.Chain(_layer_steps(L, x, got, resid), m=m)
    assert ch.workgroups >= 256
    ch.run()
    ch.status()
    for name in want:
        assert (_bits(got[name]) == _bits(want[name])).all(), name
    # the first step against the oracle
    yq = oracle.mm_batch(L["q"][1], L["q"][2], x.cpu().numpy())
    for t in range(m):
        assert normwise_rel(got["q"].cpu().numpy()[t], yq[t]) <= GEMV_TOL
    ch.free()
    for w, _, _ in L.values():
        w.free()


def _three_layer_plan(Ls, x0, xa, xb, bufs, resid):
    """Layer i reads ins[i] and its down step writes outs[i] (xa is written
    by layer 0, read by layer 1 and written again by layer 2); every layer
    writes the same q, o, g, u buffers, each re-read by the next step."""
    ins, outs = [x0, xa, xb], [xa, xb, xa]
    steps = []
    for i, L in enumerate(Ls):
        steps += [([L["q"][0]], ins[i], [bufs["q"]]),
                  ([L["o"][0]], bufs["q"], [bufs["o"]]),
                  ([L["g"][0], L["u"][0]], bufs["o"], [bufs["g"], bufs["u"]]),
                  ([L["d"][0]], bufs["g"], [outs[i]], [resid])]
    return steps


def test_chain_three_layers_reused_buffers(q, wl, gpu):
    """Three layers in one launch, their buffers reused from layer to layer
    (each re-read after it was written again): re-read activations must come
    from the coherence point, not from a cache line that held the earlier
    layer's values.  The launch is queued twice back to back (the first's
    last workgroup resets the counters); both give the sequential bits."""
    import torch
    m = 1
    Ls = [_layer_weights(q, wl, 0xC500 + 16 * i) for i in range(3)]
    x0 = torch.from_numpy(wl.gen_act(0xC5F0, m, 5120) * np.float32(1e-3)).to(gpu)
    resid = torch.from_numpy(wl.gen_act(0xC5F1, m, 5120)).to(gpu)

    def buffers():
        b = _bufs(torch, gpu, m)
        return b, torch.empty((m, 5120), device=gpu), torch.empty((m, 5120), device=gpu)
    wb, wxa, wxb = buffers()
    for ws, x, ys, *rs in _three_layer_plan(Ls, x0, wxa, wxb, wb, resid):
        if len(ws) == 1:
            q.matmul(ws[0], x, ys[0], m=m)
        else:
            q.matmul_multi(ws, x, ys, m=m)
        if rs:
            ys[0] += rs[0][0]
    torch.cuda.synchronize()
    gb, gxa, gxb = buffers()
    ch = q.Chain(_three_layer_plan(Ls, x0, gxa, gxb, gb, resid), m=m)
    for rep in range(2):
        for t in list(gb.values()) + [gxa, gxb]:
            t.fill_(float("nan"))
        ch.run()
        ch.run()
        ch.status()
        for name in ("q", "o", "g", "u"):
            assert (_bits(gb[name]) == _bits(wb[name])).all(), (rep, name)
        assert (_bits(gxa) == _bits(wxa)).all() and (_bits(gxb) == _bits(wxb)).all(), rep
    ch.free()
    for L in Ls:
        for w, _, _ in L.values():
            w.free()


def test_chain_in_a_graph(q, wl, gpu):
    """A chain launch captured into a HIP graph: replays with eager library
    calls in between give the eager bits (no counter clearing is recorded:
    the kernel resets its counters itself)."""
    import torch
    m = 2
    L = _layer_weights(q, wl, 0xC600)
    x = torch.from_numpy(wl.gen_act(0xC610, m, 5120)).to(gpu)
    resid = torch.from_numpy(wl.gen_act(0xC611, m, 5120)).to(gpu)
    want = _bufs(torch, gpu, m)
    _layer_sequential(q, L, x, want, resid, m)
    got = _bufs(torch, gpu, m)
    ch = q.Chain(_layer_steps(L, x, got, resid), m=m)
    ch.run()                                   # warm
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ch.run()
    torch.cuda.synchronize()
    other = torch.empty((m, 4096), device=gpu)
    for r in range(3):
        for b in got.values():
            b.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for name in want:
            assert (_bits(got[name]) == _bits(want[name])).all(), (r, name)
        q.matmul(L["q"][0], x, other, m=m)     # eager work between replays
        torch.cuda.synchronize()
    ch.status()
    del g
    ch.free()
    for w, _, _ in L.values():
        w.free()


def test_chain_residual_in_place(q, wl, gpu):
    """The model's residual stream: the last step writes x + down(...) back
    into the layer input x, which the first step read (the last step waits
    for every earlier one, so the first step's reads are done).  Two layers
    in one launch, the second reading the x the first updated; bits equal
    to the same calls made one by one."""
    import torch
    m = 2
    Ls = [_layer_weights(q, wl, 0xC800 + 16 * i) for i in range(2)]
    x0 = torch.from_numpy(wl.gen_act(0xC8F0, m, 5120) * np.float32(0.01)).to(gpu)

    def plan(x, B):
        steps = []
        for L in Ls:
            steps += [([L["q"][0]], x, [B["q"]]),
                      ([L["o"][0]], B["q"], [B["o"]]),
                      ([L["g"][0], L["u"][0]], B["o"], [B["g"], B["u"]]),
                      ([L["d"][0]], B["g"], [x], [x])]
        return steps
    xw = x0.clone()
    Bw = _bufs(torch, gpu, m)
    for ws, x, ys, *rs in plan(xw, Bw):
        if len(ws) == 1:
            q.matmul(ws[0], x, ys[0] if not rs else Bw["d"], m=m)
        else:
            q.matmul_multi(ws, x, ys, m=m)
        if rs:
            xw += Bw["d"]
    torch.cuda.synchronize()
    xg = x0.clone()
    Bg = _bufs(torch, gpu, m)
    ch = q.Chain(plan(xg, Bg), m=m)
    ch.run()
    ch.status()
    assert (_bits(xg) == _bits(xw)).all()
    for name in ("q", "o", "g", "u"):
        assert (_bits(Bg[name]) == _bits(Bw[name])).all(), name
    ch.free()
    for L in Ls:
        for w, _, _ in L.values():
            w.free()


def test_chain_refuses_other_shapes(q, wl, gpu):
    """Weights beyond the row-split GEMV's K range (here 168 blocks) and
    m outside 1..8 are refused with an error, nothing launched."""
    import torch
    W, sc = wl.gen_weight(0xC700, 256, 168 * 128)
    w = q.Weight(W, sc)
    x = torch.zeros((1, 168 * 128), device=gpu)
    y = torch.empty((1, 256), device=gpu)
    with pytest.raises(q.Q35mmError, match="row-split"):
        q.Chain([([w], x, [y])], m=1)
    W2, sc2 = wl.gen_weight(0xC701, 256, 1024)
    w2 = q.Weight(W2, sc2)
    with pytest.raises(q.Q35mmError, match="m=9"):
        q.Chain([([w2], torch.zeros((9, 1024), device=gpu), [torch.empty((9, 256), device=gpu)])], m=9)
    w.free()
    w2.free()


def _random_chains(count=40, seed=0xC5EED):
    """Seeded step lists over a pool of P activation buffers [m][D]: each
    step 1..3 weights (D x D) reading one buffer and writing others (never
    its own x), each output with no residual, itself (y += product, in
    place) or another buffer not written by the step (x included)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        D = int(rng.choice([1024, 2048]))
        m = int(rng.choice([1, 2, 3, 5, 8]))
        P = int(rng.integers(3, 7))
        steps = []
        for _s in range(int(rng.integers(1, 9))):
            xb = int(rng.integers(0, P))
            others = [b for b in range(P) if b != xb]
            nw = int(rng.integers(1, min(3, len(others)) + 1))
            outs = [int(b) for b in rng.choice(others, size=nw, replace=False)]
            ws = [int(i) for i in rng.choice(6, size=nw, replace=False)]
            res = []
            for o in outs:
                u = rng.random()
                res.append(None if u < 0.6 else o if u < 0.8 else int(rng.choice([b for b in range(P) if b not in outs])))
            steps.append((ws, xb, outs, res))
        out.append((D, m, P, steps))
    return out


def test_chain_random_step_lists(q, wl, gpu):
    """Random chains: which buffers each step reads and writes decide
    whether its activations are loaded cached or at the coherence point
    (reads and writes of earlier steps, on whole cache lines), and every
    step waits for all earlier ones (so a buffer read earlier may be
    overwritten).  After two launches of each chain every buffer has the
    bits of the same steps called one after another (q35mm_matmul_multi,
    then the residual added)."""
    import torch
    pools = {}
    for c, (D, m, P, steps) in enumerate(_random_chains()):
        if D not in pools:
            pools[D] = [q.Weight(*wl.gen_weight(0xC5000 + D + i, D, D)) for i in range(6)]
        W = pools[D]
        init = [torch.from_numpy(wl.gen_act(0xC6000 + 97 * c + b, m, D)).to(gpu) for b in range(P)]
        want = [t.clone() for t in init]
        for ws, xb, outs, res in steps:
            tmp = [torch.empty((m, D), device=gpu) for _ in outs]
            q.matmul_multi([W[i] for i in ws], want[xb], tmp, m=m)
            new = [tmp[j] + want[r] if r is not None else tmp[j] for j, r in enumerate(res)]
            for j, o in enumerate(outs):
                want[o] = new[j]
        got = [t.clone() for t in init]
        ch = q.Chain([([W[i] for i in ws], got[xb], [got[o] for o in outs],
                       [got[r] if r is not None else None for r in res]) for ws, xb, outs, res in steps], m=m)
        for rep in range(2):
            if rep:
                for g, t in zip(got, init):
                    g.copy_(t)
            ch.run()
            ch.status()
            torch.cuda.synchronize()
            for b in range(P):
                assert (_bits(got[b]) == _bits(want[b])).all(), (c, D, m, steps, rep, b)
        ch.free()
    for ws in pools.values():
        for w in ws:
            w.free()
