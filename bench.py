"""Benchmark of the MI355X FP8-E4M3 128x128 block-dequant matmul.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--pool P] [--no-prefill]
                    [--no-sweep] [--no-cpu] [--eager]

One step = one pass of the decode hot path over one layer at M=1 token: the
five projections 5120->6144 (qkv), 4096->5120 (o_proj), 5120->17408 (gate),
5120->17408 (up), 17408->5120 (down), called as the reference's decode
calls them: gate and up share x and go through one q35_mm_fp8_multi4-style
call (qwen35-c/src/q35_model.c:930-934), the others one call each -- four
launches of the decode GEMV kernels, with weights and activations resident
in HBM before timing starts.  Steps rotate over a pool of P distinct layer
copies (default 8 x 320 MB = 2.56 GB) so the 256 MB Infinity Cache and the
L2 cannot serve repeats.  The copies are one generated layer with per-row
sign patterns flipped (code ^ 0x80 on a pseudo-random half of the rows), so
every copy is distinct data of the same distribution.

Also the full decode-token weight stream: a stack of 64 such layers (20.5 GB
of distinct FP8 weights resident) run back to back at M=1, 256 launches per
token (--stack-layers, 0 to skip), the BF16 lm_head matvec (q35_mm_bf16,
248320 x 5120, two resident copies alternated), and one MLP block at M=1
(RMSNorm, gate+up, SwiGLU, down, residual add on device).

value = algorithmic bytes of K steps / elapsed seconds (HIP events on the
launch stream, launches replayed from a HIP graph), in GB/s.  The timed
region starts right after a device synchronize, and the first few hundred
microseconds after one run slower (the device ramps back up), so the
defaults time long regions: K = 256 steps (~18 ms) and 100 prefill calls
per shape; 64 steps read ~3% lower, 10 prefill calls ~15% lower.  Algorithmic
bytes per matmul = N*K (e4m3) + 4*ceil(N/128)*ceil(K/128) (fp32 scales) +
4*M*K (x) + 4*M*N (y).

Also reported: the M=2/4/8 decode sweep, the M=512 prefill GEMM (TFLOP/s
vs the bf16 dense MFMA peak) and the same shapes at 64 and 128 tokens
(prefill_short: short prompts, on the narrow 128 x 512 tiles), and the
reference's own CPU path (AVX2 + OpenMP, oracle/_ref) timed on this host's
cores on one layer at M=1.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "qwen38-in-c_amd")
sys.path.insert(0, PKG)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = "M=1 FP8 GEMV HBM GB/s (% peak); M=512 prefill GEMM TFLOP/s (% MFMA peak)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def row_sign_mask(n: int, variant: int):
    import numpy as np
    r = np.arange(n, dtype=np.uint64)
    salt = np.uint64((variant * 0x632BE59BD9B4E019) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        h = (r * np.uint64(0x9E3779B97F4A7C15) + salt) >> np.uint64(63)
    return (h.astype(np.uint8) << 7)[:, None]


def make_layer_pool(q, wl, pool: int):
    """pool x {qkv, o_proj, gate, up, down} resident weights + host base.
    Copy v is the base layer with row_sign_mask(n, v) applied."""
    base = []
    for i, (name, k, n) in enumerate(wl.DECODE_SHAPES):
        t = time.time()
        W, sc = wl.gen_weight(wl.SEED_BASE + 1 + 16 * i, n, k)
        base.append((name, k, n, W, sc))
        log(f"  generated {name} {n}x{k} in {time.time() - t:.1f}s")
    layers = []
    for v in range(pool):
        ws = []
        for name, k, n, W, sc in base:
            Wv = W if v == 0 else (W ^ row_sign_mask(n, v))
            ws.append(q.Weight(Wv, sc))
        layers.append(ws)
    return base, layers


def time_graph(torch, fn, steps: int, warmup: int, use_graph: bool):
    """Run fn(i) for i in range(steps) (each i = one step), timed with events
    on the current stream.  With use_graph the steps are captured once into
    a HIP graph and replayed."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    if use_graph:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                for i in range(steps):
                    fn(i)
        torch.cuda.synchronize()
        g.replay()          # one untimed replay
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        g.replay()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / 1e3, g
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for i in range(steps):
        fn(i)
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / 1e3, None


def clock_peak_tflops(cus: int):
    """Dense bf16 MFMA peak from this device's peak engine clock (HIP's
    hipDeviceAttributeClockRate, kHz) and CU count: 4 SIMDs per CU, one
    32x32x16 MFMA (32768 flop) per 32 cycles per SIMD.  None when the
    runtime does not say."""
    import ctypes as C
    try:
        hip = C.CDLL("libamdhip64.so")
        v = C.c_int(0)
        if hip.hipDeviceGetAttribute(C.byref(v), 5, 0) != 0 or v.value <= 0:   # 5: hipDeviceAttributeClockRate
            return None
    except OSError:
        return None
    mhz = v.value / 1e3
    return {"TFLOP/s": round(cus * 4 * 1024 * mhz * 1e6 / 1e12, 1), "clock_MHz": mhz, "CUs": cus}


def measured_traffic(profile: str, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch of a line's dominant kernel from the committed
    rocprofv3 counter summary (FETCH_SIZE and WRITE_SIZE, calibrated against
    a copy of known size), or None if that summary is absent."""
    path = os.path.join(ROOT, "profiles", profile)
    try:
        for ln in open(path):
            if ln.startswith(key + " "):
                return int(ln.split()[1])
    except OSError:
        pass
    return None


def host_cpu_info() -> dict:
    """The host's CPU as lscpu reports it (the whole machine, not this
    process's share)."""
    info = {"model": "unknown", "sockets": None, "cores_per_socket": None, "threads_per_core": None,
            "numa_nodes": None, "logical_cpus": os.cpu_count()}
    keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "NUMA node(s)": "numa_nodes"}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for ln in out.splitlines():
            k, _, v = ln.partition(":")
            if k.strip() in keys:
                v = v.strip()
                info[keys[k.strip()]] = int(v) if v.isdigit() else v
    except Exception:
        try:
            for ln in open("/proc/cpuinfo"):
                if ln.startswith("model name"):
                    info["model"] = ln.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    return info


CPU_CHILD = "--cpu-child"
SINGLE_COPIES = 41   # configuration 0: distinct 26 MB weight copies, 1.07 GB (GPU and CPU alike)


def cpu_child(budget_s: float) -> None:
    """The CPU baseline, run in a child process (no torch, no GPU) so that
    OMP_NUM_THREADS / OMP_PROC_BIND apply to the OpenMP runtime the
    reference's matmul starts: the reference's compiled q35_mm.c
    (oracle/_ref, AVX2 + FMA + OpenMP), or the oracle port if that build is
    absent, on the GPU workloads' inputs (same seeds).  Prints one JSON line."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import workload as wl
    from oracle import Oracle, RefMM
    ref = RefMM.available()
    impl = RefMM() if ref else Oracle()
    kind = "reference" if ref else "port"

    def med_time(fn, budget, at_least=3, at_most=200):
        fn()   # warm: page in, start the threads
        times, t_end = [], time.time() + budget
        while time.time() < t_end or len(times) < at_least:
            t = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t)
            if len(times) >= at_most:
                break
        return float(np.median(times)), len(times)

    out = {"kind": kind, "threads": int(os.environ.get("OMP_NUM_THREADS", "0") or 0),
           "omp_proc_bind": os.environ.get("OMP_PROC_BIND"), "omp_places": os.environ.get("OMP_PLACES")}
    # one layer's decode projections at M = 1, gate and up through multi4 as
    # the reference's decode calls them (qwen35-c/src/q35_model.c:930-937)
    base = []
    for i, (name, k, n) in enumerate(wl.DECODE_SHAPES):
        W, sc = wl.gen_weight(wl.SEED_BASE + 1 + 16 * i, n, k)
        base.append((name, k, n, W, sc))
    xs = [wl.gen_act(7 + i, 1, k)[0] for i, (_, k, _, _, _) in enumerate(base)]
    xs[3] = xs[2]

    def layer():
        for j in (0, 1):
            impl.mm(base[j][3], base[j][4], xs[j])
        if ref:
            impl.multi4([base[2][3], base[3][3]], [base[2][4], base[3][4]], xs[2])
        else:
            impl.mm(base[2][3], base[2][4], xs[2])
            impl.mm(base[3][3], base[3][4], xs[3])
        impl.mm(base[4][3], base[4][4], xs[4])
    lb = sum(wl.algorithmic_bytes(1, k, n) for _, k, n, _, _ in base)
    t, cnt = med_time(layer, budget_s)
    out["layer"] = {"GBps": round(lb / t / 1e9, 3), "ms": round(t * 1e3, 3), "passes": cnt, "bytes": lb}
    del base
    # configuration 0: one 5120 x 5120 GEMV, each call on the next of 41
    # distinct copies (1.07 GB, as on the GPU): one 26 MB weight called over
    # and over would be served by the host's last-level cache, not DRAM
    _, k, n = wl.SINGLE_SHAPE
    W, sc = wl.gen_weight(wl.SEED_BASE + 0, n, k)
    x = wl.gen_act(wl.SEED_BASE + 0x100, 1, k)[0]
    copies = [W] + [np.ascontiguousarray(W ^ row_sign_mask(n, v)) for v in range(1, SINGLE_COPIES)]
    turn = [0]

    def single_call():
        impl.mm(copies[turn[0] % len(copies)], sc, x)
        turn[0] += 1
    t, cnt = med_time(single_call, budget_s / 4, at_least=2 * len(copies))
    b0 = wl.algorithmic_bytes(1, k, n)
    out["single"] = {"GBps": round(b0 / t / 1e9, 3), "ms": round(t * 1e3, 3), "passes": cnt,
                     "copies": len(copies), "pool_MB": round(len(copies) * W.nbytes / 1e6, 1)}
    del W, copies
    # the prefill GEMM shapes on a sample of the 512 tokens (bf16-representable)
    mt = 64
    pre = {"tokens": mt}
    tot_f, tot_t = 0, 0.0
    for i, (name, k, n) in enumerate(wl.PREFILL_SHAPES):
        W, sc = wl.gen_weight(wl.SEED_BASE + 2 + 32 * i, n, k)
        X = wl.gen_act(wl.SEED_BASE + 3 + i, 512, k, bf16=True)[:mt].copy()
        t, cnt = med_time(lambda: impl.mm_batch(W, sc, X), 0.0, at_least=2, at_most=2)
        f = wl.flops(mt, k, n)
        pre[name] = {"ms": round(t * 1e3, 2), "TFLOPs": round(f / t / 1e12, 4)}
        tot_f += f
        tot_t += t
        del W
    pre["TFLOPs"] = round(tot_f / tot_t / 1e12, 4)
    out["prefill_sample"] = pre
    print(json.dumps(out), flush=True)


def cpu_baseline(budget_s: float = 12.0):
    """Runs cpu_child in a child process on this host's CPU share:
    OMP_NUM_THREADS from the environment (the box's share) or the visible
    CPUs, threads bound close to their cores."""
    import subprocess
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
    env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="close", OMP_PLACES="cores")
    res = subprocess.run([sys.executable, os.path.abspath(__file__), CPU_CHILD, str(budget_s)], env=env,
                         capture_output=True, text=True, timeout=900)
    if res.returncode != 0:
        raise RuntimeError("CPU baseline child failed:\n" + res.stderr[-3000:])
    out = json.loads(res.stdout.strip().splitlines()[-1])
    host = host_cpu_info()
    phys = (host.get("sockets") or 1) * (host.get("cores_per_socket") or 0)
    if isinstance(phys, int) and phys > 0:
        # the reference CLI's own default: min(5/3 x physical cores, OpenMP's maximum)
        # (qwen35-c/src/cli/cli_common.c:96-105), computed for the whole host
        out["reference_auto_threads"] = min(phys * 5 // 3, host.get("logical_cpus") or phys * 5 // 3)
    out["host"] = host
    return out

def write_safetensors(path: str, tensors) -> int:
    """tensors: (name, dtype, shape, numpy array); returns bytes written."""
    import numpy as np
    hdr, off = {}, 0
    for name, dt, shape, arr in tensors:
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + arr.nbytes]}
        off += arr.nbytes
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little") + h)
        for _, _, _, arr in tensors:
            f.write(np.ascontiguousarray(arr).tobytes())
    return 8 + len(h) + off


def variant_pool(q, wl, seed, n, k, copies):
    """copies distinct resident weights of one shape: a generated weight and
    its row-sign variants (row_sign_mask)."""
    W, sc = wl.gen_weight(seed, n, k)
    return [q.Weight(W if v == 0 else (W ^ row_sign_mask(n, v)), sc) for v in range(copies)]


# What one launch of this shape can reach at all: a raw read (no arithmetic)
# of the same codes in the row-split decomposition, one graph-replayed
# launch per copy of the weight; a figure of the committed profile, not
# measured in this run.
SINGLE_LAUNCH_CEILING = {"us": 6.36, "GBps": 4120.0, "frac_of_hbm_peak": 0.515,
                         "source": "profiles/ceilings_raw_read_and_mfma_rate.md (read single 5120->5120, "
                                   "tiles/2, graph)"}


def bench_single(q, wl, torch, dev, steps, warmup, use_graph, pool_bytes=1 << 30):
    """Configuration 0: one 5120 x 5120 GEMV at M = 1, calls rotating over
    distinct resident copies totalling at least pool_bytes (more than the 256
    MB Infinity Cache and the L2s can hold)."""
    _, k, n = wl.SINGLE_SHAPE
    copies = max(8, -(-pool_bytes // (n * k)))
    ws = variant_pool(q, wl, wl.SEED_BASE + 0, n, k, copies)
    x = torch.from_numpy(wl.gen_act(wl.SEED_BASE + 0x100, 1, k)).to(dev)
    y = torch.empty((1, n), device=dev)

    def call(i):
        q.gemv(ws[i % copies], x, y, m=1)
    el, g = time_graph(torch, call, steps, warmup, use_graph)
    del g
    b = wl.algorithmic_bytes(1, k, n)
    us = el / steps * 1e6
    for w in ws:
        w.free()
    return {"m": 1, "k": k, "n": n, "copies": copies, "pool_MB": round(copies * n * k / 1e6, 1),
            "calls": steps, "us": round(us, 3), "GBps": round(b / (us * 1e-6) / 1e9, 1),
            "frac_of_hbm_peak": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_call": b,
            "single_launch_ceiling": SINGLE_LAUNCH_CEILING}


def bench_model_token(q, wl, torch, dev, stack, use_graph, reps=3, layers=64):
    """One decode token of the reference model at M = 1, in its call order:
    per layer the DeltaNet multi4 (in_proj_qkv, in_proj_z, in_proj_a,
    in_proj_b) and out_proj, or the GQA q, k, v and o_proj, then the MLP's
    gate+up multi4 and down (qwen35-c/src/q35_model.c:903-937,
    qwen35-c/src/q35_deltanet.c:325-329,360, qwen35-c/src/q35_attn.c:262,
    273-275): 48 x 4 + 16 x 6 = 288 launches.  Every layer's weights are
    distinct and resident (the MLP weights are the stack's)."""
    n_dn = sum(1 for i in range(layers) if not wl.model_layer_is_gqa(i))
    t0 = time.time()
    dn = [variant_pool(q, wl, wl.SEED_BASE + 0x60 + j, n, k, n_dn)
          for j, (_, k, n) in enumerate(wl.MODEL_DELTANET_SHAPES)]
    gq = [variant_pool(q, wl, wl.SEED_BASE + 0x70 + j, n, k, layers - n_dn)
          for j, (_, k, n) in enumerate(wl.MODEL_GQA_SHAPES)]
    log(f"model token: {n_dn} DeltaNet + {layers - n_dn} GQA layers of projections resident "
        f"in {time.time() - t0:.1f}s")
    xs = {k: torch.randn(1, k, device=dev) for k in {5120, 6144, 17408}}
    ys = {n: torch.empty(1, n, device=dev) for n in {10240, 6144, 48, 5120, 12288, 1024, 17408}}
    ya, yb, yv = torch.empty(1, 48, device=dev), torch.empty(1, 17408, device=dev), torch.empty(1, 1024, device=dev)

    def token(_i, qkv_multi4=False):
        idn = igq = 0
        for li in range(layers):
            if wl.model_layer_is_gqa(li):
                q_, k_, v_, o_ = (gq[j][igq] for j in range(4))
                if qkv_multi4:
                    q.matmul_multi([q_, k_, v_], xs[5120], [ys[12288], ys[1024], yv], m=1)
                else:
                    q.gemv(q_, xs[5120], ys[12288], m=1)
                    q.gemv(k_, xs[5120], ys[1024], m=1)
                    q.gemv(v_, xs[5120], yv, m=1)
                q.gemv(o_, xs[6144], ys[5120], m=1)
                igq += 1
            else:
                a, z, ia, ib, out = (dn[j][idn] for j in range(5))
                q.matmul_multi([a, z, ia, ib], xs[5120], [ys[10240], ys[6144], ys[48], ya], m=1)
                q.gemv(out, xs[6144], ys[5120], m=1)
                idn += 1
            L = stack[li % len(stack)]
            q.matmul_multi([L[2], L[3]], xs[5120], [ys[17408], yb], m=1)
            q.gemv(L[4], xs[17408], ys[5120], m=1)
    el, g = time_graph(torch, token, reps, 1, use_graph)
    del g
    torch.cuda.synchronize()
    qkv_sep = [t.clone() for t in (ys[12288], ys[1024], yv)]
    # The GQA layer's q, k and v read the same x: one q35mm_matmul_multi of
    # three segments instead of three launches (the caller's choice; the
    # reference's multi4 entry point takes up to four weights on one x)
    el4, g = time_graph(torch, lambda i: token(i, qkv_multi4=True), reps, 1, use_graph)
    del g
    torch.cuda.synchronize()
    qkv_same = all(torch.equal(a, b) for a, b in zip(qkv_sep, (ys[12288], ys[1024], yv)))
    tok_bytes = 0
    for li in range(layers):
        shapes = wl.MODEL_GQA_SHAPES if wl.model_layer_is_gqa(li) else wl.MODEL_DELTANET_SHAPES
        tok_bytes += sum(wl.algorithmic_bytes(1, k, n) for _, k, n in shapes + wl.MODEL_MLP_SHAPES)
    for pool in dn + gq:
        for w in pool:
            w.free()
    n_gqa = sum(1 for i in range(layers) if wl.model_layer_is_gqa(i))
    n_launch = 4 * n_gqa + 2 * (layers - n_gqa) + 2 * layers
    return {"layers": layers, "deltanet_layers": n_dn, "gqa_layers": layers - n_dn,
            "launches_per_token": n_launch, "bytes_per_token": tok_bytes,
            "ms_per_token": round(el / reps * 1e3, 4), "GBps": round(tok_bytes * reps / el / 1e9, 1),
            "frac_of_hbm_peak": round(tok_bytes * reps / el / 1e9 / HBM_PEAK_GBS, 4),
            "gqa_qkv_multi4": {"launches_per_token": n_launch - 2 * n_gqa,
                               "ms_per_token": round(el4 / reps * 1e3, 4),
                               "GBps": round(tok_bytes * reps / el4 / 1e9, 1),
                               "frac_of_hbm_peak": round(tok_bytes * reps / el4 / 1e9 / HBM_PEAK_GBS, 4),
                               "q_k_v_bitwise_equal_to_separate_calls": qkv_same}}


def host_calls_lib():
    """The C driver of host-pointer call sequences (qwen38-in-c_amd/host_token.c):
    its call record and q35_host_calls_time, so a sequence of q35_mm_* calls
    runs from C, as the reference model makes them, with no Python between."""
    import ctypes as C

    class HostCall(C.Structure):
        _fields_ = [("kind", C.c_uint32), ("cols", C.c_uint32), ("W", C.c_void_p * 4), ("sc", C.c_void_p * 4),
                    ("rows", C.c_uint32 * 4), ("x", C.c_void_p), ("y", C.c_void_p * 4)]
    lib = C.CDLL(os.path.join(ROOT, "qwen38-in-c_amd", "lib", "libq35host_token.so"))
    lib.q35_host_calls_time.restype = C.c_double
    lib.q35_host_calls_time.argtypes = [C.POINTER(HostCall), C.c_uint32, C.c_uint32, C.c_uint32]
    return HostCall, lib


def fill_call(c, kind, cols, Ws, scs, x, ys):
    c.kind, c.cols = kind, cols
    for i in range(4):
        has = i < len(Ws) and Ws[i] is not None
        c.W[i] = Ws[i].ctypes.data if has else None
        c.sc[i] = scs[i].ctypes.data if has else None
        c.rows[i] = Ws[i].shape[0] if has else 0
        c.y[i] = ys[i].ctypes.data if has else None
    c.x = x.ctypes.data


def bench_host_abi(q, wl, calls=1000):
    """Per-call time of the drop-in q35_mm_fp8 (host x in, host y out,
    synchronous) at configuration 0's and the qkv projection's shape, called
    from C in a loop on an already resident weight."""
    import numpy as np
    HostCall, lib = host_calls_lib()
    out = {}
    for name, k, n, seed in (("single_5120x5120", 5120, 5120, wl.SEED_BASE + 0),
                             ("qkv_5120x6144", 5120, 6144, wl.SEED_BASE + 1)):
        W, sc = wl.gen_weight(seed, n, k)
        x = wl.gen_act(seed + 0x100, 1, k)[0]
        y = np.empty(n, np.float32)
        lst = (HostCall * 1)()
        fill_call(lst[0], 0, k, [W], [sc], x, [y])
        us = lib.q35_host_calls_time(lst, 1, 20, calls)
        out[name] = {"us_per_call": round(us, 2), "calls": calls}
        q.release(W)
    out["note"] = ("q35_mm_fp8 on host pointers from a C loop (qwen38-in-c_amd/host_token.c), weight already "
                   "resident: x staged in pinned memory and read there by the GEMV, y written by it into pinned "
                   "memory, completion flag waited for, fingerprint of the weight checked while the GPU runs")
    return out


def bench_host_token(q, wl, layers=64, variants=8, reps=3):
    """The reference model's decode token through the drop-in ABI: its 288
    q35_mm_fp8 / q35_mm_fp8_multi4 calls on host pointers in its order
    (per layer the DeltaNet multi4 and out_proj, or the GQA q, k, v and
    o_proj, then the MLP's gate+up multi4 and down; qwen35-c/src/q35_model.c:
    903-937, qwen35-c/src/q35_deltanet.c:325-329,360, qwen35-c/src/q35_attn.c:
    262,273-275), made from C.  Host weights: `variants` distinct copies of
    each projection, layer i using copy i % variants (3.9 GB of host weights,
    resident on the device after the untimed first token; the device streams
    them from HBM as it would distinct layers, 3.9 GB being far beyond its
    caches)."""
    import numpy as np
    HostCall, lib = host_calls_lib()
    t0 = time.time()

    def copies(seed, n, k):
        W, sc = wl.gen_weight(seed, n, k)
        return [W if v == 0 else (W ^ row_sign_mask(n, v)) for v in range(variants)], sc
    dn = [copies(wl.SEED_BASE + 0x80 + j, n, k) for j, (_, k, n) in enumerate(wl.MODEL_DELTANET_SHAPES)]
    gq = [copies(wl.SEED_BASE + 0x90 + j, n, k) for j, (_, k, n) in enumerate(wl.MODEL_GQA_SHAPES)]
    ml = [copies(wl.SEED_BASE + 0xA0 + j, n, k) for j, (_, k, n) in enumerate(wl.MODEL_MLP_SHAPES)]
    log(f"host token: {variants} host copies of every projection in {time.time() - t0:.1f}s")
    xs = {k: wl.gen_act(wl.SEED_BASE + 0xB0 + k, 1, k)[0] for k in (5120, 6144, 17408)}
    ybuf = {}

    def y_of(n, slot=0):
        return ybuf.setdefault((n, slot), np.empty(n, np.float32))

    # q, k and v get outputs of their own (k and v have the same length)
    def sequence(qkv_multi4):
        seq = []
        idn = igq = 0
        for li in range(layers):
            if wl.model_layer_is_gqa(li):
                v = igq % variants
                if qkv_multi4:
                    seq.append((1, 5120, [gq[j][0][v] for j in range(3)], [gq[j][1] for j in range(3)], xs[5120],
                                [y_of(gq[j][0][v].shape[0], j) for j in range(3)]))
                else:
                    for j in range(3):
                        seq.append((0, 5120, [gq[j][0][v]], [gq[j][1]], xs[5120], [y_of(gq[j][0][v].shape[0], j)]))
                seq.append((0, 6144, [gq[3][0][v]], [gq[3][1]], xs[6144], [y_of(5120)]))
                igq += 1
            else:
                v = idn % variants
                seq.append((1, 5120, [dn[j][0][v] for j in range(4)], [dn[j][1] for j in range(4)], xs[5120],
                            [y_of(dn[j][0][v].shape[0], j) for j in range(4)]))
                seq.append((0, 6144, [dn[4][0][v]], [dn[4][1]], xs[6144], [y_of(5120)]))
                idn += 1
            v = li % variants
            seq.append((1, 5120, [ml[0][0][v], ml[1][0][v]], [ml[0][1], ml[1][1]], xs[5120],
                        [y_of(17408, 0), y_of(17408, 1)]))
            seq.append((0, 17408, [ml[2][0][v]], [ml[2][1]], xs[17408], [y_of(5120)]))
        lst = (HostCall * len(seq))()
        for c, (kind, cols, Ws, scs, x, ys) in zip(lst, seq):
            fill_call(c, kind, cols, Ws, scs, x, ys)
        return seq, lst
    seq, lst = sequence(False)
    t0 = time.time()
    us = lib.q35_host_calls_time(lst, len(seq), 1, reps)
    log(f"host token: {len(seq)} calls, {us / 1e3:.3f} ms per token ({time.time() - t0:.1f}s incl. first-use uploads)")
    qkv_sep = [y_of(gq[j][0][0].shape[0], j).copy() for j in range(3)]
    seq4, lst4 = sequence(True)
    us4 = lib.q35_host_calls_time(lst4, len(seq4), 1, reps)
    qkv_same = all(np.array_equal(a, y_of(gq[j][0][0].shape[0], j)) for j, a in enumerate(qkv_sep))
    log(f"host token, GQA q/k/v as one multi4 call: {len(seq4)} calls, {us4 / 1e3:.3f} ms per token")
    tok_bytes = 0
    for li in range(layers):
        shapes = wl.MODEL_GQA_SHAPES if wl.model_layer_is_gqa(li) else wl.MODEL_DELTANET_SHAPES
        tok_bytes += sum(wl.algorithmic_bytes(1, k, n) for _, k, n in shapes + wl.MODEL_MLP_SHAPES)
    for pool in dn + gq + ml:
        for W in pool[0]:
            q.release(W)
    return {"calls_per_token": len(seq), "host_weight_copies": variants, "ms_per_token": round(us / 1e3, 4),
            "GBps": round(tok_bytes / (us * 1e-6) / 1e9, 1), "bytes_per_token": tok_bytes,
            "gqa_qkv_multi4": {"calls_per_token": len(seq4), "ms_per_token": round(us4 / 1e3, 4),
                               "GBps": round(tok_bytes / (us4 * 1e-6) / 1e9, 1),
                               "q_k_v_bitwise_equal_to_separate_calls": qkv_same},
            "note": "the reference's 288 q35_mm_fp8 / q35_mm_fp8_multi4 calls of one decode token on host "
                    "pointers, in its order, from a C loop (qwen38-in-c_amd/host_token.c); synchronous calls, "
                    "each x in and y out through pinned memory"}


def bench_upload(q, wl, base, reps: int = 3):
    """Load one layer's five FP8 projections (320 MB, plus bf16 scales) from a
    safetensors file in the page cache into resident tiled weights
    (q35mm_st_load_fp8), and quantize a 17408 x 5120 BF16 tensor on load
    (q35mm_st_load_ab); best of reps, GB/s of file bytes."""
    import tempfile
    import numpy as np
    import torch
    tmp = tempfile.mkdtemp(prefix="q35mm_upload_")
    try:
        tensors = []
        for name, k, n, W, sc in base:
            tensors.append((f"layer.{name}.weight", "F8_E4M3", (n, k), W))
            tensors.append((f"layer.{name}.weight_scale_inv", "BF16", sc.shape, sc))
        gen = torch.Generator().manual_seed(wl.SEED_BASE + 7)
        wbf = (torch.randn(17408, 5120, generator=gen) * 0.02).to(torch.bfloat16).view(torch.int16).numpy()
        tensors.append(("layer.bf16.weight", "BF16", wbf.shape, wbf))
        path = os.path.join(tmp, "layer.safetensors")
        write_safetensors(path, tensors)
        fp8_bytes = sum(W.nbytes + sc.nbytes for _, _, _, W, sc in base)
        ck = q.Checkpoint(path)
        best_fp8 = best_ab = None
        for _ in range(reps):
            t0 = time.perf_counter()
            ws = [ck.load_fp8(f"layer.{name}.weight", n, k) for name, k, n, _, _ in base]
            t1 = time.perf_counter()
            for w in ws:
                w.free()
            t2 = time.perf_counter()
            wa = ck.load_ab("layer.bf16.weight", 17408, 5120)
            t3 = time.perf_counter()
            wa.free()
            best_fp8 = min(best_fp8 or 1e9, t1 - t0)
            best_ab = min(best_ab or 1e9, t3 - t2)
        ck.close()
        return {"fp8_layer": {"tensors": len(base), "bytes": fp8_bytes, "ms": round(best_fp8 * 1e3, 2),
                              "GBps": round(fp8_bytes / best_fp8 / 1e9, 2)},
                "bf16_quantize_17408x5120": {"bytes": wbf.nbytes, "ms": round(best_ab * 1e3, 2),
                                             "GBps": round(wbf.nbytes / best_ab / 1e9, 2)},
                "note": "safetensors file in the page cache -> pinned chunks (reader threads) -> HBM -> "
                        "lane-order tiles (and the device quantizer for BF16); includes allocation of the "
                        "resident weights; best of %d" % reps}
    finally:
        for f in os.listdir(tmp):
            os.remove(os.path.join(tmp, f))
        os.rmdir(tmp)


def bench_stragglers(q, wl, torch, dev, use_graph: bool, n: int = 512):
    """The reference's prefill calls DeltaNet out_proj and attention o_proj
    (both 6144 -> 5120) once per token (qwen35-c/src/q35_deltanet.c:498,
    qwen35-c/src/q35_attn.c:262).  Time n per-token calls against one batch
    call, on device pointers and through the host-pointer ABI."""
    import numpy as np
    k, nrows = 6144, 5120
    W, sc = wl.gen_weight(wl.SEED_BASE + 8, nrows, k)
    w = q.Weight(W, sc)
    X = wl.gen_act(wl.SEED_BASE + 9, n, k)
    dX = torch.from_numpy(X).to(dev)
    dY = torch.empty((n, nrows), device=dev)

    def per_token(_i):
        for t in range(n):
            q.gemv(w, dX[t:t + 1], dY[t:t + 1], m=1)

    def batched(_i):
        q.matmul(w, dX, dY)
    el_t, g1 = time_graph(torch, per_token, 1, 1, use_graph)
    del g1
    el_b, g2 = time_graph(torch, batched, 5, 2, use_graph)
    del g2
    # the drop-in calls from C (bench helper library), into output buffers
    # the caller reuses: n q35_mm_fp8 calls, then one q35_mm_fp8_batch
    HostCall, hlib = host_calls_lib()
    Yh = np.empty((n, nrows), np.float32)
    Yb = np.empty((n, nrows), np.float32)
    per = (HostCall * n)()
    for t in range(n):
        fill_call(per[t], 0, k, [W], [sc], X[t], [Yh[t]])
    bat = (HostCall * 1)()
    fill_call(bat[0], 2, k, [W], [sc], X, [Yb])
    bat[0].rows[1] = n
    us_t = hlib.q35_host_calls_time(per, n, 1, 3)
    us_b = hlib.q35_host_calls_time(bat, 1, 2, 10)
    rel = float(np.linalg.norm(Yb.astype(np.float64) - Yh) / np.linalg.norm(Yh.astype(np.float64)))
    q.release(W)
    w.free()
    flops = 2.0 * n * k * nrows
    return {"shape": f"{k}->{nrows}", "tokens": n,
            "device_per_token_ms": round(el_t * 1e3, 3), "device_batched_ms": round(el_b / 5 * 1e3, 3),
            "device_speedup": round(el_t / (el_b / 5), 1),
            "device_batched_TFLOPs": round(flops / (el_b / 5) / 1e12, 1),
            "host_abi_per_token_ms": round(us_t * 1e-3, 2), "host_abi_batched_ms": round(us_b * 1e-3, 3),
            "batched_vs_per_token_rel_l2": rel,
            "note": "per-token = n q35_mm_fp8 / q35mm_gemv(m=1) calls (fp32 GEMV); batched = one "
                    "q35_mm_fp8_batch / q35mm_matmul(m=n) call (bf16 GEMM at n >= 64; Q35MM_GEMM_MIN_M=0 keeps "
                    "it on the GEMV, bitwise equal to per-token); host_abi_* = the drop-in calls from a C loop "
                    "on host buffers the caller reuses (mean of 3 / 10 passes)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--pool", type=int, default=8)
    ap.add_argument("--eager", action="store_true", help="launch steps eagerly instead of from a HIP graph")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill-reps", type=int, default=100)
    ap.add_argument("--prefill-short", type=lambda v: [int(t) for t in v.split(",") if t], default=[64, 128],
                    help="token counts of the short-prompt prefill GEMMs timed beside M=512 (comma list; '' = none)")
    ap.add_argument("--no-blas", dest="blas", action="store_false",
                    help="skip the vendor bf16 GEMM (torch.mm -> hipBLASLt) timed beside the prefill GEMM")
    ap.add_argument("--no-mlp", dest="mlp", action="store_false",
                    help="skip the MLP block (RMSNorm, gate/up, SwiGLU, down, residual) at M=1")
    ap.add_argument("--no-stragglers", dest="stragglers", action="store_false",
                    help="skip per-token vs batched out_proj/o_proj at 512 tokens")
    ap.add_argument("--no-upload", dest="upload", action="store_false",
                    help="skip the safetensors -> HBM load of one layer")
    ap.add_argument("--no-lm-head", dest="lm_head", action="store_false",
                    help="skip the BF16 lm_head matvec (248320 x 5120)")
    ap.add_argument("--stack-layers", type=int, default=64,
                    help="distinct layers of the full-token weight stream (0: skip)")
    ap.add_argument("--no-single", dest="single", action="store_false",
                    help="skip configuration 0 (one 5120 x 5120 GEMV over a >= 1 GB pool of copies)")
    ap.add_argument("--no-model-token", dest="model_token", action="store_false",
                    help="skip the reference model's decode token (288 calls in its order)")
    ap.add_argument("--no-chain", dest="chain", action="store_false",
                    help="skip the layer step as one persistent q35mm_chain launch")
    ap.add_argument("--no-host-abi", dest="host_abi", action="store_false",
                    help="skip the per-call time of the drop-in q35_mm_fp8 on host pointers")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU time per CPU-baseline measurement")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="first run one plain device-to-device copy of MIB MiB (a known-size reference "
                         "kernel for hardware byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(a multi-GPU FP8 matmul would shard weights by 128-row groups; not built here)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import q35mm as q
    import workload as wl

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(0)
    log(f"device: {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")

    if args.calib_copy:
        n = args.calib_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {args.calib_copy} MiB read + {args.calib_copy} MiB written")
        del src, dst

    steps = max(1, args.steps)   # step i runs layer copy i % pool
    t = time.time()
    n_lay = max(args.pool, args.stack_layers)
    base, stack = make_layer_pool(q, wl, n_lay)
    layers = stack[: args.pool]
    log(f"{n_lay} distinct layers resident ({sum(w.nbytes for w in stack[0]) * n_lay / 1e9:.2f} GB) "
        f"in {time.time() - t:.1f}s; the first {args.pool} are the headline pool")

    # Projection order in DECODE_SHAPES: qkv, o_proj, gate, up, down; gate
    # and up read the same x.
    GATE, UP = 2, 3

    def layer_call(L, xs, ys, m):
        q.gemv(L[0], xs[0], ys[0], m=m)
        q.gemv(L[1], xs[1], ys[1], m=m)
        q.matmul_multi([L[GATE], L[UP]], xs[GATE], [ys[GATE], ys[UP]], m=m)
        q.gemv(L[4], xs[4], ys[4], m=m)

    def layer_inputs(x0, Y, m):
        """What each projection of a layer reads: qkv the layer input x0, every
        later one an output of the projection before it in the same layer
        (o_proj the first m*4096 floats of qkv's, gate and up o_proj's, down
        gate's), so each launch depends on the previous one's result."""
        k_o = base[1][1]
        return [x0, Y[0].view(-1)[: m * k_o].view(m, k_o), Y[1], Y[1], Y[GATE]]

    def decode_step_fn(m: int, lays, nout: int):
        x0 = torch.from_numpy(wl.gen_act(100, m, base[0][1])).to(dev)
        ys = [[torch.empty((m, n), dtype=torch.float32, device=dev) for (_, _, n, _, _) in base]
              for _ in range(nout)]
        xss = [layer_inputs(x0, Y, m) for Y in ys]

        def fn(i):
            li = i % len(lays)
            layer_call(lays[li], xss[li % nout], ys[li % nout], m)
        return fn, xss[0], ys

    step_bytes = {m: sum(wl.algorithmic_bytes(m, k, n) for _, k, n, _, _ in base) for m in (1, 2, 4, 8)}

    # ---- headline: M = 1 ----
    fn, xs, ys = decode_step_fn(1, layers, args.pool)
    el, g = time_graph(torch, fn, steps, args.warmup, not args.eager)
    value = step_bytes[1] * steps / el / 1e9
    ms_per_step = el / steps * 1e3
    # the graph's outputs must equal an eager run of the same step
    if g is not None:
        ref_out = [y.clone() for y in ys[(steps - 1) % args.pool]]
        fn(steps - 1)
        torch.cuda.synchronize()
        for a, b in zip(ref_out, ys[(steps - 1) % args.pool]):
            assert torch.equal(a, b), "graph replay differs from eager launch"
    log(f"M=1: {value:.1f} GB/s, {ms_per_step * 1e3:.1f} us/step ({'graph' if g is not None else 'eager'})")
    n_launch = steps * 4
    rows_split_off = os.environ.get("Q35MM_GEMV_ROWSPLIT", "1") == "0"   # the library's default: on
    roof = {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("decode_gemv_kernels_m1_layer.md"),
            "traffic_source": "profile, not this run: profiles/decode_gemv_kernels_m1_layer.md (rocprofv3 --pmc "
                              "FETCH_SIZE x2.0 + WRITE_SIZE x1.0 per launch, factors from a 512 MiB copy)",
            "kernel": ("gemv_fp8_kernel (stream-K)" if rows_split_off else
                       "gemv_rows_kernel (qkv, o_proj, gate+up, down)"), "launches": n_launch,
            "avg_launch_us": round(el / n_launch * 1e6, 3),
            "bytes_per_launch": step_bytes[1] // 4}
    del g

    # ---- the same layer step as ONE persistent launch (q35mm_chain) ----
    chain_out = None
    if args.chain:
        chains = [q.Chain([([L[0]], xs_c[0], [Y[0]]), ([L[1]], xs_c[1], [Y[1]]),
                           ([L[GATE], L[UP]], xs_c[GATE], [Y[GATE], Y[UP]]), ([L[4]], xs_c[4], [Y[4]])])
                  for L, Y, xs_c in ((layers[li], ys[li], layer_inputs(xs[0], ys[li], 1))
                                     for li in range(args.pool))]
        want = [y.clone() for y in ys[(steps - 1) % args.pool]]

        def chain_step(i):
            chains[i % args.pool].run()
        for y in ys[(steps - 1) % args.pool]:
            y.fill_(float("nan"))
        el_c, gc = time_graph(torch, chain_step, steps, args.warmup, not args.eager)
        del gc
        for c in chains:
            c.status()
        for a, b in zip(want, ys[(steps - 1) % args.pool]):
            assert torch.equal(a, b), "chain launch differs from the four launches"
        chain_out = {"us_per_layer": round(el_c / steps * 1e6, 2),
                     "GBps": round(step_bytes[1] * steps / el_c / 1e9, 1),
                     "frac_of_hbm_peak": round(step_bytes[1] * steps / el_c / 1e9 / HBM_PEAK_GBS, 4),
                     "launches_per_layer": 1, "workgroups": chains[0].workgroups,
                     "vs_four_launches": round(el / el_c, 3),
                     "note": "each layer's four steps (qkv, o_proj, gate+up, down; each reads the previous "
                             "one's output) as one q35mm_chain launch; outputs bit-identical to the four "
                             "launches (checked here)"}
        for c in chains:
            c.free()
        log(f"chain: {chain_out}")

    # ---- full decode token: the whole stack back to back at M = 1 ----
    stack_out = None
    if args.stack_layers:
        sfn, sxs, sys_ = decode_step_fn(1, stack, 1)
        nl = len(stack)

        def token(i):
            for li in range(nl):
                sfn(li)
        reps = 3
        el_s, gs = time_graph(torch, token, reps, 1, not args.eager)
        tok_bytes = step_bytes[1] * nl
        stack_out = {"layers": nl, "launches_per_token": 4 * nl, "bytes_per_token": tok_bytes,
                     "ms_per_token": round(el_s / reps * 1e3, 4),
                     "GBps": round(tok_bytes * reps / el_s / 1e9, 1),
                     "frac_of_hbm_peak": round(tok_bytes * reps / el_s / 1e9 / HBM_PEAK_GBS, 4)}
        del gs
        if args.chain:
            # the whole token as one launch: 4 steps per layer, every layer's
            # buffers shared (re-read buffers are read at the coherence point)
            Y = sys_[0]
            tok = q.Chain([st for L in stack for st in (
                ([L[0]], sxs[0], [Y[0]]), ([L[1]], sxs[1], [Y[1]]), ([L[GATE], L[UP]], sxs[GATE], [Y[GATE], Y[UP]]),
                ([L[4]], sxs[4], [Y[4]]))])
            want = [y.clone() for y in Y]
            el_t, gt = time_graph(torch, lambda _i: tok.run(), reps, 1, not args.eager)
            del gt
            tok.status()
            for a, b in zip(want, Y):
                assert torch.equal(a, b), "token chain differs from the launches"
            tok.free()
            stack_out["chain_ms_per_token"] = round(el_t / reps * 1e3, 4)
            stack_out["chain_GBps"] = round(tok_bytes * reps / el_t / 1e9, 1)
            stack_out["chain_note"] = "the same token as one q35mm_chain launch of 4 x layers steps"
        log(f"stack: {stack_out}")

    # ---- configuration 0: one 5120 x 5120 GEMV over a >= 1 GB pool ----
    single = None
    if args.single:
        single = bench_single(q, wl, torch, dev, max(steps, 64), args.warmup, not args.eager)
        log(f"single: {single}")

    # ---- the reference model's decode token: 288 calls in its order ----
    model_token = None
    if args.model_token and args.stack_layers:
        model_token = bench_model_token(q, wl, torch, dev, stack, not args.eager)
        log(f"model token: {model_token}")

    # ---- the drop-in ABI on host pointers: per-call time, and the model's
    # 288-call token ----
    host_abi = None
    if args.host_abi:
        host_abi = bench_host_abi(q, wl)
        if single:
            host_abi["single_5120x5120"]["device_kernel_us"] = single["us"]
            host_abi["single_5120x5120"]["overhead_us"] = round(host_abi["single_5120x5120"]["us_per_call"]
                                                                - single["us"], 2)
        if args.model_token:
            tok = bench_host_token(q, wl)
            if model_token:
                tok["device_api_ms_per_token"] = model_token["ms_per_token"]
                tok["overhead_us_per_call"] = round((tok["ms_per_token"] - model_token["ms_per_token"]) * 1e3
                                                    / tok["calls_per_token"], 2)
            host_abi["model_token"] = tok
        log(f"host abi: {host_abi}")

    # ---- MLP block at M = 1: RMSNorm -> gate/up -> SwiGLU -> down -> residual ----
    mlp_out = None
    if args.mlp:
        H, I = base[GATE][1], base[GATE][2]
        mlp_pair = os.environ.get("Q35MM_MLP_PAIR", "1")   # the library's default: paired gate and up
        gen = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 6)
        nws = [torch.randn(H, device=dev, generator=gen) * 0.1 for _ in range(args.pool)]
        xres = torch.randn((1, H), device=dev, generator=gen)
        xn = torch.randn((1, H), device=dev, generator=gen)
        gu = [torch.empty((1, I), device=dev) for _ in range(2)]
        yd = torch.empty((1, H), device=dev)

        def block(i):
            L = layers[i % args.pool]
            q.mlp(L[GATE], L[UP], L[4], nws[i % args.pool], xres)

        def matmuls(i):
            L = layers[i % args.pool]
            q.matmul_multi([L[GATE], L[UP]], xn, gu)
            q.gemv(L[4], gu[0], yd)
        blk_bytes = sum(wl.algorithmic_bytes(1, k, n) for _, k, n, _, _ in base[GATE:])
        el_b, gb = time_graph(torch, block, steps, 2, not args.eager)
        del gb
        el_m, gm = time_graph(torch, matmuls, steps, 2, not args.eager)
        del gm
        mlp_out = {"m": 1, "H": H, "I": I, "bytes_per_block": blk_bytes,
                   "us_per_block": round(el_b / steps * 1e6, 2),
                   "GBps": round(blk_bytes * steps / el_b / 1e9, 1),
                   "frac_of_hbm_peak": round(blk_bytes * steps / el_b / 1e9 / HBM_PEAK_GBS, 4),
                   "us_matmuls_only": round(el_m / steps * 1e6, 2),
                   "launches_per_block": 2 if rows_split_off or mlp_pair == "1" else 3 if mlp_pair == "2" else 4,
                   "note": ("q35mm_mlp at M=1: "
                            + ("RMSNorm (exact eight-lane order) inside the gate+up GEMV; SwiGLU and the residual "
                               "add inside the down GEMV"
                               if rows_split_off else
                               "RMSNorm (exact eight-lane order, every workgroup) and SwiGLU inside one row-split "
                               "launch over gate and up (16 rows of each per workgroup, one MFMA tile), the "
                               "residual add inside the down GEMV"
                               if mlp_pair == "1" else
                               "RMSNorm as its own kernel, SwiGLU inside the paired gate+up launch, the residual "
                               "add inside the down GEMV"
                               if mlp_pair == "2" else
                               "RMSNorm and SwiGLU as their own kernels (gate, up and down run the row-split "
                               "GEMV, which takes plain activations), the residual add inside the down GEMV")
                            + "; us_matmuls_only = the gate+up and down GEMV launches on ready activations")}
        # the same block on the prefill path: 512 tokens (256 x 256 tiles) and
        # 128 (a short prompt: 128 x 512 tiles cut along K)
        for mp in (512, 128):
            xres_p = torch.randn((mp, H), device=dev, generator=gen)

            def block_p(i):
                L = layers[i % args.pool]
                q.mlp(L[GATE], L[UP], L[4], nws[i % args.pool], xres_p)
            reps_p = max(args.pool, args.prefill_reps // args.pool * args.pool)
            el_p, gp = time_graph(torch, block_p, reps_p, 2, not args.eager)
            del gp
            flops_p = 2 * mp * H * I * 3
            mlp_out[f"prefill_m{mp}"] = {
                "us_per_block": round(el_p / reps_p * 1e6, 2),
                "TFLOPs": round(flops_p * reps_p / el_p / 1e12, 1),
                "note": f"q35mm_mlp at {mp} tokens: the RMSNorm written straight into the bf16 activations of one "
                        "GEMM launch over gate and up, whose paired tiles (or, for tiles cut along K, their slice "
                        "sum) write silu(gate) * up as the down GEMM's bf16 activations, the down GEMM adding the "
                        "residual in its epilogue or slice sum"}
        log(f"mlp block: {mlp_out}")

    # ---- decode sweep M = 1, 2, 4, 8 (per shape) ----
    sweep = {}
    if not args.no_sweep:
        for m in (1, 2, 4, 8):
            fn_m, xs_m, ys_m = decode_step_fn(m, layers, args.pool)
            per_shape = {}
            for j, (name, k, n, _, _) in enumerate(base):
                def one(i, j=j):
                    li = i % args.pool
                    q.gemv(layers[li][j], xs_m[j], ys_m[li][j], m=m)
                el_j, gj = time_graph(torch, one, steps, 2, not args.eager)
                per_shape[name] = round(wl.algorithmic_bytes(m, k, n) * steps / el_j / 1e9, 1)
                del gj
            el_m, gm = time_graph(torch, fn_m, steps, 2, not args.eager)
            sweep[f"M{m}"] = {"layer_GBps": round(step_bytes[m] * steps / el_m / 1e9, 1),
                              "us_per_layer": round(el_m / steps * 1e6, 2), "per_shape_GBps": per_shape}
            del gm
            log(f"M={m}: {sweep[f'M{m}']}")

    # ---- prefill GEMM at M = 512 ----
    prefill = None
    prefill_short = {}
    if not args.no_prefill:
        calls = {}
        for i, (name, k, n) in enumerate(wl.PREFILL_SHAPES):
            W, sc = wl.gen_weight(wl.SEED_BASE + 2 + 32 * i, n, k)
            w = q.Weight(W, sc)
            del W
            X = torch.from_numpy(wl.gen_act(wl.SEED_BASE + 3 + i, 512, k, bf16=True)).to(dev)
            Y = torch.empty((512, n), dtype=torch.float32, device=dev)

            def call(_i, w=w, X=X, Y=Y):
                q.gemm(w, X, Y)
            el_p, gp = time_graph(torch, call, args.prefill_reps, 2, not args.eager)
            tf = wl.flops(512, k, n) * args.prefill_reps / el_p / 1e12
            calls[name] = {"m": 512, "k": k, "n": n, "TFLOPs": round(tf, 1),
                           "us": round(el_p / args.prefill_reps * 1e6, 1)}
            log(f"prefill {name}: {tf:.1f} TFLOP/s")
            del gp
            # short prompts: the first m tokens, on the narrow 128 x 512 tiles
            for ms in args.prefill_short:
                Xs = X[:ms].contiguous()
                Ys = torch.empty((ms, n), dtype=torch.float32, device=dev)

                def call_s(_i, w=w, Xs=Xs, Ys=Ys):
                    q.gemm(w, Xs, Ys)
                el_s, gs = time_graph(torch, call_s, args.prefill_reps, 2, not args.eager)
                prefill_short[f"{name}_m{ms}"] = {
                    "m": ms, "k": k, "n": n, "us": round(el_s / args.prefill_reps * 1e6, 1),
                    "TFLOPs": round(wl.flops(ms, k, n) * args.prefill_reps / el_s / 1e12, 1),
                    "weight_GBps": round(wl.algorithmic_bytes(ms, k, n) * args.prefill_reps / el_s / 1e9, 1)}
                log(f"prefill {name} m={ms}: {prefill_short[f'{name}_m{ms}']}")
                del gs, Xs, Ys
            w.free()
            if args.blas:
                # Context, not a baseline of the same op: the vendor library's
                # plain bf16 x bf16 -> bf16 GEMM of the same shape (no fp8
                # decode, no block scales, half the output bytes).
                Wb = torch.randn((n, k), device=dev, dtype=torch.bfloat16)
                Xb = X.to(torch.bfloat16)
                Yb = torch.empty((512, n), device=dev, dtype=torch.bfloat16)

                def call_blas(_i, Wb=Wb, Xb=Xb, Yb=Yb):
                    torch.mm(Xb, Wb.t(), out=Yb)
                el_b, gb = time_graph(torch, call_blas, args.prefill_reps, 2, not args.eager)
                calls[name]["hipblaslt_bf16_TFLOPs"] = round(wl.flops(512, k, n) * args.prefill_reps / el_b / 1e12, 1)
                log(f"prefill {name}: hipBLASLt bf16 {calls[name]['hipblaslt_bf16_TFLOPs']} TFLOP/s")
                del gb, Wb, Xb, Yb
            del X, Y
            torch.cuda.empty_cache()
        tot_flops = sum(wl.flops(512, k, n) for _, k, n in wl.PREFILL_SHAPES)
        tot_us = sum(v["us"] for v in calls.values())
        tf_all = tot_flops / (tot_us * 1e-6) / 1e12
        # the headline's schema: one step = one gate+up call and one down call
        prefill = {
            "metric": "M=512 prefill GEMM TFLOP/s (% MFMA peak)",
            "value": round(tf_all, 1), "unit": "TFLOP/s", "n_gpus": 1,
            "steps": args.prefill_reps, "warmup": 2, "ms_per_step": round(tot_us / 1e3, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16 MFMA, fp32 accumulation (fp32 activations rounded to bf16 once per call; "
                     "e4m3 weights exact in bf16; fp32 block scales)",
            "data": "synthetic (seeded N(0,0.02) weights quantized per 128x128 block, bf16-representable "
                    "N(0,1) activations)",
            "config": {"workload": "prefill GEMM at 512 tokens: 5120->34816 (gate and up of the MLP as one "
                                   "weight) then 17408->5120 (down); one step = both calls, each from fp32 "
                                   "activations in HBM to fp32 outputs in HBM",
                       "m": 512, "shapes": [[k, n] for _, k, n in wl.PREFILL_SHAPES], "launch": (
                           "hip graph" if not args.eager else "eager")},
            "roofline": {"bound": "mfma", "achieved": round(tf_all, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf_all / BF16_PEAK_TFLOPS, 4),
                         "traffic": measured_traffic("gemm_kernels_prefill_m512.md",
                                                     "prefill_traffic_bytes_per_launch"),
                         "traffic_source": "profile, not this run: profiles/gemm_kernels_prefill_m512.md "
                                           "(rocprofv3 --pmc FETCH_SIZE x2.0 + WRITE_SIZE x1.0 of the gate+up "
                                           "GEMM launch, the dominant kernel; factors from a 512 MiB copy)",
                         "kernel": "gemm_fp8_kernel (+ act_to_bf16_kernel, gemm_tail_kernel / "
                                   "gemm_reduce_kernel): whole calls",
                         "flops_per_step": tot_flops,
                         "flops_per_call": {name: wl.flops(512, k, n) for name, k, n in wl.PREFILL_SHAPES},
                         "peak_from_clock": clock_peak_tflops(props.multi_processor_count)},
            "cpu_baseline": None,
            "calls": calls,
            "note": "value = 2*M*N*K of both calls / the time of both whole calls (the fp32->bf16 activation "
                    "prepass, the GEMM and its tail or K-slice reduction); hipblaslt_bf16_TFLOPs = torch.mm "
                    "of bf16 operands of the same shape (bf16 output), for context",
        }

    # ---- BF16 lm_head matvec (q35_mm_bf16): 248320 x 5120 ----
    lm_head = None
    if args.lm_head:
        rows, cols = 248320, 5120
        # two distinct resident copies (2 x 2.54 GB), alternated: no cache reuse
        gen = torch.Generator(device=dev).manual_seed(wl.SEED_BASE + 5)
        pool2 = [(torch.randn(rows, cols, device=dev, generator=gen) * 0.02).to(torch.bfloat16).view(torch.int16)
                 for _ in range(2)]
        xh = torch.randn(cols, device=dev, generator=gen)
        yh = torch.empty(rows, dtype=torch.float32, device=dev)

        def lm_call(i):
            q.bf16_gemv(pool2[i % 2], xh, yh)
        reps = 20
        el_h, gh = time_graph(torch, lm_call, reps, 2, not args.eager)
        lm_bytes = rows * cols * 2 + cols * 4 + rows * 4
        lm_head = {"rows": rows, "cols": cols, "us": round(el_h / reps * 1e6, 1),
                   "GBps": round(lm_bytes * reps / el_h / 1e9, 1),
                   "frac_of_hbm_peak": round(lm_bytes * reps / el_h / 1e9 / HBM_PEAK_GBS, 4),
                   "numerics": "bit-identical to the reference's q35_mm_bf16 order"}
        log(f"lm_head: {lm_head}")
        del gh, pool2

    # ---- prefill stragglers: per-token out_proj / o_proj vs one batch ----
    stragglers = None
    if args.stragglers:
        stragglers = bench_stragglers(q, wl, torch, dev, not args.eager)
        log(f"stragglers: {stragglers}")

    # ---- checkpoint -> HBM: one layer's FP8 weights from a safetensors file ----
    upload = None
    if args.upload:
        upload = bench_upload(q, wl, base)
        log(f"upload: {upload}")

    cpu = None
    cpu_run = None if args.no_cpu else cpu_baseline(args.cpu_budget)
    if cpu_run:
        host = cpu_run["host"]
        hdesc = (f"{host.get('model')}, {host.get('sockets')} socket(s) x {host.get('cores_per_socket')} cores x "
                 f"{host.get('threads_per_core')} threads, {host.get('numa_nodes')} NUMA node(s)")
        cpu = {"value": cpu_run["layer"]["GBps"], "unit": "GB/s", "cores": cpu_run["threads"],
               "kind": cpu_run["kind"],
               "sample": f"{cpu_run['layer']['passes']} passes of one layer's 5 projections at M=1 (gate+up via "
                         f"multi4), {cpu_run['layer']['bytes'] / 1e6:.1f} MB each, median "
                         f"{cpu_run['layer']['ms']} ms/pass; "
                         + ("oracle/_ref = the reference's q35_mm.c" if cpu_run["kind"] == "reference"
                            else "oracle port") +
                         f", OMP_NUM_THREADS={cpu_run['threads']} OMP_PROC_BIND={cpu_run['omp_proc_bind']} "
                         f"OMP_PLACES={cpu_run['omp_places']} in a child process; host: {hdesc}",
               "host": host, "threads": cpu_run["threads"], "omp_proc_bind": cpu_run["omp_proc_bind"],
               "reference_auto_threads": cpu_run.get("reference_auto_threads")}
        if single:
            single["cpu_baseline"] = {"value": cpu_run["single"]["GBps"], "unit": "GB/s",
                                      "ms": cpu_run["single"]["ms"], "cores": cpu_run["threads"],
                                      "kind": cpu_run["kind"]}
        if prefill:
            ps = cpu_run["prefill_sample"]
            prefill["cpu_baseline"] = {"value": ps["TFLOPs"], "unit": "TFLOP/s", "cores": cpu_run["threads"],
                                       "kind": cpu_run["kind"],
                                       "sample": f"first {ps['tokens']} of the 512 tokens of both shapes, "
                                                 f"{ps}"}

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 weights x fp32 activations, fp32 accumulation",
        "data": "synthetic (seeded N(0,0.02) weights quantized per 128x128 block, N(0,1) activations)",
        "config": {"workload": "decode GEMV, M=1, one layer's projections 5120->6144, 4096->5120, "
                               "5120->17408 x2 (gate+up as one multi4 call), 17408->5120 per step, "
                               "each reading the previous projection's output",
                   "m": 1, "pool_layers": args.pool, "bytes_per_step": step_bytes[1],
                   "launch": "hip graph" if not args.eager else "eager"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "decode_sweep": sweep or None,
        "decode_chain": chain_out,
        "decode_stack": stack_out,
        "single": single,
        "decode_model_token": model_token,
        "host_abi": host_abi,
        "prefill": prefill,
        "prefill_short": prefill_short or None,
        "lm_head_bf16": lm_head,
        "mlp_block": mlp_out,
        "upload": upload,
        "prefill_stragglers": stragglers,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    if len(sys.argv) > 2 and sys.argv[1] == CPU_CHILD:
        cpu_child(float(sys.argv[2]))
    else:
        main()
