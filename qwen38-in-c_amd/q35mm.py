"""Python view of libq35mm.so through its C ABI (ctypes).

Two layers, mirroring the two headers:

* Drop-in ABI (include/q35/q35_mm.h): ``mm_fp8``, ``mm_fp8_batch``,
  ``mm_fp8_multi4``, ``mm_bf16`` take numpy host arrays exactly as the
  reference's q35_mm_fp8 / q35_mm_fp8_batch / q35_mm_fp8_multi4 / q35_mm_bf16
  take host pointers (qwen35-c/include/q35/q35_mm.h:24-45); outputs are
  token-major like the reference's (qwen35-c/src/q35_mm.c:168).
* Device API (include/q35mm/q35mm.h): ``Weight`` keeps a resident copy in
  HBM; ``matmul`` / ``gemv`` / ``gemm`` / ``matmul_multi`` run on device
  pointers (torch tensors on the GPU are accepted and their current stream
  is used).

There is no fallback: if the library is missing or fails to load, import
raises.  The GPU is touched only by calls that need it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "lib", "libq35mm.so")

_u8p = C.POINTER(C.c_uint8)
_u16p = C.POINTER(C.c_uint16)
_u32p = C.POINTER(C.c_uint32)
_f32p = C.POINTER(C.c_float)

# Every function declared by include/q35/q35_mm.h and include/q35mm/q35mm.h.
DROPIN_SYMBOLS = ("q35_mm_init", "q35_mm_e4m3_to_f32", "q35_mm_bf16_to_f32", "q35_mm_fp8",
                  "q35_mm_fp8_batch", "q35_mm_fp8_multi4", "q35_mm_bf16", "q35_mm_impl_fp8")
DATA_SYMBOLS = ("q35_mm_fp8_lut",)


class Q35mmError(RuntimeError):
    pass


class ChainStep(C.Structure):
    """q35mm_chain_step (include/q35mm/q35mm.h)."""
    _fields_ = [("nw", C.c_uint32), ("w", C.c_void_p * 4), ("x", C.c_void_p), ("y", C.c_void_p * 4),
                ("resid", C.c_void_p * 4)]


def _load(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise Q35mmError(f"libq35mm.so not built at {path}; run __graft_entry__.build() "
                         "or python qwen38-in-c_amd/build.py")
    # One HIP runtime per process: torch ships its own libamdhip64 /
    # libhsa-runtime64 and loads them under a different needed-name, so if
    # libq35mm.so pulled in /opt/rocm's copy first, torch would load a second
    # runtime and one of the two would find no device.  Importing torch first
    # makes libq35mm.so bind to the runtime torch already loaded (same SONAME).
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(path)
    lib.q35_mm_init.argtypes = []
    lib.q35_mm_e4m3_to_f32.restype = C.c_float
    lib.q35_mm_e4m3_to_f32.argtypes = [C.c_uint8]
    lib.q35_mm_bf16_to_f32.restype = C.c_float
    lib.q35_mm_bf16_to_f32.argtypes = [C.c_uint16]
    lib.q35_mm_fp8.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, _f32p, _f32p]
    lib.q35_mm_fp8_batch.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, C.c_uint32, _f32p, _f32p]
    lib.q35_mm_fp8_multi4.argtypes = [C.POINTER(_u8p), C.POINTER(_u16p), _u32p, C.c_uint32, _f32p,
                                      C.POINTER(_f32p)]
    lib.q35_mm_bf16.argtypes = [_u16p, C.c_uint32, C.c_uint32, _f32p, _f32p]
    lib.q35_mm_impl_fp8.restype = C.c_char_p
    vp = C.c_void_p
    lib.q35mm_init.argtypes = [C.c_int]
    lib.q35mm_weight_create.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, C.POINTER(vp)]
    lib.q35mm_weight_create_f32scale.argtypes = [_u8p, _f32p, C.c_uint32, C.c_uint32, C.POINTER(vp)]
    lib.q35mm_weight_destroy.argtypes = [vp]
    lib.q35mm_weight_destroy.restype = None
    lib.q35mm_weight_shape.argtypes = [vp, _u32p, _u32p]
    lib.q35mm_weight_bytes.argtypes = [vp]
    lib.q35mm_weight_bytes.restype = C.c_size_t
    for name in ("q35mm_matmul", "q35mm_gemv", "q35mm_gemm", "q35mm_matmul_noalloc"):
        getattr(lib, name).argtypes = [vp, C.c_uint32, vp, vp, vp]
    lib.q35mm_matmul_multi.argtypes = [C.POINTER(vp), C.c_uint32, C.c_uint32, vp, C.POINTER(vp), vp]
    lib.q35mm_dequant_f32.argtypes = [vp, vp, vp]
    lib.q35mm_decode_bf16.argtypes = [vp, vp, vp]
    lib.q35mm_bf16_gemv.argtypes = [vp, C.c_uint32, C.c_uint32, vp, vp, vp]
    lib.q35mm_rmsnorm.argtypes = [vp, vp, vp, C.c_uint32, C.c_uint32, C.c_float, vp]
    lib.q35mm_swiglu.argtypes = [vp, vp, vp, C.c_size_t, vp]
    lib.q35mm_mlp.argtypes = [vp, vp, vp, vp, C.c_float, C.c_uint32, vp, vp]
    lib.q35mm_quantize_f32.argtypes = [vp, C.c_uint32, C.c_uint32, vp, vp, vp]
    lib.q35mm_st_open.argtypes = [C.c_char_p, C.POINTER(vp)]
    lib.q35mm_st_close.argtypes = [vp]
    lib.q35mm_st_close.restype = None
    lib.q35mm_st_count.argtypes = [vp]
    lib.q35mm_st_count.restype = C.c_uint32
    lib.q35mm_st_name.argtypes = [vp, C.c_uint32]
    lib.q35mm_st_name.restype = C.c_char_p
    lib.q35mm_st_info.argtypes = [vp, C.c_char_p, C.POINTER(C.c_char_p), _u32p, _u32p, C.POINTER(C.c_uint64)]
    lib.q35mm_st_read.argtypes = [vp, C.c_char_p, vp, C.c_uint64]
    for name in ("q35mm_st_load_fp8", "q35mm_st_load_ab"):
        getattr(lib, name).argtypes = [vp, C.c_char_p, C.c_uint32, C.c_uint32, C.POINTER(vp)]
    lib.q35mm_st_load_bf16.argtypes = [vp, C.c_char_p, C.c_uint32, C.c_uint32, C.POINTER(vp)]
    lib.q35mm_free.argtypes = [vp]
    lib.q35mm_free.restype = None
    lib.q35mm_release.argtypes = [vp]
    lib.q35mm_release.restype = None
    lib.q35mm_release_all.argtypes = []
    lib.q35mm_release_all.restype = None
    lib.q35mm_shutdown.argtypes = []
    lib.q35mm_shutdown.restype = None
    lib.q35mm_last_error.restype = C.c_char_p
    lib.q35mm_resident_count.restype = C.c_size_t
    lib.q35mm_stream_release.argtypes = [vp]
    lib.q35mm_chain_create.argtypes = [C.POINTER(ChainStep), C.c_uint32, C.c_uint32, C.POINTER(vp)]
    lib.q35mm_chain_run.argtypes = [vp, vp]
    lib.q35mm_chain_status.argtypes = [vp]
    lib.q35mm_chain_workgroups.argtypes = [vp]
    lib.q35mm_chain_workgroups.restype = C.c_uint32
    lib.q35mm_chain_destroy.argtypes = [vp]
    lib.q35mm_chain_destroy.restype = None
    lib.q35mm_debug_counters.argtypes = [vp, C.c_int, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
    return lib


lib = _load()


def _p(a: np.ndarray, ptype):
    if not a.flags["C_CONTIGUOUS"]:
        raise Q35mmError("arrays passed to libq35mm must be C-contiguous")
    return a.ctypes.data_as(ptype)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        err = Q35mmError(f"{what} failed ({rc}): {lib.q35mm_last_error().decode()}")
        err.code = rc
        raise err


# ---------------------------------------------------------------------------
# Drop-in ABI (host pointers)
# ---------------------------------------------------------------------------
def init(device: int = -1) -> None:
    """q35mm_init: select and initialise the device (-1: the default)."""
    _check(lib.q35mm_init(device), "q35mm_init")


def impl() -> str:
    return lib.q35_mm_impl_fp8().decode()


def lut() -> np.ndarray:
    arr = (C.c_float * 256).in_dll(lib, "q35_mm_fp8_lut")
    return np.frombuffer(arr, np.float32).copy()


def e4m3_to_f32(v: int) -> float:
    return float(lib.q35_mm_e4m3_to_f32(v))


def bf16_to_f32(v: int) -> float:
    return float(lib.q35_mm_bf16_to_f32(v))


def _check_fp8(W: np.ndarray, sc: np.ndarray):
    if W.dtype != np.uint8 or W.ndim != 2:
        raise Q35mmError("W must be a 2-D uint8 array of e4m3 codes")
    rows, cols = W.shape
    want = ((rows + 127) // 128, (cols + 127) // 128)
    if sc.dtype != np.uint16 or sc.size != want[0] * want[1]:
        raise Q35mmError(f"scale must be uint16 bf16 bits with {want[0]}x{want[1]} entries")
    return rows, cols


def mm_fp8(W: np.ndarray, sc: np.ndarray, x: np.ndarray) -> np.ndarray:
    """q35_mm_fp8: y[r] = sum_c e4m3(W[r][c]) * s[r/128][c/128] * x[c]."""
    rows, cols = _check_fp8(W, sc)
    x = np.ascontiguousarray(x, np.float32)
    if x.size != cols:
        raise Q35mmError("x must have cols elements")
    y = np.empty(rows, np.float32)
    lib.q35_mm_fp8(_p(W, _u8p), _p(np.ascontiguousarray(sc), _u16p), rows, cols, _p(x, _f32p), _p(y, _f32p))
    return y


def mm_fp8_batch(W: np.ndarray, sc: np.ndarray, X: np.ndarray) -> np.ndarray:
    """q35_mm_fp8_batch: X [n][cols] -> Y [n][rows] (token-major)."""
    rows, cols = _check_fp8(W, sc)
    X = np.ascontiguousarray(X, np.float32).reshape(-1, cols)
    n = X.shape[0]
    Y = np.empty((n, rows), np.float32)
    lib.q35_mm_fp8_batch(_p(W, _u8p), _p(np.ascontiguousarray(sc), _u16p), rows, cols, n,
                         _p(X, _f32p), _p(Y, _f32p))
    return Y


def mm_fp8_multi4(Ws, scs, x: np.ndarray):
    """q35_mm_fp8_multi4: up to four (W, scale) pairs sharing x and cols.
    ``None`` entries are skipped (rows = 0), as in the reference."""
    Ws = list(Ws) + [None] * (4 - len(Ws))
    scs = list(scs) + [None] * (4 - len(scs))
    cols = next(W.shape[1] for W in Ws if W is not None)
    x = np.ascontiguousarray(x, np.float32)
    wp = (_u8p * 4)()
    sp = (_u16p * 4)()
    rows = (C.c_uint32 * 4)()
    yp = (_f32p * 4)()
    outs = []
    keep = []
    for s in range(4):
        if Ws[s] is None:
            rows[s] = 0
            outs.append(None)
            continue
        r, c = _check_fp8(Ws[s], scs[s])
        if c != cols:
            raise Q35mmError("multi4 segments must share cols")
        sc = np.ascontiguousarray(scs[s])
        keep.append(sc)
        y = np.empty(r, np.float32)
        wp[s] = _p(Ws[s], _u8p)
        sp[s] = _p(sc, _u16p)
        rows[s] = r
        yp[s] = _p(y, _f32p)
        outs.append(y)
    lib.q35_mm_fp8_multi4(wp, sp, rows, cols, _p(x, _f32p), yp)
    return outs


def mm_bf16(W16: np.ndarray, x: np.ndarray) -> np.ndarray:
    """q35_mm_bf16: y[r] = sum_c bf16(W[r][c]) * x[c]."""
    if W16.dtype != np.uint16 or W16.ndim != 2:
        raise Q35mmError("W must be a 2-D uint16 array of bf16 bits")
    rows, cols = W16.shape
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    lib.q35_mm_bf16(_p(W16, _u16p), rows, cols, _p(x, _f32p), _p(y, _f32p))
    return y


def release(W: np.ndarray) -> None:
    lib.q35mm_release(W.ctypes.data)


def release_all() -> None:
    lib.q35mm_release_all()


def resident_count() -> int:
    return int(lib.q35mm_resident_count())


# ---------------------------------------------------------------------------
# Device API
# ---------------------------------------------------------------------------
def _dptr(t) -> int:
    """Device pointer of a torch tensor (or an int)."""
    if isinstance(t, int):
        return t
    if not t.is_cuda or not t.is_contiguous():
        raise Q35mmError("device arguments must be contiguous GPU tensors")
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is not None:
        return int(stream)
    try:
        import torch
        if torch.cuda.is_available():
            return int(torch.cuda.current_stream().cuda_stream)
    except ImportError:
        pass
    return None


class Weight:
    """A resident FP8 weight (q35mm_weight_create)."""

    def __init__(self, W: np.ndarray, sc: np.ndarray):
        self.rows, self.cols = W.shape
        h = C.c_void_p()
        W = np.ascontiguousarray(W, np.uint8)
        if sc.dtype == np.float32:
            rc = lib.q35mm_weight_create_f32scale(_p(W, _u8p), _p(np.ascontiguousarray(sc), _f32p),
                                                  self.rows, self.cols, C.byref(h))
        else:
            _check_fp8(W, sc)
            rc = lib.q35mm_weight_create(_p(W, _u8p), _p(np.ascontiguousarray(sc), _u16p),
                                         self.rows, self.cols, C.byref(h))
        _check(rc, "q35mm_weight_create")
        self.handle = h

    @property
    def nbytes(self) -> int:
        return int(lib.q35mm_weight_bytes(self.handle))

    def free(self) -> None:
        if self.handle:
            lib.q35mm_weight_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Chain:
    """q35mm_chain_*: decode GEMVs run as one persistent launch.  steps is a
    list of (weights, x, ys) or (weights, x, ys, resids): 1..4 Weights
    sharing cols, the device activations x [m][cols] and one output (and
    optional residual, or None) per weight; x may be an output of an earlier
    step.  The tensors are kept referenced while the chain lives."""

    def __init__(self, steps, m: int = 1):
        arr = (ChainStep * len(steps))()
        self._keep = []
        for i, st in enumerate(steps):
            ws, x, ys = st[0], st[1], st[2]
            rs = st[3] if len(st) > 3 and st[3] is not None else [None] * len(ws)
            if not 1 <= len(ws) <= 4 or len(ys) != len(ws) or len(rs) != len(ws):
                raise Q35mmError("a chain step holds 1..4 weights, one output (and residual) each")
            arr[i].nw = len(ws)
            arr[i].x = _dptr(x)
            for j, (w, y, r) in enumerate(zip(ws, ys, rs)):
                arr[i].w[j] = w.handle
                arr[i].y[j] = _dptr(y)
                arr[i].resid[j] = _dptr(r) if r is not None else None
            self._keep.append((ws, x, ys, rs))
        h = C.c_void_p()
        _check(lib.q35mm_chain_create(arr, len(steps), m, C.byref(h)), "q35mm_chain_create")
        self.handle = h
        self.steps = len(steps)

    @property
    def workgroups(self) -> int:
        return int(lib.q35mm_chain_workgroups(self.handle))

    def run(self, stream=None) -> None:
        _check(lib.q35mm_chain_run(self.handle, _stream(stream)), "q35mm_chain_run")

    def status(self) -> None:
        """Waits for the device; raises if a launch gave up waiting."""
        _check(lib.q35mm_chain_status(self.handle), "q35mm_chain_status")

    def free(self) -> None:
        if self.handle:
            lib.q35mm_chain_destroy(self.handle)
            self.handle = None
            self._keep = []

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def matmul(w: Weight, X, Y, m: int | None = None, stream=None) -> None:
    m = X.shape[0] if m is None else m
    _check(lib.q35mm_matmul(w.handle, m, _dptr(X), _dptr(Y), _stream(stream)), "q35mm_matmul")


def matmul_noalloc(w: Weight, X, Y, m: int | None = None, stream=None) -> None:
    """q35mm_matmul_noalloc: q35mm_matmul on the library's fixed scratch."""
    m = X.shape[0] if m is None else m
    _check(lib.q35mm_matmul_noalloc(w.handle, m, _dptr(X), _dptr(Y), _stream(stream)), "q35mm_matmul_noalloc")


def gemv(w: Weight, X, Y, m: int | None = None, stream=None) -> None:
    m = X.shape[0] if m is None else m
    _check(lib.q35mm_gemv(w.handle, m, _dptr(X), _dptr(Y), _stream(stream)), "q35mm_gemv")


def gemm(w: Weight, X, Y, m: int | None = None, stream=None) -> None:
    m = X.shape[0] if m is None else m
    _check(lib.q35mm_gemm(w.handle, m, _dptr(X), _dptr(Y), _stream(stream)), "q35mm_gemm")


def matmul_multi(ws, X, Ys, m: int | None = None, stream=None) -> None:
    m = X.shape[0] if m is None else m
    n = len(ws)
    hs = (C.c_void_p * n)(*[w.handle for w in ws])
    ys = (C.c_void_p * n)(*[_dptr(y) for y in Ys])
    _check(lib.q35mm_matmul_multi(hs, n, m, _dptr(X), ys, _stream(stream)), "q35mm_matmul_multi")


def dequant_f32(w: Weight, out, stream=None) -> None:
    _check(lib.q35mm_dequant_f32(w.handle, _dptr(out), _stream(stream)), "q35mm_dequant_f32")


def decode_bf16(w: Weight, out, stream=None) -> None:
    _check(lib.q35mm_decode_bf16(w.handle, _dptr(out), _stream(stream)), "q35mm_decode_bf16")


def bf16_gemv(W16, x, y, stream=None) -> None:
    rows, cols = W16.shape
    _check(lib.q35mm_bf16_gemv(_dptr(W16), rows, cols, _dptr(x), _dptr(y), _stream(stream)),
           "q35mm_bf16_gemv")


def rmsnorm(X, w, Y, eps: float = 1e-6, stream=None) -> None:
    """Row-wise zero-centred RMSNorm (q35_kern_rmsnorm) of X [rows][n]."""
    n = X.shape[-1]
    rows = X.numel() // n if n else 0
    if w.numel() != n or Y.numel() != X.numel():
        raise Q35mmError("rmsnorm: shapes disagree")
    _check(lib.q35mm_rmsnorm(_dptr(X), _dptr(w), _dptr(Y), rows, n, eps, _stream(stream)), "q35mm_rmsnorm")


def swiglu(G, U, Y, stream=None) -> None:
    """Y = silu(G) * U elementwise (q35_kern_swiglu)."""
    if G.numel() != U.numel() or Y.numel() != G.numel():
        raise Q35mmError("swiglu: sizes disagree")
    _check(lib.q35mm_swiglu(_dptr(G), _dptr(U), _dptr(Y), G.numel(), _stream(stream)), "q35mm_swiglu")


def mlp(gate: Weight, up: Weight, down: Weight, norm_w, X, eps: float = 1e-6, m: int | None = None,
        stream=None) -> None:
    """One MLP block in place on the residual stream X [m][H]."""
    m = X.shape[0] if m is None else m
    _check(lib.q35mm_mlp(gate.handle, up.handle, down.handle, _dptr(norm_w), eps, m, _dptr(X),
                         _stream(stream)), "q35mm_mlp")


def quantize_f32(W, codes, scale, stream=None) -> None:
    """Device quantizer (q35mm_quantize_f32): W [rows][cols] fp32 ->
    codes [rows][cols] uint8, scale [ceil(rows/128)][ceil(cols/128)] bf16 bits."""
    rows, cols = W.shape
    _check(lib.q35mm_quantize_f32(_dptr(W), rows, cols, _dptr(codes), _dptr(scale), _stream(stream)),
           "q35mm_quantize_f32")


class Checkpoint:
    """A safetensors file or shard directory (q35mm_st_open)."""

    def __init__(self, path: str):
        h = C.c_void_p()
        _check(lib.q35mm_st_open(os.fsencode(path), C.byref(h)), "q35mm_st_open")
        self.handle = h

    def close(self) -> None:
        if self.handle:
            lib.q35mm_st_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def names(self) -> list:
        return [lib.q35mm_st_name(self.handle, i).decode() for i in range(lib.q35mm_st_count(self.handle))]

    def info(self, name: str):
        """(dtype, shape, nbytes)"""
        dt = C.c_char_p()
        nd = C.c_uint32()
        shape = (C.c_uint32 * 8)()
        nb = C.c_uint64()
        _check(lib.q35mm_st_info(self.handle, name.encode(), C.byref(dt), C.byref(nd), shape, C.byref(nb)),
               "q35mm_st_info")
        return dt.value.decode(), tuple(shape[: nd.value]), nb.value

    def read(self, name: str) -> bytes:
        _, _, nb = self.info(name)
        buf = C.create_string_buffer(max(nb, 1))
        _check(lib.q35mm_st_read(self.handle, name.encode(), buf, nb), "q35mm_st_read")
        return buf.raw[:nb]

    def _load(self, fn, name, rows, cols) -> "Weight":
        w = Weight.__new__(Weight)
        w.rows, w.cols = rows, cols
        h = C.c_void_p()
        _check(getattr(lib, fn)(self.handle, name.encode(), rows, cols, C.byref(h)), fn)
        w.handle = h
        return w

    def load_fp8(self, name: str, rows: int, cols: int) -> "Weight":
        return self._load("q35mm_st_load_fp8", name, rows, cols)

    def load_ab(self, name: str, rows: int, cols: int) -> "Weight":
        return self._load("q35mm_st_load_ab", name, rows, cols)

    def load_bf16(self, name: str, rows: int, cols: int) -> int:
        """Device pointer of a new bf16 buffer (free with free())."""
        p = C.c_void_p()
        _check(lib.q35mm_st_load_bf16(self.handle, name.encode(), rows, cols, C.byref(p)), "q35mm_st_load_bf16")
        return p.value


def free(dptr: int) -> None:
    lib.q35mm_free(dptr)


def shutdown() -> None:
    lib.q35mm_shutdown()


def stream_release(stream=None) -> None:
    """q35mm_stream_release: free the scratch of a stream (default: torch's
    current stream) before it is destroyed."""
    _check(lib.q35mm_stream_release(_stream(stream)), "q35mm_stream_release")


def debug_counters(stream=None, noalloc: bool = False) -> tuple[int, int]:
    """q35mm_debug_counters: (nonzero words, words) among the arrival
    counters of a stream's scratch, or of the allocation-free scratch."""
    nz, n = C.c_uint64(), C.c_uint64()
    _check(lib.q35mm_debug_counters(_stream(stream), 1 if noalloc else 0, C.byref(nz), C.byref(n)),
           "q35mm_debug_counters")
    return int(nz.value), int(n.value)
