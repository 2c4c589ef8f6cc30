"""ctypes wrapper around the CPU oracle (oracle/liboracle.so) and, when built,
the reference's own compiled matmul and elementwise kernels
(oracle/_ref/libq35ref*.so, oracle/_ref/libq35kern.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check in
__graft_entry__.py and by the cpu_baseline leg of bench.py.  The product
library never loads it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libq35ref.so")
REF_SCALAR_PATH = os.path.join(HERE, "_ref", "libq35ref_scalar.so")
REF_KERN_PATH = os.path.join(HERE, "_ref", "libq35kern.so")

_u8p = C.POINTER(C.c_uint8)
_u16p = C.POINTER(C.c_uint16)
_u32p = C.POINTER(C.c_uint32)
_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    targets = ["oracle", "ref"] if ref else ["oracle"]
    subprocess.run(["make", "-s", "-C", HERE] + targets, check=True)


def _p(a: np.ndarray, ptype):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ptype)


class Oracle:
    """numpy-facing view of the C restatement."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            build(ref=False)
        self.lib = L = C.CDLL(path)
        L.orc_e4m3_to_f32.restype = C.c_float
        L.orc_e4m3_to_f32.argtypes = [C.c_uint8]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_fill_lut.argtypes = [_f32p]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_f32_to_e4m3.restype = C.c_uint8
        L.orc_f32_to_e4m3.argtypes = [C.c_float]
        L.orc_quantize_fp8.argtypes = [_f32p, C.c_uint32, C.c_uint32, _u8p, _u16p]
        L.orc_dequant.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, _f32p]
        L.orc_dequant_f32scale.argtypes = [_u8p, _f32p, C.c_uint32, C.c_uint32, _f32p]
        L.orc_mm_fp8.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, _f32p, _f32p]
        L.orc_mm_fp8_batch.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, C.c_uint32,
                                       _f32p, _f32p]
        L.orc_mm_fp8_rows.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, C.c_uint32,
                                      _f32p, _u32p, C.c_uint32, _f32p]
        L.orc_mm_fp8_batch_f32scale.argtypes = [_u8p, _f32p, C.c_uint32, C.c_uint32,
                                                C.c_uint32, _f32p, _f32p]
        L.orc_mm_fp8_f64.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, C.c_uint32,
                                     _f32p, _f64p]
        L.orc_mm_bf16.argtypes = [_u16p, C.c_uint32, C.c_uint32, _f32p, _f32p]
        L.orc_fnv1a64.restype = C.c_uint64
        L.orc_fnv1a64.argtypes = [C.c_void_p, C.c_size_t]
        L.orc_fnv1a64_q35test.restype = C.c_uint64
        L.orc_fnv1a64_q35test.argtypes = [C.c_void_p, C.c_size_t]
        L.orc_fnv1a32.restype = C.c_uint32
        L.orc_fnv1a32.argtypes = [C.c_void_p, C.c_size_t]
        L.orc_num_threads.restype = C.c_int
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_uint32, C.c_uint32, C.c_float]
        L.orc_silu.argtypes = [_f32p, _f32p, C.c_size_t]
        L.orc_swiglu.argtypes = [_f32p, _f32p, _f32p, C.c_size_t]
        L.orc_add_inplace.argtypes = [_f32p, _f32p, C.c_size_t]
        L.orc_expf.argtypes = [_f32p, _f32p, C.c_size_t]

    # ---- decoders / quantizer ----
    def lut(self) -> np.ndarray:
        out = np.empty(256, np.float32)
        self.lib.orc_fill_lut(_p(out, _f32p))
        return out

    def f32_to_bf16(self, a: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, np.float32).ravel()
        return np.array([self.lib.orc_f32_to_bf16(float(v)) for v in a], np.uint16)

    def f32_to_e4m3(self, a: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, np.float32).ravel()
        f = self.lib.orc_f32_to_e4m3
        return np.array([f(v) for v in a.tolist()], np.uint8)

    def quantize(self, w: np.ndarray):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        q = np.empty((rows, cols), np.uint8)
        sc = np.empty(((rows + 127) // 128, (cols + 127) // 128), np.uint16)
        self.lib.orc_quantize_fp8(_p(w, _f32p), rows, cols, _p(q, _u8p), _p(sc, _u16p))
        return q, sc

    def dequant(self, W: np.ndarray, sc: np.ndarray) -> np.ndarray:
        W = np.ascontiguousarray(W, np.uint8)
        rows, cols = W.shape
        out = np.empty((rows, cols), np.float32)
        if sc.dtype == np.float32:
            self.lib.orc_dequant_f32scale(_p(W, _u8p), _p(np.ascontiguousarray(sc), _f32p),
                                          rows, cols, _p(out, _f32p))
        else:
            self.lib.orc_dequant(_p(W, _u8p), _p(np.ascontiguousarray(sc, np.uint16), _u16p),
                                 rows, cols, _p(out, _f32p))
        return out

    # ---- matmul ----
    def mm_batch(self, W: np.ndarray, sc: np.ndarray, X: np.ndarray) -> np.ndarray:
        """Y[t][r] = row_r . X[t] with the reference's arithmetic."""
        W = np.ascontiguousarray(W, np.uint8)
        rows, cols = W.shape
        X = np.ascontiguousarray(X, np.float32).reshape(-1, cols)
        n = X.shape[0]
        Y = np.empty((n, rows), np.float32)
        if sc.dtype == np.float32:
            self.lib.orc_mm_fp8_batch_f32scale(_p(W, _u8p), _p(np.ascontiguousarray(sc), _f32p),
                                               rows, cols, n, _p(X, _f32p), _p(Y, _f32p))
        else:
            self.lib.orc_mm_fp8_batch(_p(W, _u8p), _p(np.ascontiguousarray(sc, np.uint16), _u16p),
                                      rows, cols, n, _p(X, _f32p), _p(Y, _f32p))
        return Y

    def mm(self, W, sc, x) -> np.ndarray:
        return self.mm_batch(W, sc, np.asarray(x, np.float32).reshape(1, -1))[0]

    def mm_rows(self, W, sc, X, rows_idx) -> np.ndarray:
        W = np.ascontiguousarray(W, np.uint8)
        rows, cols = W.shape
        X = np.ascontiguousarray(X, np.float32).reshape(-1, cols)
        idx = np.ascontiguousarray(rows_idx, np.uint32)
        Y = np.empty((X.shape[0], idx.size), np.float32)
        self.lib.orc_mm_fp8_rows(_p(W, _u8p), _p(np.ascontiguousarray(sc, np.uint16), _u16p),
                                 rows, cols, X.shape[0], _p(X, _f32p), _p(idx, _u32p),
                                 idx.size, _p(Y, _f32p))
        return Y

    def mm_f64(self, W, sc, X) -> np.ndarray:
        W = np.ascontiguousarray(W, np.uint8)
        rows, cols = W.shape
        X = np.ascontiguousarray(X, np.float32).reshape(-1, cols)
        Y = np.empty((X.shape[0], rows), np.float64)
        self.lib.orc_mm_fp8_f64(_p(W, _u8p), _p(np.ascontiguousarray(sc, np.uint16), _u16p),
                                rows, cols, X.shape[0], _p(X, _f32p), _p(Y, _f64p))
        return Y

    def mm_bf16(self, W16: np.ndarray, x: np.ndarray) -> np.ndarray:
        W16 = np.ascontiguousarray(W16, np.uint16)
        rows, cols = W16.shape
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(rows, np.float32)
        self.lib.orc_mm_bf16(_p(W16, _u16p), rows, cols, _p(x, _f32p), _p(y, _f32p))
        return y

    # ---- MLP neighbours (qwen35-c/src/q35_kern.c) ----
    def rmsnorm(self, X: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
        """Row-wise zero-centred RMSNorm of X [rows][n] (or one vector)."""
        X = np.ascontiguousarray(X, np.float32)
        n = X.shape[-1]
        rows = X.size // n if n else 0
        w = np.ascontiguousarray(w, np.float32)
        assert w.shape == (n,)
        Y = np.empty_like(X)
        if X.size:
            self.lib.orc_rmsnorm(_p(X, _f32p), _p(w, _f32p), _p(Y, _f32p), rows, n, eps)
        return Y

    def silu(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.orc_silu(_p(x, _f32p), _p(y, _f32p), x.size)
        return y

    def swiglu(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        assert g.shape == u.shape
        y = np.empty_like(g)
        self.lib.orc_swiglu(_p(g, _f32p), _p(u, _f32p), _p(y, _f32p), g.size)
        return y

    def add(self, x: np.ndarray, y: np.ndarray) -> np.ndarray:
        """x + y elementwise as the residual update (returns a new array)."""
        out = np.array(x, np.float32, copy=True, order="C")
        y = np.ascontiguousarray(y, np.float32)
        assert out.shape == y.shape
        self.lib.orc_add_inplace(_p(out, _f32p), _p(y, _f32p), out.size)
        return out

    def expf(self, x: np.ndarray) -> np.ndarray:
        """libm expf per element (what the reference's sigmoid calls)."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.orc_expf(_p(x, _f32p), _p(y, _f32p), x.size)
        return y

    def mlp(self, x: np.ndarray, norm_w: np.ndarray, gate, up, down, eps: float = 1e-6) -> np.ndarray:
        """One MLP block on token-major x [m][H]: post-attention RMSNorm,
        gate/up, SwiGLU, down, residual add (qwen35-c/src/q35_model.c:927-939,
        :964-978).  gate/up/down are (codes, bf16 scale) pairs.  Returns the
        new residual stream and the intermediates as a dict."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, norm_w.shape[0])
        xn = self.rmsnorm(x, norm_w, eps)
        g = self.mm_batch(gate[0], gate[1], xn)
        u = self.mm_batch(up[0], up[1], xn)
        mid = self.swiglu(g, u)
        y = self.mm_batch(down[0], down[1], mid)
        return {"xn": xn, "gate": g, "up": u, "mid": mid, "y": y, "out": self.add(x, y)}

    # ---- hashes ----
    def fnv64(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        return int(self.lib.orc_fnv1a64(a.ctypes.data, a.nbytes))

    def fnv64_q35test(self, a: np.ndarray) -> int:
        """The FNV-1a-64 variant the reference mm test prints."""
        a = np.ascontiguousarray(a)
        return int(self.lib.orc_fnv1a64_q35test(a.ctypes.data, a.nbytes))

    def fnv32(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        return int(self.lib.orc_fnv1a32(a.ctypes.data, a.nbytes))

    def threads(self) -> int:
        return int(self.lib.orc_num_threads())


class RefMM:
    """The reference's compiled q35_mm.c (oracle/_ref); None-safe loader."""

    def __init__(self, path: str = REF_PATH):
        self.path = path
        self.lib = L = C.CDLL(path)
        L.q35_mm_init.argtypes = []
        L.q35_mm_e4m3_to_f32.restype = C.c_float
        L.q35_mm_e4m3_to_f32.argtypes = [C.c_uint8]
        L.q35_mm_bf16_to_f32.restype = C.c_float
        L.q35_mm_bf16_to_f32.argtypes = [C.c_uint16]
        L.q35_mm_fp8.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, _f32p, _f32p]
        L.q35_mm_fp8_batch.argtypes = [_u8p, _u16p, C.c_uint32, C.c_uint32, C.c_uint32,
                                       _f32p, _f32p]
        L.q35_mm_fp8_multi4.argtypes = [C.POINTER(_u8p), C.POINTER(_u16p), _u32p,
                                        C.c_uint32, _f32p, C.POINTER(_f32p)]
        L.q35_mm_bf16.argtypes = [_u16p, C.c_uint32, C.c_uint32, _f32p, _f32p]
        L.q35_mm_impl_fp8.restype = C.c_char_p
        L.q35_mm_init()

    @staticmethod
    def available(path: str = REF_PATH) -> bool:
        return os.path.exists(path)

    def impl(self) -> str:
        return self.lib.q35_mm_impl_fp8().decode()

    def lut(self) -> np.ndarray:
        arr = (C.c_float * 256).in_dll(self.lib, "q35_mm_fp8_lut")
        return np.frombuffer(arr, np.float32).copy()

    def mm_batch(self, W, sc, X) -> np.ndarray:
        W = np.ascontiguousarray(W, np.uint8)
        rows, cols = W.shape
        X = np.ascontiguousarray(X, np.float32).reshape(-1, cols)
        Y = np.empty((X.shape[0], rows), np.float32)
        self.lib.q35_mm_fp8_batch(_p(W, _u8p), _p(np.ascontiguousarray(sc, np.uint16), _u16p),
                                  rows, cols, X.shape[0], _p(X, _f32p), _p(Y, _f32p))
        return Y

    def mm(self, W, sc, x) -> np.ndarray:
        W = np.ascontiguousarray(W, np.uint8)
        rows, cols = W.shape
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(rows, np.float32)
        self.lib.q35_mm_fp8(_p(W, _u8p), _p(np.ascontiguousarray(sc, np.uint16), _u16p),
                            rows, cols, _p(x, _f32p), _p(y, _f32p))
        return y

    def mm_bf16(self, W16, x) -> np.ndarray:
        W16 = np.ascontiguousarray(W16, np.uint16)
        rows, cols = W16.shape
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(rows, np.float32)
        self.lib.q35_mm_bf16(_p(W16, _u16p), rows, cols, _p(x, _f32p), _p(y, _f32p))
        return y

    def multi4(self, Ws, scs, x) -> list:
        """q35_mm_fp8_multi4 over up to four weights sharing x
        (qwen35-c/src/q35_mm.c:176-198)."""
        n = len(Ws)
        assert 1 <= n <= 4
        Ws = [np.ascontiguousarray(W, np.uint8) for W in Ws]
        scs = [np.ascontiguousarray(sc, np.uint16) for sc in scs]
        cols = Ws[0].shape[1]
        x = np.ascontiguousarray(x, np.float32)
        ys = [np.empty(W.shape[0], np.float32) for W in Ws]
        wp = (_u8p * 4)(*[_p(W, _u8p) for W in Ws], *[None] * (4 - n))
        sp = (_u16p * 4)(*[_p(sc, _u16p) for sc in scs], *[None] * (4 - n))
        rows = (C.c_uint32 * 4)(*[W.shape[0] for W in Ws], *[0] * (4 - n))
        yp = (_f32p * 4)(*[_p(y, _f32p) for y in ys], *[None] * (4 - n))
        self.lib.q35_mm_fp8_multi4(wp, sp, rows, cols, _p(x, _f32p), yp)
        return ys


class RefKern:
    """The reference's compiled q35_kern.c (oracle/_ref/libq35kern.so)."""

    def __init__(self, path: str = REF_KERN_PATH):
        self.lib = L = C.CDLL(path)
        for nm in ("q35_kern_rmsnorm", "q35_kern_rmsnorm_scalar"):
            getattr(L, nm).argtypes = [_f32p, _f32p, _f32p, C.c_size_t, C.c_float]
        for nm in ("q35_kern_silu", "q35_kern_silu_scalar"):
            getattr(L, nm).argtypes = [_f32p, _f32p, C.c_size_t]
        for nm in ("q35_kern_swiglu", "q35_kern_swiglu_scalar"):
            getattr(L, nm).argtypes = [_f32p, _f32p, _f32p, C.c_size_t]

    @staticmethod
    def available(path: str = REF_KERN_PATH) -> bool:
        return os.path.exists(path)

    def rmsnorm(self, x, w, eps=1e-6, scalar=False) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        y = np.empty_like(x)
        fn = self.lib.q35_kern_rmsnorm_scalar if scalar else self.lib.q35_kern_rmsnorm
        fn(_p(x, _f32p), _p(w, _f32p), _p(y, _f32p), x.size, eps)
        return y

    def silu(self, x, scalar=False) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        fn = self.lib.q35_kern_silu_scalar if scalar else self.lib.q35_kern_silu
        fn(_p(x, _f32p), _p(y, _f32p), x.size)
        return y

    def swiglu(self, g, u, scalar=False) -> np.ndarray:
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        y = np.empty_like(g)
        fn = self.lib.q35_kern_swiglu_scalar if scalar else self.lib.q35_kern_swiglu
        fn(_p(g, _f32p), _p(u, _f32p), _p(y, _f32p), g.size)
        return y
