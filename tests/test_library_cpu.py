"""CPU-side checks of libq35mm.so: it loads, it exports every symbol its
headers declare, and its host-only functions (decoders, LUT, impl name) are
bit-exact.  Nothing here launches a kernel."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT


def header_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(q35\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


HEADERS = [os.path.join(ROOT, "include", "q35", "q35_mm.h"),
           os.path.join(ROOT, "include", "q35mm", "q35mm.h")]


def test_headers_declare_the_reference_entry_points():
    names = header_functions(HEADERS[0])
    for n in ("q35_mm_init", "q35_mm_e4m3_to_f32", "q35_mm_bf16_to_f32", "q35_mm_fp8",
              "q35_mm_fp8_batch", "q35_mm_fp8_multi4", "q35_mm_bf16", "q35_mm_impl_fp8"):
        assert n in names


def test_library_exports_every_declared_symbol(q):
    out = subprocess.run(["nm", "-D", "--defined-only", q.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1]: ln.split()[-2] for ln in out.splitlines() if len(ln.split()) >= 3}
    for h in HEADERS:
        for name in header_functions(h):
            assert exported.get(name) == "T", f"{name} not exported as a function"
    assert exported.get("q35_mm_fp8_lut") in ("B", "D"), "q35_mm_fp8_lut data symbol missing"
    # nothing from the internal namespace leaks except the kernel stubs HIP
    # registers with its runtime
    assert not [n for n in exported if n.startswith("_ZN5q35mm") and "_kernel" not in n]


def test_lut_and_decoders_bit_exact(q, oracle):
    q.lib.q35_mm_init()
    q.lib.q35_mm_init()   # idempotent
    assert (q.lut().view(np.uint32) == oracle.lut().view(np.uint32)).all()
    for c in range(256):
        a = np.float32(q.e4m3_to_f32(c))
        b = np.float32(oracle.lib.orc_e4m3_to_f32(c))
        assert a.view(np.uint32) == b.view(np.uint32), hex(c)
    for bits in (0, 1, 0x3F80, 0x7F80, 0x8000, 0xFF7F, 0x0001, 0x7FC0):
        a = np.float32(q.bf16_to_f32(bits))
        assert a.view(np.uint32) == np.uint32(bits << 16)


def test_lut_is_filled_at_load_without_init():
    # a fresh process that reads the table before any call
    code = ("import ctypes,sys;sys.path.insert(0,%r);import q35mm;"
            "import numpy as np;l=q35mm.lut();print(l[0x38],l[0x7e],np.isnan(l[0x7f]))" %
            os.path.join(ROOT, "qwen38-in-c_amd"))
    out = subprocess.run(["python3", "-c", code], capture_output=True, text=True, check=True).stdout
    assert out.split() == ["1.0", "448.0", "True"]


def test_impl_name(q):
    assert q.impl() == "hip-gfx950"


def test_reference_header_signatures_kept():
    """The drop-in header keeps the reference's parameter lists
    (qwen35-c/include/q35/q35_mm.h:24-45)."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADERS[0]).read(), flags=re.S)
    text = " ".join(text.split())
    for sig in (
        "void q35_mm_fp8(const uint8_t *W, const uint16_t *scale_bf16, uint32_t rows, uint32_t cols, "
        "const float *x, float *y);",
        "void q35_mm_fp8_batch(const uint8_t *W, const uint16_t *scale_bf16, uint32_t rows, uint32_t cols, "
        "uint32_t n, const float *X, float *Y);",
        "void q35_mm_fp8_multi4(const uint8_t *W[4], const uint16_t *sc[4], uint32_t rows[4], uint32_t cols, "
        "const float *x, float *y[4]);",
        "void q35_mm_bf16(const uint16_t *W, uint32_t rows, uint32_t cols, const float *x, float *y);",
        "extern float q35_mm_fp8_lut[256];",
        "float q35_mm_e4m3_to_f32(uint8_t v);",
        "float q35_mm_bf16_to_f32(uint16_t v);",
        "const char *q35_mm_impl_fp8(void);",
        "void q35_mm_init(void);",
    ):
        assert sig in text, sig


def test_device_api_rejects_null_handles(q):
    rc = q.lib.q35mm_matmul(None, 1, None, None, None)
    assert rc < 0
    assert q.lib.q35mm_last_error().decode()


def test_python_wrapper_validates_shapes(q):
    W = np.zeros((10, 20), np.uint8)
    with pytest.raises(q.Q35mmError):
        q.mm_fp8(W, np.zeros((2, 2), np.uint16), np.zeros(20, np.float32))
    with pytest.raises(q.Q35mmError):
        q.mm_fp8(W.astype(np.int8), np.zeros((1, 1), np.uint16), np.zeros(20, np.float32))


def test_lut_seen_by_a_linked_c_caller(q, oracle, tmp_path):
    """A C program linked with -lq35mm (as the reference's model code links
    its matmul) reads q35_mm_fp8_lut through a copy relocation; the table must
    be right before and after q35_mm_init(), and the reference loader's
    nearest-code search over it (qwen35-c/src/q35_model.c:41-57) must pick the
    oracle's codes."""
    import shutil
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    exe = str(tmp_path / "lut_link")
    libdir = os.path.dirname(q.LIB_PATH)
    subprocess.run(["gcc", "-O1", "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "c", "lut_link.c"),
                    "-o", exe, "-L", libdir, "-lq35mm", "-Wl,-rpath," + libdir, "-Wl,-rpath-link,/opt/rocm/lib",
                    "-lm"], check=True, capture_output=True)
    rel = subprocess.run(["readelf", "-r", exe], capture_output=True, text=True, check=True).stdout
    assert "q35_mm_fp8_lut" in rel   # the executable holds the table's copy
    vals = np.array([1.0, -3.3, 0.0017, 500.0, -448.0, 1e-6, 0.0009765625, 0.0029296875, 240.0, 232.0,
                     -0.013671875, 0.0], np.float32)
    out = subprocess.run([exe] + [repr(float(v)) for v in vals], capture_output=True, text=True,
                         check=True).stdout.split("\n")
    want = oracle.lut().view(np.uint32)
    for line, tag in zip(out[:2], ("before", "after")):
        words = line.split()
        assert words[0] == tag
        got = np.array([int(w, 16) for w in words[1:]], np.uint32)
        assert (got == want).all(), f"table {tag} q35_mm_init differs from the oracle"
    codes = [int(c) for c in out[2].split()[1:]]
    assert codes == [int(oracle.lib.orc_f32_to_e4m3(float(v))) for v in vals]
