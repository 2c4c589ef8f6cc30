"""The reference's own matmul tests, unchanged, through the drop-in library.

oracle/Makefile compiles qwen35-c/tests/test_mm.c and test_batch_mm.c (the
reference's ctest targets mm and batch_mm, qwen35-c/CMakeLists.txt:76-78,
118-120) against include/q35/q35_mm.h and links them to
qwen38-in-c_amd/lib/libq35mm.so, so every q35_mm_* call they make runs on
the GPU through the C ABI on host pointers:

- test_mm (qwen35-c/tests/test_mm.c:25-90) runs every case of a fixture
  manifest against the reference's float64 .yref at its tolerance (5e-4
  absolute + relative) and prints an FNV-1a hash of the outputs.  It runs
  on tests/golden/mm, the reference's fixtures without qkvlike_fp8 and
  deep_bf16, whose weight files the reference checkout lacks.  The BF16
  case (q35_mm_bf16) is bit-identical to the reference, so its printed hash
  must equal the one the compiled reference prints (manifest fnv_q35test).
- test_batch_mm (qwen35-c/tests/test_batch_mm.c:12-71): q35_mm_fp8_batch of
  5 tokens at 10240 x 5120 must equal five q35_mm_fp8 calls bit for bit,
  and q35_mm_fp8_multi4 the batch's first token; it prints ALL OK.

The binaries are built here and carried to the GPU host beside the library;
a missing binary fails the test (the build step makes them).
"""
import json
import os
import re
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref")
MM_DIR = os.path.join(ROOT, "tests", "golden", "mm")


def _run(name, *args):
    exe = os.path.join(REF, name)
    assert os.path.exists(exe), f"{exe} missing: build() compiles it from the reference's sources"
    print(f"running {name} {' '.join(args)}", flush=True)
    r = subprocess.run([exe, *args], capture_output=True, text=True, timeout=120, cwd=ROOT)
    print(r.stdout, r.stderr, flush=True)
    return r


def test_reference_test_mm_on_fixtures():
    r = _run("test_mm", MM_DIR)
    manifest = json.load(open(os.path.join(MM_DIR, "manifest.json")))
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"{len(manifest)} cases, 0 failed" in r.stdout
    printed = dict(re.findall(r"^ok (\S+) .* fnv=([0-9a-f]{16})", r.stdout, re.M))
    assert sorted(printed) == sorted(c["name"] for c in manifest)
    for c in manifest:
        if not c["fp8"]:
            assert printed[c["name"]] == c["fnv_q35test"], c["name"]


def test_reference_test_batch_mm():
    r = _run("test_batch_mm")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL OK" in r.stdout
    assert "MISMATCH" not in r.stdout
