"""Builds libq35mm.so (HIP kernels + C-ABI host layer) in-tree for gfx950.

    python qwen38-in-c_amd/build.py          # build
    python qwen38-in-c_amd/build.py --asm    # also dump device assembly to _build/

The library is written to qwen38-in-c_amd/lib/libq35mm.so; tests, the
benchmark and the smoke check load it from there.  The ceiling probe
(probes/q35mm_probe.hip: raw weight-read rate, MFMA issue rate) is built
beside it as lib/q35mm_probe.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libq35mm.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed fp32 math (v_pk_*_f32) is disabled for all device code.
DEVICE_FLAGS = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
                f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + sorted(glob.glob(os.path.join(CSRC, "*.cpp")))


def build_library(verbose: bool = False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *DEVICE_FLAGS, *COMMON_FLAGS, "-shared", "-Wl,-Bsymbolic-functions", "-o", tmp, *sources()]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature and says so.
    noise = ("packed-fp32-ops", "is not a recognized feature", "warning: argument unused")
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if ln.strip() and not any(n in ln for n in noise)]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if msgs and verbose:
        print("\n".join(msgs))
    os.replace(tmp, LIB)
    return LIB


PROBE_SRC = os.path.join(PKG, "probes", "q35mm_probe.hip")
PROBE = os.path.join(LIBDIR, "q35mm_probe")


def build_probe(verbose: bool = False) -> str:
    """The ceiling probe (raw weight reads, MFMA issue rate): a separate
    executable, not part of the library."""
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = PROBE + ".tmp"
    cmd = [HIPCC, *DEVICE_FLAGS, "-O3", "-std=c++17", "-o", tmp, PROBE_SRC]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed on the probe:\n" + res.stdout + res.stderr)
    os.replace(tmp, PROBE)
    return PROBE


def dump_asm(outdir: str) -> None:
    os.makedirs(outdir, exist_ok=True)
    for src in glob.glob(os.path.join(CSRC, "*.hip")):
        out = os.path.join(outdir, os.path.basename(src).replace(".hip", ".s"))
        subprocess.run([HIPCC, *DEVICE_FLAGS, *COMMON_FLAGS, "--cuda-device-only", "-S", "-o", out, src],
                       check=True, capture_output=True)


if __name__ == "__main__":
    print(build_library(verbose=True))
    print(build_probe())
    if "--asm" in sys.argv:
        dump_asm(os.path.join(ROOT, "_build", "asm"))
