"""Builds libq35mm.so (HIP kernels + C-ABI host layer) in-tree for gfx950.

    python qwen38-in-c_amd/build.py          # build
    python qwen38-in-c_amd/build.py --asm    # also dump device assembly to _build/

The library is written to qwen38-in-c_amd/lib/libq35mm.so; tests, the
benchmark and the smoke check load it from there.
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


def _run(cmd: list[str]) -> list[str]:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature and says so.
    noise = ("packed-fp32-ops", "is not a recognized feature", "warning: argument unused")
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if ln.strip() and not any(n in ln for n in noise)]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + "\n".join(msgs))
    return msgs


def build_library(verbose: bool = False) -> str:
    """Compiles every source to an object (in parallel) under _build/obj,
    then links lib/libq35mm.so."""
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(ROOT, "_build", "obj")
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(objdir, os.path.basename(s) + ".o") for s in srcs]
    cmds = [[HIPCC, *DEVICE_FLAGS, *COMMON_FLAGS, "-c", "-o", o, s] for s, o in zip(srcs, objs)]
    if verbose:
        for c in cmds:
            print(" ".join(c), flush=True)
    from concurrent.futures import ThreadPoolExecutor
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as ex:
        msgs = [m for ms in ex.map(_run, cmds) for m in ms]
    tmp = LIB + ".tmp"
    msgs += _run([HIPCC, *DEVICE_FLAGS, "-shared", "-fPIC", "-Wl,-Bsymbolic-functions", "-o", tmp, *objs])
    if msgs and verbose:
        print("\n".join(msgs))
    os.replace(tmp, LIB)
    build_host_token()
    return LIB


HOST_TOKEN = os.path.join(LIBDIR, "libq35host_token.so")


def build_host_token() -> str:
    """The benchmark's C driver of host-pointer call sequences
    (host_token.c), linked to lib/libq35mm.so."""
    cc = os.environ.get("CC", "gcc")
    subprocess.run([cc, "-O2", "-std=gnu11", "-fPIC", "-shared", f"-I{os.path.join(ROOT, 'include')}",
                    "-o", HOST_TOKEN, os.path.join(PKG, "host_token.c"), f"-L{LIBDIR}", "-lq35mm",
                    "-Wl,-rpath,$ORIGIN"], check=True)
    return HOST_TOKEN


def dump_asm(outdir: str) -> None:
    os.makedirs(outdir, exist_ok=True)
    for src in glob.glob(os.path.join(CSRC, "*.hip")):
        out = os.path.join(outdir, os.path.basename(src).replace(".hip", ".s"))
        subprocess.run([HIPCC, *DEVICE_FLAGS, *COMMON_FLAGS, "--cuda-device-only", "-S", "-o", out, src],
                       check=True, capture_output=True)


if __name__ == "__main__":
    print(build_library(verbose=True))
    if "--asm" in sys.argv:
        dump_asm(os.path.join(ROOT, "_build", "asm"))
