"""Copies the reference's RMSNorm / SiLU / SwiGLU fixtures (data only) from
qwen35-c/tests/fixtures/kern/ into tests/golden/kern/ and writes
manifest.json: the reference manifest's fields for those cases plus
`fnv1a_ref`, the FNV-1a-32 of the fp32 output of the reference's own
compiled q35_kern.c (oracle/_ref/libq35kern.so) on the fixture inputs, so the
oracle's bit equality with the reference is checked on any machine.

Run where the reference tree and oracle/_ref exist:

    python tests/golden/copy_kern_fixtures.py
"""
from __future__ import annotations

import json
import os
import shutil
import sys
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SRC = "/root/reference/qwen35-c/tests/fixtures/kern"
DST = os.path.join(HERE, "kern")
CASES = ("rmsnorm_5120", "silu_17408", "swiglu_17408")

sys.path.insert(0, os.path.join(ROOT, "oracle"))
from oracle import Oracle, RefKern  # noqa: E402


def parse_manifest(path):
    out = {}
    for line in open(path):
        line = line.strip()
        if not line or line.startswith("#"):
            continue
        name, *kv = line.split()
        out[name] = dict(x.split("=", 1) for x in kv)
    return out


def main():
    man = parse_manifest(os.path.join(SRC, "manifest.txt"))
    os.makedirs(DST, exist_ok=True)
    ref = RefKern()
    orc = Oracle()
    res = {}
    for name in CASES:
        c = man[name]
        ins = c["in"].split(",")
        for f in ins + [c["out"]]:
            shutil.copyfile(os.path.join(SRC, f), os.path.join(DST, f))
        out_bytes = open(os.path.join(DST, c["out"]), "rb").read()
        assert "%08x" % (zlib.crc32(out_bytes) & 0xFFFFFFFF) == c["crc32"], name
        arrs = [np.fromfile(os.path.join(DST, f), np.float32) for f in ins]
        if c["kernel"] == "rmsnorm":
            y = ref.rmsnorm(arrs[0], arrs[1], float(c["eps"]))
        elif c["kernel"] == "silu":
            y = ref.silu(arrs[0])
        else:
            y = ref.swiglu(arrs[0], arrs[1])
        res[name] = {
            "kernel": c["kernel"], "in": ins, "out": c["out"], "n": int(c["n"]),
            "atol": float(c["atol"]), "rtol": float(c["rtol"]), "crc32": c["crc32"],
            **({"eps": float(c["eps"])} if "eps" in c else {}),
            "fnv1a_ref": "%08x" % orc.fnv32(y),
        }
    with open(os.path.join(DST, "manifest.json"), "w") as f:
        json.dump(res, f, indent=1, sort_keys=True)
        f.write("\n")
    print(json.dumps(res, indent=1))


if __name__ == "__main__":
    main()
