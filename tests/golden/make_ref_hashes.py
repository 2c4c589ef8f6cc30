"""Writes tests/golden/ref_hashes.json: FNV-1a-64 hashes of the outputs of
the reference's own compiled matmul (oracle/_ref/libq35ref.so, built from
qwen35-c/src/q35_mm.c) on seeded synthetic workloads, together with hashes of
the generated inputs.

The oracle restatement must reproduce these hashes bit for bit; the tests
check that on any machine, with or without the reference tree.  Run here,
where oracle/_ref can be built:

    python tests/golden/make_ref_hashes.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "qwen38-in-c_amd"))

import workload as wl  # noqa: E402
from oracle import Oracle, RefMM  # noqa: E402


def cases():
    """(name, m, k, n, weight kind, activation kwargs, seed)."""
    b = wl.SEED_BASE
    out = [("single_m1_5120x5120", 1, 5120, 5120, "normal", {}, b + 0)]
    for i, (nm, k, n) in enumerate(wl.DECODE_SHAPES):
        for m in (1, 2, 8):
            out.append((f"decode_{nm}_m{m}", m, k, n, "normal", {}, b + 1 + 16 * i))
    out.append(("prefill_m512_5120x256", 512, 5120, 256, "normal", {"bf16": True}, b + 2))
    out.append(("prefill_m512_17408x128", 512, 17408, 128, "normal", {"bf16": True}, b + 3))
    out.append(("ragged_m37_4736x3000", 37, 4736, 3000, "ragged", {"outlier_frac": 0.01}, b + 4))
    out.append(("kpartial_m5_4700x3000", 5, 4700, 3000, "ragged", {"outlier_frac": 0.01}, b + 5))
    out.append(("edge_m3_129x129", 3, 129, 129, "normal", {}, b + 6))
    out.append(("tiny_m1_5x3", 1, 5, 3, "normal", {}, b + 7))
    out.append(("small_n48_m1_5120x48", 1, 5120, 48, "normal", {}, b + 8))
    # The reference's decode projections besides the MLP: DeltaNet in_proj_qkv
    # and in_proj_z (its multi4, qwen35-c/src/q35_deltanet.c:325-329; the 48-row
    # in_proj_a/b are small_n48 above), GQA q and k/v
    # (qwen35-c/src/q35_attn.c:273-275), out_proj / o_proj 6144 -> 5120
    # (qwen35-c/src/q35_deltanet.c:360, qwen35-c/src/q35_attn.c:262).
    for i, (nm, k, n) in enumerate((("dn_qkv", 5120, 10240), ("dn_z", 5120, 6144), ("attn_q", 5120, 12288),
                                    ("attn_kv", 5120, 1024), ("out_proj", 6144, 5120))):
        out.append((f"model_{nm}_m1_{k}x{n}", 1, k, n, "normal", {}, b + 0x20 + i))
    # out_proj / o_proj over a prefill's tokens as one batch instead of the
    # reference's per-token calls (qwen35-c/src/q35_deltanet.c:498,
    # qwen35-c/src/q35_attn.c:262,311): 63 tokens (decode GEMV) and 512
    # (prefill GEMM); activations plain fp32, as those callers pass them.
    out.append(("straggler_m63_6144x5120", 63, 6144, 5120, "normal", {}, b + 0x30))
    out.append(("straggler_m512_6144x5120", 512, 6144, 5120, "normal", {}, b + 0x31))
    return out


def make_inputs(m, k, n, kind, act_kw, seed):
    if kind == "ragged":
        W, sc = wl.gen_weight_ragged(seed, n, k)
    else:
        W, sc = wl.gen_weight(seed, n, k)
    X = wl.gen_act(seed + 0x100, m, k, **act_kw)
    return W, sc, X


def main():
    o = Oracle()
    r = RefMM()
    doc = {"generator": "qwen38-in-c_amd/workload.py (gen_weight / gen_weight_ragged / gen_act)",
           "reference": "oracle/_ref/libq35ref.so = qwen35-c/src/q35_mm.c, gcc -O2 -mavx2 -mfma "
                        "-ffp-contract=off -fopenmp",
           "hash": "FNV-1a-64, standard offset basis, over the little-endian bytes",
           "cases": []}
    for name, m, k, n, kind, act_kw, seed in cases():
        W, sc, X = make_inputs(m, k, n, kind, act_kw, seed)
        Y = r.mm_batch(W, sc, X)
        doc["cases"].append(dict(name=name, m=m, k=k, n=n, kind=kind, act=act_kw, seed=seed,
                                 fnv_codes=f"{o.fnv64(W):016x}", fnv_scales=f"{o.fnv64(sc):016x}",
                                 fnv_x=f"{o.fnv64(X):016x}", fnv_y_ref=f"{o.fnv64(Y):016x}",
                                 y_head=[float(v) for v in Y.ravel()[:4]]))
        print(name, doc["cases"][-1]["fnv_y_ref"], flush=True)
    with open(os.path.join(HERE, "ref_hashes.json"), "w") as f:
        json.dump(doc, f, indent=1)


if __name__ == "__main__":
    main()
