import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen38-in-c_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ORACLE_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: large inputs (seconds of CPU oracle time)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    """The reference's own compiled q35_mm.c (oracle/_ref), when built."""
    from oracle import RefMM
    if not RefMM.available():
        pytest.skip("oracle/_ref not built (reference tree absent when built)")
    return RefMM()


@pytest.fixture(scope="session")
def refkern():
    """The reference's own compiled q35_kern.c (oracle/_ref), when built."""
    from oracle import RefKern
    if not RefKern.available():
        pytest.skip("oracle/_ref not built (reference tree absent when built)")
    return RefKern()


@pytest.fixture(scope="session")
def q():
    import q35mm
    return q35mm


@pytest.fixture(scope="session")
def wl():
    import workload
    return workload


@pytest.fixture(scope="session")
def gpu():
    if not gpu_available():
        pytest.skip("no GPU visible")
    import torch
    return torch.device("cuda:0")


def load_fixture(name: str):
    """A reference mm fixture from tests/golden/mm (copied data files of
    qwen35-c/tests/fixtures/mm)."""
    man = {c["name"]: c for c in json.load(open(os.path.join(GOLDEN, "mm", "manifest.json")))}
    c = man[name]
    d = os.path.join(GOLDEN, "mm", name)
    x = np.fromfile(d + ".x", np.float32)
    yref = np.fromfile(d + ".yref", np.float64)
    if c["fp8"]:
        W = np.fromfile(d + ".w8", np.uint8).reshape(c["rows"], c["cols"])
        sc = np.fromfile(d + ".sc", np.uint16).reshape(c["sr"], c["sc"])
        return c, W, sc, x, yref
    W = np.fromfile(d + ".w16", np.uint16).reshape(c["rows"], c["cols"])
    return c, W, None, x, yref


def fixture_names(fp8=True):
    man = json.load(open(os.path.join(GOLDEN, "mm", "manifest.json")))
    return [c["name"] for c in man if c["fp8"] == fp8]


def kern_manifest():
    return json.load(open(os.path.join(GOLDEN, "kern", "manifest.json")))


def load_kern_fixture(name: str):
    """(case, inputs, expected) of a reference kernel fixture copied to
    tests/golden/kern (qwen35-c/tests/fixtures/kern)."""
    c = kern_manifest()[name]
    d = os.path.join(GOLDEN, "kern")
    ins = [np.fromfile(os.path.join(d, f), np.float32) for f in c["in"]]
    return c, ins, np.fromfile(os.path.join(d, c["out"]), np.float32)


def within_kern_tol(y, yref, atol, rtol) -> bool:
    """The reference kernel test's acceptance rule
    (qwen35-c/tests/test_kern.c:112-121): |y - ref| <= atol + rtol*|ref|."""
    y = np.asarray(y, np.float64)
    yref = np.asarray(yref, np.float64)
    return bool((np.abs(y - yref) <= atol + rtol * np.abs(yref)).all())


def goldens():
    return json.load(open(os.path.join(GOLDEN, "ref_hashes.json")))


def unit_scale_act(X, k: int, std: float = 0.02):
    """X times the power of two 2^-e, e = max(0, ceil(log2(std * sqrt(k)))):
    with weights ~N(0, std^2), outputs of K = k terms then have an RMS of at
    most 1, the scale the GEMM's absolute max-error bar is stated for.  The
    factor is exact (bf16-representable activations stay so) and leaves every
    relative error unchanged."""
    e = max(0, int(np.ceil(np.log2(std * np.sqrt(k)))))
    return np.ascontiguousarray(X * np.float32(2.0 ** -e)) if e else X


def normwise_rel(y, yref) -> float:
    """||y - yref||_inf / ||yref||_inf in float64."""
    y = np.asarray(y, np.float64)
    yref = np.asarray(yref, np.float64)
    den = np.abs(yref).max()
    return float(np.abs(y - yref).max() / (den if den > 0 else 1.0))
