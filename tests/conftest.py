"""Shared test setup: the `gpu` marker, repo-root imports, and the golden-fixture reader."""
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_golden(name):
    """Reads a reference fixture (<name>.json manifest + <name>.bin float32 LE), the format of the reference's
    tools/autograd_oracle.py:22-33; returns {tensor name: float32 array}."""
    with open(os.path.join(GOLDEN, name + ".json")) as f:
        man = json.load(f)
    flat = np.fromfile(os.path.join(GOLDEN, name + ".bin"), dtype="<f4")
    out = {}
    for k, v in man["tensors"].items():
        n = int(np.prod(v["shape"])) if v["shape"] else 1
        out[k] = flat[v["offset"]:v["offset"] + n].reshape(v["shape"]).astype(np.float32)
    return out


def scaled(a, b, floor=1e-12):
    """Scaled error max|a-b| / max(max|b|, floor) (tests/OneModel.Tests/Tensors/AutogradModelTests.cs:20-30)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))) if b.size else 0.0, floor)) if b.size else 0.0


@pytest.fixture(scope="session")
def oracle():
    from oracle import tape
    tape.lib()
    return tape
