import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "codec_golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X")


@pytest.fixture(scope="session")
def golden():
    z = np.load(GOLDEN)
    cases = {}
    for name in z["names"]:
        name = str(name)
        d = {k: z[f"{name}/{k}"] for k in ("w", "m8", "e4", "rp", "er", "ec", "ev", "dec")}
        d["base"] = int(z[f"{name}/base"])
        d["ch"] = int(z[f"{name}/ch"])
        cases[name] = d
    return cases


def ref_dict(g):
    """Golden codec dict in the reference's key layout (numpy arrays)."""
    N, K = g["w"].shape
    return {"m8": g["m8"], "e4": g["e4"], "base": g["base"], "rp": g["rp"], "er": g["er"], "ec": g["ec"],
            "ev": g["ev"], "N": N, "K": K, "CH": g["ch"]}


def same_bf16(a, b):
    """bit-exact equality of bf16 bit arrays, with any NaN equal to any NaN"""
    a = np.asarray(a, np.uint16)
    b = np.asarray(b, np.uint16)
    na = ((a & 0x7F80) == 0x7F80) & ((a & 0x7F) != 0)
    nb = ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb]))
