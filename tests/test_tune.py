"""Tuning-cache robustness without a GPU (the reference's
ramvi/engine/tests/legacy/test_f31.py:8-18): a corrupt cache is ignored, a
shape where every candidate fails raises and leaves the cache untouched, and a
good cache is read back into CFG1 / CFGT."""
import json

import pytest

from ai_amd import tune, wcomp


@pytest.fixture
def fake(monkeypatch):
    monkeypatch.setattr(tune, "_device", lambda: "test|gfx950")
    monkeypatch.setattr(tune, "_version", lambda: "v1")
    monkeypatch.setattr(tune, "_sample", lambda N, K, mode: ([None] * 3, None, None))
    return monkeypatch


def test_corrupt_cache_ignored_and_failures_not_cached(fake, tmp_path):
    p = tmp_path / "tune.json"
    p.write_text("{bad")
    fake.setattr(tune, "_try", lambda f: float("inf"))
    logs = []
    tune.tune([], log=logs.append, cache=str(p))
    assert logs
    with pytest.raises(RuntimeError):
        tune.tune([(16, 256, 0)], log=logs.append, cache=str(p))
    assert p.read_text() == "{bad"


def test_results_are_cached_and_read_back(fake, tmp_path):
    p = tmp_path / "tune.json"
    calls = []

    def timing(f):
        calls.append(1)
        return float(len(calls))  # the first candidate of each list is the fastest

    fake.setattr(tune, "_try", timing)
    tune.tune([(4096, 4096, 1)], log=lambda *a: None, cache=str(p))
    d = json.loads(p.read_text())
    assert d["version"] == "v1"
    e = d["entries"]["test|gfx950|(4096, 4096, 1)"]
    assert tuple(e["one"]) == tune.ONE[0] and tuple(e["batch"]) == tune.BATCH[0]
    assert wcomp.CFG1[(4096, 4096, 1)] == tune.ONE[0][:2]
    n = len(calls)
    tune.tune([(4096, 4096, 1)], log=lambda *a: None, cache=str(p))   # from the cache: no timing
    assert len(calls) == n
    fake.setattr(tune, "_version", lambda: "v2")                        # another build: tuned again
    tune.tune([(4096, 4096, 1)], log=lambda *a: None, cache=str(p))
    assert len(calls) > n
    wcomp.CFG1.clear()
    wcomp.CFGT.clear()
