"""The tuner's cache contract without a GPU (the reference's
ramvi/engine/tests/legacy/test_f31.py:8-18): an unreadable cache is reported
and ignored, a shape for which every candidate fails raises and leaves the
cache untouched, and measured results are cached per library + device and
read back into CFG1 / CFGT in the reference's (BN, w, S) format."""
import json

import pytest

from ai_amd import tune, wcomp

VEC = [(1, 1, 8, 1), (1, 2, 8, 1), (1, 1, 4, 2)]
MFMA = [(2, 2, 8, 1), (2, 1, 4, 1)]


@pytest.fixture
def fake(monkeypatch):
    monkeypatch.setattr(tune, "_identity", lambda: "lib0|gfx950|test")
    monkeypatch.setattr(tune, "candidates", lambda N, K, T: VEC if T == 1 else MFMA)
    yield monkeypatch
    wcomp.CFG1.clear()
    wcomp.CFGT.clear()


def test_unreadable_cache_ignored_and_failures_not_cached(fake, tmp_path):
    p = tmp_path / "tune.json"
    p.write_text("{bad")
    fake.setattr(tune, "_measure", lambda N, K, mode, T, shp, mb, reps, rms=False: {s: float("inf") for s in shp})
    logs = []
    tune.tune([], log=logs.append, cache=str(p))
    assert logs and "ignoring" in logs[0]
    with pytest.raises(RuntimeError):
        tune.tune([(16, 256, 0)], log=logs.append, cache=str(p))
    assert p.read_text() == "{bad"


def test_fastest_shape_cached_and_read_back(fake, tmp_path):
    p = tmp_path / "tune.json"
    calls = []

    def measure(N, K, mode, T, shp, mb, reps, rms=False):
        calls.append(T)
        # the last candidate is the fastest; a failing one never wins
        return {s: (float("inf") if i == 0 else 10.0 - i) for i, s in enumerate(shp)}

    fake.setattr(tune, "_measure", measure)
    tune.tune([(4096, 4096, 1)], log=lambda *a: None, cache=str(p))
    d = json.loads(p.read_text())
    assert d["identity"] == "lib0|gfx950|test"
    e = d["entries"]["4096x4096|1"]
    assert tuple(e["one"]) == VEC[-1] and tuple(e["batch"]) == MFMA[-1]
    assert wcomp.CFG1[(4096, 4096, 1)] == (16, 4, 2)          # BN = 16 rows, 4 waves, 2 splits
    assert wcomp.CFGT[(4096, 4096, 1)] == (16 * 1 * 4, 4, 1)   # BN = row blocks per wave x waves x 16
    n = len(calls)
    tune.tune([(4096, 4096, 1)], log=lambda *a: None, cache=str(p))   # from the cache
    assert len(calls) == n
    fake.setattr(tune, "_identity", lambda: "lib1|gfx950|test")        # a rebuilt library measures again
    tune.tune([(4096, 4096, 1)], log=lambda *a: None, cache=str(p))
    assert len(calls) > n


def test_reference_cfg_maps_back_to_the_shape():
    """wcomp._launch turns the stored (BN, w, S) back into the tuned shape."""
    for shape, T in ((VEC[1], 1), (VEC[2], 1), (MFMA[0], 16), (MFMA[1], 16), ((3, 2, 8, 1), 8), ((3, 1, 4, 3), 4)):
        bn, w, s = tune.as_reference_cfg(shape)
        c = wcomp._launch(bn, w, s, T)
        assert (c.kernel, c.rb, c.waves, c.splits) == shape


def test_rms_shapes_measured_with_the_prologue_and_cached_apart(fake, tmp_path):
    """A shape with rms=True is timed with the RMSNorm prologue and cached
    under its own key; the plain shape of the same (N, K, MODE) is another
    entry."""
    p = tmp_path / "tune.json"
    seen = []

    def measure(N, K, mode, T, shp, mb, reps, rms=False):
        seen.append((N, K, mode, T, rms))
        return {s: 10.0 - i for i, s in enumerate(shp)}

    fake.setattr(tune, "_measure", measure)
    out = tune.tune([(6144, 4096, 0, True), (4096, 12288, 2)], log=lambda *a: None, cache=str(p))
    assert (6144, 4096, 0, True, 1) in [s[:3] + (s[4], s[3]) for s in seen]
    assert all(r for N, K, m, T, r in seen if N == 6144) and not any(r for N, K, m, T, r in seen if N == 4096)
    d = json.loads(p.read_text())
    assert set(d["entries"]) == {"6144x4096|0|rms", "4096x12288|2"}
    assert (6144, 4096, 0, True) in out and (4096, 12288, 2) in out
    n = len(seen)
    tune.tune([(6144, 4096, 0)], log=lambda *a: None, cache=str(p))  # the plain shape is measured on its own
    assert len(seen) > n
    assert set(json.loads(p.read_text())["entries"]) == {"6144x4096|0|rms", "4096x12288|2", "6144x4096|0"}
