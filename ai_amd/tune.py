"""Launch-shape autotuning for the fused decode-linear, per (N, K, MODE).

Mirrors ramvi/engine/ramvi_engine/planning/tune.py:21-88: each candidate is
timed as the median of 8 HIP-graph replays over three distinct random
matrices (beyond the caches), the best one per shape goes into
`wcomp.CFG1` (one token) and `wcomp.CFGT` (16 tokens) as the reference's
(BN, w) / (BN, w, S) tuples, and the results are kept in a JSON cache keyed
by the library build, torch, and the device, so later runs read them back.
A corrupt cache is ignored; a shape for which no candidate runs raises
RuntimeError and is not cached (ramvi/engine/tests/legacy/test_f31.py:8-18).

    from ai_amd import tune
    tune.tune([(6144, 4096, 0), (4096, 4096, 1), (24576, 4096, 0), (4096, 12288, 2)])
"""
import hashlib
import json
import math
import os
import statistics
import tempfile

import torch

from . import wcomp
from .wcomp import compress, gemvc1, gemvc_tc

CACHE = os.environ.get("RV12_TUNE_CACHE", os.path.join(os.path.expanduser("~"), ".cache", "ai_amd", "tune.json"))

# candidates: BN = rows per workgroup (row blocks of 16), w = waves per workgroup, S = K splits
ONE = [(bn, w, s) for bn in (16, 32) for w in (4, 8, 16) for s in (1, 2, 4) if not (bn == 32 and w == 16)]
BATCH = [(16 * rbw * w, w, 0) for rbw in (1, 2) for w in (4, 8)]


def _bench(f, n=8):
    f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        f()
    g.replay()
    torch.cuda.synchronize()
    r = []
    for _ in range(n):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        g.replay()
        e.record()
        torch.cuda.synchronize()
        r.append(s.elapsed_time(e))
    return statistics.median(r)


def _try(f):
    try:
        return _bench(f)
    except Exception:
        return float("inf")


def _sample(N, K, mode):
    """Three distinct random matrices of the shape (compressed, packed) and
    16 activation / output rows."""
    cs = [wcomp.compact(compress((torch.randn(N, K, device="cuda") * 0.02).bfloat16())) for _ in range(3)]
    x = torch.randn(16, K * (2 if mode == 2 else 1), device="cuda")
    y = torch.zeros(16, N, device="cuda")
    return cs, x, y


def _version():
    """The library build and this module's Python mirror, and torch."""
    h = hashlib.sha256()
    from . import _lib
    for p in (_lib.LIB_PATH, wcomp.__file__):
        try:
            h.update(open(p, "rb").read())
        except OSError:
            h.update(p.encode())
    return h.hexdigest() + "|" + torch.__version__


def _device():
    p = torch.cuda.get_device_properties(torch.cuda.current_device())
    return f"{p.name}|{getattr(p, 'gcnArchName', '')}"


def _load(path, version, log):
    try:
        if not os.path.exists(path):
            return {}
        with open(path, encoding="utf-8") as h:
            cached = json.load(h)
        db = cached.get("entries", {}) if isinstance(cached, dict) and cached.get("version") == version else {}
        return db if isinstance(db, dict) else {}
    except (ValueError, OSError):
        log("tuning cache unreadable; tuning again")
        return {}


def tune(shapes, log=print, cache=None):
    """shapes: list of (N, K, MODE).  Fills wcomp.CFG1 and wcomp.CFGT."""
    cache = cache or CACHE
    dev = _device()
    version = _version()
    db = _load(cache, version, log)
    todo = [s for s in shapes if f"{dev}|{tuple(s)}" not in db]
    for N, K, mode in todo:
        log(f"  tuning {N}x{K} (mode {mode})...")
        cs, x, y = _sample(N, K, mode)
        r1 = min(((_try(lambda: [gemvc1(x[:1], c, y[:1], mode, bn, w) if s == 1 else
                                 gemvc_tc(x[:1], c, y[:1], mode, 1, bn, w, s) for c in cs]), bn, w, s)
                  for bn, w, s in ONE if N % bn == 0), default=(float("inf"),))
        rt = min(((_try(lambda: [gemvc_tc(x, c, y, mode, 16, bn, w, s or None) for c in cs]), bn, w, s)
                  for bn, w, s in BATCH if N % bn == 0), default=(float("inf"),))
        if not math.isfinite(r1[0]) or not math.isfinite(rt[0]):
            raise RuntimeError(f"no working launch shape for {N}x{K}")
        db[f"{dev}|{(N, K, mode)}"] = {"one": list(r1[1:]), "batch": list(rt[1:])}
        del cs
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
    if todo:
        os.makedirs(os.path.dirname(cache), exist_ok=True)
        tmp = None
        try:
            with tempfile.NamedTemporaryFile("w", dir=os.path.dirname(cache), delete=False) as h:
                tmp = h.name
                json.dump({"version": version, "entries": db}, h, indent=1)
            os.replace(tmp, cache)
        finally:
            if tmp and os.path.exists(tmp):
                os.unlink(tmp)
    for N, K, mode in shapes:
        d = db[f"{dev}|{(N, K, mode)}"]
        bn, w, s = d["one"]
        wcomp.CFG1[(N, K, mode)] = (bn, w) if s == 1 else (bn, w, s)
        bn, w, s = d["batch"]
        wcomp.CFGT[(N, K, mode)] = (bn, w, s or None)
