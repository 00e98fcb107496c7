"""Launch-shape tuning of the fused decode-linear on the device it runs on.

For each linear (N, K, MODE) of a model the tuner measures the library's own
launch space (rv12_launch: kernel, row blocks, waves, K splits) and stores the
fastest shape in `wcomp.CFG1` (one token, the decode step) and `wcomp.CFGT`
(16 tokens, the batched pass), in the reference's value format
(ramvi/engine/ramvi_engine/kernels/wcomp.py:115, 222: (BN, w) or (BN, w, S)).
A shape may carry a fourth entry, rms: True times every candidate with the
RMSNorm prologue the engine fuses into that linear (a bf16 weight vector),
since the prologue moves the best launch shape; MODE 2 is always timed with
its silu(g) * u prologue.  The engine tunes its four layer linears with the
prologues it runs them with (Engine(tune=True), as the reference's engine
does at load, core/engine.py:207-208).

Measurement.  The MI355X keeps 256 MB in its memory-side cache, more than any
single Qwen3 matrix, so a shape is timed over distinct matrices that together
exceed `min_bytes` (1 GiB by default), launched back to back from one HIP
graph and replayed; the time per launch is the replays' total over the
launches (HIP events on the graph's stream).  Every candidate's output is
compared with the built-in shape's before it may win.

Cache.  Results go to a JSON file keyed by the library binary's sha256, the
GPU architecture and the device name, so a rebuilt library or another GPU
measures again.  The tuning contract of the reference
(ramvi/engine/tests/legacy/test_f31.py:8-18) holds: an unreadable cache is
reported and ignored, and a shape for which no candidate runs raises
RuntimeError and leaves the cache file untouched.

    from ai_amd import tune
    tune.tune([(6144, 4096, 0), (4096, 4096, 1), (24576, 4096, 0), (4096, 12288, 2)])
"""
import hashlib
import json
import math
import os

from . import _lib, wcomp

CACHE = os.environ.get("RV12_TUNE_CACHE", os.path.join(os.path.expanduser("~"), ".cache", "ai_amd", "tune.json"))
TOKENS = {"one": 1, "batch": 16}

_ident = None


def _identity():
    """Key of the measurements: library binary, GPU architecture, device."""
    global _ident
    if _ident is None:
        import torch
        h = hashlib.sha256(open(_lib.LIB_PATH, "rb").read()).hexdigest()[:16]
        p = torch.cuda.get_device_properties(0)
        _ident = f"{h}|{getattr(p, 'gcnArchName', '?')}|{p.name}"
    return _ident


def candidates(N, K, T):
    """The launch shapes to measure for N x K at T tokens, as (kernel, rb,
    waves, splits), the built-in one first; every entry is one the library
    accepts (rv12_launch_shape)."""
    L = _lib.lib()
    nsteps = K // 32
    raw = [(0, 0, 0, 0)]
    if T <= 2:
        raw += [(1, rb, w, s) for rb in (1, 2) for w in (4, 8, 16) for s in (0, 2, 3, 4)]
    else:
        raw += [(2, rb, w, 0) for rb in (1, 2, 4) for w in (4, 8)]
        # kernel 3 with fewer row blocks than waves (as_reference_cfg tells
        # the two MFMA kernels apart by BN < 16 waves)
        raw += [(3, rb, w, s) for rb in (1, 2, 4) for w in (4, 8) if rb < w for s in (0, 2)]
    out = []
    for c in raw:
        if c[3] > nsteps:
            continue
        r = _lib.Launch()
        if L.rv12_launch_shape(N, K, T, _lib.Launch(*c), r) == 0:
            shape = (r.kernel, r.rb, r.waves, r.splits)
            if shape not in out:
                out.append(shape)
    return out


def as_reference_cfg(shape):
    """(kernel, rb, waves, splits) -> the reference's (BN, w, S): BN rows per
    workgroup, w waves, S K splits (wcomp._launch maps it back)."""
    kernel, rb, waves, splits = shape
    bn = 16 * rb if kernel in (1, 3) else 16 * rb * waves
    return (bn, waves, splits)


def _measure(N, K, mode, T, shapes, min_bytes, reps, rms=False):
    """us per launch of every shape (inf where it fails or disagrees with the
    built-in shape's output), over distinct random matrices of > min_bytes;
    rms: with the RMSNorm prologue (a bf16 weight vector of K entries)."""
    import ctypes

    import torch
    dev = torch.device("cuda")
    L = _lib.lib()
    copies = max(2, math.ceil(min_bytes / (1.5 * N * K)))
    g = torch.Generator(device=dev).manual_seed(N * 31 + K)
    mats = []
    for _ in range(copies):
        w = torch.randn(N, K, device=dev, generator=g).mul_(0.02).bfloat16()
        mats.append(wcomp.compact(wcomp.compress(w)))
        del w
    xs = 2 * K if mode == 2 else K
    x = torch.randn(T, xs, device=dev, generator=g).bfloat16().float()
    y = torch.zeros(T, N, device=dev)
    lnw = (torch.rand(K, device=dev, generator=g) + 0.5).bfloat16() if rms else None
    st = torch.cuda.current_stream()
    mstructs = [wcomp._matrix(c) for c in mats]
    times, ref = {}, None
    for shape in shapes:
        cfg = _lib.Launch(*shape)
        need = max(16, L.rv12_workspace_bytes(N, K, T, shape[3]))
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        p = lambda t: ctypes.c_void_p(t.data_ptr())

        def launches():
            for m in mstructs:
                rc = L.rv12_gemm(ctypes.byref(m), p(x), p(y), T, None if lnw is None else p(lnw), 1e-6, mode,
                                 ctypes.byref(cfg), p(ws), need,
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                if rc:
                    raise ValueError(_lib.strerror(rc))

        try:
            y.zero_()
            launches()
            torch.cuda.synchronize()
            out = y.clone()
            if ref is None:
                ref = out
            elif not torch.allclose(out, ref, rtol=1e-3, atol=1e-3):
                times[shape] = float("inf")
                continue
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                launches()
            graph.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            for _ in range(reps):
                graph.replay()
            e1.record(st)
            torch.cuda.synchronize()
            times[shape] = e0.elapsed_time(e1) * 1e3 / (reps * copies)
            del graph
        except (ValueError, RuntimeError):
            times[shape] = float("inf")
    del mats
    torch.cuda.empty_cache()
    return times


def _read(path, log):
    try:
        with open(path) as f:
            d = json.load(f)
        if isinstance(d, dict) and isinstance(d.get("entries"), dict):
            return d
        log(f"tune: ignoring {path}: not a tuning cache")
    except FileNotFoundError:
        pass
    except (OSError, ValueError) as e:
        log(f"tune: ignoring unreadable cache {path}: {e}")
    return None


def _write(path, d):
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    tmp = f"{path}.{os.getpid()}.part"
    with open(tmp, "w") as f:
        json.dump(d, f, indent=1, sort_keys=True)
    os.replace(tmp, path)


def _key(N, K, mode, rms):
    return f"{N}x{K}|{mode}" + ("|rms" if rms else "")


def tune(shapes, log=print, cache=None, min_bytes=1 << 30, reps=10):
    """Fill wcomp.CFG1 / CFGT for every (N, K, MODE) or (N, K, MODE, rms) in
    shapes, from the cache where it holds this library and device, else by
    measurement (with the RMSNorm prologue where rms is true)."""
    path = cache or CACHE
    stored = _read(path, log)
    ident = _identity()
    entries = dict(stored["entries"]) if stored and stored.get("identity") == ident else {}
    changed = False
    shapes = [tuple(s) + (False,) * (4 - len(s)) for s in shapes]
    for N, K, mode, rms in shapes:
        key = _key(N, K, mode, rms)
        e = entries.get(key)
        if e is None:
            e = {}
            for name, T in TOKENS.items():
                shp = candidates(N, K, T)
                t = _measure(N, K, mode, T, shp, min_bytes, reps, rms=bool(rms)) if shp else {}
                good = {s: v for s, v in t.items() if math.isfinite(v)}
                if not good:
                    raise RuntimeError(f"tune: no launch shape runs for {N}x{K} mode {mode} at {T} tokens")
                best = min(good, key=good.get)
                e[name] = list(best)
                log(f"tune: {N}x{K} mode {mode}{' rms' if rms else ''} {T} tok: {best} {good[best]:.2f} us "
                    f"(built-in {t.get(shp[0], float('inf')):.2f} us)")
            entries[key] = e
            changed = True
        wcomp.CFG1[(N, K, mode)] = as_reference_cfg(tuple(e["one"]))
        wcomp.CFGT[(N, K, mode)] = as_reference_cfg(tuple(e["batch"]))
    if changed:
        _write(path, {"identity": ident, "entries": entries})
    return {k[:3] if not k[3] else k: entries[_key(*k)] for k in shapes}
