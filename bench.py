"""Benchmark: fused 12-bit decode + GEMV over the Qwen3-8B linear layers on one MI355X.

Workload (the isolated kernel sweep the headline GB/s is quoted on): every
Qwen3-8B linear of one decode token at batch 1 — 36 layers x {qkv 6144x4096
(RMSNorm prologue), o 4096x4096 (accumulate), gu 24576x4096 (RMSNorm
prologue), down 4096x12288 (silu(g)*u prologue, accumulate)} + lm_head
151936x4096 — 145 distinct matrices, 11.35 GB of 12-bit weights, random bf16
weights N(0, sigma), sigma ~ U(0.01, 0.05) per matrix, 0.1% of output rows
scaled x20, packed with the 12-bit codec; activations N(0, 1) rounded to bf16.
A step is one pass over all 145 matrices, replayed from a HIP graph, inputs
resident in HBM.  The working set (11.35 GB) is far above the 256 MB Infinity
Cache, so every step streams from HBM.

value = compressed-weight bytes per step (the reference codec's sizes:
1.5 N K + 12 E + 4 (N + 1) per matrix) / step time, in GB/s.

    python bench.py [--steps K] [--warmup W] [--only SHAPE] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM = 8000.0  # GB/s, MI355X HBM3E
# HBM bytes per launch of the dominant kernel (vector-FMA linear over the 144
# layer matrices of a Qwen3-8B token, mean per launch) from the rocprofv3
# FETCH_SIZE and WRITE_SIZE counters, each scaled by what it reads for a 1 GiB
# device copy (--copy-calibration): profiles/k_gemv_qwen3-8b_token.md
TRAFFIC_BYTES_PER_LAUNCH = 73326808
D, FF, L, V = 4096, 12288, 36, 151936
QKV = (32 + 2 * 8) * 128
LAYER = [("qkv", QKV, D, 0, True), ("o", D, 32 * 128, 1, False), ("gu", 2 * FF, D, 0, True),
         ("down", D, FF, 2, False)]
# Qwen3-14B skinny-GEMM shapes (N, K): fused as the engine runs them, and unfused
SWEEP_14B = {"qkv": (7168, 5120), "o": (5120, 5120), "gu": (34816, 5120), "down": (5120, 17408),
             "q": (5120, 5120), "k_v": (1024, 5120), "gate_up": (17408, 5120)}
SWEEP_M = (1, 2, 4, 8, 16)
PEAK_BF16 = 2500.0  # TFLOP/s, MI355X dense bf16 MFMA
SWEEP = {"q_o": (4096, 4096, 0), "k_v": (1024, 4096, 0), "gate_up": (12288, 4096, 0),
         "down": (4096, 12288, 0), "lm_head": (151936, 4096, 0), "qkv": (6144, 4096, 0),
         "gu": (24576, 4096, 0)}


def make_matrix(N, K, gen, dev, outliers="rows"):
    """N(0, sigma) bf16 weights, sigma ~ U(0.01, 0.05), with 0.1 % of the
    output rows (or of the input columns) x20."""
    sigma = float(torch.empty(1).uniform_(0.01, 0.05, generator=gen))
    seed = int(torch.randint(0, 2**31 - 1, (1,), generator=gen))
    w = torch.randn(N, K, device=dev, generator=torch.Generator(device=dev).manual_seed(seed))
    w.mul_(sigma)
    if outliers == "rows":
        rows = torch.randperm(N, generator=gen)[: max(1, N // 1000)].to(dev)
        w[rows] *= 20
    else:
        cols = torch.randperm(K, generator=gen)[: max(1, K // 1000)].to(dev)
        w[:, cols] *= 20
    return w.bfloat16()


def comp_bytes(c):
    N, K = c["N"], c["K"]
    return int(1.5 * N * K) + 12 * int(c["er"].numel()) + 4 * (N + 1)


def alg_bytes(c, mode, rms, T=1):
    """Algorithmic bytes of one call: weights + exceptions + activations
    (+ lnw) + outputs (read and written when accumulating)."""
    N, K = c["N"], c["K"]
    kin = 2 * K if mode == 2 else K
    return comp_bytes(c) + T * kin * 4 + (2 * K if rms else 0) + T * N * 4 * (2 if mode else 1)


class Graph:
    """Capture a list of launches once, replay it as one unit."""

    def __init__(self, fn):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.g):
            fn()
        torch.cuda.synchronize()

    def replay(self):
        self.g.replay()


def time_graph(g, reps, warm=2):
    """Average ms per replay over `reps` replays, HIP events on the stream the
    graph runs on."""
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def build_model(dev, seed=0):
    from ai_amd import wcomp
    gen = torch.Generator().manual_seed(seed)
    layers = []
    for _ in range(L):
        lay = {}
        for name, N, K, mode, rms in LAYER:
            c = wcomp.compress(make_matrix(N, K, gen, dev))
            lay[name] = wcomp.compact(c)
        layers.append(lay)
        torch.cuda.empty_cache()
    head = wcomp.compact(wcomp.compress(make_matrix(V, D, gen, dev)))
    return layers, head


def token_linears(layers, head, bufs, with_head=True):
    """The 4 x 36 (+ 1) launches of one decode token, in engine order
    (ramvi/engine/ramvi_engine/core/engine.py:335-340)."""
    from ai_amd import wcomp
    x, qkv, att, gu, ln, logits = bufs["x"], bufs["qkv"], bufs["att"], bufs["gu"], bufs["ln"], bufs["logits"]
    for lay in layers:
        wcomp.gemvc1(x, lay["qkv"], qkv, 0, lnw=ln)
        wcomp.gemvc1(att, lay["o"], x, 1)
        wcomp.gemvc1(x, lay["gu"], gu, 0, lnw=ln)
        wcomp.gemvc1(gu, lay["down"], x, 2)
    if with_head:
        wcomp.gemvc1(x, head, logits, 0)


def run_token_bench(args, dev):
    """Two graphs over the same resident weights: the whole token (145
    launches: value, tok/s) and the 144 layer launches alone, which are all
    the dominant kernel (vector-FMA linear, one token; two row blocks per
    workgroup for qkv, one for the others): the
    roofline figure is its algorithmic bytes over its measured time."""
    layers, head = build_model(dev)
    g = torch.Generator(device=dev).manual_seed(1)
    rnd = lambda n: torch.randn(n, device=dev, generator=g).bfloat16().float()
    bufs = {"x": rnd(D), "qkv": torch.zeros(QKV, device=dev), "att": rnd(32 * 128),
            "gu": rnd(2 * FF), "ln": torch.ones(D, device=dev, dtype=torch.bfloat16),
            "logits": torch.zeros(V, device=dev)}
    x0 = bufs["x"].clone()

    def step(with_head=True):
        bufs["x"].copy_(x0)  # keep the residual stream the same on every replay
        token_linears(layers, head, bufs, with_head)

    graph = Graph(step)
    cb = sum(comp_bytes(lay[n]) for lay in layers for n, *_ in LAYER) + comp_bytes(head)
    ab_layers = sum(alg_bytes(lay[n], m, r) for lay in layers for n, _, _, m, r in LAYER)
    ab = ab_layers + alg_bytes(head, 0, False)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    ms = time_graph(graph, args.steps, warm=0)
    del graph
    lgraph = Graph(lambda: step(False))
    ms_layers = time_graph(lgraph, args.steps, warm=args.warmup)
    del lgraph
    return {"ms": ms, "comp_bytes": cb, "alg_bytes": ab, "ms_layers": ms_layers, "alg_bytes_layers": ab_layers,
            "launches_layers": 4 * L, "layers": layers, "head": head, "bufs": bufs}


def copy_calibration(dev, reps=20):
    """A plain 1 GiB device copy (torch's copy kernel), for scaling the HBM
    byte counters: FETCH_SIZE and WRITE_SIZE of this kernel should each read
    1 GiB per launch."""
    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": 4 * n, "launches": reps}), flush=True)


def measure_hbm(dev, reps=10):
    """HBM rates torch's own kernels reach on this device, next to the
    published 8 TB/s: a 2 GiB device-to-device copy (bytes read + written per
    second), a read-only reduction of the same 2 GiB, and a plain bf16
    matrix-vector product over a 2 GiB matrix (65536 x 16384, the library
    GEMV of uncompressed weights; bytes read per second), HIP events over
    `reps` launches after one warm launch."""
    n = 1 << 29
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    acc = torch.empty((), dtype=torch.float32, device=dev)
    a = torch.full((1 << 16, 1 << 14), 0.5, dtype=torch.bfloat16, device=dev)
    xv = torch.ones(1 << 14, dtype=torch.bfloat16, device=dev)
    yv = torch.empty(1 << 16, dtype=torch.bfloat16, device=dev)

    def rate(fn, nbytes):
        fn()
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            fn()
        e1.record(st)
        torch.cuda.synchronize()
        return nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9

    copy = rate(lambda: dst.copy_(src), 8 * n)
    read = rate(lambda: torch.sum(src, 0, out=acc), 4 * n)
    mv = rate(lambda: torch.mv(a, xv, out=yv), 2 * a.numel())
    del src, dst, a
    torch.cuda.empty_cache()
    return {"copy_GBs": round(copy, 1), "sum_read_GBs": round(read, 1), "bf16_gemv_read_GBs": round(mv, 1),
            "read_GBs": round(max(read, mv), 1),
            "method": "torch copy_, sum and bf16 mv over 2 GiB; read_GBs = the faster read; HIP events, 10 launches"}


def run_e2e(dev, size="8b", prompt_len=2048, new=256, seed=0, batch=None, prefill="blocked", stream_layers=0):
    """Greedy decode of a random-init Qwen3 (8b: a 2048-token random-id
    prompt, 256 new tokens; 32b: 4096 and
    128; bf16 KV cache): decode-only tok/s from the graph replays after the
    prefill (the reference's blocked prefill: each matrix decoded once for the
    whole prompt).  batch=T adds the reference's "batch": one pass of T tokens of the
    same sequence through every layer (_batch_layer), replayed from a graph
    at the position after the prompt; tok/s = T / pass time."""
    from ai_amd.engine import Engine
    from ai_amd.model import QWEN3, RandomCkpt
    ck = RandomCkpt(QWEN3[size], seed=seed)
    t0 = time.time()
    eng = Engine(ck, maxt=prompt_len + new + (batch or 0), kv_dtype=torch.bfloat16, prefill=prefill,
                 stream_layers=stream_layers)
    load_s = time.time() - t0
    prompt = [int(t) for t in np.random.default_rng(seed).integers(0, ck.V, prompt_len)]
    eng.generate(prompt[:64], 8)  # capture + warm
    if prefill == "blocked" and prompt_len >= eng.prefill_min:
        eng.generate(prompt[:eng.prefill_min + 8], 2)  # the blocked prefill's GEMM shapes
    ids, prefill_ms, decode_ms = eng.generate(prompt, new, timing=True)
    per_tok = decode_ms / (new - 1)
    out = {"model": f"qwen3-{size} random init", "prompt": prompt_len, "new_tokens": new, "kv_cache": "bf16",
           "tok_s": round(1e3 / per_tok, 2), "ms_per_token": round(per_tok, 4), "prefill_ms": round(prefill_ms, 1),
           "prefill": prefill if prefill != "blocked" or prompt_len >= eng.prefill_min else "legacy (below the blocked minimum)",
           "load_s": round(load_s, 1), "first_ids": ids[:8]}
    if stream_layers:
        gb = eng.streamer.bytes_per_pass / 1e9
        out["streamed"] = {"layers": stream_layers, "of_layers": eng.L, "slots": eng.streamer.S,
                           "GB_per_token": round(gb, 4), "h2d_GBs_per_token_time": round(gb / per_tok * 1e3, 1)}
    if new <= 64:
        out["ids"] = ids
    if batch:
        ms = eng.batch_pass_ms(batch, prompt_len)
        out["batch_pass"] = {"tokens_per_pass": batch, "ms_per_pass": round(ms, 3), "tok_s": round(batch * 1e3 / ms, 2),
                             "semantics": "T tokens of one sequence per pass (the reference's _batch_layer), "
                                          "not independent sequences"}
    del eng
    torch.cuda.empty_cache()
    return out


def run_prefill(dev, size="8b", prompt_len=2048, reps=3, seed=0):
    """The blocked prefill alone (every layer's fused linears and prompt
    attention over the whole prompt, then the head's pick), `reps` times
    after a warm pass: ms per prompt."""
    from ai_amd.engine import Engine
    from ai_amd.model import QWEN3, RandomCkpt
    ck = RandomCkpt(QWEN3[size], seed=seed)
    eng = Engine(ck, maxt=prompt_len + 8, kv_dtype=torch.bfloat16, prefill="blocked")
    prompt = [int(t) for t in np.random.default_rng(seed).integers(0, ck.V, prompt_len)]
    eng.prefill(prompt)
    torch.cuda.synchronize()
    ms = []
    for _ in range(reps):
        eng.reset()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        eng.prefill(prompt)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
        print(f"# prefill {prompt_len} tokens: {ms[-1]:.1f} ms", file=sys.stderr, flush=True)
    del eng
    torch.cuda.empty_cache()
    return {"model": f"qwen3-{size} random init", "prompt": prompt_len, "kv_cache": "bf16", "prefill_ms": ms}


def measure_h2d(dev, nbytes=1 << 30, reps=5):
    """Pinned host -> HBM copy rate (one 1 GiB hipMemcpyAsync, HIP events):
    the ceiling of the streamed placement."""
    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    d = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    d.copy_(host, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        d.copy_(host, non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del host, d
    torch.cuda.empty_cache()
    return round(nbytes / ms / 1e6, 1)


def run_attn(dev, reps=20, layers=36, positions=(100, 1000, 2100)):
    """Decode-step attention of the Qwen3-8B shape alone (32 q / 8 kv heads,
    head dim 128, 2304-position bf16 caches, one per layer, 340 MB in all, so
    the caches stream from HBM as in the decode): k_rope_attn + k_attn_combine
    for `layers` layers replayed from a HIP graph, us per layer at each
    position (HIP events)."""
    from ai_amd.attn import RopeAttn
    H, KV, HD, maxt = 32, 8, 128, 2304
    att = RopeAttn(H, KV, HD, maxt, torch.bfloat16, 1e-6, dev)
    g = torch.Generator(device=dev).manual_seed(0)
    qkv = torch.randn((H + 2 * KV) * HD, device=dev, generator=g)
    qn, kn = torch.ones(HD, device=dev), torch.ones(HD, device=dev)
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    kcs = [torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16() for _ in range(layers)]
    vcs = [torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16() for _ in range(layers)]
    out = torch.zeros(H * HD, device=dev)
    res = {}
    for pos in positions:
        p = torch.tensor([pos], device=dev)

        def fn():
            for l in range(layers):
                att(qkv, qn, kn, inv, p, kcs[l], vcs[l], out)

        res[pos] = round(time_graph(Graph(fn), reps) / layers * 1e3, 2)
    return {"heads": H, "kv_heads": KV, "head_dim": HD, "maxt": maxt, "splits": att.a.splits,
            "kv_bytes_per_layer_at_2100": 2 * KV * 2101 * HD * 2, "us_per_layer": res}


def run_shape(name, reps, dev, min_bytes=1.2e9, outliers="rows"):
    """Qwen3-8B linear-shape sweep entry: one shape, distinct copies totalling > 1 GB
    replayed round-robin from a graph; ms per launch.  outliers: the x20
    outliers on 0.1 % of the output rows or of the input columns."""
    from ai_amd import wcomp
    N, K, mode = SWEEP[name]
    gen = torch.Generator().manual_seed(100 + sorted(SWEEP).index(name))
    per = 1.5 * N * K
    ncopy = max(1, int(np.ceil(min_bytes / per)))
    cs = [wcomp.compact(wcomp.compress(make_matrix(N, K, gen, dev, outliers))) for _ in range(ncopy)]
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn(K * (2 if mode == 2 else 1), device=dev, generator=g).bfloat16().float()
    y = torch.zeros(N, device=dev)

    def fn():
        for c in cs:
            wcomp.gemvc1(x, c, y, mode)

    graph = Graph(fn)
    ms = time_graph(graph, reps) / ncopy
    cb = sum(comp_bytes(c) for c in cs) / ncopy
    ab = sum(alg_bytes(c, mode, False) for c in cs) / ncopy
    exc = sum(int(c["er"].numel()) for c in cs) / ncopy / (N * K)
    r = {"shape": name, "N": N, "K": K, "copies": ncopy, "us": ms * 1e3, "comp_GBs": cb / ms / 1e6,
         "alg_GBs": ab / ms / 1e6, "frac_peak": cb / ms / 1e6 / PEAK_HBM, "exception_frac": exc}
    st = stream_ceiling(cs, N, K, reps)
    if st:
        r.update(st)
        r["ceiling_frac"] = r["stream_us"] / r["us"]  # the linear's rate over the pure stream's
    del cs, graph
    torch.cuda.empty_cache()
    return r


def stream_ceiling(cs, N, K, reps):
    """The pure weight stream of the same launch (ai_amd/csrc/rv12_probe.hip:
    the vector linear's grid, waves, step order, loads and loop at one token,
    without decode, activations, FMAs or exceptions) over the same copies, at
    4, 6 and 8 steps in flight per wave: the fastest is what a launch of this
    shape can reach on its 12-bit bytes."""
    import ctypes
    from ai_amd import _lib, build
    if not os.path.exists(build.PROBE_OUT):
        return None
    P = ctypes.CDLL(build.PROBE_OUT)
    P.rv12_probe_stream.restype = ctypes.c_int
    P.rv12_probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    c = _lib.Launch()
    if _lib.lib().rv12_launch_shape(N, K, 1, None, ctypes.byref(c)) or c.kernel != 1 or c.splits != 1:
        return None
    nblk = (N + 15) // 16
    out = torch.empty(((nblk + c.rb - 1) // c.rb) * c.waves * 64, dtype=torch.int32, device="cuda")
    best = None
    for depth in (4, 6, 8):
        def fn(depth=depth):
            for m in cs:
                rc = P.rv12_probe_stream(ctypes.c_void_p(m["q16_tiles"].data_ptr()), N, K, c.rb, c.waves, depth,
                                         ctypes.c_void_p(out.data_ptr()),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                assert rc == 0, rc

        graph = Graph(fn)
        ms = time_graph(graph, reps) / len(cs)
        del graph
        if best is None or ms < best[0]:
            best = (ms, depth)
    ms, depth = best
    tb = 1.5 * ((N + 15) // 16 * 16) * K
    return {"stream_us": ms * 1e3, "stream_GBs": tb / ms / 1e6, "stream_frac_peak": tb / ms / 1e6 / PEAK_HBM,
            "stream_depth": depth}


ARRIVAL_MODES = {0: "vector, alone", 1: "scalar, alone", 2: "vector, weight stream", 3: "scalar, weight stream"}


def arrival(dev, shapes=(("q_o", 4096, 4096, 8), ("k_v", 1024, 4096, 8)), min_bytes=1.0e9):
    """When the activations reach LDS inside one launch of the vector linear's
    one-token shape (ai_amd/csrc/rv12_probe.hip, k_arrival): each workgroup
    stages the K floats with vector loads (the linear's way) or with scalar
    loads of 64 bytes (two 128-byte pieces in flight per wave), alone or
    followed by the weight stream of its row block (6 steps in flight per
    wave).  Weights are random bytes of the 12-bit size, distinct copies over
    >= 1 GB; each launch reads its own activation vector, written by a copy
    kernel just before it, as the engine's previous launch writes it.  Per
    wave the 100 MHz real-time counter is read at entry, after the barrier
    that ends the staging, and at the end; times are from the launch's
    earliest entry."""
    import ctypes
    from ai_amd import build
    if not os.path.exists(build.PROBE_OUT):
        raise RuntimeError("librv12probe.so is not built")
    P = ctypes.CDLL(build.PROBE_OUT)
    P.rv12_probe_arrival.restype = ctypes.c_int
    P.rv12_probe_arrival.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    out = []
    for name, N, K, W in shapes:
        nbytes = N * K * 3 // 2
        ncopy = max(2, int(np.ceil(min_bytes / nbytes)))
        g = torch.Generator(device=dev).manual_seed(11)
        ws = [torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev, generator=g)
              for _ in range(ncopy)]
        xsrc = torch.randn(K, device=dev, generator=g)
        xs = [torch.empty(K, device=dev) for _ in range(ncopy)]
        nwg = (N + 15) // 16
        sink = torch.empty(nwg * W * 64, dtype=torch.int32, device=dev)
        ts = torch.zeros(ncopy, nwg, W, 3, dtype=torch.int64, device=dev)
        for mode, what in ARRIVAL_MODES.items():
            def fn():
                st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                for i in range(ncopy):
                    xs[i].copy_(xsrc)
                    rc = P.rv12_probe_arrival(ctypes.c_void_p(ws[i].data_ptr()), N, K, W, mode,
                                              ctypes.c_void_p(xs[i].data_ptr()), ctypes.c_void_p(sink.data_ptr()),
                                              ctypes.c_void_p(ts[i].data_ptr()), st)
                    assert rc == 0, rc

            graph = Graph(fn)
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            t = ts.cpu().numpy().astype(np.int64)
            del graph
            base = t[:, :, :, 0].min(axis=(1, 2))[:, None]  # earliest entry of each launch
            arr = (t[:, :, :, 1].max(axis=2) - base) * 0.01  # per workgroup, us
            own = (t[:, :, :, 1].max(axis=2) - t[:, :, :, 0].min(axis=2)) * 0.01
            end = (t[:, :, :, 2].max(axis=(1, 2)) - base[:, 0]) * 0.01
            r = {"shape": name, "N": N, "K": K, "waves": W, "workgroups": nwg, "launches": ncopy, "mode": mode,
                 "staging": what, "arrive_us_median": round(float(np.median(arr)), 3),
                 "arrive_us_p90": round(float(np.percentile(arr, 90)), 3),
                 "arrive_us_max": round(float(arr.max(axis=1).mean()), 3),
                 "arrive_from_own_entry_us_median": round(float(np.median(own)), 3),
                 "launch_span_us_median": round(float(np.median(end)), 3)}
            out.append(r)
            print(f"# arrival {name} {what}: median {r['arrive_us_median']:.2f} us, p90 {r['arrive_us_p90']:.2f}, "
                  f"last {r['arrive_us_max']:.2f}; span {r['launch_span_us_median']:.2f} us", file=sys.stderr,
                  flush=True)
        del ws, xs
        torch.cuda.empty_cache()
    return out


def cache_warm(dev, reps=10, rounds=5):
    """What the next launch gains from its first weight bytes in the caches:
    per shape, 40 distinct copies, each linear (built-in launch) preceded by
    a probe (ai_amd/csrc/rv12_probe.hip, k_warm) that reads, with ordinary
    loads, the first 6 (or 16) steps per wave of the same matrix or of
    another copy (same cost); us per pair, median of interleaved rounds."""
    import ctypes
    import statistics
    from ai_amd import build, wcomp
    P = ctypes.CDLL(build.PROBE_OUT)
    P.rv12_probe_warm.restype = ctypes.c_int
    P.rv12_probe_warm.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_void_p, ctypes.c_void_p]
    out = []
    for name, N, K, mode, W in (("q_o", 4096, 4096, 1, 8), ("qkv", 6144, 4096, 0, 8), ("down", 4096, 12288, 2, 16)):
        gen = torch.Generator().manual_seed(9)
        ncopy = 40
        cs = [wcomp.compact(wcomp.compress(make_matrix(N, K, gen, dev))) for _ in range(ncopy)]
        x = torch.randn(K * (2 if mode == 2 else 1), device=dev).bfloat16().float()
        y = torch.zeros(N, device=dev)
        sink = torch.empty(((N + 15) // 16) * 1024, dtype=torch.int32, device=dev)

        def graph(shift, depth):
            def fn():
                st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                for i, c in enumerate(cs):
                    if depth:
                        w = cs[(i + shift) % ncopy]
                        rc = P.rv12_probe_warm(ctypes.c_void_p(w["q16_tiles"].data_ptr()), N, K, W, depth,
                                               ctypes.c_void_p(sink.data_ptr()), st)
                        assert rc == 0, rc
                    wcomp.gemvc1(x, c, y, mode)
            return Graph(fn)

        gs = {"linear alone": graph(0, 0)}
        for depth in (6, 16):
            gs[f"same matrix, {depth} steps per wave"] = graph(0, depth)
            gs[f"other matrix, {depth} steps per wave"] = graph(ncopy // 2, depth)
        t = {k: [] for k in gs}
        for _ in range(rounds):
            for k, g in gs.items():
                t[k].append(time_graph(g, reps) / ncopy * 1e3)
        r = {"shape": name, "N": N, "K": K, "us_per_pair": {k: round(statistics.median(v), 3) for k, v in t.items()}}
        out.append(r)
        print(f"# cache warm {name}: " + ", ".join(f"{k} {v:.2f}" for k, v in r["us_per_pair"].items()), file=sys.stderr,
              flush=True)
        del gs, cs
        torch.cuda.empty_cache()
    return out


LOAD_WIDTH_SHAPES = (("q_o", 4096, 4096, 8), ("qkv", 6144, 4096, 8), ("down", 4096, 12288, 16),
                     ("gu", 24576, 4096, 4), ("lm_head", 151936, 4096, 8))


def load_width(dev, reps=10, min_bytes=1.2e9):
    """The pure weight stream of one row block per workgroup read with the
    layout's 12-byte loads (k_stream: 6 of them, 768 bytes, per wave and K
    step) against 16-byte loads of the same bytes (k_stream16: the row
    block's bytes in 3 KB chunks, three 1 KB loads each), at 3, 4.5-6 and
    6-9 KB in flight per wave, over >= 1.2 GB of distinct random byte
    copies per shape (ai_amd/csrc/rv12_probe.hip)."""
    import ctypes
    from ai_amd import build
    P = ctypes.CDLL(build.PROBE_OUT)
    for f in (P.rv12_probe_stream, P.rv12_probe_stream16):
        f.restype = ctypes.c_int
    P.rv12_probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    P.rv12_probe_stream16.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_void_p]
    res = []
    for name, N, K, W in LOAD_WIDTH_SHAPES:
        nb = N * K * 3 // 2
        ncopy = max(2, int(np.ceil(min_bytes / nb)))
        g = torch.Generator(device=dev).manual_seed(21)
        ws = [torch.randint(-2**31, 2**31 - 1, (nb // 4,), dtype=torch.int32, device=dev, generator=g)
              for _ in range(ncopy)]
        out = torch.empty(((N + 15) // 16) * 16 * 64, dtype=torch.int32, device=dev)
        for kind, depths in (("12-byte", (4, 6, 8)), ("16-byte", (1, 2, 3))):
            for d in depths:
                def fn():
                    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                    for w in ws:
                        if kind == "12-byte":
                            rc = P.rv12_probe_stream(ctypes.c_void_p(w.data_ptr()), N, K, 1, W, d,
                                                     ctypes.c_void_p(out.data_ptr()), st)
                        else:
                            rc = P.rv12_probe_stream16(ctypes.c_void_p(w.data_ptr()), N, K, W, d,
                                                       ctypes.c_void_p(out.data_ptr()), st)
                        assert rc == 0, rc

                graph = Graph(fn)
                us = time_graph(graph, reps) / ncopy * 1e3
                del graph
                r = {"shape": name, "loads": kind, "waves": W, "depth": d,
                     "KB_in_flight_per_wave": round((768 * d if kind == "12-byte" else 3072 * d) / 1024, 1),
                     "us": round(us, 2), "frac_peak": round(nb / us / 1e3 / PEAK_HBM, 4)}
                res.append(r)
                print(f"# load width {name} {kind} depth {d}: {us:.2f} us ({r['frac_peak']:.1%})", file=sys.stderr,
                      flush=True)
        del ws
        torch.cuda.empty_cache()
    return res


def run_skinny(name, reps, dev, min_bytes=1.2e9):
    """Qwen3-14B skinny-GEMM entry: one shape at every M of SWEEP_M, weights
    N(0, 0.02) bf16 with 0.1% of output rows x20, distinct copies totalling
    > 1 GB replayed round-robin, with the library's built-in kernel choice:
    the vector kernel at one token and, up to 4 tokens, where its activations
    fit the LDS unsplit on the smaller matrices (qkv and k/v at 4 tokens, o at
    2 and 3, down and gate/up at 2), else the bf16 MFMA kernel (3 MFMAs per
    tile: the hi/mid/lo split of x)."""
    from ai_amd import wcomp
    N, K = SWEEP_14B[name]
    gen = torch.Generator().manual_seed(200 + sorted(SWEEP_14B).index(name))
    ncopy = max(1, int(np.ceil(min_bytes / (1.5 * N * K))))
    cs = []
    for _ in range(ncopy):
        w = torch.randn(N, K, device=dev, generator=torch.Generator(device=dev).manual_seed(
            int(torch.randint(0, 2**31 - 1, (1,), generator=gen)))).mul_(0.02)
        w[torch.randperm(N, generator=gen)[: max(1, N // 1000)].to(dev)] *= 20
        cs.append(wcomp.compact(wcomp.compress(w.bfloat16())))
        del w
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(16, K, device=dev, generator=g).bfloat16().float()
    y = torch.zeros(16, N, device=dev)
    out = []
    for M in SWEEP_M:
        def fn():
            for c in cs:
                wcomp.gemvc_tc(x, c, y, 0, M)

        graph = Graph(fn)
        ms = time_graph(graph, reps) / ncopy
        del graph
        cb = sum(comp_bytes(c) for c in cs) / ncopy
        mfma = wcomp.launch_shape(N, K, M)[0] == 2
        r = {"shape": name, "N": N, "K": K, "M": M, "copies": ncopy, "kernel": "k_gemm" if mfma else "k_gemv",
             "us": round(ms * 1e3, 3), "comp_GBs": round(cb / ms / 1e6, 1), "frac_peak": round(cb / ms / 1e6 / PEAK_HBM, 4),
             "alg_TFLOPs": round(2 * M * N * K / ms / 1e9, 3)}
        if mfma:  # issued: 3 MFMAs over 16 token columns per tile
            r["mfma_TFLOPs"] = round(3 * 2 * 16 * N * K / ms / 1e9, 2)
            r["mfma_frac"] = round(r["mfma_TFLOPs"] / PEAK_BF16, 4)
        out.append(r)
    del cs
    torch.cuda.empty_cache()
    return out


def _cpu_threads():
    """Threads of the CPU legs: every core this process may run on
    (sched_getaffinity), capped by OMP_NUM_THREADS where the host sets it (the
    GPU hosts give each GPU a share of their cores that way)."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    return (min(aff, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else aff), aff, omp


def _timed(fn, budget):
    """(passes, seconds) of fn repeated for about `budget` seconds (at least once)."""
    fn()  # warm: page in, thread pool up
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget:
            return n, dt


def cpu_baseline(dev, gpu_ids_0_6b=None, budget=0.7):
    """The reference's CPU paths restated in C (oracle/), timed on this host:
      gemv_12bit  the 12-bit block decode + dot product of the native CPU path
                  (native/qmm.cpp:195-212: decode a 256-chunk of a row to fp32,
                  dot it with every token), from the reference codec's own
                  arrays, per Qwen3-8B shape at M=1;
      matmat16    the CPU layer's bf16 linear (cpu/cpu_layer.py:35-48), per shape;
      e2e_qwen3_0_6b  Qwen3-0.6B end to end: CpuLayer.__call__ over 28 layers +
                  the exact greedy head (cpu/cpu_layer.py:155-175,
                  generation/head.py:19-26), 128-token prompt, 64 new tokens.
    value: the gemv_12bit leg over one Qwen3-8B layer's qkv / o / gu / down
    (with their RMS and silu prologues), compressed GB/s, the same bytes as the
    GPU line's value."""
    from ai_amd import wcomp
    from ai_amd.model import QWEN3, RandomCkpt
    from oracle import cpu_qwen3, cref
    if not os.path.exists(cref.LIB_PATH):
        cref.build()
    threads, aff, omp = _cpu_threads()
    gen = torch.Generator().manual_seed(7)
    rng = np.random.default_rng(0)

    def host_codec(w):
        c = wcomp.compress(w)
        return {k: (c[k].cpu().numpy() if torch.is_tensor(c[k]) else c[k]) for k in
                ("m8", "e4", "base", "rp", "er", "ec", "ev", "N", "K", "CH")}

    legs = {"gemv_12bit": {}, "matmat16": {}}
    for name, (N, K, _) in SWEEP.items():
        w = make_matrix(N, K, gen, dev)
        c = host_codec(w)
        wb = w.view(torch.int16).cpu().numpy().view(np.uint16)
        del w
        # distinct copies of > 1 GB in all, so that no pass is served from the
        # host's last-level cache
        copies = max(1, -(-(1 << 30) // (2 * N * K)))
        cs = [c] + [{k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in c.items()} for _ in range(copies - 1)]
        wbs = [wb] + [wb.copy() for _ in range(copies - 1)]
        x = rng.standard_normal((1, K)).astype(np.float32)
        y = np.zeros((1, N), np.float32)
        cb = int(1.5 * N * K) + 12 * int(c["er"].size) + 4 * (N + 1)
        n, dt = _timed(lambda: [cref.gemv_12bit(ci, x, y, 0, threads=threads) for ci in cs], budget)
        n *= copies
        legs["gemv_12bit"][name] = {"us": round(dt / n * 1e6, 1), "comp_GBs": round(cb * n / dt / 1e9, 2),
                                    "copies": copies}
        n, dt = _timed(lambda: [cref.gemv_bf16(wi, x, y, add=False, threads=threads) for wi in wbs], budget)
        n *= copies
        legs["matmat16"][name] = {"us": round(dt / n * 1e6, 1), "bf16_GBs": round(2 * N * K * n / dt / 1e9, 2),
                                  "comp_equiv_GBs": round(cb * n / dt / 1e9, 2), "copies": copies}
        del c, wb, cs, wbs
    # value: one Qwen3-8B layer through the 12-bit leg, prologues included
    layer, cbytes = [], 0
    for name, N, K, mode, rms in LAYER:
        c = host_codec(make_matrix(N, K, gen, dev))
        X = rng.standard_normal((1, 2 * K if mode == 2 else K)).astype(np.float32)
        lnw = np.ones(K, np.uint16) * 0x3F80 if rms else None
        layer.append((c, X, np.zeros((1, N), np.float32), mode, lnw))
        cbytes += int(1.5 * N * K) + 12 * int(c["er"].size) + 4 * (N + 1)

    def one_layer():
        for c, X, Y, mode, lnw in layer:
            cref.gemv_12bit(c, X, Y, mode, lnw=lnw, threads=threads)

    n, dt = _timed(one_layer, 3.0)  # 0.33 GB of codec arrays per pass: beyond the host caches
    value = cbytes * n / dt / 1e9
    del layer
    # Qwen3-0.6B end to end (weights drawn on the GPU, as the GPU engine's)
    ck = RandomCkpt(QWEN3["0.6b"], seed=0)
    m = cpu_qwen3.load(ck, dev)
    prompt = [int(t) for t in np.random.default_rng(0).integers(0, ck.V, 128)]
    ids, pre_s, dec_s = cpu_qwen3.generate(m, prompt, 64, threads=threads)
    e2e = {"model": "qwen3-0.6b random init", "prompt": 128, "new_tokens": 64, "kv_cache": "fp32",
           "decode_tok_s": round(63 / dec_s, 2), "ms_per_token": round(dec_s / 63 * 1e3, 2),
           "prefill_s": round(pre_s, 2), "first_ids": ids[:8]}
    if gpu_ids_0_6b:
        e2e["ids_equal_to_gpu_engine"] = sum(a == b for a, b in zip(ids, gpu_ids_0_6b))
        e2e["gpu_engine_kv_cache"] = "bf16"
    del m
    return {"value": round(value, 3), "unit": "GB/s (compressed bytes)", "cores": threads, "kind": "port",
            "sample": f"{n} passes over one Qwen3-8B layer's qkv/o/gu/down at M=1 (12-bit block decode + dot, "
                      f"RMS and silu prologues) in {dt:.1f} s; per-shape legs {budget} s each; config-1 decode "
                      f"of 64 tokens",
            "nproc": os.cpu_count(), "affinity_cores": aff, "omp_num_threads": omp, "cpu_model": _cpu_model(),
            "legs": legs, "e2e_qwen3_0_6b": e2e}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=sorted(SWEEP), help="time one Qwen3-8B linear shape only (for profiling)")
    ap.add_argument("--reps", type=int, default=20, help="graph replays per sweep shape")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the Qwen3-8B end-to-end decode")
    ap.add_argument("--no-14b", action="store_true", help="skip the Qwen3-14B skinny-GEMM sweep")
    ap.add_argument("--no-32b", action="store_true", help="skip the Qwen3-32B end-to-end decode")
    ap.add_argument("--only-14b", action="store_true", help="run only the Qwen3-14B skinny-GEMM sweep (for profiling)")
    ap.add_argument("--only-attn", action="store_true", help="run only the Qwen3-8B decode attention (for profiling)")
    ap.add_argument("--only-e2e", nargs="?", const="8b", choices=("8b", "0.6b"),
                    help="run only one end-to-end decode (for profiling): 8b (the default: 2048-token prompt, 256 "
                         "tokens) or 0.6b (128-token prompt, 64 tokens, as in the default run)")
    ap.add_argument("--only-prefill", action="store_true",
                    help="run only the Qwen3-8B blocked prefill of a 2048-token prompt, 3 times (for profiling)")
    ap.add_argument("--only-cache-warm", action="store_true",
                    help="run only the probe of a linear preceded by a read of its first weight bytes (three shapes)")
    ap.add_argument("--only-load-width", action="store_true",
                    help="run only the pure-stream probe with 12-byte against 16-byte loads (five Qwen3-8B shapes)")
    ap.add_argument("--only-arrival", action="store_true",
                    help="run only the activation-arrival probe (vector against scalar staging, q/o and k/v shapes)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 1 GiB device copy (scale factor of the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the 12-bit decode-linear runs on a single MI355X "
              "(multi-GPU sharding is designed, not built)", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    from ai_amd import _lib
    _lib.lib()

    if args.copy_calibration:
        copy_calibration(dev)
        return
    if args.only:
        r = run_shape(args.only, args.reps, dev)
        print(json.dumps(r), flush=True)
        return
    if args.only_14b:
        print(json.dumps([r for name in SWEEP_14B for r in run_skinny(name, args.reps, dev)]), flush=True)
        return
    if args.only_attn:
        print(json.dumps(run_attn(dev, args.reps)), flush=True)
        return
    if args.only_e2e:
        r = run_e2e(dev) if args.only_e2e == "8b" else run_e2e(dev, "0.6b", prompt_len=128, new=64)
        print(json.dumps(r), flush=True)
        return
    if args.only_prefill:
        print(json.dumps(run_prefill(dev)), flush=True)
        return
    if args.only_arrival:
        print(json.dumps(arrival(dev)), flush=True)
        return
    if args.only_load_width:
        print(json.dumps(load_width(dev)), flush=True)
        return
    if args.only_cache_warm:
        print(json.dumps(cache_warm(dev)), flush=True)
        return

    tok = run_token_bench(args, dev)
    ms = tok["ms"]
    value = tok["comp_bytes"] / ms / 1e6
    achieved_alg = tok["alg_bytes_layers"] / tok["ms_layers"] / 1e6
    us_launch = tok["ms_layers"] * 1e3 / tok["launches_layers"]
    print(f"# token linears: {ms:.3f} ms, {value:.0f} GB/s compressed; layer launches {us_launch:.2f} us avg, "
          f"{achieved_alg:.0f} GB/s algorithmic", file=sys.stderr, flush=True)
    del tok["layers"], tok["head"]
    torch.cuda.empty_cache()

    sweep, sweep_cols = [], []
    if not args.no_sweep:
        for name in ("q_o", "k_v", "gate_up", "down", "lm_head", "qkv", "gu"):
            r = run_shape(name, args.reps, dev)
            print(f"# {name}: {r['us']:.1f} us/launch, {r['comp_GBs']:.0f} GB/s ({r['frac_peak']:.1%}); pure "
                  f"stream {r.get('stream_us', 0):.1f} us ({r.get('stream_frac_peak', 0):.1%}), linear at "
                  f"{r.get('ceiling_frac', 0):.1%} of it", file=sys.stderr, flush=True)
            sweep.append({k: (round(v, 6) if isinstance(v, float) else v) for k, v in r.items()})
        for name in ("q_o", "k_v", "gate_up", "down", "lm_head", "qkv", "gu"):
            r = run_shape(name, args.reps, dev, outliers="columns")
            print(f"# {name} (outlier input columns): {r['us']:.1f} us/launch, {r['comp_GBs']:.0f} GB/s "
                  f"({r['frac_peak']:.1%})", file=sys.stderr, flush=True)
            sweep_cols.append({k: (round(v, 6) if isinstance(v, float) else v) for k, v in r.items()})

    sweep14 = []
    if not args.no_14b:
        for name in SWEEP_14B:
            rs = run_skinny(name, args.reps, dev)
            print("# 14b " + name + ": " + ", ".join(f"M{r['M']} {r['us']:.1f} us {r['frac_peak']:.1%}" for r in rs),
                  file=sys.stderr, flush=True)
            sweep14 += rs

    e2e = None
    if not args.no_e2e:
        e2e = run_e2e(dev)
        print(f"# qwen3-8b decode: {e2e['tok_s']} tok/s ({e2e['ms_per_token']} ms/token), prefill "
              f"{e2e['prefill_ms']} ms for {e2e['prompt']} tokens", file=sys.stderr, flush=True)

    e2e06 = None
    if not args.no_e2e:
        e2e06 = run_e2e(dev, "0.6b", prompt_len=128, new=64)
        e2e06["reference_published"] = {"tok_s": 290, "hardware": "RTX 5060 Laptop 8 GB (other hardware)",
                                        "source": "ramvi/docs/architecture/COMPATIBILITY.md:72"}
        print(f"# qwen3-0.6b decode: {e2e06['tok_s']} tok/s ({e2e06['ms_per_token']} ms/token), prefill "
              f"{e2e06['prefill_ms']} ms for {e2e06['prompt']} tokens", file=sys.stderr, flush=True)

    e2e_st = None
    if not args.no_e2e:
        # the reference's "stream" placement: 12 of the 36 layers in pinned host
        # memory, copied into two HBM slots every token
        e2e_st = run_e2e(dev, "8b", prompt_len=512, new=64, stream_layers=12)
        e2e_st["h2d_measured_GBs"] = measure_h2d(dev)
        print(f"# qwen3-8b, 12 layers streamed: {e2e_st['tok_s']} tok/s, {e2e_st['streamed']['GB_per_token']} GB "
              f"per token over PCIe ({e2e_st['streamed']['h2d_GBs_per_token_time']} GB/s of token time; pinned "
              f"copy {e2e_st['h2d_measured_GBs']} GB/s)", file=sys.stderr, flush=True)

    e2e32 = None
    if not args.no_e2e and not args.no_32b:
        e2e32 = run_e2e(dev, "32b", prompt_len=4096, new=128, batch=8)
        print(f"# qwen3-32b decode: {e2e32['tok_s']} tok/s ({e2e32['ms_per_token']} ms/token), prefill "
              f"{e2e32['prefill_ms']} ms for {e2e32['prompt']} tokens; 8-token passes "
              f"{e2e32['batch_pass']['tok_s']} tok/s", file=sys.stderr, flush=True)

    hbm = measure_hbm(dev)
    print(f"# measured HBM: copy {hbm['copy_GBs']:.0f} GB/s, sum {hbm['sum_read_GBs']:.0f} GB/s read, bf16 mv "
          f"{hbm['bf16_gemv_read_GBs']:.0f} GB/s read", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(dev, e2e06.get("ids") if e2e06 else None)
        print(f"# cpu ({cpu['cores']} threads of {cpu['nproc']}, {cpu['cpu_model']}): 8B layer 12-bit "
              f"{cpu['value']} GB/s; " + ", ".join(f"{k} {v['comp_GBs']}" for k, v in cpu["legs"]["gemv_12bit"].items())
              + f"; 0.6B decode {cpu['e2e_qwen3_0_6b']['decode_tok_s']} tok/s", file=sys.stderr, flush=True)
    line = {
        "metric": "Qwen3-8B bs1 decode tok/s; fused GEMV effective HBM GB/s vs peak",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (random bf16 weights, 12-bit coded; N(0,1) activations)",
        "config": {"workload": "qwen3-8b-linear-sweep", "layers": L, "matrices_per_step": 4 * L + 1,
                   "shapes_NxK": {"qkv": [QKV, D], "o": [D, 4096], "gu": [2 * FF, D], "down": [D, FF],
                                  "lm_head": [V, D]},
                   "tokens": 1, "compressed_GB_per_step": round(tok["comp_bytes"] / 1e9, 4)},
        "linear_only_tok_s": round(1e3 / ms, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved_alg, 2), "peak": PEAK_HBM, "unit": "GB/s",
                     "frac": round(achieved_alg / PEAK_HBM, 4), "traffic": TRAFFIC_BYTES_PER_LAUNCH,
                     "kernel": "k_gemv<T=1> (vector-FMA linear, 1 token, RMS / silu prologue variants; RB=2 for qkv, RB=1 otherwise): the 144 layer launches of one token",
                     "avg_launch_us": round(us_launch, 3),
                     "alg_bytes_per_launch": round(tok["alg_bytes_layers"] / tok["launches_layers"]),
                     "frac_of_measured_read": round(achieved_alg / hbm["read_GBs"], 4)},
        "hbm_measured": hbm,
        "e2e_decode": e2e,
        "e2e_decode_0_6b": e2e06,
        "e2e_decode_32b": e2e32,
        "e2e_decode_8b_streamed": e2e_st,
        "cpu_baseline": cpu,
        "sweep_m1": sweep,
        "sweep_m1_input_column_outliers": sweep_cols,
        "sweep_14b": sweep14,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
