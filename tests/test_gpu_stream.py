"""Streamed layers (ai_amd.stream + Engine(resident=...), the reference's
"stream" placement, ramvi/engine/ramvi_engine/core/engine.py:34-326): layers
kept in host memory as packed images and copied into two device slots per
pass run the same kernels on the same bytes, so the greedy ids equal those of
the all-resident engine and of the fp32 oracle; the loader passes its errors
to the consumer and every wait is bounded."""
import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ck(seed=21):
    from ai_amd.model import RandomCkpt, tiny_config
    return RandomCkpt(tiny_config(layers=3, vocab=4096), seed=seed)


@pytest.mark.parametrize("prefill,pin_budget", [("legacy", None), ("blocked", None), ("legacy", 0)])
def test_streamed_layers_match_resident_and_oracle(prefill, pin_budget):
    from ai_amd.engine import Engine
    from oracle import qwen3
    ck = _ck()
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, ck.V, 40)]
    new = 12
    kw = dict(maxt=64, kv_dtype=torch.bfloat16, prefill=prefill, prefill_min=1)
    ref_eng = Engine(ck, **kw)
    want = ref_eng.generate(prompt, new)
    del ref_eng
    eng = Engine(ck, resident=1, pin_budget=pin_budget, **kw)
    try:
        assert eng.place == ["gpu", "stream", "stream"]
        if pin_budget == 0:
            assert eng.arena.pinned == 0 and eng.arena.plain > 0  # staged through pinned buffers
        got = eng.generate(prompt, new)
        again = eng.generate(prompt, new)
    finally:
        eng.close()
    print("streamed", got, flush=True)
    assert got == want and again == want
    ref = qwen3.argmax(ck, prompt + got[:-1], kv_dtype=torch.bfloat16)[len(prompt) - 1:]
    assert got == ref


def test_loader_passes_errors_on_and_closes():
    from ai_amd import stream
    ld = stream.Loader()
    try:
        src = torch.ones(1000, dtype=torch.uint8, pin_memory=True)
        small = torch.zeros(10, dtype=torch.uint8, device="cuda")
        mk = lambda pairs: {"l": 0, "s": 0, "pairs": pairs, "wait": None, "done": threading.Event(), "ev": None,
                            "rel": {"done": threading.Event(), "ev": None}}
        bad = mk([(src, small)])  # the image does not fit its slot: refused before any copy
        ld.q.put(bad)
        with pytest.raises(RuntimeError):
            stream.Loader.wait(bad)
        assert bad["rel"]["done"].is_set() and bad["rel"].get("error") is not None
        later = mk([(src[:5], small)])  # every job after a failure fails too
        ld.q.put(later)
        with pytest.raises(RuntimeError):
            stream.Loader.wait(later)
    finally:
        ld.close()
    assert not ld.thread.is_alive()


def test_loader_copies_in_chunks_from_plain_and_pinned_memory():
    from ai_amd import stream
    ld = stream.Loader()
    try:
        n = 3 * stream.Loader.CHUNK + 12345
        src_plain = torch.randint(0, 255, (n,), dtype=torch.uint8)
        src_pinned = src_plain.clone().pin_memory()
        for src in (src_plain, src_pinned):
            dst = torch.zeros(n + 100, dtype=torch.uint8, device="cuda")
            job = {"l": 0, "s": 0, "pairs": [(src, dst)], "wait": None, "done": threading.Event(), "ev": None,
                   "rel": None}
            ld.q.put(job)
            stream.Loader.wait(job)
            torch.cuda.current_stream().wait_event(job["ev"])
            assert torch.equal(dst[:n].cpu(), src_plain) and not bool(dst[n:].any())
    finally:
        ld.close()
