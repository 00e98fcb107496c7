"""End-to-end greedy decoding through the 12-bit linears against the fp32
oracle (teacher-forced argmax over prompt + generated tokens, the reference's
selftest criterion: ramvi/engine/tools/checks/selftest.py:63-78)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _check(ck, prompt, new, kv_dtype=torch.float32, maxt=None, prefill="legacy"):
    from ai_amd.engine import Engine
    from oracle import qwen3
    eng = Engine(ck, maxt=maxt or len(prompt) + new + 8, kv_dtype=kv_dtype, prefill=prefill, prefill_min=1)
    ids = eng.generate(prompt, new)
    again = eng.generate(prompt, new)  # graph replays are repeatable
    assert ids == again
    ref, margins = qwen3.argmax(ck, prompt + ids[:-1], kv_dtype=kv_dtype, margins=True)
    want = ref[len(prompt) - 1:]
    bad = [i for i in range(new) if ids[i] != want[i]]
    m = margins[len(prompt) - 1:]
    print(f"generated {new}, mismatches {bad}, smallest top-2 margin {min(m):.3g}", flush=True)
    assert not bad, [(i, ids[i], want[i], m[i]) for i in bad]
    del eng
    torch.cuda.empty_cache()
    return ids


def test_tiny_model_greedy_matches_oracle():
    from ai_amd.model import RandomCkpt, tiny_config
    ck = RandomCkpt(tiny_config(layers=2, vocab=4096), seed=11)
    prompt = [int(t) for t in np.random.default_rng(1).integers(0, ck.V, 37)]
    _check(ck, prompt, 24)


@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
def test_tiny_model_blocked_prefill(kv_dtype):
    """The reference's blocked prefill (RAMVI_PREFILL=blocked): the whole
    prompt in one pass per layer, each matrix decoded once."""
    from ai_amd.model import RandomCkpt, tiny_config
    ck = RandomCkpt(tiny_config(layers=2, vocab=4096), seed=14)
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, ck.V, 300)]
    _check(ck, prompt, 16, kv_dtype=kv_dtype, prefill="blocked")


def test_tiny_model_bf16_cache():
    from ai_amd.model import RandomCkpt, tiny_config
    ck = RandomCkpt(tiny_config(layers=3, vocab=4096), seed=12)
    prompt = [int(t) for t in np.random.default_rng(2).integers(0, ck.V, 20)]
    _check(ck, prompt, 16, kv_dtype=torch.bfloat16)


def test_checkpoint_folder_round_trip(tmp_path):
    """A model written as config.json + model.safetensors (the reference
    loader's format) decodes the same as the in-memory one."""
    from ai_amd.engine import Engine
    from ai_amd.model import Ckpt, RandomCkpt, tiny_config, write_checkpoint
    ck = RandomCkpt(tiny_config(layers=1, vocab=2048), seed=13)
    prompt = list(range(100, 118))
    a = Engine(ck, maxt=64).generate(prompt, 8)
    b = Engine(Ckpt(write_checkpoint(ck, str(tmp_path / "m"))), maxt=64).generate(prompt, 8)
    assert a == b


def test_qwen3_0_6b_64_tokens():
    """Qwen3-0.6B architecture, random init: 128-token random prompt, 64
    greedy tokens, all equal to the fp32 oracle's."""
    from ai_amd.model import QWEN3, RandomCkpt
    ck = RandomCkpt(QWEN3["0.6b"], seed=0)
    prompt = [int(t) for t in np.random.default_rng(0).integers(0, ck.V, 128)]
    _check(ck, prompt, 64, maxt=256)
