"""The CPU restatement of the reference CPU layer (oracle/cpu_qwen3.py over
oracle/c/rv12_oracle.c: rms_rows, qk_rope_attn, silu_mul, matmat16; the CPU
baseline of the end-to-end decode) against the torch float32 forward
(oracle/qwen3.py, itself pinned by Transformers' Qwen3 logits): the greedy
ids of a tiny random Qwen3 agree wherever the top-2 logit margin is clear,
and planted RoPE frequencies from an off-by-one head size break the
agreement of the hidden states."""
import numpy as np
import pytest

from ai_amd.model import RandomCkpt, tiny_config
from oracle import cpu_qwen3, cref, qwen3


@pytest.fixture(scope="module")
def model():
    if not __import__("os").path.exists(cref.LIB_PATH):
        cref.build()
    ck = RandomCkpt(tiny_config(layers=2, vocab=2048), seed=21, gen_device="cpu")
    return ck, cpu_qwen3.load(ck)


def test_greedy_ids_match_the_torch_forward(model):
    ck, m = model
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, ck.V, 23)]
    ids, _, _ = cpu_qwen3.generate(m, prompt, 10, threads=2)
    want, margin = qwen3.argmax(ck, prompt + ids[:-1], margins=True, first=len(prompt) - 1)
    bad = [i for i in range(10) if ids[i] != want[i] and margin[i] > 1e-4]
    assert not bad, (ids, want)
    assert sum(a == b for a, b in zip(ids, want)) >= 9


def test_prefill_rows_match_the_torch_hidden_states(model):
    """Every prompt row after both layers and the final norm, against the
    torch forward (float32 tolerance)."""
    ck, m = model
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, ck.V, 17)]
    T = len(prompt)
    caches = [(np.zeros((ck.KV, T, ck.HD), np.float32), np.zeros((ck.KV, T, ck.HD), np.float32))
              for _ in range(ck.L)]
    X = np.ascontiguousarray(cpu_qwen3._embed(m, prompt))
    for l in range(ck.L):
        cpu_qwen3._layer(m, l, X, 0, caches, 2)
    h = np.empty_like(X)
    cref.rms_rows(X, m["norm"], h, m["eps"])
    ref = qwen3.hidden(ck, prompt).numpy()
    assert np.allclose(h, ref, rtol=2e-4, atol=2e-4), float(np.abs(h - ref).max())
    # planted: RoPE frequencies from an off-by-one head size, 1 / theta^(2i / (HD - 1))
    bad = dict(m, inv=(1.0 / (ck.theta ** (np.arange(0, ck.HD, 2) / (ck.HD - 1)))).astype(np.float32))
    caches = [(np.zeros((ck.KV, T, ck.HD), np.float32), np.zeros((ck.KV, T, ck.HD), np.float32))
              for _ in range(ck.L)]
    X = np.ascontiguousarray(cpu_qwen3._embed(bad, prompt))
    for l in range(ck.L):
        cpu_qwen3._layer(bad, l, X, 0, caches, 2)
    cref.rms_rows(X, m["norm"], h, m["eps"])
    assert not np.allclose(h, ref, rtol=2e-4, atol=2e-4)
