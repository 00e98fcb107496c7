"""Pinning the fp32 Qwen3 oracle (CPU): against Hugging Face Transformers'
Qwen3ForCausalLM (eager attention, float32) on a small random checkpoint
written to disk, the same cross-check the reference runs
(ramvi/engine/tools/checks/check_reference.py:14-19, 104-107); a planted RoPE
mistake fails it; the greedy argmax and its tie rule."""
import numpy as np
import pytest
import torch

from ai_amd.model import Ckpt, RandomCkpt, tiny_config, write_checkpoint
from oracle import qwen3


@pytest.fixture(scope="module")
def ckdir(tmp_path_factory):
    ck = RandomCkpt(tiny_config(layers=2, vocab=2048), seed=7, gen_device="cpu")
    return write_checkpoint(ck, str(tmp_path_factory.mktemp("qwen3tiny")))


def _hf_logits(path, tokens):
    transformers = pytest.importorskip("transformers")
    m = transformers.Qwen3ForCausalLM.from_pretrained(path, dtype=torch.float32, attn_implementation="eager")
    m.eval()
    with torch.no_grad():
        return m(torch.tensor([tokens])).logits[0]


def test_logits_match_transformers(ckdir):
    ck = Ckpt(ckdir)
    toks = [int(t) for t in np.random.default_rng(0).integers(0, ck.V, 40)]
    ours = qwen3.logits(ck, toks)
    ref = _hf_logits(ckdir, toks)
    assert ours.shape == ref.shape
    assert torch.allclose(ours, ref, atol=2e-5, rtol=1e-4), float((ours - ref).abs().max())
    assert qwen3.argmax(ck, toks) == ref.argmax(-1).tolist()


def test_planted_rope_mistake_is_caught(ckdir):
    """Interleaved-pair rotation instead of rotate-half: the logits move far
    beyond the tolerance the previous test applies."""
    ck = Ckpt(ckdir)
    toks = list(range(3, 35))

    def interleaved(t):
        a, b = t[..., 0::2], t[..., 1::2]
        return torch.stack([-b, a], -1).flatten(-2)

    bad = qwen3.logits(ck, toks, rotate=interleaved)
    ref = _hf_logits(ckdir, toks)
    assert (bad - ref).abs().max() > 1e-2


def test_argmax_chunks_and_ties():
    """Chunked argmax equals the full argmax, and a tie picks the smallest id."""
    ck = RandomCkpt(tiny_config(layers=1, vocab=3000), seed=2, gen_device="cpu")
    toks = list(range(10, 30))
    full = qwen3.logits(ck, toks).argmax(-1).tolist()
    assert qwen3.argmax(ck, toks, head_chunk=700) == full

    class Tied(RandomCkpt):
        """Untied head that is zero except rows 5 and 9, which are equal: every
        logit row is a tie, between 5 and 9 (when positive) or among zeros."""
        def t(self, name, device="cpu"):
            if name == "lm_head.weight":
                w = torch.zeros(self.V, self.D, dtype=torch.bfloat16)
                u = torch.randn(self.D, generator=torch.Generator().manual_seed(0)).bfloat16()
                w[5] = u
                w[9] = u
                return w.to(device)
            return super().t(name, device)

    cfg = dict(tiny_config(layers=1, vocab=3000), tie_word_embeddings=False)
    tk = Tied(cfg, seed=2, gen_device="cpu")
    h = qwen3.hidden(tk, toks)
    s = h @ tk.t("lm_head.weight").float()[5]
    ids, margins = qwen3.argmax(tk, toks, head_chunk=7, margins=True)
    assert (s > 0).any() and (s < 0).any()
    assert ids == [5 if v > 0 else 0 for v in s.tolist()]
    assert all(m == 0.0 for m in margins)


def test_argmax_pick_gaps():
    """The gap of a pick is 0 for the argmax itself and best - logit(pick)
    for any other token, across head chunks."""
    ck = RandomCkpt(tiny_config(layers=1, vocab=3000), seed=3, gen_device="cpu")
    toks = list(range(40, 52))
    lg = qwen3.logits(ck, toks)
    best = lg.argmax(-1)
    _, gap = qwen3.argmax(ck, toks, head_chunk=700, picks=best.tolist())
    assert all(g == 0.0 for g in gap)
    other = ((best + 1234) % 3000).tolist()
    ids, m, gap = qwen3.argmax(ck, toks, head_chunk=700, margins=True, picks=other[2:], first=2)
    want = (lg.max(-1).values - lg.gather(1, torch.tensor(other)[:, None])[:, 0])[2:]
    assert ids == best.tolist()[2:]
    assert torch.allclose(torch.tensor(gap), want, rtol=1e-6, atol=1e-6)
