"""GPU test of rv12_decode_advance, the decode step's bookkeeping after the
greedy pick: the id goes to out[steps] (only inside [0, out_len)), becomes
the next token, its bf16 embedding row (id clamped into [0, vocab)) becomes
the float32 activations, pos and steps advance."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(ids, emb, x, out, steps, pos, tok, out_len=None):
    from ai_amd import _lib, wcomp
    L = _lib.lib()
    return L.rv12_decode_advance(wcomp._ptr(ids), wcomp._ptr(emb), emb.shape[0], emb.shape[1], wcomp._ptr(x),
                                 wcomp._ptr(out), out.numel() if out_len is None else out_len, wcomp._ptr(steps),
                                 wcomp._ptr(pos), wcomp._ptr(tok), None)


def test_decode_advance_records_embeds_and_counts():
    g = torch.Generator(device="cuda").manual_seed(3)
    V, H = 1000, 4096
    emb = torch.randn(V, H, device="cuda", generator=g).bfloat16()
    x = torch.full((2, H), 7.0, device="cuda")
    out = torch.full((8,), -5, dtype=torch.long, device="cuda")
    steps = torch.tensor([3], dtype=torch.long, device="cuda")
    pos = torch.tensor([100], dtype=torch.long, device="cuda")
    tok = torch.zeros(16, dtype=torch.long, device="cuda")
    ids = torch.tensor([417, 9], dtype=torch.long, device="cuda")
    assert _call(ids, emb, x, out, steps, pos, tok) == 0
    torch.cuda.synchronize()
    assert torch.equal(x[0], emb[417].float()) and torch.all(x[1] == 7.0)
    assert out.tolist() == [-5, -5, -5, 417, -5, -5, -5, -5]
    assert steps.item() == 4 and pos.item() == 101 and tok[0].item() == 417 and tok[1].item() == 0
    # steps outside [0, out_len): nothing recorded, counters still advance;
    # an id past the vocabulary takes the last row; tok may be NULL
    ids[0] = V + 50
    steps.fill_(8)
    assert _call(ids, emb, x, out, steps, pos, None) == 0
    torch.cuda.synchronize()
    assert torch.equal(x[0], emb[V - 1].float())
    assert out.tolist() == [-5, -5, -5, 417, -5, -5, -5, -5]
    assert steps.item() == 9 and pos.item() == 102 and tok[0].item() == 417
    ids[0] = 5
    steps.fill_(2)
    assert _call(ids, emb, x, out, steps, pos, tok, out_len=2) == 0  # out_len bounds the write
    torch.cuda.synchronize()
    assert out.tolist() == [-5, -5, -5, 417, -5, -5, -5, -5] and torch.equal(x[0], emb[5].float())


@pytest.mark.parametrize("H", [1024, 1004, 10240, 12])
def test_decode_advance_row_widths(H):
    """The embedding row copy at widths that take the 16-byte path (1024,
    10240: more than one round of loads per thread) and the element path
    (1004 and 12: rows not 16-byte aligned); nothing past the row is written."""
    g = torch.Generator(device="cuda").manual_seed(H)
    V = 64
    emb = torch.randn(V, H, device="cuda", generator=g).bfloat16()
    x = torch.full((H + 8,), 7.0, device="cuda")
    out = torch.full((4,), -5, dtype=torch.long, device="cuda")
    steps = torch.tensor([0], dtype=torch.long, device="cuda")
    pos = torch.tensor([0], dtype=torch.long, device="cuda")
    for i, tid in enumerate((37, 1, V - 1)):
        ids = torch.tensor([tid], dtype=torch.long, device="cuda")
        assert _call(ids, emb, x, out, steps, pos, None) == 0
        torch.cuda.synchronize()
        assert torch.equal(x[:H], emb[tid].float()) and torch.all(x[H:] == 7.0)
        assert out[i].item() == tid and steps.item() == i + 1 and pos.item() == i + 1
