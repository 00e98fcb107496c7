"""float32 Qwen3 forward for greedy-token parity.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates the reference's independent fp32 oracle, `Reference.argmax`
(ramvi/engine/ramvi_engine/core/reference.py:24-61): one teacher-forced pass
over prompt + generated tokens in plain torch float32 on the CPU (Hugging Face
Qwen3 math: RMSNorm, q/k head norms, rotate-half RoPE with
inv = 1 / theta^(2i / HD), grouped-query causal attention, SwiGLU MLP, final
norm, lm_head), returning the argmax at every position with the smallest id
on ties (reference.py:52-60, head.py:76-79).

kv_dtype: the keys and values are rounded to this dtype before attention, as
an engine with a cache of that dtype stores them
(ramvi/engine/ramvi_engine/kernels/tkernels.py:187-190; the reference's
validation oracle rounds to its fp16 cache the same way).

device: where the float32 forward runs.  Only "cpu" is accepted: the oracle
runs on the host, apart from the GPU code it checks.  Token ids and picks are
range-checked on the host before any indexing.
"""
import torch


def _host(device):
    dev = torch.device(device)
    if dev.type != "cpu":
        raise ValueError("the oracle runs on the CPU only (device must be 'cpu')")
    return dev


def _ids_in_range(ids, V, what):
    bad = [i for i in ids if not 0 <= int(i) < V]
    if bad:
        raise ValueError(f"{what} outside [0, {V}): {bad[:8]}")


def rms(x, w, eps):
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def rotate_half(t):
    HD = t.shape[-1]
    return torch.cat([-t[..., HD // 2:], t[..., :HD // 2]], -1)


@torch.no_grad()
def hidden(ck, tokens, kv_dtype=torch.float32, rotate=rotate_half, device="cpu"):
    """Final-norm hidden states [T, D] of a teacher-forced pass over `tokens`
    (reference.py:26-51)."""
    H, KV, HD, eps, F = ck.H, ck.KV, ck.HD, ck.eps, ck.FF
    T = len(tokens)
    dev = _host(device)
    _ids_in_range(tokens, ck.V, "tokens")
    emb = ck.t("model.embed_tokens.weight", dev)
    x = emb[torch.tensor(tokens, device=dev)].float()
    del emb
    inv = (1.0 / (ck.theta ** (torch.arange(0, HD, 2, dtype=torch.int64).float() / HD))).to(dev)
    fr = torch.arange(T, device=dev).float()[:, None] * inv[None]
    e = torch.cat([fr, fr], -1)
    cos, sin = e.cos(), e.sin()
    mask = torch.full((T, T), float("-inf"), device=dev).triu(1)
    for i in range(ck.L):
        w = {k: v.float() for k, v in ck.layer(i, dev).items()}
        h = rms(x, w["ln1"], eps)
        qkv = h @ w["qkv"].T
        q = rms(qkv[:, :H * HD].view(T, H, HD), w["qn"], eps)
        k = rms(qkv[:, H * HD:(H + KV) * HD].view(T, KV, HD), w["kn"], eps)
        v = qkv[:, (H + KV) * HD:].view(T, KV, HD)
        q = q * cos[:, None] + rotate(q) * sin[:, None]
        k = k * cos[:, None] + rotate(k) * sin[:, None]
        k, v = k.to(kv_dtype).float(), v.to(kv_dtype).float()
        k, v = k.repeat_interleave(H // KV, 1), v.repeat_interleave(H // KV, 1)
        qh, kt, vh = q.transpose(0, 1).contiguous(), k.permute(1, 2, 0).contiguous(), v.transpose(0, 1).contiguous()
        del q, k, v
        a = torch.softmax((qh @ kt) * HD ** -0.5 + mask, -1)
        del qh, kt
        x = x + (a @ vh).transpose(0, 1).reshape(T, H * HD) @ w["o"].T
        del a, vh
        h = rms(x, w["ln2"], eps)
        gu = h @ w["gu"].T
        x = x + (torch.nn.functional.silu(gu[:, :F]) * gu[:, F:]) @ w["down"].T
        del w
    return rms(x, ck.t("model.norm.weight", dev).float(), eps)


@torch.no_grad()
def logits(ck, tokens, kv_dtype=torch.float32, **kw):
    """Full-vocabulary float32 logits [T, V] (small vocabularies only)."""
    h = hidden(ck, tokens, kv_dtype, **kw)
    return h @ ck.t(ck.head_name(), h.device).float().T


@torch.no_grad()
def argmax(ck, tokens, kv_dtype=torch.float32, head_chunk=16384, margins=False, device="cpu", first=0, picks=None):
    """Greedy next-token ids at every position of `tokens` (a list of ints)
    from position `first` on, smallest id on ties (reference.py:52-60).  With
    margins=True also the gap between the best and the second-best logit of
    each position; with picks (one token id per position from `first` on)
    also the gap between the best logit and the logit of each pick."""
    h = hidden(ck, tokens, kv_dtype, device=device)[first:]
    T = h.shape[0]
    dev = h.device
    head = ck.t(ck.head_name(), dev)
    best = torch.full((T,), -float("inf"), device=dev)
    second = torch.full((T,), -float("inf"), device=dev)
    arg = torch.zeros(T, dtype=torch.long, device=dev)
    if picks is not None:
        if len(picks) != T:
            raise ValueError(f"picks must hold one id per position from first on ({T})")
        _ids_in_range(picks, head.shape[0], "picks")
    pk = None if picks is None else torch.tensor(picks, dtype=torch.long, device=dev)
    pick_logit = torch.zeros(T, device=dev)
    for i in range(0, head.shape[0], head_chunk):
        lg = h @ head[i:i + head_chunk].float().T
        if pk is not None:
            inside = (pk >= i) & (pk < i + lg.shape[1])
            col = (pk - i).clamp(0, lg.shape[1] - 1)
            pick_logit = torch.where(inside, lg.gather(1, col[:, None])[:, 0], pick_logit)
        v, j = lg.max(-1)                      # first maximum inside the chunk
        if margins:                            # running second-best logit
            top2 = lg.topk(min(2, lg.shape[1]), -1).values
            c2 = top2[:, 1] if top2.shape[1] > 1 else torch.full((T,), -float("inf"), device=dev)
            second = torch.stack([second, c2, torch.minimum(best, v)], 1).max(1).values
        better = v > best                      # an earlier chunk wins a tie: smallest id
        arg = torch.where(better, j + i, arg)
        best = torch.where(better, v, best)
    out = [arg.tolist()]
    if margins:
        out.append((best - second).tolist())
    if pk is not None:
        out.append((best - pick_logit).tolist())
    return out[0] if len(out) == 1 else tuple(out)
