"""Blocked prefill on MI355X: the reference's opt-in prompt path
(ramvi/engine/ramvi_engine/kernels/prefill.py, RAMVI_PREFILL=blocked, from
RAMVI_PREFILL_MIN_TOKENS = 256 prompt tokens on): every weight matrix is
decoded exactly once per prompt and multiplied with ALL prompt tokens in one
dense GEMM, instead of passes of 16 tokens through the fused decode-linear.

    enabled(n)                                       prefill.py:14-20  (same variables, same errors)
    matrix(x, c, y, add)                             prefill.py:66-78
    layer(eng, l, weights, x, start, kc, vc, gguf)   prefill.py:81-121 (same signature)

MI355X form of `matrix`: the 12-bit matrix is decoded to its exact bf16 bits
(rv12_decode_rows), and the fp32 activations are split into three bf16 parts
x = hi + mid + lo (the reference's own split for bf16 matrix units,
ramvi/engine/ramvi_engine/kernels/wcomp.py:130-140; the parts carry all 24
significand bits of a normal fp32 value).  One hipBLASLt GEMM over the stacked
parts [hi; mid; lo] (3T x K) with fp32 output runs on the bf16 MFMA units;
every product w * part is exact in fp32 and the sums are fp32, and
(hi + mid) + lo is added in fp32.  The reference computes the same sums with
IEEE fp32 products (prefill_kernels.py:8-26, input_precision='ieee'); both
are fp32 evaluations of the same closed form, held to the same error bound in
the tests.  The decode of a matrix is bit-exact, so the weights are the
reference's, not a re-quantisation.

Attention over the prompt (prefill_kernels.py:35-60, att_k) is the same causal
softmax in fp32, computed in query blocks of ATT_BLOCK tokens with fp32 IEEE
batched products over the whole cache prefix.
"""
import os

import torch

from . import wcomp

ATT_BLOCK = 256  # query tokens per attention block


def enabled(n=None):
    """RAMVI_PREFILL=blocked and at least RAMVI_PREFILL_MIN_TOKENS (256)
    prompt tokens (prefill.py:14-20)."""
    mode = os.environ.get("RAMVI_PREFILL", "legacy")
    if mode not in ("legacy", "blocked"):
        raise ValueError("RAMVI_PREFILL должен быть legacy или blocked (RAMVI_PREFILL must be legacy or blocked)")
    minimum = int(os.environ.get("RAMVI_PREFILL_MIN_TOKENS", "256"))
    if minimum < 0:
        raise ValueError("RAMVI_PREFILL_MIN_TOKENS должен быть неотрицательным (must not be negative)")
    return mode == "blocked" and (n is None or n >= minimum)


def split3(x):
    """fp32 [T, K] -> bf16 [3T, K]: hi, mid, lo with hi + mid + lo = x."""
    hi = x.bfloat16()
    r = x - hi.float()
    mid = r.bfloat16()
    lo = (r - mid.float()).bfloat16()
    return torch.cat([hi, mid, lo], 0)


def matrix(x, c, y, add=False):
    """y (=|+=) x . W^T for every token row of x (fp32 [T, K]); W decoded
    exactly from the 12-bit codec (prefill.py:66-78)."""
    T = x.shape[0]
    N = int(c["N"])
    w = wcomp.decode_rows(c, 0, N, torch.bfloat16)  # exact bf16 bits of W
    parts = torch.mm(split3(x), w.t(), out_dtype=torch.float32)  # [3T, N]
    del w
    v = parts[:T]
    v.add_(parts[T:2 * T]).add_(parts[2 * T:])
    if add:
        y.add_(v)
    else:
        y.copy_(v)


def _rms(x, w, eps):
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def _rot(t):
    h = t.shape[-1] // 2
    return torch.cat([-t[..., h:], t[..., :h]], -1)


def attention(eng, q, start, kc, vc):
    """Causal grouped-query attention of the T prompt rows q (fp32 [T, H, HD],
    positions start..start+T-1) over positions 0..start+T-1 of the caches
    kc / vc [KV, maxt, HD], in query blocks (prefill_kernels.py:35-60)."""
    T = q.shape[0]
    H, KV, HD = eng.H, eng.KV, eng.HD
    G = H // KV
    n = start + T
    Kf = kc[:, :n].float()                             # [KV, n, HD]
    Kt = Kf.transpose(1, 2).contiguous()               # [KV, HD, n]
    Vf = vc[:, :n].float().contiguous()                # [KV, n, HD]
    del Kf
    out = torch.empty(T, H * HD, device=q.device)
    cols = torch.arange(n, device=q.device)
    for b0 in range(0, T, ATT_BLOCK):
        b1 = min(T, b0 + ATT_BLOCK)
        tb = b1 - b0
        qg = q[b0:b1].view(tb, KV, G, HD).permute(1, 2, 0, 3).reshape(KV, G * tb, HD)
        sc = torch.bmm(qg, Kt).view(KV, G, tb, n) * HD ** -0.5
        rows = start + torch.arange(b0, b1, device=q.device)
        sc.masked_fill_(cols[None, None, None, :] > rows[None, None, :, None], float("-inf"))
        a = torch.softmax(sc, -1).view(KV, G * tb, n)
        o = torch.bmm(a, Vf).view(KV, G, tb, HD).permute(2, 0, 1, 3).reshape(tb, H * HD)
        out[b0:b1].copy_(o)
    return out


def layer(eng, l, weights, x, start, kc, vc, gguf=False):
    """One layer over all prompt rows x (fp32 [T, D], updated in place) at
    positions start.. (prefill.py:81-121, same signature): RMSNorm, qkv, q/k
    head norms, RoPE, K/V into the caches kc / vc (rounded to their dtype),
    causal attention, o (residual add), RMSNorm, gate/up, silu(g) * u, down
    (residual add).  weights: the layer's fused 12-bit matrices qkv, o, gu,
    down; eng supplies the dimensions, eng.small[l] the norm weights and
    eng.inv the RoPE frequencies.  gguf=True (separate q/k/v and gate/up GGUF
    matrices) belongs to the reference's GGUF engine, which is not on this
    path."""
    if gguf:
        raise NotImplementedError("GGUF weights are not on the 12-bit path")
    T = x.shape[0]
    H, KV, HD, FF, eps = eng.H, eng.KV, eng.HD, eng.FF, eng.eps
    W = weights
    s = eng.small[l]
    norm = _rms(x, s["ln1"].float(), eps)
    qkv = torch.empty(T, (H + 2 * KV) * HD, device=x.device)
    matrix(norm, W["qkv"], qkv)
    q = _rms(qkv[:, :H * HD].view(T, H, HD), s["qn"], eps)
    k = _rms(qkv[:, H * HD:(H + KV) * HD].view(T, KV, HD), s["kn"], eps)
    v = qkv[:, (H + KV) * HD:].view(T, KV, HD)
    p = start + torch.arange(T, device=x.device)
    ang = p[:, None].float() * eng.inv[None]
    e = torch.cat([ang, ang], -1)
    cos, sin = e.cos()[:, None], e.sin()[:, None]
    q = q * cos + _rot(q) * sin
    k = k * cos + _rot(k) * sin
    kc.index_copy_(1, p, k.to(kc.dtype).transpose(0, 1))
    vc.index_copy_(1, p, v.to(vc.dtype).transpose(0, 1))
    del qkv, k, v
    att = attention(eng, q, start, kc, vc)
    del q
    matrix(att, W["o"], x, add=True)
    del att
    norm = _rms(x, s["ln2"].float(), eps)
    gu = torch.empty(T, 2 * FF, device=x.device)
    matrix(norm, W["gu"], gu)
    del norm
    g = gu[:, :FF]
    mid = g / (1.0 + torch.exp(-g)) * gu[:, FF:]
    del gu
    matrix(mid, W["down"], x, add=True)
