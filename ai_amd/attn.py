"""Attention of one layer through librv12.so: q/k head RMSNorm, RoPE at a
device-side position, K/V into the cache, grouped-query attention.  One token
(rv12_rope_attn: the reference's rope_attn_k,
ramvi/engine/ramvi_engine/kernels/tkernels.py:164-213) or a batch of up to 16
tokens of one sequence, each attending causally (rv12_rope_attn_batch: the
reference's qk_rope_cache_k + attn_k, tkernels.py:82-150), or a whole prompt
block (rv12_prefill_rope_attn: qk_rope_cache_k + att_k of the blocked prefill,
ramvi/engine/ramvi_engine/kernels/prefill.py:100-103,
prefill_kernels.py:29-54)."""
import ctypes

import torch

from ._lib import Attn, check, lib


SPAN = 80  # positions one workgroup covers at most
LONG_SPAN = 256  # one split per kv head covers up to this many (no combine pass)
MAX_SPLITS = 128


def default_splits(n_kv, maxt, kv_bf16=True, head_dim=128):
    """Position splits: one for a context of up to 256 positions (one
    workgroup per kv head, no combine launch; not for float32 caches of
    128-dim heads, whose long-span workgroup would spill registers); else
    each workgroup covers at most 80 positions, and there are at least 256
    workgroups while each keeps >= 16 positions."""
    if maxt <= LONG_SPAN and (kv_bf16 or head_dim <= 64):
        return 1
    need = -(-maxt // SPAN)
    want = min(-(-256 // n_kv), -(-maxt // 16))
    s = max(1, need, want)
    if s > MAX_SPLITS:
        raise ValueError("the attention kernel covers at most 10240 positions")
    return int(s)


class RopeAttn:
    """Launch parameters and workspace for one model's caches."""

    def __init__(self, n_heads, n_kv, head_dim, maxt, kv_dtype, eps, device, splits=None):
        if kv_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("the cache must be float32 or bfloat16")
        bf16 = kv_dtype == torch.bfloat16
        self.a = Attn(n_heads, n_kv, head_dim, maxt, 1 if bf16 else 0,
                      splits or default_splits(n_kv, maxt, bf16, head_dim), float(eps), float(head_dim ** -0.5))
        need = lib().rv12_attn_workspace_bytes(ctypes.byref(self.a))
        self.ws = torch.empty(max(need, 16), dtype=torch.uint8, device=device)
        need = lib().rv12_attn_batch_workspace_bytes(ctypes.byref(self.a), 16)
        self.wsb = torch.empty(max(need, 16), dtype=torch.uint8, device=device)

    def _check(self, qkv, qn, kn, inv, pos, kc, vc, out, T):
        """The tensors' dtypes, layouts, sizes and device: the C ABI sees only
        pointers, so a cache of another dtype or shape than this object's
        would be written out of bounds."""
        a = self.a
        for t in (qkv, qn, kn, inv, out):
            if t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError("qkv, qn, kn, inv and out must be contiguous float32")
        if pos.dtype != torch.int64 or pos.numel() < 1:
            raise ValueError("pos must be int64")
        dev = qkv.device
        if any(t.device != dev for t in (qn, kn, inv, pos, kc, vc, out)):
            raise ValueError("every tensor must be on the device of qkv")
        if qkv.numel() < T * (a.n_heads + 2 * a.n_kv) * a.head_dim or out.numel() < T * a.n_heads * a.head_dim:
            raise ValueError(f"qkv and out need {T} rows")
        if qn.numel() < a.head_dim or kn.numel() < a.head_dim or inv.numel() < a.head_dim // 2:
            raise ValueError("qn, kn need head_dim entries and inv head_dim / 2")
        want = torch.bfloat16 if a.kv_bf16 else torch.float32
        for c in (kc, vc):
            if c.dtype != want or not c.is_contiguous() or tuple(c.shape) != (a.n_kv, a.maxt, a.head_dim):
                raise ValueError(f"kc and vc must be contiguous {want} caches of shape "
                                 f"({a.n_kv}, {a.maxt}, {a.head_dim})")

    def __call__(self, qkv, qn, kn, inv, pos, kc, vc, out):
        self._check(qkv, qn, kn, inv, pos, kc, vc, out, 1)
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        rc = lib().rv12_rope_attn(ctypes.byref(self.a), p(qkv), p(qn), p(kn), p(inv), p(pos), p(kc), p(vc), p(out),
                                  p(self.ws), self.ws.numel(),
                                  ctypes.c_void_p(torch.cuda.current_stream(qkv.device).cuda_stream))
        check(rc, "rope_attn")

    def batch(self, qkv, qn, kn, inv, pos, kc, vc, out, T):
        """T <= 16 tokens at positions pos .. pos + T - 1: rows of qkv in, rows
        of out written; K/V of the T positions into the caches."""
        self._check(qkv, qn, kn, inv, pos, kc, vc, out, int(T))
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        rc = lib().rv12_rope_attn_batch(ctypes.byref(self.a), int(T), p(qkv), p(qn), p(kn), p(inv), p(pos), p(kc),
                                        p(vc), p(out), p(self.wsb), self.wsb.numel(),
                                        ctypes.c_void_p(torch.cuda.current_stream(qkv.device).cuda_stream))
        check(rc, "rope_attn_batch")

    def prefill(self, qkv, qn, kn, inv, pos, kc, vc, out, T):
        """A prompt block of T tokens at positions pos .. pos + T - 1 (pos a
        device int64): rows of qkv in, rows of out written; K/V of the T
        positions into the caches.  The q rows live in a workspace kept for
        the largest T seen."""
        self._check(qkv, qn, kn, inv, pos, kc, vc, out, int(T))
        L = lib()
        need = L.rv12_prefill_attn_workspace_bytes(ctypes.byref(self.a), int(T))
        if need == 0:
            raise ValueError("prefill attention: unsupported block (tokens, context or head size)")
        ws = getattr(self, "wsp", None)
        if ws is None or ws.numel() < need:
            ws = self.wsp = torch.empty(need, dtype=torch.uint8, device=qkv.device)
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        rc = L.rv12_prefill_rope_attn(ctypes.byref(self.a), int(T), p(qkv), p(qn), p(kn), p(inv), p(pos), p(kc),
                                      p(vc), p(out), p(ws), ws.numel(),
                                      ctypes.c_void_p(torch.cuda.current_stream(qkv.device).cuda_stream))
        check(rc, "prefill_rope_attn")
