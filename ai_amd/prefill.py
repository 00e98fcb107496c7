"""Blocked prefill on MI355X: the reference's opt-in prompt path
(ramvi/engine/ramvi_engine/kernels/prefill.py, RAMVI_PREFILL=blocked, from
RAMVI_PREFILL_MIN_TOKENS = 256 prompt tokens on): every weight matrix is
decoded exactly once per prompt and multiplied with ALL prompt tokens in one
dense GEMM, instead of passes of 16 tokens through the fused decode-linear.

    enabled(n)                                       prefill.py:14-20  (same variables, same errors)
    matrix(x, c, y, add)                             prefill.py:66-78
    layer(eng, l, weights, x, start, kc, vc, gguf)   prefill.py:81-121 (same signature)

MI355X form of `matrix`: one fused kernel chain in librv12
(rv12_prefill_linear): the fp32 activations of all prompt tokens are split
once into three bf16 parts (24 significand bits, after an exact per-token
power-of-two scale, the reference's own split for bf16 matrix units,
ramvi/engine/ramvi_engine/kernels/wcomp.py:130-140), and a hand-written
bf16 MFMA GEMM reads each weight once in its 12-bit packed form (the Q16
tiles are the MFMA's A operand), accumulates in fp32 and adds the
exceptions; no wider copy of W is ever written.  The reference computes the
same sums with IEEE fp32 products after decoding W to fp32
(prefill_kernels.py:8-26, 58-110); both are fp32 evaluations of the same
closed form, held to the same error bound in the tests.

The q/k head norms, RoPE, the cache writes and the attention over the prompt
(qk_rope_cache_k, tkernels.py:82-150, and att_k, prefill_kernels.py:29-54)
are one library call, rv12_prefill_rope_attn: the same causal softmax with
float32 products, on the float32 matrix cores.
"""
import os

import torch

from . import wcomp
from .attn import RopeAttn


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


_WS = {}  # device -> workspace of the prefill linear (the split activations)


def _linear(x, c, y, mode, lnw=None, eps=1e-6):
    """y (=|+=) W x' over every token row of x (fp32 [T, K], [T, 2K] in mode
    2); lnw (bf16 [K]) fuses the row's RMSNorm, as gemvc1 does."""
    import ctypes
    from . import _lib
    T = x.shape[0]
    K, N = int(c["K"]), int(c["N"])
    if x.dtype != torch.float32 or y.dtype != torch.float32 or not x.is_contiguous() or not y.is_contiguous():
        raise ValueError("prefill: x and y must be contiguous float32")
    if x.shape[1] != (2 * K if mode == 2 else K) or y.numel() < T * N:
        raise ValueError("prefill: x or y has the wrong shape")
    if lnw is not None and (lnw.dtype != torch.bfloat16 or not lnw.is_contiguous() or lnw.numel() < K):
        raise ValueError("prefill: lnw must be a contiguous bf16 vector of K entries")
    L = _lib.lib()
    need = L.rv12_prefill_workspace_bytes(N, K, T)
    if need == 0:
        raise ValueError("prefill: too many tokens")
    key = str(x.device)
    if key not in _WS or _WS[key].numel() < need:
        _WS[key] = torch.empty(need, dtype=torch.uint8, device=x.device)
    ws = _WS[key]
    rc = L.rv12_prefill_linear(ctypes.byref(wcomp._matrix(c)), ctypes.c_void_p(x.data_ptr()),
                               ctypes.c_void_p(y.data_ptr()), T,
                               None if lnw is None else ctypes.c_void_p(lnw.data_ptr()), float(eps), int(mode),
                               ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                               ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream))
    _lib.check(rc, "prefill")


def matrix(x, c, y, add=False, lnw=None, eps=1e-6):
    """y (=|+=) x . W^T for every token row of x (fp32 [T, K]); W read once
    in its 12-bit form (prefill.py:66-78).  lnw: the rows' RMSNorm (rmsg_k,
    prefill.py:94) fused into the linear."""
    _linear(x, c, y, 1 if add else 0, lnw, eps)


_ATT = {}  # (dimensions, cache, device) -> RopeAttn launch parameters and workspace
_POS = {}  # device -> the block's first position (int64 on the device)


def _attn(eng, kc):
    key = (eng.H, eng.KV, eng.HD, kc.shape[1], kc.dtype, float(eng.eps), str(kc.device))
    if key not in _ATT:
        _ATT[key] = RopeAttn(eng.H, eng.KV, eng.HD, kc.shape[1], kc.dtype, eng.eps, kc.device)
    return _ATT[key]


def _pos(device, start):
    key = str(device)
    if key not in _POS:
        _POS[key] = torch.zeros(1, dtype=torch.int64, device=device)
    return _POS[key].fill_(start)


def layer(eng, l, weights, x, start, kc, vc, gguf=False):
    """One layer over all prompt rows x (fp32 [T, D], updated in place) at
    positions start.. (prefill.py:81-121, same signature): RMSNorm fused into
    qkv, q/k head norms, RoPE, K/V into the caches kc / vc (rounded to their
    dtype), causal attention, o (residual add), RMSNorm fused into gate/up,
    silu(g) * u fused into down (residual add): five library calls.  weights: the layer's fused 12-bit matrices qkv, o, gu,
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
    bf = lambda t: t.to(torch.bfloat16).contiguous()
    qkv = torch.empty(T, (H + 2 * KV) * HD, device=x.device)
    matrix(x, W["qkv"], qkv, lnw=bf(s["ln1"]), eps=eps)
    f32 = lambda t: t.float().contiguous()
    att = torch.empty(T, H * HD, device=x.device)
    _attn(eng, kc).prefill(qkv, f32(s["qn"]), f32(s["kn"]), f32(eng.inv), _pos(x.device, start), kc, vc, att, T)
    del qkv
    matrix(att, W["o"], x, add=True)
    del att
    gu = torch.empty(T, 2 * FF, device=x.device)
    matrix(x, W["gu"], gu, lnw=bf(s["ln2"]), eps=eps)
    _linear(gu, W["down"], x, 2)  # silu(g) * u fused into the linear's prologue
    del gu
