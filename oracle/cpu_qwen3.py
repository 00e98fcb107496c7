"""Qwen3 greedy decoding on the CPU through the C oracle: the reference CPU
layer (CpuLayer.__call__, ramvi/engine/ramvi_engine/cpu/cpu_layer.py:155-175:
rms_rows, matmat16 for qkv, qk_rope_attn with float32 caches, matmat16 for o
into the residual, rms_rows, matmat16 for gate/up, silu_mul, matmat16 for
down into the residual) over every layer, the final RMSNorm, and the exact
head over the whole vocabulary (bf16 rows, fp32 sums; the greedy id with the
smallest id on ties, ramvi/engine/ramvi_engine/generation/head.py:19-26,
76-79).  The prompt goes through each layer as one batch of rows, then one
token per step.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the CPU baseline of the
end-to-end decode in bench.py.
"""
import time

import numpy as np

from . import cref


def _bits(t):
    import torch
    return np.ascontiguousarray(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def _f32(t):
    return np.ascontiguousarray(t.float().cpu().numpy())


def load(ck, device="cpu"):
    """Host copies of a checkpoint's tensors (bf16 bits for the matrices and
    the embedding, float32 for the norms); tensors are produced on `device`
    (a RandomCkpt draws its values there) and copied to host memory."""
    layers = []
    for i in range(ck.L):
        w = ck.layer(i, device)
        layers.append({"qkv": _bits(w["qkv"]), "o": _bits(w["o"]), "gu": _bits(w["gu"]), "down": _bits(w["down"]),
                       "ln1": _f32(w["ln1"]), "ln2": _f32(w["ln2"]), "qn": _f32(w["qn"]), "kn": _f32(w["kn"])})
        del w
    emb = _bits(ck.t("model.embed_tokens.weight", device))
    head = emb if ck.head_name() == "model.embed_tokens.weight" else _bits(ck.t(ck.head_name(), device))
    inv = (1.0 / (ck.theta ** (np.arange(0, ck.HD, 2, dtype=np.int64).astype(np.float32) / ck.HD))).astype(np.float32)
    return {"layers": layers, "emb": emb, "head": head, "norm": _f32(ck.t("model.norm.weight", device)),
            "inv": inv, "H": ck.H, "KV": ck.KV, "HD": ck.HD, "FF": ck.FF, "D": ck.D, "eps": float(ck.eps)}


def _layer(m, l, X, pos0, caches, threads):
    """CpuLayer.__call__ (cpu_layer.py:155-175) on rows X [T, D], in place."""
    T = X.shape[0]
    H, KV, HD, FF, eps = m["H"], m["KV"], m["HD"], m["FF"], m["eps"]
    w = m["layers"][l]
    h = np.empty_like(X)
    cref.rms_rows(X, w["ln1"], h, eps)
    qkv = np.empty((T, (H + 2 * KV) * HD), np.float32)
    cref.gemv_bf16(w["qkv"], h, qkv, add=False, threads=threads)
    att = np.empty((T, H * HD), np.float32)
    Kc, Vc = caches[l]
    cref.qk_rope_attn(qkv, w["qn"], w["kn"], m["inv"], pos0, Kc, Vc, att, H, KV, HD, eps, threads)
    cref.gemv_bf16(w["o"], att, X, add=True, threads=threads)
    cref.rms_rows(X, w["ln2"], h, eps)
    gu = np.empty((T, 2 * FF), np.float32)
    cref.gemv_bf16(w["gu"], h, gu, add=False, threads=threads)
    mid = np.empty((T, FF), np.float32)
    cref.silu_mul(gu, mid, FF)
    cref.gemv_bf16(w["down"], mid, X, add=True, threads=threads)


def _pick(m, x, threads):
    """Exact greedy id of the last row of x: final norm, every logit, the
    first maximum (smallest id on ties)."""
    h = np.empty((1, m["D"]), np.float32)
    cref.rms_rows(np.ascontiguousarray(x[-1:]), m["norm"], h, m["eps"])
    lg = np.empty((1, m["head"].shape[0]), np.float32)
    cref.gemv_bf16(m["head"], h, lg, add=False, threads=threads)
    return int(np.argmax(lg[0]))


def _embed(m, tokens):
    return (m["emb"][np.asarray(tokens)].astype(np.uint32) << 16).view(np.float32)


def generate(m, prompt, new, threads=0, maxt=None):
    """(ids, prefill seconds, decode seconds) of `new` greedy tokens after
    `prompt`."""
    maxt = maxt or len(prompt) + new
    L, KV, HD = len(m["layers"]), m["KV"], m["HD"]
    caches = [(np.zeros((KV, maxt, HD), np.float32), np.zeros((KV, maxt, HD), np.float32)) for _ in range(L)]
    t0 = time.perf_counter()
    X = np.ascontiguousarray(_embed(m, prompt))
    for l in range(L):
        _layer(m, l, X, 0, caches, threads)
    ids = [_pick(m, X, threads)]
    t1 = time.perf_counter()
    pos = len(prompt)
    while len(ids) < new:
        x = np.ascontiguousarray(_embed(m, ids[-1:]))
        for l in range(L):
            _layer(m, l, x, pos, caches, threads)
        ids.append(_pick(m, x, threads))
        pos += 1
    t2 = time.perf_counter()
    return ids, t1 - t0, t2 - t1
