"""Closed forms of the reference's fused decode-linears, in float64.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Both reference kernels compute, for T token rows,
    Y[t] (=|+=) W_dec . x'[t]
with W_dec the exactly decoded weights (wcomp.py:48-54 plus the exception list)
and the input prologue
    MODE 0, 1 : x'[t] = X[t, 0:K]                               (wcomp.py:57-64)
    MODE 2    : x'[t] = g / (1 + exp(-g)) * u, g = X[t, 0:K], u = X[t, K:2K]
    RMS       : x'[t] = lnw * (x'[t] * rs),
                rs = rsqrt(sum_k X[t, k]^2 / K + eps)             (wcomp.py:75-86)
and the epilogue MODE 0 store, MODE 1/2 accumulate (wcomp.py:109-112, 210-219).
X rows are 2K floats apart in MODE 2 and K floats otherwise (wcomp.py:166);
Y rows are N floats apart (wcomp.py:199).
"""
import numpy as np

from .codec import decode_f32


def prologue(X, K, mode, lnw=None, eps=1e-6):
    """x' (float64[T, K]) from the float32 activation rows X[T, K or 2K]."""
    X = np.asarray(X, dtype=np.float64)
    if X.ndim == 1:
        X = X[None, :]
    if mode == 2:
        g, u = X[:, :K], X[:, K:2 * K]
        with np.errstate(over="ignore"):
            xp = g / (1.0 + np.exp(-g)) * u
    elif mode in (0, 1):
        xp = X[:, :K].copy()
    else:
        raise ValueError("mode must be 0, 1 or 2")
    if lnw is not None:
        rs = 1.0 / np.sqrt((X[:, :K] ** 2).sum(1, keepdims=True) / K + eps)
        xp = np.asarray(lnw, dtype=np.float64)[None, :] * (xp * rs)
    return xp


def linear(c, X, mode, y_prev=None, lnw=None, eps=1e-6, W=None):
    """Y (float64[T, N]) = prologue(X) @ W_dec^T, plus y_prev for MODE 1/2."""
    N, K = c["N"], c["K"]
    if W is None:
        W = decode_f32(c).astype(np.float64)
    xp = prologue(X, K, mode, lnw, eps)
    with np.errstate(invalid="ignore", over="ignore"):
        out = xp @ W.T
    if mode == 0:
        return out
    if y_prev is None:
        raise ValueError("MODE 1/2 accumulate into y_prev")
    return np.asarray(y_prev, dtype=np.float64).reshape(out.shape) + out


def error_bound(c, X, mode, lnw=None, eps=1e-6, W=None):
    """Forward-error scale of an fp32 evaluation: K * 2^-24 * sum_k |w_k x'_k|
    per output (the textbook bound for a K-term fp32 dot product), plus the
    rounding of the prologue itself."""
    N, K = c["N"], c["K"]
    if W is None:
        W = decode_f32(c).astype(np.float64)
    xp = prologue(X, K, mode, lnw, eps)
    with np.errstate(invalid="ignore", over="ignore"):
        mag = np.abs(xp) @ np.abs(W).T
    return (K + 8) * 2.0 ** -24 * mag


def brute_force(c, X, mode, y_prev=None, lnw=None, eps=1e-6):
    """Loop form of `linear` for tiny shapes: one scalar sum per output."""
    import math
    N, K = c["N"], c["K"]
    W = decode_f32(c)
    X = np.atleast_2d(np.asarray(X, dtype=np.float64))
    T = X.shape[0]
    Y = np.zeros((T, N))
    for t in range(T):
        if lnw is not None:
            ss = 0.0
            for k in range(K):
                ss += X[t, k] * X[t, k]
            rs = 1.0 / math.sqrt(ss / K + eps)
        for n in range(N):
            s = 0.0
            for k in range(K):
                if mode == 2:
                    g, u = X[t, k], X[t, K + k]
                    xk = g / (1.0 + math.exp(-g)) * u
                else:
                    xk = X[t, k]
                if lnw is not None:
                    xk = float(lnw[k]) * (xk * rs)
                s += float(W[n, k]) * xk
            Y[t, n] = s if mode == 0 else float(np.asarray(y_prev).reshape(T, N)[t, n]) + s
    return Y
