"""ctypes binding of the C oracle (oracle/c/rv12_oracle.c).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Build with `make -C oracle`.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "librvoracle.so")
_lib = None


def build():
    import subprocess
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"C oracle not built: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        P, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.rvo_compress.restype = I64
        L.rvo_compress.argtypes = [P, I, I, I, P, P, P, P, P, P, I64, ctypes.POINTER(I)]
        L.rvo_choose_base.restype = I
        L.rvo_choose_base.argtypes = [P, I64]
        L.rvo_decode.restype = None
        L.rvo_decode.argtypes = [P, P, I, P, P, P, I64, I, I, I, P]
        L.rvo_gemv_bf16.restype = None
        L.rvo_gemv_bf16.argtypes = [P, P, P, I, I, I, I, I]
        L.rvo_gemv_12bit.restype = I
        L.rvo_gemv_12bit.argtypes = [P, P, I, P, P, P, P, P, P, F, I, I, I, I, I, I]
        L.rvo_rms_rows.restype = None
        L.rvo_rms_rows.argtypes = [P, P, P, I, I, F]
        L.rvo_qk_rope_attn.restype = None
        L.rvo_qk_rope_attn.argtypes = [P, P, P, P, I, P, P, I, P, I, I, I, I, F, I]
        L.rvo_silu_mul.restype = None
        L.rvo_silu_mul.argtypes = [P, P, I, I]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def compress(w_bits, CH=256):
    """Same dict as oracle.codec.compress, computed in C (for large matrices)."""
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    N, K = w_bits.shape
    m8 = np.empty((N, K), np.uint8)
    e4 = np.zeros((N, K // 2), np.uint8)
    rp = np.empty(N + 1, np.int32)
    base = ctypes.c_int(0)
    cap = max(1024, N * K // 256)
    while True:
        er = np.empty(cap, np.int32)
        ec = np.empty(cap, np.int32)
        ev = np.empty(cap, np.float32)
        E = lib().rvo_compress(_p(w_bits), N, K, CH, _p(m8), _p(e4), _p(rp), _p(er), _p(ec), _p(ev), cap,
                               ctypes.byref(base))
        if E == -1:
            raise ValueError("bad shape")
        if E >= 0:
            break
        cap = int(rp[-1]) + 1
    return {"m8": m8, "e4": e4, "base": base.value, "rp": rp, "er": er[:E].copy(), "ec": ec[:E].copy(),
            "ev": ev[:E].copy(), "N": N, "K": K, "CH": CH}


def decode_f32(c):
    out = np.empty((c["N"], c["K"]), np.float32)
    er, ec, ev = (np.ascontiguousarray(c[k]) for k in ("er", "ec", "ev"))
    lib().rvo_decode(_p(np.ascontiguousarray(c["m8"])), _p(np.ascontiguousarray(c["e4"])), int(c["base"]),
                     _p(er), _p(ec), _p(ev), int(er.size), c["N"], c["K"], c["CH"], _p(out))
    return out


def gemv_bf16(W_bits, X, Y, add, threads=0):
    """matmat16 restatement: Y[t] (+)= W X[t] (fp32)."""
    N, K = W_bits.shape
    T = X.shape[0]
    lib().rvo_gemv_bf16(_p(W_bits), _p(X), _p(Y), N, K, T, int(add), threads)


def gemv_12bit(c, X, Y, mode, lnw=None, eps=1e-6, threads=0):
    """12-bit decode + product on the CPU; Y[T, N] float32 updated in place."""
    T = X.shape[0]
    rc = lib().rvo_gemv_12bit(_p(np.ascontiguousarray(c["m8"])), _p(np.ascontiguousarray(c["e4"])),
                              int(c["base"]), _p(np.ascontiguousarray(c["rp"])), _p(np.ascontiguousarray(c["ec"])),
                              _p(np.ascontiguousarray(c["ev"])), _p(X), _p(Y), _p(lnw), eps, c["N"], c["K"],
                              c["CH"], T, mode, threads)
    if rc:
        raise ValueError(f"rvo_gemv_12bit: {rc}")


def rms_rows(X, w, out, eps):
    """rms_rows restatement (cpu_layer.py:51-59)."""
    T, D = X.shape
    lib().rvo_rms_rows(_p(X), _p(w), _p(out), T, D, eps)


def qk_rope_attn(QKV, qn, kn, inv, pos0, Kc, Vc, out, H, KV, HD, eps, threads=0):
    """qk_rope_attn restatement (cpu_layer.py:62-131), float32 caches [KV, maxt, HD]."""
    lib().rvo_qk_rope_attn(_p(QKV), _p(qn), _p(kn), _p(inv), int(pos0), _p(Kc), _p(Vc), Kc.shape[1], _p(out),
                           QKV.shape[0], H, KV, HD, eps, threads)


def silu_mul(GU, M, FF):
    """silu_mul restatement (cpu_layer.py:134-140)."""
    lib().rvo_silu_mul(_p(GU), _p(M), GU.shape[0], FF)
