"""numpy restatement of the reference 12-bit lossless bf16 codec.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the product path never calls
this module.

Format (ramvi/engine/ramvi_engine/kernels/wcomp.py:1-7, 13-32), for a bf16
matrix W[N, K] with K % CH == 0:
  e      = (bits >> 7) & 0xFF                       biased exponent
  base   = first argmax over b of #{e in [b, b+14]}  one value per matrix
  code   = e - base, or 15 when e is outside the window (an exception)
  m8     = sign << 7 | mantissa7                    uint8[N, K]
  e4     = per CH-chunk, byte i = code[i] | code[CH/2 + i] << 4    uint8[N, K/2]
  rp/er/ec/ev = exceptions in row-major order: CSR row pointer int32[N+1],
           row int32[E], column int32[E], value float32[E] (exact copy)
"""
import numpy as np

WINDOW = 15          # exponents base .. base+14 are coded, code 15 escapes
ESCAPE = 15


def bf16_to_f32(bits):
    """bf16 bit patterns (uint16) -> float32 values, exact (NaN payload kept)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(x, nan=0xFFFF):
    """float32 -> bf16 bits with round-to-nearest-even; every NaN -> `nan`.

    This is the conversion `Tensor.bfloat16()` applies, which the reference
    `decompress` ends with (wcomp.py:45).  The NaN it produces depends on the
    torch build and device (0xFFFF from the CPU conversion of torch 2.10, as the
    golden vectors record; 0x7FC0 or 0x7FFF elsewhere), so tests compare NaN
    positions with isnan and every other bit pattern exactly."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(np.asarray(x, dtype=np.float32)), np.uint16(nan), r)


def choose_base(e):
    """First start b in [0, 241] of the 15-wide exponent window holding the most
    weights (wcomp.py:19-21: bincount, cumsum, window differences, argmax)."""
    cnt = np.bincount(np.asarray(e, dtype=np.int64).ravel(), minlength=256)
    cs = np.concatenate([[0], np.cumsum(cnt)])
    win = cs[WINDOW:] - cs[:-WINDOW]          # win[b] = count of e in [b, b+14]
    return int(np.argmax(win))                # numpy argmax returns the first maximum


def compress(w_bits, CH=256):
    """bf16 bits uint16[N, K] -> codec dict (wcomp.py:13-32)."""
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    N, K = w_bits.shape
    if K % CH:
        raise ValueError("K must be a multiple of CH")
    b = w_bits.astype(np.int64)
    e = (b >> 7) & 0xFF
    base = choose_base(e)
    code = e - base
    exc = (code < 0) | (code > WINDOW - 1)
    code = np.where(exc, ESCAPE, code)
    m8 = (((b >> 15) << 7) | (b & 0x7F)).astype(np.uint8)
    c4 = code.reshape(N, K // CH, 2, CH // 2)
    e4 = (c4[:, :, 0] | (c4[:, :, 1] << 4)).astype(np.uint8).reshape(N, K // 2)
    r, col = np.nonzero(exc)                  # row-major order
    rp = np.zeros(N + 1, dtype=np.int32)
    rp[1:] = np.cumsum(np.bincount(r, minlength=N))
    return {"m8": m8, "e4": e4, "base": base, "rp": rp, "er": r.astype(np.int32),
            "ec": col.astype(np.int32), "ev": bf16_to_f32(w_bits[r, col]).copy(),
            "N": N, "K": K, "CH": CH}


def codes(c):
    """Per-weight 4-bit codes int64[N, K] unpacked from e4 (wcomp.py:38-39)."""
    N, K, CH = c["N"], c["K"], c["CH"]
    e4 = np.asarray(c["e4"]).astype(np.int64).reshape(N, K // CH, CH // 2)
    return np.stack([e4 & 15, e4 >> 4], 2).reshape(N, K)


def decode_f32(c):
    """Decoded weights as float32 values (wcomp.py:40-44); NaN payloads kept."""
    code = codes(c)
    m = np.asarray(c["m8"]).astype(np.int64)
    bits = ((m >> 7) << 31) | ((code + c["base"]) << 23) | ((m & 0x7F) << 16)
    bits = np.where(code == ESCAPE, 0, bits).astype(np.uint32)
    W = bits.view(np.float32).copy()
    W[np.asarray(c["er"], dtype=np.int64), np.asarray(c["ec"], dtype=np.int64)] = c["ev"]
    return W


def decode_exact(c):
    """Lossless inverse: the original bf16 bit patterns, NaN payloads included."""
    return (decode_f32(c).view(np.uint32) >> 16).astype(np.uint16)


def decompress(c):
    """Reference `decompress` result (wcomp.py:35-45): decode then `.bfloat16()`,
    which replaces every NaN payload by one canonical NaN."""
    return f32_to_bf16_rne(decode_f32(c))


def compressed_bytes(c):
    """Bytes of the reference codec for one matrix: m8 + e4 + rp + er/ec/ev."""
    N, K = c["N"], c["K"]
    E = int(np.asarray(c["er"]).size)
    return N * K + N * K // 2 + 4 * (N + 1) + 12 * E
