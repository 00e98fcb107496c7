"""numpy model of the Q16 tile layout the HIP kernels use (ai_amd/csrc/rv12_kernels.hip).

Test helper: it restates, in array form, what k_retile writes and what the
kernels read back, so the layout's arithmetic (pair packing, exponent codes,
the 2^(base-1) rescale, the exception convention) is checked on the CPU
against the oracle before any kernel runs.
"""
import numpy as np

from oracle.codec import codes

M_PAIR = np.uint32(0x87FF87FF)


def scale_exp(base):
    """sc: h << 16 read as a float32 is the weight times 2^-sc."""
    return max(int(base) - 1, 0)


def h_values(c):
    """16-bit h per weight: sign<<15 | c'<<7 | m7 with c' = e - sc for
    in-window weights (code + 1 when base >= 1, the exponent itself when
    base == 0) and h = 0 for exceptions."""
    code = codes(c)
    m = np.asarray(c["m8"]).astype(np.uint32)
    sm = ((m >> 7) << 15) | (m & 0x7F)
    base = int(c["base"])
    cc = (code + base - scale_exp(base)).astype(np.uint32)
    h = np.where(code == 15, 0, sm | (cc << 7))
    return h.astype(np.uint32)


def retile(c):
    """uint32 tiles [nblk, nsteps, 64, 3] as k_retile writes them."""
    N, K = c["N"], c["K"]
    h = h_values(c)
    nblk = (N + 15) // 16
    hp = np.zeros((nblk * 16, K), np.uint32)
    hp[:N] = h
    # [blk, row16, step, quarter, 8] -> [blk, step, quarter, row16, 8]
    g = hp.reshape(nblk, 16, K // 32, 4, 8).transpose(0, 2, 3, 1, 4).reshape(nblk, K // 32, 64, 8)
    p = g[..., 0::2] | (g[..., 1::2] << 16)
    p0, p1, p2, p3 = p[..., 0], p[..., 1], p[..., 2], p[..., 3]
    d0 = p0 | ((p3 & 0x000F000F) << 11)
    d1 = p1 | ((p3 & 0x00F000F0) << 7)
    d2 = p2 | ((p3 & 0x07000700) << 3) | ((p3 & 0x80008000) >> 1)
    return np.stack([d0, d1, d2], -1).astype(np.uint32)


def unpack(tiles):
    """pairs [..., 4] from the three dwords, as unpack_pairs does."""
    d0, d1, d2 = tiles[..., 0], tiles[..., 1], tiles[..., 2]
    p3 = (((d0 >> 11) & 0x000F000F) | ((d1 >> 7) & 0x00F000F0) | ((d2 >> 3) & 0x07000700)
          | ((d2 << 1) & 0x80008000))
    return np.stack([d0 & M_PAIR, d1 & M_PAIR, d2 & M_PAIR, p3.astype(np.uint32)], -1)


def h_from_tiles(tiles, N, K):
    """h [N, K] back from the tiles (inverse of retile's permutation)."""
    nblk = tiles.shape[0]
    p = unpack(tiles)
    g = np.empty(p.shape[:-1] + (8,), np.uint32)
    g[..., 0::2] = p & 0xFFFF
    g[..., 1::2] = p >> 16
    hp = g.reshape(nblk, K // 32, 4, 16, 8).transpose(0, 3, 1, 2, 4).reshape(nblk * 16, K)
    return hp[:N]


def bf16_from_h(h, base):
    """original bf16 bits from h (before the exception scatter), as h_to_bf16."""
    cc = (h >> 7) & 15
    return np.where(cc != 0, (h.astype(np.int64) + (scale_exp(base) << 7)) & 0xFFFF, h).astype(np.uint16)


def scaled_dot(c, xp):
    """sum_k h_k x'_k computed in float64 with h as a float32 value, rescaled by
    2^sc, plus the exceptions: the kernels' formula in exact arithmetic."""
    h = h_values(c)
    wh = (h.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    y = np.ldexp(xp @ wh.T, scale_exp(c["base"]))
    er, ec, ev = (np.asarray(c[k]) for k in ("er", "ec", "ev"))
    for j in range(er.size):
        y[:, er[j]] += ev[j].astype(np.float64) * xp[:, ec[j]]
    return y
