"""numpy model of the packed form the HIP kernels read (ai_amd/csrc/rv12_device.h).

Test helper: it restates, in array form, what the pack kernels write and what
the linear kernels read back, so the layout's arithmetic (row exponent
windows, pair packing, the 2^sc rescale, the exception convention) is checked
on the CPU against the oracle before any kernel runs.
"""
import numpy as np

from oracle.codec import choose_base

M_PAIR = np.uint32(0x87FF87FF)


def scale_exp(base):
    """sc: h << 16 read as a float32 is the weight times 2^-sc."""
    return max(int(base) - 1, 0)


def row_bases(w_bits):
    """Window start of each row: the reference's whole-matrix rule (first
    argmax of the 15-wide window counts) applied to the row."""
    w = np.asarray(w_bits, np.uint16)
    e = (w.astype(np.int64) >> 7) & 0xFF
    return np.array([choose_base(e[n]) for n in range(w.shape[0])], np.int64)


def h_values(w_bits, rbase):
    """16-bit h per weight: sign<<15 | c<<7 | m7 with c = e - sc of the row
    for weights inside the row window, h = 0 outside it."""
    w = np.asarray(w_bits, np.uint16).astype(np.int64)
    base = np.asarray(rbase, np.int64)[:, None]
    sc = np.maximum(base - 1, 0)
    e = (w >> 7) & 0xFF
    code = e - base
    inside = (code >= 0) & (code <= 14)
    h = np.where(inside, (w & 0x807F) | ((e - sc) << 7), 0)
    return h.astype(np.uint32), ~inside


def pack(w_bits):
    """(tiles [nblk, nsteps, 64, 3] uint32, rbase, rp, er, ec, ev) as the pack kernels write them."""
    w = np.asarray(w_bits, np.uint16)
    N, K = w.shape
    rbase = row_bases(w)
    h, out = h_values(w, rbase)
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
    tiles = np.stack([d0, d1, d2], -1).astype(np.uint32)
    er, ec = np.nonzero(out)
    rp = np.zeros(N + 1, np.int32)
    rp[1:] = np.cumsum(np.bincount(er, minlength=N))
    ev = (w[er, ec].astype(np.uint32) << 16).view(np.float32)
    return tiles, rbase, rp, er.astype(np.int32), ec.astype(np.int32), ev


def unpack(tiles):
    """pairs [..., 4] from the three dwords, as unpack_pairs does."""
    d0, d1, d2 = tiles[..., 0], tiles[..., 1], tiles[..., 2]
    p3 = (((d0 >> 11) & 0x000F000F) | ((d1 >> 7) & 0x00F000F0) | ((d2 >> 3) & 0x07000700)
          | ((d2 << 1) & 0x80008000))
    return np.stack([d0 & M_PAIR, d1 & M_PAIR, d2 & M_PAIR, p3.astype(np.uint32)], -1)


def h_from_tiles(tiles, N, K):
    """h [N, K] back from the tiles (inverse of pack's permutation)."""
    nblk = tiles.shape[0]
    p = unpack(tiles)
    g = np.empty(p.shape[:-1] + (8,), np.uint32)
    g[..., 0::2] = p & 0xFFFF
    g[..., 1::2] = p >> 16
    hp = g.reshape(nblk, K // 32, 4, 16, 8).transpose(0, 3, 1, 2, 4).reshape(nblk * 16, K)
    return hp[:N]


def bf16_from_h(h, rbase):
    """bf16 bits from h (before the exception scatter), as h_to_bf16."""
    sc = np.maximum(np.asarray(rbase, np.int64) - 1, 0)[:, None]
    cc = (h >> 7) & 15
    return np.where(cc != 0, (h.astype(np.int64) + (sc << 7)) & 0xFFFF, h).astype(np.uint16)


def decode(tiles, rbase, er, ec, ev, N, K):
    """The exact bf16 bits of the packed matrix."""
    bits = bf16_from_h(h_from_tiles(tiles, N, K), rbase)
    bits[np.asarray(er, np.int64), np.asarray(ec, np.int64)] = (np.asarray(ev, np.float32).view(np.uint32)
                                                                 >> 16).astype(np.uint16)
    return bits


def scaled_dot(w_bits, xp):
    """sum_k h_k x'_k in float64 with h read as a float32 value, each row
    rescaled by 2^sc of its window, plus the row-window exceptions: the
    kernels' formula in exact arithmetic."""
    tiles, rbase, rp, er, ec, ev = pack(w_bits)
    N, K = np.asarray(w_bits).shape
    h = h_from_tiles(tiles, N, K)
    wh = (h.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    sc = np.maximum(rbase - 1, 0)
    y = np.ldexp(xp @ wh.T, sc[None, :])
    for j in range(er.size):
        y[:, er[j]] += ev[j].astype(np.float64) * xp[:, ec[j]]
    return y
