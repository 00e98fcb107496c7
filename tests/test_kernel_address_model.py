"""CPU model of the addresses the decode step's kernels form, at the real
shapes of Qwen3-0.6B/8B/14B/32B and the launch shapes the library picks:
every index a thread can compute stays inside its buffer, and every 32-bit
byte offset or descriptor range stays below 2^32 (2^31 where the kernel
treats it as signed).  The formulas are those of k_gemv (rv12_gemv.hip:
steps 0-6), k_splitk_reduce, k_pick, k_rope_attn and k_attn_combine
(rv12_attn.hip), both forms of the MFMA linear k_gemm (rv12_gemm.hip) and the
exception epilogue of the prefill GEMM k_prefill_mm (rv12_prefill.hip),
written here from the kernels' own index expressions."""
import ctypes

import pytest

from ai_amd import _lib

MODELS = {  # D, H, KV, HD, FF, V
    "0.6b": (1024, 16, 8, 128, 3072, 151936),
    "8b": (4096, 32, 8, 128, 12288, 151936),
    "14b": (5120, 40, 8, 128, 17408, 151936),
    "32b": (5120, 64, 8, 128, 25600, 151936),
}
U32, I32 = 1 << 32, 1 << 31


def _layer_linears(D, H, KV, HD, FF, V):
    # (name, N, K, mode, rms)
    return [("qkv", (H + 2 * KV) * HD, D, 0, True), ("o", D, H * HD, 1, False), ("gu", 2 * FF, D, 0, True),
            ("down", D, FF, 2, False), ("head", V, D, 0, True)]


def _shape(N, K, T):
    c = _lib.Launch()
    assert _lib.lib().rv12_launch_shape(N, K, T, None, ctypes.byref(c)) == 0
    return c.kernel, c.rb, c.waves, c.splits


@pytest.mark.parametrize("model", sorted(MODELS))
@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_vector_linear_addresses(model, T):
    D, H, KV, HD, FF, V = MODELS[model]
    for name, N, K, mode, rms in _layer_linears(D, H, KV, HD, FF, V):
        kernel, RB, W, S = _shape(N, K, T)
        if kernel != 1:
            continue
        nthr, nsteps = 64 * W, K // 32
        nblk = (N + 15) // 16
        grid = (nblk + RB - 1) // RB
        npad = nblk * 16
        xs = 2 * K if mode == 2 else K
        n_exc = N * K // 64  # far above the densest Qwen3 matrix (0.1 % outlier rows give 0.08 %)
        # step 0: the owner's row, clamped; old y at (min(tok, T-1), row)
        for blk in (0, grid - 1):
            n0 = blk * RB * 16
            for orow in (0, RB * 16 - 1):
                onc = min(n0 + orow, N - 1)
                assert 0 <= onc < N and onc + 1 <= N  # rbase[onc], rp[onc], rp[onc + 1]
                assert (T - 1) * N + onc < T * N
            assert min(n0 + RB * 16, N) <= N  # rp[...] of the exception range
        # step 1: activations of split sp, chunk offsets i < krange
        for sp in (0, S - 1):
            s_lo, s_hi = sp * nsteps // S, (sp + 1) * nsteps // S
            assert (sp + 1) * nsteps < U32  # the split bounds are computed in 32 bits
            k_lo, krange = s_lo * 32, (s_hi - s_lo) * 32
            i_max = krange - 4
            k = k_lo + i_max
            assert k + 3 < K and (T - 1) * xs + (K if mode == 2 else 0) + k + 3 < T * xs
            if rms:
                assert k + 3 < K  # lnw (4 bf16 per chunk)
        # step 2: weights through one descriptor per workgroup over its row
        # blocks' bytes; a step's offset is all in the 32-bit vector offset,
        # and a step past the split's end takes 2^31 plus the row-block
        # offset, past the descriptor's range without wrapping
        blk_bytes = nsteps * 768
        assert RB * blk_bytes < I32  # the descriptor's range, below 2^31
        assert (RB - 1) * blk_bytes + (nsteps - 1) * 768 + 63 * 12 + 12 <= RB * blk_bytes
        assert I32 + (RB - 1) * blk_bytes + 63 * 12 + 12 <= U32
        # step 3: the exception entries through descriptors of min(n_exc, 2^28) * 4 bytes
        assert min(n_exc, 1 << 28) * 4 < U32 and (n_exc - 1) * 4 < 0xFFFFFFF0
        # step 5/6: stores and partials
        assert (T - 1) * N + N - 1 < T * N
        if S > 1:
            assert ((S - 1) * T + T - 1) * npad + npad - 1 < S * T * npad
            assert (S + 16) * T * npad * 4 < I32  # the reduce's 32-bit byte offsets (host-checked)
        # fused greedy pick: pairs [T][grid]
        if name == "head":
            assert (T - 1) * grid + grid - 1 < T * grid


@pytest.mark.parametrize("model", sorted(MODELS))
def test_decode_attention_long_span_addresses(model):
    """One split over a short cache (the 1024-thread workgroup, up to 256
    positions, one workgroup per q head): the positions its threads address
    stay inside the span, the cache rows inside the cache, the offsets in 32
    bits; workgroup h reads q row h, the k and v rows of kv head h / G and
    that head's cache, writes output row h, and only the first q head of each
    kv head writes the cache (one writer per kv head)."""
    D, H, KV, HD, FF, V = MODELS[model]
    from ai_amd.attn import LONG_SPAN, default_splits
    NT, P = 1024, 256
    G = H // KV
    assert P == LONG_SPAN
    qkv_floats = (H + 2 * KV) * HD
    writers = {}
    for h in range(H):  # grid over the q heads
        g = h // G
        assert 0 <= g < KV
        assert (h * HD + HD - 1) < H * HD                                   # q row h (its own head)
        assert ((H + g) * HD + HD - 1) < qkv_floats                         # k row of kv head g
        assert ((H + KV + g) * HD + HD - 1) < qkv_floats                    # v row of kv head g
        assert h * HD + HD - 1 < H * HD                                     # output row h
        if h == g * G:
            writers[g] = writers.get(g, 0) + 1
    assert writers == {g: 1 for g in range(KV)}
    for maxt, eb in ((81, 2), (192, 2), (256, 2), (256, 4)):
        S = default_splits(KV, maxt, eb == 2, HD)
        if S != 1:
            continue
        for pos in (0, maxt // 2, maxt - 1):
            n = pos + 1
            lo, hi = 0, n
            assert hi - lo <= P
            # score threads: position t / 4 < P; value threads: group t / (HD / 2) of P / groups positions
            groups = NT // (HD // 2)
            assert (NT - 1) // 4 < P and (groups - 1) * (P // groups) + P // groups - 1 < P
            assert ((lo + P - 1) * HD + HD - 1) * eb < I32 and min(hi, n - 1) * HD * eb < U32
            assert (KV - 1) * maxt * HD + pos * HD + HD - 1 < KV * maxt * HD


@pytest.mark.parametrize("model", sorted(MODELS))
def test_decode_attention_addresses(model):
    D, H, KV, HD, FF, V = MODELS[model]
    from ai_amd.attn import SPAN, default_splits
    G = H // KV
    for maxt, eb in ((2304, 2), (4224, 2), (10240, 2), (2304, 4)):
        S = default_splits(KV, maxt)
        assert (maxt + S - 1) // S <= SPAN
        for pos in (0, maxt // 2, maxt - 1):
            n = pos + 1
            assert S * n < U32 and (S + 1) * n < U32  # split bounds in 32 bits
            for sp in (0, S - 1):
                lo, hi = sp * n // S, (sp + 1) * n // S
                assert hi - lo <= SPAN
                cbytes = min(hi, n - 1) * HD * eb
                assert cbytes < U32
                # key quarter rows and value pairs of positions lo..lo+79 (past hi: zeros by the descriptor)
                assert ((lo + SPAN - 1) * HD + HD - 1) * eb < I32
            # the step's k/v slot and the caches' rows, 64-bit
            row0 = (KV - 1) * maxt * HD
            assert row0 + pos * HD + HD - 1 < KV * maxt * HD
        # partials [n_kv][S][G][HD + 2] and the combine's ranges
        part = KV * S * G * (HD + 2)
        assert ((KV - 1) * S + S - 1) * G * (HD + 2) + G * (HD + 2) - 1 < part
        stride = G * (HD + 2) * 4
        assert (S - 1) * stride + (HD + 2) * 4 < U32
        # batch: T <= 16 rows per token, R = 16 G rows per kv head
        R = 16 * G
        assert ((KV - 1) * S + S - 1) * R * (HD + 2) + R * (HD + 2) - 1 < KV * S * R * (HD + 2)
        assert (S - 1) * R * (HD + 2) * 4 + (HD + 2) * 4 < U32


def _prefill_exception_reads(rp, N, blk0, wb=4, eb=8):
    """The exception-list indices k_prefill_mm's epilogue (rv12_prefill.hip,
    step (b)) reads for the row tile starting at row block blk0: the entries
    [e_lo, e_hi) of rows blk0*16 .. +16 wb, fetched eb at a time with each
    index clamped to e_hi - 1, the first batch only when the range is not
    empty, the next one only while it starts below e_hi."""
    rlo = blk0 * 16
    if rlo >= N:
        return []
    e_lo, e_hi = rp[rlo], rp[min(rlo + 16 * wb, N)]
    reads = []

    def fetch(e0):
        reads.extend(min(e0 + j, e_hi - 1) for j in range(eb))

    if e_lo < e_hi:
        fetch(e_lo)
    e0 = e_lo
    while e0 < e_hi:
        if e0 + eb < e_hi:
            fetch(e0 + eb)
        e0 += eb
    return reads


@pytest.mark.parametrize("case", ["no_exceptions", "first_tile_empty", "last_tile_only", "dense"])
def test_prefill_exception_epilogue_reads_inside_the_list(case):
    """Every exception entry the prefill GEMM's epilogue reads lies inside
    [e_lo, e_hi) of its row tile, so inside the list: with no exceptions at
    all (the list may be a null pointer) nothing is read, and a row tile with
    no entries before or inside it reads nothing (the first fetch is guarded)."""
    import numpy as np
    N = 1000
    per_row = np.zeros(N, np.int64)
    if case == "first_tile_empty":
        per_row[64:] = 1
    elif case == "last_tile_only":
        per_row[-3:] = 5
    elif case == "dense":
        per_row[:] = np.random.default_rng(0).integers(0, 20, N)
    rp = np.concatenate([[0], np.cumsum(per_row)]).tolist()
    n_exc = rp[-1]
    nblk = (N + 15) // 16
    total = 0
    for blk0 in range(0, nblk, 4):
        reads = _prefill_exception_reads(rp, N, blk0)
        rlo = blk0 * 16
        e_lo, e_hi = rp[rlo], rp[min(rlo + 64, N)]
        assert all(e_lo <= e < e_hi for e in reads), (case, blk0)
        assert all(0 <= e < n_exc for e in reads)
        if e_lo == e_hi:
            assert not reads
        total += len(set(reads))
    assert total == n_exc  # every entry is read, each tile its own


def _mfma_layout_bytes(nst, TP, W, RBW, ks):
    """End of k_gemm's LDS layout (rv12_gemm.hip): x' parts [nst][3][4 TP]
    16-byte groups, the exception sums [W * ORB * 16 rows][16 tokens], with
    the waves splitting K their sums [W][RBW][64] 16-byte values, then the
    sums of squares [W][16], the range flags [W] and the slow path's
    exponents [W][16]."""
    G = 4 * TP
    orb = 1 if ks else RBW
    return nst * 3 * G * 16 + W * orb * 256 * 4 + (W * RBW * 64 * 16 if ks else 0) + W * 16 * 4 + W * 4 + W * 16 * 4


@pytest.mark.parametrize("model", ["8b", "14b", "32b"])
@pytest.mark.parametrize("kernel", [2, 3])
def test_mfma_linear_addresses(model, kernel):
    """k_gemm at the real shapes, 3..16 tokens: the built-in launch (kernel 2)
    and kernel 3 (the waves splitting K) at every row-block count and wave
    count the library accepts.  Every LDS index lies inside the layout, which
    fits 160 KB; the grid covers every row block once per split; every global
    index lies inside its buffer; the 32-bit offsets stay in range."""
    D, H, KV, HD, FF, V = MODELS[model]
    for name, N, K, mode, rms in _layer_linears(D, H, KV, HD, FF, V):
        nblk, nsteps = (N + 15) // 16, K // 32
        npad = nblk * 16
        xs = 2 * K if mode == 2 else K
        for T in (3, 4, 5, 8, 9, 16):
            TP = 4 if T <= 4 else (8 if T <= 8 else 16)
            G = 4 * TP
            if kernel == 2:
                shapes = [_shape(N, K, T)] if _shape(N, K, T)[0] == 2 else []
            else:
                shapes = []
                for rb in (1, 2, 4):
                    for w in (4, 8):
                        c = _lib.Launch()
                        if rb <= w and _lib.lib().rv12_launch_shape(N, K, T, _lib.Launch(3, rb, w, 0),
                                                                    ctypes.byref(c)) == 0:
                            shapes.append((c.kernel, c.rb, c.waves, c.splits))
            for kn, RBW, W, S in shapes:
                assert kn == kernel
                ks = kernel == 3
                per_wg = RBW * (1 if ks else W)
                grid = (nblk + per_wg - 1) // per_wg
                # every row block in exactly one workgroup of each split
                covered = [0] * nblk
                for bx in range(grid):
                    for w in range(1 if ks else W):
                        for b in range(RBW):
                            blk = bx * per_wg + w * RBW + b
                            if blk < nblk:
                                covered[blk] += 1
                assert covered == [1] * nblk, (name, T, kn, RBW, W, S)
                for sp in range(S):
                    s_lo, s_hi = sp * nsteps // S, (sp + 1) * nsteps // S
                    nst = s_hi - s_lo
                    assert (sp + 1) * nsteps < U32
                    assert _mfma_layout_bytes(nst, TP, W, RBW, ks) <= 160 * 1024, (name, T, kn, RBW, W, S)
                    # staging: group g < nst G at step g / G, k-group (g % G) / TP, token g % TP
                    g_max = nst * G - 1
                    assert (g_max // G) * 3 * G + g_max % G + 2 * G < nst * 3 * G
                    k_max = s_lo * 32 + (g_max // G) * 32 + ((g_max % G) // TP) * 8 + 7
                    assert k_max < K
                    assert (T - 1) * xs + (K if mode == 2 else 0) + k_max < T * xs  # x (and u) of token T - 1
                    # main loop: lane l reads group (l / 16) TP + l % 16 for l % 16 < TP, three parts
                    assert 3 * TP + TP - 1 + 2 * G < 3 * G
                    # exception x' reads: step c / 32, group ((c % 32) / 8) TP + token, element c % 8
                    c = nst * 32 - 1
                    o = ((c >> 5) * 3 * G + ((c & 31) >> 3) * TP + (T - 1)) * 16 + (c & 7) * 2
                    assert o + 2 * G * 16 + 1 < nst * 3 * G * 16
                # weights: one descriptor over the loading wave's (KS: the
                # workgroup's) row blocks; a step's offset is all in the 32-bit
                # vector offset, a step past the split's end takes 2^31 plus the
                # row-block offset, past the descriptor's range without wrapping
                blk_bytes = nsteps * 768
                assert RBW * blk_bytes < I32
                assert (RBW - 1) * blk_bytes + (nsteps - 1) * 768 + 63 * 12 + 12 <= RBW * blk_bytes
                assert I32 + (RBW - 1) * blk_bytes + 63 * 12 + 12 <= U32
                # output rows: KS wave b < RBW takes row block b, its 16 rows hold every exception row index
                orb = 1 if ks else RBW
                assert orb * 16 * 16 <= 256 * orb  # excw [orb * 16 rows][16 tokens] of the wave
                # y and rbase through descriptors; their 32-bit byte ranges and offsets
                assert T * N * 4 < U32 and ((T - 1) * N + npad) * 4 < I32 and N * 4 < U32
                if S > 1:
                    assert ((S - 1) * T + T - 1) * npad + npad - 1 < S * T * npad
                    assert (S + 16) * T * npad * 4 < I32


def test_attention_split_bounds_by_multiplier():
    """The attention kernels divide by a multiplier the host computes,
    floor(2^32 / v) + 1 (v >= 2), and a mulhi: the decode step's split bounds
    (sp n) / S for n <= 10240 positions and S <= 128 splits (a < 2^21), and
    the combine's row quotients h / R and i / G (below 2^16, R and G up to
    1024).  Exhaustive against integer division over those ranges."""
    import numpy as np

    def mulhi_div(a, v):
        m = np.uint64((1 << 32) // v + 1)
        return (a.astype(np.uint64) * m) >> np.uint64(32)

    a = np.arange(1 << 21, dtype=np.uint64)
    for S in range(2, 129):
        assert np.array_equal(mulhi_div(a, S), a // np.uint64(S)), S
    h = np.arange(1 << 16, dtype=np.uint64)
    for v in range(2, 1025):
        assert np.array_equal(mulhi_div(h, v), h // np.uint64(v)), v
