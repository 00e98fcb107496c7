"""GPU parity of the greedy pick over the 12-bit lm_head (rv12_head_argmax
through wcomp.greedy), the reference's greedy branch of Head.pick
(ramvi/engine/ramvi_engine/generation/head.py:59-88): the id of the largest
logit, the smallest id on ties (:76-79).

Pinned by: rows made identical bit for bit give identical logits, so the
smallest of them must win a tie by construction; one row with a NaN weight
wins (NaN counts as the largest value, as torch.argmax and numpy.argmax order
it), the smaller of two such rows; the ids equal numpy's first argmax over
the logits the same launch writes; and, where the fp64 closed form's best
logit leads the second by more than the fp32 error bound, they equal the
closed form's argmax.  Every launch family is covered: the fused pick of the
vector kernel (one, two and four row blocks per workgroup), the vector kernel
with a K split and the MFMA kernel (logits, then the two-pass pick)."""
import numpy as np
import pytest
import torch

from oracle import codec, linear

pytestmark = pytest.mark.gpu

BF16_NAN = 0x7FC0


def _matrix(N, K, seed, tied=(), nan_rows=()):
    """bf16 bits of N(0, 0.02) weights; rows `tied` are copies of one row
    scaled x8 (so their logit is the largest for x = sign(row)); rows
    `nan_rows` carry one NaN weight."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(N, K, device="cuda", generator=g) * 0.02
    if tied:
        w[list(tied)] = w[tied[0]] * 8
    bits = w.bfloat16().view(torch.int16).cpu().numpy().view(np.uint16).copy()
    for r in nan_rows:
        bits[r, 5] = BF16_NAN
    return bits


def _pick(cg, X, lnw=None, launch=None, want_logits=True):
    """(ids, logits) of rv12_head_argmax for the rows of X."""
    import ctypes
    from ai_amd import _lib, wcomp
    T, K = X.shape
    N = int(cg["N"])
    x = torch.from_numpy(X).cuda()
    ids = torch.full((16,), -1, dtype=torch.int64, device="cuda")
    lg = torch.full((T, N), float("nan"), device="cuda") if want_logits else None
    ln = None if lnw is None else torch.from_numpy(lnw.view(np.int16).copy()).view(torch.bfloat16).cuda()
    if launch is None:
        wcomp.greedy(x, cg, T, ids, lnw=ln, logits=lg)
    else:
        L = _lib.lib()
        cfg = _lib.Launch(*launch)
        need = L.rv12_head_workspace_bytes(N, K, T, ctypes.byref(cfg))
        assert need > 0
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
        _lib.check(L.rv12_head_argmax(ctypes.byref(wcomp._matrix(cg)), p(x), T, p(ln), 1e-6, p(lg), p(ids), ctypes.byref(cfg),
                                      p(ws), need, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                   "rv12_head_argmax")
    torch.cuda.synchronize()
    got = ids.cpu().numpy()
    assert (got[T:] == -1).all()  # only T ids are written
    return got[:T], (None if lg is None else lg.cpu().numpy())


def _compress(bits):
    from ai_amd import wcomp
    return codec.compress(bits), wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())


LAUNCHES = [None, (1, 1, 4, 1), (1, 2, 8, 1), (1, 4, 8, 1), (1, 1, 4, 3), (2, 1, 4, 0), (2, 2, 8, 0)]


def _fits(launch, T):
    return launch is None or launch[0] == 2 or T <= 4


@pytest.mark.parametrize("launch", LAUNCHES)
def test_ties_pick_the_smallest_row(launch):
    """Rows 17, 2600 and 4999 are one row (x8) and hold the largest logit for
    x = sign of that row: every launch picks 17, with or without logits."""
    N, K = 5000, 1024
    tied = (2600, 17, 4999)
    bits = _matrix(N, K, 3, tied=tied)
    cnp, cg = _compress(bits)
    row = codec.decode_f32(cnp)[17]
    for T in (1, 2, 3, 8, 16):
        if not _fits(launch, T):
            continue
        X = np.tile(np.sign(row).astype(np.float32), (T, 1))
        X[1:] *= np.linspace(0.5, 2.0, T - 1, dtype=np.float32)[:, None] if T > 1 else 1
        print("launch", launch, "T", T, flush=True)
        ids, lg = _pick(cg, X, launch=launch)
        assert (ids == 17).all(), (launch, T, ids)
        assert np.array_equal(lg[:, 17], lg[:, 2600]) and np.array_equal(lg[:, 17], lg[:, 4999])
        ids2, _ = _pick(cg, X, launch=launch, want_logits=False)
        assert np.array_equal(ids, ids2)


@pytest.mark.parametrize("launch", [None, (1, 2, 8, 1), (1, 1, 4, 3), (2, 1, 8, 0)])
def test_nan_row_wins(launch):
    """A NaN logit counts as the largest value; of two, the smaller row."""
    N, K = 3000, 512
    bits = _matrix(N, K, 4, nan_rows=(2100, 777))
    cnp, cg = _compress(bits)
    rng = np.random.default_rng(0)
    for T in (1, 2, 5):
        if not _fits(launch, T):
            continue
        X = rng.standard_normal((T, K)).astype(np.float32)
        ids, lg = _pick(cg, X, launch=launch)
        assert np.isnan(lg[:, 777]).all() and (ids == 777).all(), (launch, T, ids)


@pytest.mark.parametrize("launch", LAUNCHES)
def test_ids_match_logits_and_closed_form(launch):
    """Random heads with the final RMSNorm fused: ids equal numpy's first
    argmax of the launch's own logits, and the fp64 closed form's argmax
    wherever its top two logits are further apart than the fp32 bound."""
    from ai_amd import wcomp
    N, K = 20000, 1024
    bits = _matrix(N, K, 5)
    cnp, cg = _compress(bits)
    W = codec.decode_f32(cnp).astype(np.float64)
    rng = np.random.default_rng(1)
    lnw = codec.f32_to_bf16_rne((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    lw = codec.bf16_to_f32(lnw)
    checked = 0
    for T in (1, 2, 4, 7, 16):
        if not _fits(launch, T):
            continue
        X = rng.standard_normal((T, K)).astype(np.float32)
        ids, lg = _pick(cg, X, lnw=lnw, launch=launch)
        assert np.array_equal(ids, np.argmax(lg, 1)), (launch, T)
        ref = linear.linear(cnp, X, 0, lnw=lw, W=W)
        bound = linear.error_bound(cnp, X, 0, lnw=lw, W=W)
        top2 = np.sort(ref, 1)[:, -2:]
        clear = top2[:, 1] - top2[:, 0] > 8 * bound.max(1)
        assert np.array_equal(ids[clear], np.argmax(ref, 1)[clear]), (launch, T)
        checked += int(clear.sum())
        # the same pick without logits, through the Python mirror
        if launch is None:
            out = torch.zeros(16, dtype=torch.int64, device="cuda")
            wcomp.greedy(torch.from_numpy(X).cuda(), cg, T, out,
                         lnw=torch.from_numpy(lnw.view(np.int16).copy()).view(torch.bfloat16).cuda())
            assert np.array_equal(out[:T].cpu().numpy(), ids)
    assert checked > 0


def test_vocabulary_head_full_size():
    """The Qwen3-8B head (151936 x 4096) with the final norm at one and two
    tokens (the fused pick, two passes over 9496 workgroup pairs) and at 16
    (MFMA, logits): ids equal the first argmax of the logits."""
    from ai_amd import wcomp
    N, K = 151936, 4096
    bits = _matrix(N, K, 6, tied=(151000, 9, 70000))
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    rng = np.random.default_rng(2)
    lnw = codec.f32_to_bf16_rne((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    row = codec.bf16_to_f32(bits[9])
    del bits
    for T in (1, 2, 16):
        X = rng.standard_normal((T, K)).astype(np.float32)
        X[0] = np.sign(row) * 3.0  # token 0: rows 9, 70000, 151000 tie at the top
        print("T", T, flush=True)
        ids, lg = _pick(cg, X, lnw=lnw)
        assert ids[0] == 9
        assert np.array_equal(ids, np.argmax(lg, 1))
    del cg
    torch.cuda.empty_cache()


def test_head_class_greedy_and_sampling():
    """ai_amd.head.Head with the reference's interface: greedy picks equal
    wcomp.greedy's; sampling at a tiny temperature picks the greedy id where
    there is no tie, and top_p = 0 keeps only the most likely id."""
    from ai_amd.head import Head
    N, K = 4000, 256
    bits = _matrix(N, K, 8, tied=(30, 3000))
    hd = Head(bits, TM=16)
    row = codec.bf16_to_f32(bits[30])
    rng = np.random.default_rng(3)
    X = rng.standard_normal((4, K)).astype(np.float32)
    X[0] = np.sign(row)
    h = torch.from_numpy(X).cuda()
    ids = hd.pick(h, 4)
    assert ids[0] == 30
    want, _ = _pick(hd.c, X)
    assert ids == want.tolist()
    # token 0 ties rows 30 and 3000: sampling may take either, top_p = 0 keeps
    # the first of the stable order (the smaller id)
    assert hd.pick(h, 4, temperature=1e-6, rng=np.random.default_rng(0))[1:] == ids[1:]
    assert hd.pick(h, 4, temperature=1.0, top_p=0.0, rng=np.random.default_rng(0)) == ids
