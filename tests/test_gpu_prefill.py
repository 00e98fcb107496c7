"""GPU parity of the blocked prefill's linear (ai_amd.prefill.matrix ->
rv12_prefill_linear: the 12-bit decode fused into a bf16x3 MFMA GEMM over all
tokens) against the oracle's float64 closed form: 1e-3 abs + 1e-2 rel and 4x
the fp32 forward-error bound, for store, residual add and the silu(g) * u
prologue, ragged token counts and row counts, on the golden matrices, a
matrix with exceptions in many rows, activations of very different scales,
and (at the Qwen3-8B gu shape over 2048 tokens, beyond what the float64
oracle finishes in seconds) sampled rows against the decode kernels."""
import numpy as np
import pytest
import torch

from conftest import ref_dict
from oracle import codec, linear

pytestmark = pytest.mark.gpu


def _check(cnp, T, seed, add, mode=None, scales=None, rms=False):
    from ai_amd import prefill, wcomp
    rng = np.random.default_rng(seed)
    N, K = cnp["N"], cnp["K"]
    mode = (1 if add else 0) if mode is None else mode
    X = rng.standard_normal((T, 2 * K if mode == 2 else K)) * 2
    if scales is not None:  # MODE 2: g and u each by the square root, so that x' ~ the scale
        sc = np.asarray(scales, np.float64)[:T, None]
        X *= np.sqrt(sc) if mode == 2 else sc
    X = X.astype(np.float32)
    Y0 = rng.standard_normal((T, N)).astype(np.float32)
    lnw = lw = ln = None
    if rms:  # the RMSNorm prologue (rmsg_k fused): a bf16 weight of K entries
        lnw = codec.f32_to_bf16_rne((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32))
        lw = codec.bf16_to_f32(lnw)
        ln = torch.from_numpy(lnw.view(np.int16).copy()).view(torch.bfloat16).cuda()
    W = codec.decode_f32(cnp).astype(np.float64)
    ref = linear.linear(cnp, X, mode, Y0 if mode else None, lnw=lw, W=W)
    bound = linear.error_bound(cnp, X, mode, lnw=lw, W=W)
    c = wcomp.prepare({k: (torch.from_numpy(np.ascontiguousarray(v)) if isinstance(v, np.ndarray) else v)
                       for k, v in cnp.items()})
    y = torch.from_numpy(Y0.copy()).cuda()
    if mode == 2:
        prefill._linear(torch.from_numpy(X).cuda(), c, y, 2)
    else:
        prefill.matrix(torch.from_numpy(X).cuda(), c, y, add=add, lnw=ln)
    torch.cuda.synchronize()
    got = y.cpu().numpy().astype(np.float64)
    # outputs beyond the float32 range: the closed form rounded to float32
    # (inf), as an fp32 evaluation must produce
    with np.errstate(over="ignore"):
        ref = ref.astype(np.float32).astype(np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])
    err = np.abs(got[fin] - ref[fin])
    assert np.all(err <= 1e-3 + 1e-2 * np.abs(ref[fin])), float(err.max())
    # plus the rounding of the final add into y (2^-23 |y|) where y is accumulated
    tight = 4 * bound[fin] + (2.0 ** -23 * np.abs(ref[fin]) if mode else 0.0) + 1e-30
    assert np.all(err <= tight), float((err - tight).max())


@pytest.mark.parametrize("case", ["prefill_seed7", "outliers_rows_cols", "chunk128", "subnormal_heavy"])
def test_matrix_on_golden_dicts(golden, case):
    cnp = ref_dict(golden[case])
    for add in (False, True):
        _check(cnp, 300, 1, add)


def test_matrix_with_exceptions_in_many_rows():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((777, 1024)) * 0.02).astype(np.float32)
    idx = rng.choice(w.size, 400, replace=False)
    w.reshape(-1)[idx[::2]] = 3e4
    w.reshape(-1)[idx[1::2]] = -1e-30
    w[5] *= 20
    cnp = codec.compress(codec.f32_to_bf16_rne(w))
    assert cnp["er"].size > 100
    _check(cnp, 513, 2, True)


@pytest.mark.parametrize("T", [1, 17, 128, 129, 300])
def test_ragged_tokens_rows_and_modes(T):
    """Token counts around the 128-token tile, a row count that is not a
    multiple of the 256-row tile, every mode, and the RMSNorm prologue
    (store and accumulate)."""
    rng = np.random.default_rng(T)
    w = (rng.standard_normal((300, 512)) * 0.02).astype(np.float32)
    w[rng.choice(300, 2)] *= 20
    cnp = codec.compress(codec.f32_to_bf16_rne(w))
    for mode in (0, 1, 2):
        print("T", T, "mode", mode, flush=True)
        _check(cnp, T, T + mode, mode != 0, mode=mode)
    for mode in (0, 1):
        print("T", T, "mode", mode, "rms", flush=True)
        _check(cnp, T, T + 7 + mode, mode != 0, mode=mode, rms=True)


def test_rms_prologue_on_golden_dicts_and_scales(golden):
    """The fused RMSNorm (rs per token over its full row, lnw x staged) on
    the golden matrices, and over tokens scaled by 2^-60 .. 2^60: the sum of
    squares runs over (x 2^-32)^2, so no token overflows or vanishes."""
    for case in ("prefill_seed7", "outliers_rows_cols"):
        _check(ref_dict(golden[case]), 300, 5, False, rms=True)
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((200, 1024)) * 0.02).astype(np.float32)
    cnp = codec.compress(codec.f32_to_bf16_rne(w))
    T = 40
    scales = [2.0 ** e for e in np.linspace(-60, 60, T)]
    _check(cnp, T, 13, False, mode=0, scales=scales, rms=True)


def test_rms_prologue_rejected_in_mode_2():
    import ctypes
    from ai_amd import _lib, wcomp
    rng = np.random.default_rng(1)
    cnp = codec.compress(codec.f32_to_bf16_rne((rng.standard_normal((32, 256)) * 0.02).astype(np.float32)))
    c = wcomp.prepare({k: (torch.from_numpy(np.ascontiguousarray(v)) if isinstance(v, np.ndarray) else v)
                       for k, v in cnp.items()})
    x = torch.zeros(4, 512, device="cuda")
    y = torch.zeros(4, 32, device="cuda")
    ln = torch.ones(256, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    L = _lib.lib()
    rc = L.rv12_prefill_linear(ctypes.byref(wcomp._matrix(c)), ctypes.c_void_p(x.data_ptr()),
                               ctypes.c_void_p(y.data_ptr()), 4, ctypes.c_void_p(ln.data_ptr()), 1e-6, 2,
                               ctypes.c_void_p(ws.data_ptr()), ws.numel(), None)
    assert rc == _lib.RV12_E_MODE


def test_token_scales():
    """Tokens scaled by 2^-60 .. 2^60 (and one of zeros) in one prompt: each
    token's exact power-of-two scale keeps the fp32 bound."""
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((200, 1024)) * 0.02).astype(np.float32)
    cnp = codec.compress(codec.f32_to_bf16_rne(w))
    T = 40
    scales = [2.0 ** e for e in np.linspace(-60, 60, T)]
    scales[7] = 0.0
    for mode in (0, 2):
        _check(cnp, T, 11 + mode, False, mode=mode, scales=scales)


def test_qwen3_8b_gu_2048_tokens_against_the_decode_kernels():
    """The 24576 x 4096 gu matrix over 2048 tokens: sampled token rows equal
    the MFMA decode-linear's (rv12_gemm at 16 tokens) within the tolerance,
    and a 64-token slice of rows equals the float64 closed form."""
    from ai_amd import prefill, wcomp
    g = torch.Generator(device="cuda").manual_seed(8)
    N, K, T = 24576, 4096, 2048
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02)
    w[torch.randperm(N, device="cuda", generator=g)[:24]] *= 20
    w = w.bfloat16()
    c = wcomp.compress(w)
    x = torch.randn(T, K, device="cuda", generator=g)
    y = torch.zeros(T, N, device="cuda")
    prefill.matrix(x, c, y)
    pick = torch.tensor([0, 1, 127, 128, 1000, 1777, 2046, 2047, 5, 6, 7, 8, 9, 10, 11, 12], device="cuda")
    xs = x[pick].contiguous()
    ys = torch.zeros(16, N, device="cuda")
    wcomp.gemvc_tc(xs, c, ys, 0, 16)
    torch.cuda.synchronize()
    ref = ys.cpu().numpy().astype(np.float64)
    got = y[pick].cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref)), float(np.abs(got - ref).max())
    # 64 rows against float64
    rows = slice(4096, 4160)
    W64 = w[rows].float().cpu().numpy().astype(np.float64)
    want = x[:64].cpu().numpy().astype(np.float64) @ W64.T
    mag = np.abs(x[:64].cpu().numpy().astype(np.float64)) @ np.abs(W64).T
    err = np.abs(y[:64, rows].cpu().numpy() - want)
    assert np.all(err <= 4 * (K + 8) * 2.0 ** -24 * mag + 1e-30), float(err.max())
    del c, w, x, y
    torch.cuda.empty_cache()


@pytest.mark.parametrize("K", [160, 224, 288])
def test_step_counts_off_the_ring(K):
    """K / 32 steps that are not a multiple of the kernel's four-slot load
    ring (5, 7, 9 steps): the padded steps of the last round load zeros
    through the 0-byte descriptors and add nothing; every mode, with and
    without the RMS prologue, exceptions in many rows."""
    rng = np.random.default_rng(K)
    w = (rng.standard_normal((300, K)) * 0.02).astype(np.float32)
    w[rng.choice(300, 3)] *= 20
    w.reshape(-1)[rng.choice(w.size, 60, replace=False)] = 1e-30
    cnp = codec.compress(codec.f32_to_bf16_rne(w), CH=32)
    assert cnp["er"].size > 30
    for T in (17, 130):
        for mode in (0, 1, 2):
            print("K", K, "T", T, "mode", mode, flush=True)
            _check(cnp, T, K + T + mode, mode != 0, mode=mode)
        _check(cnp, T, K + T + 7, False, mode=0, rms=True)


def test_random_draws_of_shapes_tokens_and_modes():
    """24 seeded draws of row count (1-600), K (128-2048 in steps of 32,
    codec chunks of 32), token count (1-400), MODE, the RMS prologue (MODES 0
    and 1), outlier rows and exceptions (3e4, -1e-30 or 1e-35 at random
    positions), each against the float64 closed form and the fp32 bound."""
    rng = np.random.default_rng(4242)
    for d in range(24):
        N = int(rng.integers(1, 601))
        K = 32 * int(rng.integers(4, 65))
        T = int(rng.integers(1, 401))
        mode = int(rng.integers(0, 3))
        rms = bool(rng.integers(0, 2)) and mode != 2
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        nout = int(rng.integers(0, 4))
        if nout:
            w[rng.choice(N, min(N, nout), replace=False)] *= 20
        nexc = int(rng.integers(0, 1 + N * K // 500))
        if nexc:
            w.reshape(-1)[rng.choice(w.size, nexc, replace=False)] = float(rng.choice([3e4, -1e-30, 1e-35]))
        cnp = codec.compress(codec.f32_to_bf16_rne(w), CH=32)
        print("draw", d, N, K, T, mode, rms, int(cnp["er"].size), flush=True)
        _check(cnp, T, 9000 + d, mode != 0, mode=mode, rms=rms)


@pytest.mark.parametrize("case", ["special_values", "all_zero"])
def test_matrix_on_golden_special_values(golden, case):
    """Golden matrices with infinities, NaNs, subnormals and zeros among the
    weights: NaN and infinite outputs where the closed form (rounded to
    float32) has them, every finite output within the tolerance.  (The
    golden matrices of weights near the top of the float32 range, huge_with_inf
    and window_hits_inf, are decode vectors only: a sum of their products
    overflows float32 part-way in an order-dependent way, so an infinite
    weight meets an overflowed partial sum of either sign.)"""
    cnp = ref_dict(golden[case])
    for add in (False, True):
        _check(cnp, 40, 3, add)
