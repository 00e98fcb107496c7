"""GPU parity of the fused decode-linear (gemvc1 / gemvc_tc through librv12.so)
against the oracle's closed form.

Bar: |y - y_ref| <= 1e-3 + 1e-2 |y_ref| in every output.  Each
case is also held to the fp32 forward-error bound of the oracle
(oracle.linear.error_bound: (K + 8) 2^-24 sum_k |w_k x'_k|), which a dropped
exception, a wrong exponent or a transposed operand would break."""
import numpy as np
import pytest
import torch

from conftest import ref_dict
from oracle import codec, cref, linear

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _close(y, ref, bound, what, tight_bound=True):
    """ref is the float64 closed form; outputs beyond the float32 range are
    compared with the closed form rounded to float32 (inf), as an fp32
    evaluation must produce."""
    y = np.asarray(y, np.float64)
    with np.errstate(over="ignore"):
        ref = np.asarray(ref, np.float64).astype(np.float32).astype(np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(y), np.isnan(ref)), what
    assert np.array_equal(y[np.isinf(ref)], ref[np.isinf(ref)]), what
    err = np.abs(y[fin] - ref[fin])
    assert np.all(err <= ATOL + RTOL * np.abs(ref[fin])), (what, float(err.max()))
    if tight_bound:
        tight = 4 * bound[fin] + 1e-30
        bad = err > tight
        assert not bad.any(), (what, float(err[bad].max()), float(tight[bad].min()))


def _inputs(c, T, mode, seed, rms):
    rng = np.random.default_rng(seed)
    K, N = c["K"], c["N"]
    xs = 2 * K if mode == 2 else K
    X = rng.standard_normal((T, xs)).astype(np.float32)
    Y0 = rng.standard_normal((T, N)).astype(np.float32)
    lnw = None
    if rms:
        lnw = codec.f32_to_bf16_rne((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    return X, Y0, lnw


def _run(c_gpu, X, Y0, mode, T, lnw=None, BN=None, w=None, S=None, eps=1e-6, use_tc=False, launch=None):
    """One linear through the Python mirror, or with `launch` (kernel, rb,
    waves, splits) straight through the C ABI's rv12_gemm."""
    import ctypes
    from ai_amd import _lib, wcomp
    x = torch.from_numpy(X).cuda()
    y = torch.from_numpy(Y0.copy()).cuda()
    ln = None if lnw is None else torch.from_numpy(lnw.view(np.int16).copy()).view(torch.bfloat16).cuda()
    if launch is not None:
        L = _lib.lib()
        cfg = _lib.Launch(*launch)
        out = _lib.Launch()
        _lib.check(L.rv12_launch_shape(int(c_gpu["N"]), int(c_gpu["K"]), T, ctypes.byref(cfg), ctypes.byref(out)),
                   "launch")
        need = max(16, L.rv12_workspace_bytes(int(c_gpu["N"]), int(c_gpu["K"]), T, out.splits))
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
        m = wcomp._matrix(c_gpu)
        _lib.check(L.rv12_gemm(ctypes.byref(m), p(x), p(y), T, p(ln), eps, mode, ctypes.byref(cfg), p(ws), need,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "rv12_gemm")
    elif T == 1 and not use_tc:
        wcomp.gemvc1(x, c_gpu, y, mode, BN=BN, w=w, lnw=ln, eps=eps)
    elif ln is not None:  # the RMS prologue at T > 1 (an addition to the reference's gemvc_tc)
        wcomp.gemvc_tc(x, c_gpu, y, mode, T, BN=BN, w=w, S=S, lnw=ln, eps=eps)
    else:
        wcomp.gemvc_tc(x, c_gpu, y, mode, T, BN=BN, w=w, S=S)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _check(cnp, c_gpu, T, mode, rms, seed, **kw):
    X, Y0, lnw = _inputs(cnp, T, mode, seed, rms)
    W = codec.decode_f32(cnp).astype(np.float64)
    lw = None if lnw is None else codec.bf16_to_f32(lnw)
    ref = linear.linear(cnp, X, mode, Y0, lnw=lw, W=W)
    bound = linear.error_bound(cnp, X, mode, lnw=lw, W=W)
    y = _run(c_gpu, X, Y0, mode, T, lnw=lnw, **kw)
    _close(y, ref, bound, (T, mode, rms, seed, kw))


@pytest.mark.parametrize("case", ["prefill_seed7", "special_values", "outliers_rows_cols", "chunk128",
                                  "tie_spread", "subnormal_heavy"])
def test_golden_matrices_all_modes(golden, case):
    from ai_amd import wcomp
    print("case", case, flush=True)
    cnp = ref_dict(golden[case])
    cg = wcomp.prepare(ref_dict(golden[case]))
    for mode in (0, 1, 2):
        for rms in (False, True):
            _check(cnp, cg, 1, mode, rms, 3)
        for T in (2, 5, 16):
            _check(cnp, cg, T, mode, False, 4 + T, use_tc=True)


@pytest.mark.parametrize("case", ["prefill_seed7", "outliers_rows_cols", "subnormal_heavy"])
def test_rms_prologue_batched(golden, case):
    """rv12_gemm with an RMSNorm weight at 2..16 tokens with the built-in
    kernel (on these small matrices the vector kernel at 2 and 3 tokens, the
    MFMA kernel at 8 and 16), one split and several."""
    from ai_amd import wcomp
    print("case", case, flush=True)
    cnp = ref_dict(golden[case])
    cg = wcomp.prepare(ref_dict(golden[case]))
    nsteps = cnp["K"] // 32
    for T in (2, 3, 8, 16):
        for mode in (0, 1, 2):
            _check(cnp, cg, T, mode, True, 20 + T + mode, use_tc=True)
            _check(cnp, cg, T, mode, True, 30 + T + mode, use_tc=True, S=min(3, nsteps))


def _random_matrix(N, K, seed, sigma=0.02, out_rows=0.0, out_cols=0.0):
    """bf16 bits of N(0, sigma) weights with outlier rows / columns x20
    (generated on the GPU, rounded to bf16 by torch)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(N, K, device="cuda", generator=g) * sigma
    if out_rows:
        w[torch.randperm(N, device="cuda", generator=g)[: max(1, int(N * out_rows))]] *= 20
    if out_cols:
        w[:, torch.randperm(K, device="cuda", generator=g)[: max(1, int(K * out_cols))]] *= 20
    return w.bfloat16().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("N,K", [(200, 1024), (520, 2560)])
def test_vector_kernel_prefetch_depths(N, K):
    """The vector kernel at 1-4 tokens in both of its prefetch depths, straight
    through the C ABI: workgroups of 4 waves keep the deep form (6 or 8 steps),
    of 8 or 16 waves the shallow one (4 steps; at one token where their first
    weight loads reach 48 KB), one and two row blocks, a partial last row
    block, with every prologue (RMS, accumulate, silu(g)*u, both), K split
    (the built-in fill split below 128 row blocks from 2 tokens on) and
    unsplit."""
    from ai_amd import wcomp
    print("shape", N, K, flush=True)
    bits = _random_matrix(N, K, N + 3 * K, out_rows=0.01, out_cols=0.01)
    cnp = codec.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    for T in (1, 2, 3, 4):
        for rb, w in ((1, 4), (1, 8), (1, 16), (2, 4), (2, 8)):
            for S in ((0, 1) if T > 1 and w == 8 else (0,)):
                print("  T", T, "rb", rb, "waves", w, "splits", S, flush=True)
                for mode, rms in ((0, True), (1, False), (2, False), (2, True)):
                    _check(cnp, cg, T, mode, rms, 40 + 7 * T + rb + w + mode, launch=(1, rb, w, S))


@pytest.mark.parametrize("N,K", [(1, 256), (15, 256), (16, 512), (33, 1024), (100, 768), (1000, 2048)])
def test_shapes_and_launch_shapes(N, K):
    from ai_amd import wcomp
    print("shape", N, K, flush=True)
    bits = _random_matrix(N, K, N + K, out_rows=0.01, out_cols=0.01)
    cnp = codec.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    nsteps = K // 32
    # vector kernel (the built-in choice at one token): BN rows per workgroup
    for BN, w, S in ((16, 1, 1), (16, 4, 1), (32, 2, 2), (64, 4, 1), (16, 3, min(5, nsteps)), (16, 4, nsteps)):
        if N % BN:
            BN = None  # the reference's N % BN rule; the default row tiling handles any N
        print("  launch", BN, w, S, flush=True)
        for mode in (0, 2):
            _check(cnp, cg, 1, mode, mode == 0, 7, BN=BN, w=w)
            _check(cnp, cg, 2, mode, False, 8, BN=BN, w=w, S=S, use_tc=True)
    # MFMA kernel (the built-in choice on the larger matrices): every row-block count
    # per wave and wave count it takes (the split count left to the library:
    # the fewest splits whose staging fits the LDS, so long splits stage
    # groups past the 4 per thread held in registers), straight through the
    # C ABI, at token counts of each staged width (4, 8, 16 columns)
    for rb, w, S in [(rb, w, 0) for rb in (1, 2, 4) for w in (1, 2, 4, 8)] + [(1, 4, nsteps), (4, 2, nsteps // 4)]:
        print("  mfma launch", rb, w, S, flush=True)
        for T, mode, rms in ((1, 0, True), (3, 0, True), (3, 2, False), (6, 1, False), (8, 2, True), (16, 1, False),
                             (11, 2, True)):
            _check(cnp, cg, T, mode, rms, 9 + T, launch=(2, rb, w, S))
    # the MFMA kernel with the waves splitting K (kernel 3): row blocks per
    # workgroup up to the wave count, with and without a K split
    for rb, w, S in [(rb, w, 0) for rb in (1, 2, 4) for w in (1, 2, 4, 8) if rb <= w] + [(1, 4, min(3, nsteps)),
                                                                                         (2, 8, nsteps)]:
        print("  mfma k-split-waves launch", rb, w, S, flush=True)
        for T, mode, rms in ((1, 0, True), (3, 0, True), (4, 2, False), (6, 1, False), (8, 2, True), (16, 1, False),
                             (11, 2, True)):
            _check(cnp, cg, T, mode, rms, 19 + T, launch=(3, rb, w, S))


def test_bn_must_divide_rows():
    from ai_amd import wcomp
    bits = _random_matrix(24, 256, 1)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    x = torch.zeros(256, device="cuda")
    y = torch.zeros(24, device="cuda")
    with pytest.raises(ValueError):
        wcomp.gemvc1(x, cg, y, 0, BN=16, w=4)
    with pytest.raises(ValueError):
        wcomp.gemvc_tc(x, cg, y, 0, 1, BN=16, w=4, S=1)
    with pytest.raises(ValueError):
        wcomp.gemvc1(x, cg, y, 3)
    with pytest.raises(ValueError):
        wcomp.gemvc_tc(x, cg, y, 0, 17)


QWEN3_8B = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288), (6144, 4096), (24576, 4096)]


@pytest.mark.parametrize("N,K", QWEN3_8B)
def test_qwen3_8b_shapes_full_size(N, K):
    """Qwen3-8B sweep matrices (sigma ~ U(0.01, 0.05), 0.1% outlier rows x20) at full
    size against the C oracle, modes 0/1/2 and RMS, T = 1 and 8."""
    from ai_amd import wcomp
    print("shape", N, K, flush=True)
    rng = np.random.default_rng(N * 7 + K)
    sigma = float(rng.uniform(0.01, 0.05))
    bits = _random_matrix(N, K, N + 3 * K, sigma=sigma, out_rows=0.001)
    cnp = cref.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    assert cg["base"] == cnp["base"] and cg["er"].numel() == cnp["er"].size
    for T, mode, rms in ((1, 0, True), (1, 1, False), (1, 2, False), (8, 0, False), (8, 2, False)):
        X, Y0, lnw = _inputs(cnp, T, mode, 5 + T + mode, rms)
        ref = Y0.copy()
        cref.gemv_12bit(cnp, X, ref, mode, lnw=lnw)
        y = _run(cg, X, Y0, mode, T, lnw=lnw, use_tc=T > 1)
        err = np.abs(y.astype(np.float64) - ref)
        assert np.all(err <= ATOL + RTOL * np.abs(ref)), (N, K, T, mode, rms, float(err.max()))
        # both sides are fp32 sums of the same exact products: agree to ~1e-5
        assert float((err / (np.abs(ref) + 1.0)).max()) < 1e-4, (N, K, T, mode, float(err.max()))


def test_lm_head_full_size():
    """151936 x 4096 (the lm_head) at M=1 against the C oracle."""
    from ai_amd import wcomp
    N, K = 151936, 4096
    bits = _random_matrix(N, K, 99, sigma=0.02, out_rows=0.001)
    cnp = cref.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    X, Y0, _ = _inputs(cnp, 1, 0, 1, False)
    ref = np.zeros((1, N), np.float32)
    cref.gemv_12bit(cnp, X, ref, 0)
    y = _run(cg, X, Y0, 0, 1)
    err = np.abs(y.astype(np.float64) - ref)
    assert np.all(err <= ATOL + RTOL * np.abs(ref)), float(err.max())
    assert float((err / (np.abs(ref) + 1.0)).max()) < 1e-4
    del cg
    torch.cuda.empty_cache()


@pytest.mark.parametrize("N,K,shape1,shape2", [
    (1000, 2048, (1, 1, 8, 1), (1, 1, 8, 4)),    # 63 row blocks: unsplit at one token, split at two
    (4100, 1024, (1, 2, 8, 1), (1, 2, 8, 1)),    # 257 row blocks of 32 K steps: two per workgroup of 8 waves
    (6000, 4096, (1, 2, 8, 1), (1, 2, 8, 1)),    # 375 row blocks
    (8300, 1024, (1, 1, 4, 1), (1, 1, 8, 1)),    # 519 row blocks, ragged: 4 waves at one token
    (5000, 17408, (1, 2, 8, 3), (1, 2, 8, 1)),   # 313 row blocks of a long K: 3 splits fill the round at
                                                  # one token; unsplit at two (the activations fit the LDS)
])
def test_default_launch_shape_families(N, K, shape1, shape2):
    """The built-in launch shape of each row-block range (asserted), every
    mode, with and without the RMS prologue, at one and two tokens, against
    the C oracle."""
    from ai_amd import wcomp
    print("shape", N, K, flush=True)
    assert wcomp.launch_shape(N, K, 1) == shape1
    if shape2 is not None:
        assert wcomp.launch_shape(N, K, 2) == shape2
    bits = _random_matrix(N, K, N + 5 * K, out_rows=0.001, out_cols=0.001)
    cnp = cref.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    for T, mode, rms in ((1, 0, True), (1, 1, False), (1, 2, False), (2, 0, True), (2, 1, False), (2, 2, False)):
        X, Y0, lnw = _inputs(cnp, T, mode, 11 + T + mode, rms)
        ref = Y0.copy()
        cref.gemv_12bit(cnp, X, ref, mode, lnw=lnw)
        y = _run(cg, X, Y0, mode, T, lnw=lnw, use_tc=T > 1)
        err = np.abs(y.astype(np.float64) - ref)
        assert np.all(err <= ATOL + RTOL * np.abs(ref)), (N, K, T, mode, rms, float(err.max()))
        assert float((err / (np.abs(ref) + 1.0)).max()) < 1e-4, (N, K, T, mode, float(err.max()))


def test_builtin_launch_random_shapes():
    """Seeded random shapes (ragged N, K from 256 to 12288) at 1-4 tokens with
    every prologue, each through the launch the library picks for it (vector
    kernel, either prefetch depth, split or not, or the MFMA kernel), against
    the C oracle: the launch rules' every branch meets the same bar."""
    from ai_amd import wcomp
    rng = np.random.default_rng(2026)
    seen = set()
    for case in range(24):
        N = int(rng.integers(1, 9000))
        K = 256 * int(rng.integers(1, 49))
        T = int(rng.integers(1, 5))
        mode = int(rng.integers(0, 3))
        rms = bool(rng.integers(0, 2))
        shape = wcomp.launch_shape(N, K, T)
        seen.add(shape[0])
        print("case", case, N, K, T, mode, rms, shape, flush=True)
        bits = _random_matrix(N, K, 100 + case, out_rows=0.002, out_cols=0.002)
        cnp = cref.compress(bits)
        cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
        X, Y0, lnw = _inputs(cnp, T, mode, 200 + case, rms)
        ref = Y0.copy()
        cref.gemv_12bit(cnp, X, ref, mode, lnw=lnw)
        y = _run(cg, X, Y0, mode, T, lnw=lnw, use_tc=T > 1)
        err = np.abs(y.astype(np.float64) - ref)
        assert np.all(err <= ATOL + RTOL * np.abs(ref)), (case, N, K, T, mode, rms, shape, float(err.max()))
        assert float((err / (np.abs(ref) + 1.0)).max()) < 1e-4, (case, N, K, T, mode, rms, shape, float(err.max()))
        del cg
    assert seen == {1, 2}, seen  # both kernels were picked


def test_tuned_launch_shapes_keep_parity(tmp_path):
    """tune() fills CFG1 / CFGT on the GPU; the linears then run with those
    launch shapes and still match the closed form: a plain MODE 0 shape,
    MODE 2 (timed with its silu(g) * u prologue) and a MODE 0 shape timed with
    the RMSNorm prologue the engine fuses into qkv and gu, run with it."""
    from ai_amd import tune, wcomp
    N, K = 1024, 1024
    Nr = 2048
    tune.tune([(N, K, 0), (N, K, 2), (Nr, K, 0, True)], log=lambda *a: None, cache=str(tmp_path / "tune.json"))
    try:
        assert (N, K, 0) in wcomp.CFG1 and (N, K, 2) in wcomp.CFGT and (Nr, K, 0) in wcomp.CFG1
        bits = _random_matrix(N, K, 5, out_rows=0.01)
        cnp = codec.compress(bits)
        cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
        for mode in (0, 2):
            _check(cnp, cg, 1, mode, False, 21)
            _check(cnp, cg, 16, mode, False, 22, use_tc=True)
        bits = _random_matrix(Nr, K, 6, out_rows=0.01)
        cnp = codec.compress(bits)
        cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
        _check(cnp, cg, 1, 0, True, 23)
        _check(cnp, cg, 16, 0, True, 24, use_tc=True)
    finally:
        wcomp.CFG1.clear()
        wcomp.CFGT.clear()


def test_two_tokens_with_k_beyond_the_vector_staging():
    """At 2 tokens the library runs the vector kernel while its activations fit
    in registers unsplit and the MFMA kernel beyond (K > 12288 here); both
    sides of the switch, every mode, with and without the RMS prologue."""
    from ai_amd import wcomp
    for N, K in ((100, 12288), (100, 16384)):
        print("shape", N, K, flush=True)
        bits = _random_matrix(N, K, 31 + K, out_rows=0.01, out_cols=0.001)
        cnp = codec.compress(bits)
        cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
        for mode in (0, 1, 2):
            _check(cnp, cg, 2, mode, False, 40 + mode, use_tc=True)
            _check(cnp, cg, 2, mode, True, 50 + mode, use_tc=True)
        del cg
        torch.cuda.empty_cache()


def test_partial_launch_shape_sizes_its_workspace():
    """BN and w given, S left to the library, and an explicit S beyond the
    built-in shape's: the workspace is sized for the split each launch
    resolves to (the built-in 16-token launch's workspace would be too
    small for 24 splits)."""
    from ai_amd import wcomp
    N, K = 2048, 5120
    bits = _random_matrix(N, K, 77, out_rows=0.01)
    cnp = codec.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    builtin = wcomp.launch_shape(N, K, 16)[3]
    partial = wcomp.launch_shape(N, K, 16, wcomp._launch(32, 2, None, 16))
    assert partial[:3] == (2, 1, 2)
    assert wcomp.launch_shape(N, K, 16, wcomp._launch(32, 2, 24, 16)) == (2, 1, 2, 24) and 24 > builtin
    for mode in (0, 2):
        _check(cnp, cg, 16, mode, False, 60 + mode, BN=32, w=2, use_tc=True)
        _check(cnp, cg, 16, mode, False, 62 + mode, BN=32, w=2, S=24, use_tc=True)


def _check_scaled(cnp, c_gpu, T, mode, rms, seed, e, both_halves=False, **kw):
    """Activations scaled by 2^e (MODE 2: g and u by 2^(e/2) each, so x' ~ 2^e,
    or both by 2^e with both_halves), y_prev scaled like W x'; the output held
    to 4x the fp32 forward-error bound plus the rounding of the final add."""
    rng = np.random.default_rng(seed)
    K, N = cnp["K"], cnp["N"]
    xs = 2 * K if mode == 2 else K
    X = rng.standard_normal((T, xs))
    if mode == 2 and not both_halves:
        X *= 2.0 ** (e / 2)
    else:
        X *= 2.0 ** e
    X = X.astype(np.float32)
    W = codec.decode_f32(cnp).astype(np.float64)
    lnw = codec.f32_to_bf16_rne((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)) if rms else None
    lw = None if lnw is None else codec.bf16_to_f32(lnw)
    xp = linear.prologue(X, K, mode, lw)
    typ = float(np.abs(xp @ W.T).mean()) or 1.0
    Y0 = (rng.standard_normal((T, N)) * typ).astype(np.float32)
    ref = linear.linear(cnp, X, mode, Y0, lnw=lw, W=W)
    bound = linear.error_bound(cnp, X, mode, lnw=lw, W=W)
    y = _run(c_gpu, X, Y0, mode, T, lnw=lnw, **kw).astype(np.float64)
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(ref)), (T, mode, rms, e)
    err = np.abs(y - ref)
    tight = 4 * bound + 2.0 ** -23 * np.abs(ref) + 1e-300
    bad = err > tight
    assert not bad.any(), (T, mode, rms, e, both_halves, float(err[bad].max()), float(tight[bad].min()))


@pytest.mark.parametrize("e", [-60, -40, -20, 0, 20, 40, 60])
def test_activation_scale(e):
    """Activations from 2^-60 to 2^60 in every mode, with and without the RMS
    prologue, at the token counts of the vector kernel: within 4x the fp32
    bound (the kernels scale x' by an exact power of two, so tiny activations
    do not meet the Q16 weights' float32 floor)."""
    from ai_amd import wcomp
    print("scale 2^%d" % e, flush=True)
    bits = _random_matrix(300, 1024, 1234, out_rows=0.01, out_cols=0.01)
    cnp = codec.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    cases = [(1, {}), (2, {}), (3, {"launch": (1, 1, 8, 0)}), (4, {"launch": (1, 1, 8, 0)}),  # vector kernel
             (3, {"launch": (2, 1, 4, 0)}), (4, {}), (6, {}), (8, {}), (16, {}),                  # MFMA kernel
             (16, {"launch": (2, 2, 4, 0)}), (4, {"launch": (2, 1, 1, 0)}),
             (4, {"launch": (3, 2, 8, 0)}), (16, {"launch": (3, 1, 4, 0)})]                       # waves split K
    for T, kw in cases:
        use_tc = T > 1
        for mode in (0, 1, 2):
            _check_scaled(cnp, cg, T, mode, False, 70 + T + mode, e, use_tc=use_tc, **kw)
            _check_scaled(cnp, cg, T, mode, True, 80 + T + mode, e, use_tc=use_tc, **kw)
        _check_scaled(cnp, cg, T, 2, False, 90 + T, e, both_halves=True, use_tc=use_tc, **kw)


def test_random_draws_of_the_launch_space():
    """64 seeded draws of matrix, token count (1-16), MODE, RMS prologue and
    launch (kernel 0-3, row blocks, waves, splits, each possibly left to the
    library): every draw rv12_launch_shape accepts runs through rv12_gemm and
    is held to the oracle's closed form and the fp32 bound; a draw it rejects
    is skipped.  Matrices of odd row counts (one partial row block) and 2%
    outlier rows and columns."""
    import ctypes
    from ai_amd import _lib, wcomp
    L = _lib.lib()
    rng = np.random.default_rng(2026)
    pool = []
    for i, (N, K) in enumerate([(37, 256), (300, 512), (129, 1024), (513, 768), (64, 2048), (250, 1536)]):
        bits = _random_matrix(N, K, 900 + i, out_rows=0.02, out_cols=0.02)
        cnp = codec.compress(bits)
        cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
        pool.append((cnp, cg, codec.decode_f32(cnp).astype(np.float64)))
    ran, kernels = 0, set()
    for d in range(64):
        cnp, cg, W = pool[int(rng.integers(len(pool)))]
        N, K = cnp["N"], cnp["K"]
        T = int(rng.integers(1, 17))
        mode = int(rng.integers(0, 3))
        rms = bool(rng.integers(0, 2))
        launch = (int(rng.choice([0, 1, 2, 3])), int(rng.choice([0, 1, 2, 4])), int(rng.choice([0, 1, 2, 4, 8, 16])),
                  int(rng.choice([0, 0, 1, 2, 3, 5, 8])))
        out = _lib.Launch()
        if L.rv12_launch_shape(N, K, T, ctypes.byref(_lib.Launch(*launch)), ctypes.byref(out)):
            continue
        print("draw", d, N, K, T, mode, rms, launch, "->", (out.kernel, out.rb, out.waves, out.splits), flush=True)
        X, Y0, lnw = _inputs(cnp, T, mode, 5000 + d, rms)
        lw = None if lnw is None else codec.bf16_to_f32(lnw)
        ref = linear.linear(cnp, X, mode, Y0, lnw=lw, W=W)
        bound = linear.error_bound(cnp, X, mode, lnw=lw, W=W)
        y = _run(cg, X, Y0, mode, T, lnw=lnw, launch=launch)
        _close(y, ref, bound, (d, N, K, T, mode, rms, launch))
        ran += 1
        kernels.add(out.kernel)
    assert ran >= 32 and kernels == {1, 2, 3}, (ran, kernels)


STEP_SCALES = {"huge": {3: 70, 17: 70}, "tiny": {0: -80, 9: -80, 30: -75},
               "mixed": {5: 70, 12: -80, 13: -30, 21: 40}}


@pytest.mark.parametrize("pattern", sorted(STEP_SCALES))
def test_activation_scale_in_some_steps(pattern):
    """Activation columns outside the fast path's range in a few 32-column K
    steps only (2^70 or 2^-80 against N(0, 1) elsewhere; in MODE 2 the u half
    carries the scale).  In the vector kernel each wave stages the columns of
    its own steps, so only the waves owning those steps take their own scale,
    and the epilogue brings every wave's sum (and the exception products of
    those columns: 2 % of the columns are outliers) to one scale.  Held to 4x
    the fp32 forward-error bound."""
    from ai_amd import wcomp
    print("pattern", pattern, flush=True)
    bits = _random_matrix(300, 1024, 4242, out_rows=0.01, out_cols=0.02)
    cnp = codec.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    K, N = cnp["K"], cnp["N"]
    colexp = np.zeros(K)
    for s, e in STEP_SCALES[pattern].items():
        colexp[32 * s:32 * s + 32] = e
    W = codec.decode_f32(cnp).astype(np.float64)
    cases = [(1, {}), (2, {}), (1, {"launch": (1, 1, 16, 0)}), (3, {"launch": (1, 1, 8, 0)}),
             (4, {"launch": (1, 1, 4, 0)}), (2, {"launch": (1, 1, 4, 2)}), (1, {"launch": (1, 2, 8, 3)})]
    for i, (T, kw) in enumerate(cases):
        for mode in (0, 1, 2):
            for rms in (False, True):
                rng = np.random.default_rng(1000 * i + 10 * mode + rms)
                X = rng.standard_normal((T, 2 * K if mode == 2 else K))
                X[:, -K:] *= 2.0 ** colexp
                X = X.astype(np.float32)
                lnw = codec.f32_to_bf16_rne((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)) if rms else None
                lw = None if lnw is None else codec.bf16_to_f32(lnw)
                xp = linear.prologue(X, K, mode, lw)
                typ = float(np.abs(xp @ W.T).mean()) or 1.0
                Y0 = (rng.standard_normal((T, N)) * typ).astype(np.float32)
                ref = linear.linear(cnp, X, mode, Y0, lnw=lw, W=W)
                bound = linear.error_bound(cnp, X, mode, lnw=lw, W=W)
                y = _run(cg, X, Y0, mode, T, lnw=lnw, use_tc=T > 1, **kw).astype(np.float64)
                assert np.all(np.isfinite(y)) and np.all(np.isfinite(ref)), (T, kw, mode, rms)
                err = np.abs(y - ref)
                tight = 4 * bound + 2.0 ** -23 * np.abs(ref) + 1e-300
                bad = err > tight
                assert not bad.any(), (pattern, T, kw, mode, rms, float(err[bad].max()), float(tight[bad].min()))


def test_activation_scale_mixed_tokens():
    """Tokens of very different scales in one batch (2^-50, 1, 2^50, and one
    token of zeros): each keeps the fp32 bound (the MFMA kernel's scale is
    per token)."""
    from ai_amd import wcomp
    bits = _random_matrix(200, 2048, 4321, out_rows=0.01)
    cnp = codec.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    W = codec.decode_f32(cnp).astype(np.float64)
    rng = np.random.default_rng(5)
    for T, kw in ((2, {}), (4, {"launch": (1, 1, 8, 0)}), (3, {"launch": (2, 1, 4, 0)}), (4, {}), (7, {}),
                  (16, {}), (5, {"launch": (3, 2, 4, 0)})):
        for mode in (0, 2):
            K = cnp["K"]
            X = rng.standard_normal((T, 2 * K if mode == 2 else K))
            X *= np.array([2.0 ** (-50 if t % 3 == 0 else (50 if t % 3 == 1 else 0)) for t in range(T)])[:, None]
            X[T // 2] = 0.0
            X = X.astype(np.float32)
            Y0 = np.zeros((T, cnp["N"]), np.float32)
            ref = linear.linear(cnp, X, mode, Y0, W=W)
            bound = linear.error_bound(cnp, X, mode, W=W)
            y = _run(cg, X, Y0, mode, T, use_tc=True, **kw).astype(np.float64)
            err = np.abs(y - ref)
            assert not (err > 4 * bound + 2.0 ** -23 * np.abs(ref) + 1e-300).any(), (T, mode, float(err.max()))


QWEN3_14B = {"qkv": (7168, 5120), "o_q": (5120, 5120), "gu": (34816, 5120), "down": (5120, 17408),
             "k_v": (1024, 5120), "gate_up": (17408, 5120)}


@pytest.mark.parametrize("name", sorted(QWEN3_14B))
def test_qwen3_14b_skinny_shapes_full_size(name):
    """Qwen3-14B skinny-GEMM matrices (N(0, 0.02), 0.1% outlier rows x20) at
    full size, M = 1, 2, 4, 8, 16 tokens with the built-in kernel choice,
    modes 0 (with the RMS prologue), 1 and 2, against the C oracle."""
    from ai_amd import wcomp
    N, K = QWEN3_14B[name]
    print("shape", name, N, K, flush=True)
    bits = _random_matrix(N, K, N + 7 * K, sigma=0.02, out_rows=0.001)
    cnp = cref.compress(bits)
    cg = wcomp.compress(torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda())
    assert cg["base"] == cnp["base"] and cg["er"].numel() == cnp["er"].size
    for T in (1, 2, 4, 8, 16):
        print("  M", T, wcomp.launch_shape(N, K, T), flush=True)
        for mode, rms in ((0, True), (1, False), (2, False)):
            X, Y0, lnw = _inputs(cnp, T, mode, 100 + T + mode, rms)
            ref = Y0.copy()
            cref.gemv_12bit(cnp, X, ref, mode, lnw=lnw)
            y = _run(cg, X, Y0, mode, T, lnw=lnw, use_tc=T > 1)
            err = np.abs(y.astype(np.float64) - ref)
            assert np.all(err <= ATOL + RTOL * np.abs(ref)), (name, T, mode, rms, float(err.max()))
            assert float((err / (np.abs(ref) + 1.0)).max()) < 1e-4, (name, T, mode, float(err.max()))
    del cg
    torch.cuda.empty_cache()
