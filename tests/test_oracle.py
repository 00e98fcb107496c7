"""Pinning the oracle (CPU only).

codec: against the golden vectors written by the reference's own compress /
decompress (tests/golden/codec_golden.npz), and the exhaustive lossless round
trip.  linear: against closed-form special cases (identity rows, one
exception, zero weights, MODE 2 with u = 0, RMS of a constant vector) and a
scalar brute force on tiny shapes.  C oracle: against the numpy one."""
import math

import numpy as np
import pytest

from conftest import ref_dict, same_bf16
from oracle import codec, cref, linear


@pytest.fixture(scope="module", autouse=True)
def _built():
    import os
    if not os.path.exists(cref.LIB_PATH):
        cref.build()


def test_compress_matches_golden(golden):
    for name, g in golden.items():
        c = codec.compress(g["w"], CH=g["ch"])
        assert c["base"] == g["base"], name
        for k in ("m8", "e4", "rp", "er", "ec"):
            assert np.array_equal(c[k], g[k]), (name, k)
        assert np.array_equal(c["ev"].view(np.uint32), g["ev"].view(np.uint32)), name


def test_decompress_matches_golden(golden):
    for name, g in golden.items():
        d = codec.decompress(ref_dict(g))
        assert same_bf16(d, g["dec"]), name
        # the NaN the reference's .bfloat16() produced in this torch build
        assert np.array_equal(d, g["dec"]), name


def test_lossless_round_trip_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(0)
    for shape in ((256, 256), (64, 1024), (16, 4096)):
        for w in (bits[: shape[0] * shape[1]].reshape(shape), rng.permutation(bits)[: shape[0] * shape[1]].reshape(shape)):
            for ch in (256, 64, 16):
                if shape[1] % ch:
                    continue
                c = codec.compress(w, CH=ch)
                assert np.array_equal(codec.decode_exact(c), w)


def test_base_is_first_maximal_window():
    # exponents 100 and 130 equally frequent, windows [86..100]..[100..114] all tie
    e = np.array([100] * 8 + [130] * 8, np.uint16)
    w = (e << 7).reshape(1, 16)
    w = np.tile(w, (1, 16))
    c = codec.compress(w, CH=256)
    assert c["base"] == 86
    # brute force over all windows
    ex = (w.astype(np.int64) >> 7) & 0xFF
    counts = [((ex >= b) & (ex <= b + 14)).sum() for b in range(242)]
    assert c["base"] == counts.index(max(counts))


def test_nibble_order_in_chunk():
    # code of element i in the low nibble, element CH/2 + i in the high nibble
    base_e = 110
    k = np.arange(256)
    e = base_e + (k % 15)
    w = (e.astype(np.uint16) << 7).reshape(1, 256)
    c = codec.compress(w)
    assert c["base"] == base_e
    assert c["e4"][0, 3] == (3 % 15) | (((128 + 3) % 15) << 4)


def test_c_oracle_matches_numpy(golden):
    for name, g in golden.items():
        a = codec.compress(g["w"], CH=g["ch"])
        b = cref.compress(g["w"], CH=g["ch"])
        assert a["base"] == b["base"], name
        for k in ("m8", "e4", "rp", "er", "ec"):
            assert np.array_equal(a[k], b[k]), (name, k)
        assert np.array_equal(a["ev"].view(np.uint32), b["ev"].view(np.uint32)), name
        assert np.array_equal(cref.decode_f32(b).view(np.uint32), codec.decode_f32(a).view(np.uint32)), name
    rng = np.random.default_rng(5)
    w = codec.f32_to_bf16_rne((rng.standard_normal((300, 1024)) * 0.03).astype(np.float32))
    w[7] = codec.f32_to_bf16_rne((rng.standard_normal(1024) * 0.6).astype(np.float32))
    a, b = codec.compress(w), cref.compress(w)
    for k in ("m8", "e4", "rp", "er", "ec"):
        assert np.array_equal(a[k], b[k]), k


def _c_from_f32(w):
    return codec.compress(codec.f32_to_bf16_rne(np.asarray(w, np.float32)))


def test_linear_identity_rows():
    w = np.zeros((16, 256), np.float32)
    w[np.arange(16), 5 + np.arange(16) * 3] = 1.0
    c = _c_from_f32(w)
    x = np.random.default_rng(1).standard_normal((2, 256)).astype(np.float32)
    y = linear.linear(c, x, 0)
    assert np.array_equal(y, x[:, 5 + np.arange(16) * 3].astype(np.float64))


def test_linear_single_exception():
    w = np.full((4, 256), 0.01, np.float32)
    w[2, 77] = 1e20   # far outside the window: an exception
    c = _c_from_f32(w)
    assert c["er"].tolist() == [2] and c["ec"].tolist() == [77]
    x = np.zeros((1, 256), np.float32)
    x[0, 77] = 3.0
    y = linear.linear(c, x, 0)
    assert y[0, 2] == 3.0 * float(codec.bf16_to_f32(codec.f32_to_bf16_rne(np.float32(1e20))))
    assert np.all(y[0, [0, 1, 3]] == 3.0 * float(codec.bf16_to_f32(codec.f32_to_bf16_rne(np.float32(0.01)))))


def test_linear_zero_weights_and_accumulate():
    c = _c_from_f32(np.zeros((5, 256)))
    x = np.ones((3, 256), np.float32)
    prev = np.arange(15, dtype=np.float32).reshape(3, 5)
    assert np.array_equal(linear.linear(c, x, 0), np.zeros((3, 5)))
    assert np.array_equal(linear.linear(c, x, 1, prev), prev.astype(np.float64))


def test_linear_mode2_and_rms_closed_forms():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((8, 256)).astype(np.float32) * 0.05
    c = _c_from_f32(w)
    W = codec.decode_f32(c).astype(np.float64)
    g = rng.standard_normal((1, 256)).astype(np.float32)
    # u = 0: silu(g) * 0 contributes nothing
    X = np.concatenate([g, np.zeros_like(g)], 1)
    prev = np.ones((1, 8), np.float32)
    assert np.array_equal(linear.linear(c, X, 2, prev), prev.astype(np.float64))
    # u = 1: silu(g) exactly
    X = np.concatenate([g, np.ones_like(g)], 1)
    sg = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    assert np.allclose(linear.linear(c, X, 2, np.zeros((1, 8))), sg @ W.T, rtol=1e-14, atol=0)
    # RMS of a constant vector a: rs = 1/sqrt(a^2 + eps), lnw = 1 -> x' = a * rs
    a = 3.0
    X = np.full((1, 256), a, np.float32)
    y = linear.linear(c, X, 0, lnw=np.ones(256), eps=1e-6)
    assert np.allclose(y, (a / math.sqrt(a * a + 1e-6)) * W.sum(1)[None, :], rtol=1e-14)


def test_linear_matches_brute_force(golden):
    rng = np.random.default_rng(3)
    g = golden["prefill_seed43"]
    c = ref_dict(g)
    c = dict(c, m8=c["m8"][:3], e4=c["e4"][:3], rp=c["rp"][:4], N=3)
    keep = c["er"] < 3
    c = dict(c, er=c["er"][keep], ec=c["ec"][keep], ev=c["ev"][keep])
    for mode in (0, 1, 2):
        X = rng.standard_normal((2, 2 * 512 if mode == 2 else 512)).astype(np.float32)
        prev = rng.standard_normal((2, 3)).astype(np.float32)
        for lnw in (None, (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)):
            a = linear.linear(c, X, mode, prev, lnw=lnw)
            b = linear.brute_force(c, X, mode, prev, lnw=lnw)
            assert np.allclose(a, b, rtol=1e-12, atol=1e-12), (mode, lnw is None)


def test_c_gemv_12bit_within_fp32_bound(golden):
    rng = np.random.default_rng(4)
    for name in ("outliers_rows_cols", "prefill_seed109", "chunk128"):
        c = ref_dict(golden[name])
        for mode, T, rms in ((0, 1, True), (1, 3, False), (2, 2, False)):
            X = rng.standard_normal((T, 2 * c["K"] if mode == 2 else c["K"])).astype(np.float32)
            Y = rng.standard_normal((T, c["N"])).astype(np.float32)
            lnw = codec.f32_to_bf16_rne((1 + 0.1 * rng.standard_normal(c["K"])).astype(np.float32)) if rms else None
            lw = None if lnw is None else codec.bf16_to_f32(lnw)
            ref = linear.linear(c, X, mode, Y, lnw=lw)
            bound = linear.error_bound(c, X, mode, lnw=lw)
            out = Y.copy()
            cref.gemv_12bit(c, X, out, mode, lnw=lnw)
            assert np.all(np.abs(out - ref) <= 4 * bound + 1e-30), (name, mode)


def test_dropped_exception_breaks_the_bound(golden):
    """A planted oracle mistake (one exception left out) is caught by the
    bound the GPU tests apply."""
    c = ref_dict(golden["outliers_rows_cols"])
    X = np.random.default_rng(6).standard_normal((1, c["K"])).astype(np.float32)
    ref = linear.linear(c, X, 0)
    bound = linear.error_bound(c, X, 0)
    j = int(np.argmax(np.abs(c["ev"])))
    bad = dict(c, er=np.delete(c["er"], j), ec=np.delete(c["ec"], j), ev=np.delete(c["ev"], j),
               rp=np.where(np.arange(c["N"] + 1) > c["er"][j], c["rp"] - 1, c["rp"]).astype(np.int32))
    wrong = linear.linear(bad, X, 0)
    assert np.any(np.abs(wrong - ref) > 4 * bound)


def test_gemv_bf16_matches_linear():
    rng = np.random.default_rng(7)
    w = codec.f32_to_bf16_rne((rng.standard_normal((33, 512)) * 0.05).astype(np.float32))
    X = rng.standard_normal((2, 512)).astype(np.float32)
    Y = np.zeros((2, 33), np.float32)
    cref.gemv_bf16(w, X, Y, add=False)
    ref = X.astype(np.float64) @ codec.bf16_to_f32(w).astype(np.float64).T
    assert np.allclose(Y, ref, rtol=1e-5, atol=1e-5)
