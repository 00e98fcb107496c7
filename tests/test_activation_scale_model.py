"""CPU model of the linear kernels' float32 arithmetic on the Q16 h values,
with and without the activation scaling (ai_amd/csrc/rv12_device.h): the h
values are the weights times 2^-sc (sc ~ 110 for N(0, 0.02) weights), so
products with small activations fall below the float32 normal range unless x'
is scaled by 2^P first and the row rescaled by 2^(sc - P) at the end.

The model sums in float32 with numpy (subnormals kept, no flush), one product
and one add per weight in column order; the kernels' order differs, which the
4x bound absorbs.  A planted mistake (P = 0, the layout's raw floor) must
break the bound at small scales."""
import numpy as np
import pytest

import q16_model as qm
from oracle import codec, linear


def _row_dot(h_row, x, sc, P):
    hf = (h_row.astype(np.uint32) << 16).view(np.float32)
    xs = np.ldexp(x.astype(np.float32), P).astype(np.float32)  # exact power-of-two scaling, as ldexpf
    acc = np.float32(0.0)
    with np.errstate(under="ignore", over="ignore"):
        for a, b in zip(hf, xs):
            acc = np.float32(acc + np.float32(a * b))
        return float(np.ldexp(np.float64(acc), sc - P))


def _fast_path_ok(xp):
    """Every nonzero |x'| in [2^-64, 2^63): the kernels' fast path, P = 64."""
    nz = xp[xp != 0]
    e = np.frexp(nz)[1]
    return bool(nz.size == 0 or (e.min() >= -63 and e.max() <= 63))


def _scale_exp(xp):
    """P of the kernels: 64 on the fast path, else 100 - frexp exponent of max |x'|."""
    if _fast_path_ok(xp):
        return 64
    nz = np.abs(xp[np.isfinite(xp) & (xp != 0)])
    return 64 if nz.size == 0 else 100 - int(np.frexp(nz.max())[1])


def _setup(seed, K=1024, N=4):
    rng = np.random.default_rng(seed)
    bits = codec.f32_to_bf16_rne((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    rbase = qm.row_bases(bits)
    h, out = qm.h_values(bits, rbase)
    c = codec.compress(bits)
    return rng, bits, rbase, h, c


@pytest.mark.parametrize("e", [-60, -40, -20, 0, 20, 40, 60])
def test_scaled_sums_stay_within_the_fp32_bound(e):
    rng, bits, rbase, h, c = _setup(7)
    K = bits.shape[1]
    W = codec.decode_f32(c).astype(np.float64)
    x = (rng.standard_normal(K) * 2.0 ** e).astype(np.float32)
    ref = linear.linear(c, x[None], 0, W=W)[0]
    bound = linear.error_bound(c, x[None], 0, W=W)[0]
    P = _scale_exp(x)
    for n in range(bits.shape[0]):
        inside = h[n] != 0
        hw = np.where(inside, h[n], 0)
        y = _row_dot(hw, x, qm.scale_exp(rbase[n]), P)
        # the exceptions of the row window, exact products added at the end
        y += float(np.sum(W[n][~inside] * x[~inside].astype(np.float64)))
        assert abs(y - ref[n]) <= 4 * bound[n], (e, n, y, ref[n], bound[n])


def test_unscaled_floor_breaks_the_bound():
    """The planted mistake: P = 0 (raw h values times x') loses every product
    at x ~ 2^-40."""
    rng, bits, rbase, h, c = _setup(8)
    K = bits.shape[1]
    W = codec.decode_f32(c).astype(np.float64)
    x = (rng.standard_normal(K) * 2.0 ** -40).astype(np.float32)
    ref = linear.linear(c, x[None], 0, W=W)[0]
    bound = linear.error_bound(c, x[None], 0, W=W)[0]
    broke = 0
    for n in range(bits.shape[0]):
        inside = h[n] != 0
        y = _row_dot(np.where(inside, h[n], 0), x, qm.scale_exp(rbase[n]), 0)
        y += float(np.sum(W[n][~inside] * x[~inside].astype(np.float64)))
        broke += abs(y - ref[n]) > 4 * bound[n]
    assert broke == bits.shape[0]


def test_fast_path_range_and_slow_scale():
    assert _fast_path_ok(np.array([0.0, 1.0, -2.0 ** -64, 2.0 ** 62.9], np.float32))
    assert not _fast_path_ok(np.array([1.0, 2.0 ** -65], np.float32))
    assert not _fast_path_ok(np.array([1.0, 2.0 ** 63], np.float32))
    x = np.array([0.0, 2.0 ** -70, 3.0 * 2.0 ** -80], np.float32)
    P = _scale_exp(x)
    assert 2.0 ** 99 <= 2.0 ** -70 * 2.0 ** P < 2.0 ** 100
    assert _scale_exp(np.zeros(4, np.float32)) == 64
