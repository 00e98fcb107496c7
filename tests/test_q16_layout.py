"""CPU checks of the packed form (numpy model in tests/q16_model.py) against
the oracle: the layout must reproduce every weight bit-exactly and the
rescaled dot product must equal the closed form."""
import numpy as np
import pytest

from conftest import ref_dict
from oracle import codec, linear
import q16_model as q


def test_layout_round_trip_on_golden(golden):
    for name, g in golden.items():
        w = g["w"]
        N, K = w.shape
        if K % 32:
            continue
        tiles, rbase, rp, er, ec, ev = q.pack(w)
        assert np.array_equal(q.h_from_tiles(tiles, N, K), q.h_values(w, rbase)[0]), name
        assert np.array_equal(q.decode(tiles, rbase, er, ec, ev, N, K), w), name


def test_row_window_is_the_reference_rule_per_row(golden):
    """A row's window is what the reference's compress chooses for a matrix
    made of that row alone."""
    for name in ("prefill_seed7", "special_values", "outliers_rows_cols", "tie_spread", "subnormal_heavy"):
        w = golden[name]["w"]
        rb = q.row_bases(w)
        for n in range(w.shape[0]):
            one = np.tile(w[n:n + 1], (1, 1))
            assert rb[n] == codec.compress(one, CH=w.shape[1])["base"], (name, n)


def test_pairs_never_touch_spare_bits(golden):
    w = golden["all_patterns"]["w"]
    h, _ = q.h_values(w, q.row_bases(w))
    assert not np.any(h & 0x7800), "h uses bits 11..14"
    assert h.max() < 65536


def test_row_windows_shrink_outlier_row_exceptions():
    """0.1% of rows scaled x20 sit above the matrix-wide window (about a fifth
    of their weights become reference exceptions) but inside their own."""
    rng = np.random.default_rng(0)
    w = rng.standard_normal((2048, 1024)).astype(np.float32) * 0.02
    w[[3, 1500]] *= 20
    bits = codec.f32_to_bf16_rne(w)
    ref = codec.compress(bits)
    _, _, rp, er, ec, ev = q.pack(bits)
    ref_rows = np.bincount(ref["er"], minlength=2048)
    own_rows = np.diff(rp)
    assert ref_rows[3] > 100 and ref_rows[1500] > 100
    assert own_rows[3] < 10 and own_rows[1500] < 10
    assert er.size < ref["er"].size


@pytest.mark.parametrize("name", ["prefill_seed7", "outliers_rows_cols", "tie_spread", "special_values",
                                  "chunk128"])
def test_scaled_dot_equals_closed_form(golden, name):
    g = golden[name]
    c = ref_dict(g)
    rng = np.random.default_rng(0)
    X = rng.standard_normal((3, c["K"]))
    ref = linear.linear(c, X, 0)
    got = q.scaled_dot(g["w"], X)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    assert np.allclose(got[fin], ref[fin], rtol=1e-12, atol=0)


def test_scaled_dot_exact_cases():
    """Identity-like rows: y picks single activations; base 0 and a window
    reaching exponent 254 both rescale exactly, and with base 0 subnormal
    weights enter with their own value."""
    for scale in (1.0, 2.0 ** -120, 2.0 ** 100, 3.0, 2.0 ** -130, -(2.0 ** -133) * 3):
        w = np.zeros((16, 256), np.float32)
        w[np.arange(16), np.arange(16) * 7] = scale
        bits = codec.f32_to_bf16_rne(w)
        x = np.arange(256, dtype=np.float64)[None, :] + 1
        y = q.scaled_dot(bits, x)
        assert np.array_equal(y[0], (np.arange(16) * 7 + 1) * np.float64(codec.bf16_to_f32(bits[0, 0])))


def test_planted_oracle_mistake_is_caught(golden):
    """A plausible decoding slip (exponent off by one, swapped nibbles) in the
    oracle fails the golden vectors: the pinning has teeth."""
    c = ref_dict(golden["prefill_seed7"])
    bad = dict(c, base=c["base"] + 1)
    assert not np.array_equal(codec.decode_exact(bad), golden["prefill_seed7"]["w"])
    swapped = dict(c, e4=((c["e4"] >> 4) | (c["e4"] << 4)).astype(np.uint8))
    assert not np.array_equal(codec.decode_exact(swapped), golden["prefill_seed7"]["w"])
