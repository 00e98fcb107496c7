"""CPU checks of the Q16 tile layout (numpy model in tests/q16_model.py)
against the oracle: the layout must reproduce every weight bit-exactly and the
rescaled dot product must equal the closed form."""
import numpy as np
import pytest

from conftest import ref_dict
from oracle import codec, linear
import q16_model as q


def test_layout_round_trip_on_golden(golden):
    for name, g in golden.items():
        c = ref_dict(g)
        N, K = c["N"], c["K"]
        t = q.retile(c)
        h = q.h_from_tiles(t, N, K)
        assert np.array_equal(h, q.h_values(c)), name
        bits = q.bf16_from_h(h, c["base"])
        er, ec = c["er"].astype(np.int64), c["ec"].astype(np.int64)
        bits[er, ec] = (c["ev"].view(np.uint32) >> 16).astype(np.uint16)
        assert np.array_equal(bits, g["w"]), name


def test_pairs_never_touch_spare_bits(golden):
    h = q.h_values(ref_dict(golden["all_patterns"]))
    assert not np.any(h & 0x7800), "h uses bits 11..14"
    assert h.max() < 65536


@pytest.mark.parametrize("name", ["prefill_seed7", "outliers_rows_cols", "tie_spread", "special_values",
                                  "chunk128"])
def test_scaled_dot_equals_closed_form(golden, name):
    c = ref_dict(golden[name])
    rng = np.random.default_rng(0)
    X = rng.standard_normal((3, c["K"]))
    ref = linear.linear(c, X, 0)
    got = q.scaled_dot(c, X)
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
        c = codec.compress(bits)
        x = np.arange(256, dtype=np.float64)[None, :] + 1
        y = q.scaled_dot(c, x)
        assert np.array_equal(y[0], (np.arange(16) * 7 + 1) * np.float64(codec.bf16_to_f32(bits[0, 0])))


def test_planted_oracle_mistake_is_caught(golden):
    """A plausible decoding slip (exponent off by one) in the oracle fails the
    golden vectors: the pinning has teeth."""
    c = ref_dict(golden["prefill_seed7"])
    bad = dict(c, base=c["base"] + 1)
    assert not np.array_equal(codec.decode_exact(bad), golden["prefill_seed7"]["w"])
    swapped = dict(c, e4=((c["e4"] >> 4) | (c["e4"] << 4)).astype(np.uint8))
    assert not np.array_equal(codec.decode_exact(swapped), golden["prefill_seed7"]["w"])
