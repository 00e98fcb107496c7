"""GPU codec parity: compress / retile / decode against the reference codec's
golden vectors (tests/golden/codec_golden.npz) — bit-exact."""
import numpy as np
import pytest
import torch

from conftest import ref_dict, same_bf16

pytestmark = pytest.mark.gpu


def _w(bits):
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).cuda()


def test_compress_matches_reference_dict(golden):
    from ai_amd import wcomp
    for name, g in golden.items():
        print("case", name, flush=True)
        c = wcomp.compress(_w(g["w"]), CH=g["ch"])
        assert c["base"] == g["base"], name
        for k in ("m8", "e4", "rp", "er", "ec"):
            assert np.array_equal(c[k].cpu().numpy(), g[k]), (name, k)
        assert np.array_equal(c["ev"].cpu().numpy().view(np.uint32), g["ev"].view(np.uint32)), name
        assert c["N"] == g["w"].shape[0] and c["K"] == g["w"].shape[1] and c["CH"] == g["ch"]


def test_decompress_matches_reference(golden):
    from ai_amd import wcomp
    for name, g in golden.items():
        print("case", name, flush=True)
        c = wcomp.compress(_w(g["w"]), CH=g["ch"])
        d = wcomp.decompress(c).view(torch.int16).cpu().numpy().view(np.uint16)
        # lossless: the exact input bits, NaN payloads included
        assert np.array_equal(d, g["w"]), name
        # the reference decompress equals it up to its NaN canonicalisation
        assert same_bf16(d, g["dec"]), name


def test_retile_of_reference_dict_decodes_exactly(golden):
    """A dict made by the reference's own compress (the fixture) re-tiles and
    decodes to the original weights."""
    from ai_amd import wcomp
    for name, g in golden.items():
        print("case", name, flush=True)
        c = wcomp.prepare(ref_dict(g))
        d = wcomp.decompress(c).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(d, g["w"]), name


def test_pack_matches_layout_model(golden):
    """The device packer writes exactly what the CPU model of the layout
    (tests/q16_model.py) writes: tiles, row windows and exception list."""
    import q16_model as q
    from ai_amd import wcomp
    for name, g in golden.items():
        if g["w"].shape[1] % 32:
            continue
        print("case", name, flush=True)
        t, rb, rp, er, ec, ev = q.pack(g["w"])
        got = wcomp.pack(_w(g["w"]))
        assert np.array_equal(got["q16_tiles"].cpu().numpy().view(np.uint32), t.reshape(-1)), name
        assert np.array_equal(got["q16_rbase"].cpu().numpy(), rb), name
        for k, v in (("q16_rp", rp), ("q16_er", er), ("q16_ec", ec)):
            assert np.array_equal(got[k].cpu().numpy(), v), (name, k)
        assert np.array_equal(got["q16_ev"].cpu().numpy().view(np.uint32), ev.view(np.uint32)), name


def test_decode_rows_ranges_and_f32(golden):
    from ai_amd import wcomp
    g = golden["outliers_rows_cols"]
    c = wcomp.prepare(ref_dict(g))
    w32 = (g["w"].astype(np.uint32) << 16).view(np.float32)
    for first, last in ((0, 64), (2, 7), (5, 6), (15, 17), (40, 41), (63, 64), (10, 10)):
        r = wcomp.decode_rows(c, first, last).cpu().numpy()
        assert r.shape == (last - first, g["w"].shape[1])
        assert np.array_equal(r.view(np.uint32), w32[first:last].view(np.uint32)), (first, last)


def test_prefill_seed_rows_exact():
    """decode_rows(compress(w), 2, 7) == w[2:7].float() for the reference
    test's matrices (ramvi/engine/tests/legacy/test_prefill.py:25-30,
    ramvi/engine/tools/checks/check_prefill.py:38-40)."""
    from ai_amd import wcomp
    for seed in (7, 43, 109, 19, 71, 509):
        torch.manual_seed(seed)
        w = torch.randn(9, 512).bfloat16()
        w[3, 11] = 1e-30
        w[4, 92] = 1e20
        c = wcomp.compress(w.cuda())
        assert torch.equal(wcomp.weight_rows(c, 2, 7).cpu(), w[2:7].float()), seed


def test_all_bit_patterns_round_trip():
    from ai_amd import wcomp
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    for shape in ((256, 256), (128, 512), (16, 4096), (1024, 64)):
        w = bits.view(torch.bfloat16).reshape(shape).cuda()
        perm = torch.randperm(65536, generator=torch.Generator().manual_seed(shape[0]))
        for ww in (w, w.flatten()[perm.cuda()].reshape(shape)):
            c = wcomp.compress(ww, CH=min(256, shape[1]))
            d = wcomp.decompress(c)
            assert torch.equal(d.view(torch.int16), ww.view(torch.int16)), shape


def test_outlier_rows_stay_out_of_the_packed_exception_list():
    """0.1% of rows x20: the reference dict holds a fifth of such a row as
    exceptions, the packed form (one window per row) almost none; both decode
    exactly."""
    from ai_amd import wcomp
    g = torch.Generator(device="cuda").manual_seed(3)
    N, K = 4096, 4096
    w = torch.randn(N, K, device="cuda", generator=g) * 0.02
    rows = torch.randperm(N, device="cuda", generator=g)[:4]
    w[rows] *= 20
    w = w.bfloat16()
    c = wcomp.compress(w)
    ref_rows = torch.bincount(c["er"].long(), minlength=N)
    own_rows = torch.diff(c["q16_rp"].long())
    assert int(ref_rows[rows].min()) > 500
    assert int(own_rows[rows].max()) < 20
    assert torch.equal(wcomp.decompress(c).view(torch.int16), w.view(torch.int16))


def test_large_matrix_round_trip_and_exceptions():
    """Full-size lm_head-shaped matrix with outlier rows and columns: decode is
    bit-exact and the exception list is row-major and complete."""
    from ai_amd import wcomp
    g = torch.Generator(device="cuda").manual_seed(11)
    N, K = 151936, 4096
    w = torch.randn(N, K, device="cuda", generator=g) * 0.02
    rows = torch.randperm(N, device="cuda", generator=g)[: N // 1000]
    w[rows] *= 20
    w = w.bfloat16()
    c = wcomp.compress(w)
    for first in (0, 1000, N - 700):
        d = wcomp.decode_rows(c, first, first + 640, torch.bfloat16)
        assert torch.equal(d.view(torch.int16), w[first:first + 640].view(torch.int16))
    er, ec = c["er"].long(), c["ec"].long()
    key = er * K + ec
    assert bool((key[1:] > key[:-1]).all())
    e = (w.view(torch.int16).int() >> 7) & 0xFF
    exc = ((e - c["base"]) < 0) | ((e - c["base"]) > 14)
    assert int(exc.sum()) == er.numel()
    assert bool(exc[er, ec].all())
    del w, c
    torch.cuda.empty_cache()


def test_random_draws_against_the_oracle_codec():
    """20 seeded draws of shape (1-400 rows, K a multiple of the chunk),
    chunk size (32, 64, 128, 256), weight scale (which moves the exponent
    window) and special values (NaN with payloads, +-inf, zeros, subnormals,
    huge and tiny normals at random positions): the GPU compress equals the
    oracle's codec.compress (pinned by the reference's golden dicts) field by
    field, bit for bit, and the GPU decode returns the input bits."""
    from oracle import codec
    from ai_amd import wcomp
    rng = np.random.default_rng(3131)
    specials = np.array([0x7FC1, 0xFF80, 0x7F80, 0x0000, 0x8000, 0x0001, 0x807F, 0x7F7F, 0x0080, 0x3F80],
                        dtype=np.uint16)
    for d in range(20):
        CH = int(rng.choice([32, 64, 128, 256]))
        N = int(rng.integers(1, 401))
        K = CH * int(rng.integers(1, max(2, 4096 // CH) + 1))
        scale = float(2.0 ** rng.uniform(-20, 20))
        w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
        bits = codec.f32_to_bf16_rne(w)
        n_sp = int(rng.integers(0, 1 + N * K // 200))
        if n_sp:
            bits.reshape(-1)[rng.choice(bits.size, n_sp, replace=False)] = rng.choice(specials, n_sp)
        print("draw", d, N, K, CH, scale, n_sp, flush=True)
        ref = codec.compress(bits, CH=CH)
        c = wcomp.compress(_w(bits), CH=CH)
        assert c["base"] == ref["base"], d
        for k in ("m8", "e4", "rp", "er", "ec"):
            assert np.array_equal(c[k].cpu().numpy(), ref[k]), (d, k)
        assert np.array_equal(c["ev"].cpu().numpy().view(np.uint32), np.asarray(ref["ev"]).view(np.uint32)), d
        back = wcomp.decompress(c).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(back, bits), d
