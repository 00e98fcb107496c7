"""Host-side checks of the streamed-layer byte image (ai_amd.stream,
the reference's _pack/_unpack role, ramvi/engine/ramvi_engine/core/engine.py:34-56):
every packed tensor of a layer lands at a 256-byte-aligned offset of one
buffer and comes back bit for bit as a view, empty exception lists included."""
import pytest
import torch

from ai_amd.stream import ALIGN, KEYS, LayerImage


def _mat(n, k, n_exc, seed):
    g = torch.Generator().manual_seed(seed)
    return {"N": n, "K": k,
            "q16_tiles": torch.randint(-2 ** 31, 2 ** 31 - 1, (n * k * 3 // 8,), generator=g, dtype=torch.int32),
            "q16_rbase": torch.randint(0, 255, (n,), generator=g, dtype=torch.int32),
            "q16_rp": torch.arange(n + 1, dtype=torch.int32) * n_exc // n,
            "q16_er": torch.randint(0, n, (n_exc,), generator=g, dtype=torch.int32),
            "q16_ec": torch.randint(0, k, (n_exc,), generator=g, dtype=torch.int32),
            "q16_ev": torch.randn(n_exc, generator=g)}


def test_layer_image_round_trip():
    mats = {"qkv": _mat(48, 64, 7, 1), "o": _mat(32, 32, 0, 2), "gu": _mat(64, 64, 13, 3), "down": _mat(32, 96, 1, 4)}
    im = LayerImage(mats, pin=False)
    assert len(im.table) == 4 * len(KEYS)
    offs = [o for _, _, o, _, _, _ in im.table]
    assert all(o % ALIGN == 0 for o in offs) and offs == sorted(offs)
    for (_, _, o, nb, _, _), (_, _, o2, _, _, _) in zip(im.table, im.table[1:]):
        assert o + nb <= o2                                  # no overlap
    assert im.nbytes % ALIGN == 0 and im.table[-1][2] + im.table[-1][3] <= im.nbytes
    buf = torch.zeros(im.nbytes + 512, dtype=torch.uint8)
    buf[:im.nbytes].copy_(im.host)
    back = im.views(buf)
    for name, c in mats.items():
        assert back[name]["N"] == c["N"] and back[name]["K"] == c["K"]
        for k in KEYS:
            assert back[name][k].dtype == c[k].dtype and back[name][k].shape == c[k].shape
            assert torch.equal(back[name][k].view(torch.uint8), c[k].view(torch.uint8)), (name, k)
    assert back["o"]["q16_er"].numel() == 0
    # the views alias the buffer: a new image copied in shows through
    buf[:im.nbytes].zero_()
    assert int(back["gu"]["q16_rbase"].abs().sum()) == 0
    with pytest.raises(ValueError):
        im.views(torch.zeros(im.nbytes - 1, dtype=torch.uint8))
