"""The streamed layers' byte image (ai_amd.stream.pack / unpack, the
reference's _pack/_unpack, ramvi/engine/ramvi_engine/core/engine.py:34-56) on
the CPU: every tensor comes back bit for bit as a view into one buffer, each
part starting at a multiple of 256 bytes, other values kept."""
import torch

from ai_amd import stream


def _dict():
    g = torch.Generator().manual_seed(0)
    return {"q16": {"tiles": torch.randint(0, 2**31 - 1, (777,), generator=g, dtype=torch.int32),
                    "rbase": torch.randint(0, 255, (33,), generator=g, dtype=torch.int32),
                    "ev": torch.randn(5, generator=g),
                    "er": torch.zeros(0, dtype=torch.int32)},
            "N": 33, "K": 256, "name": "o"}


def test_pack_unpack_round_trip():
    c = _dict()
    img, lay = stream.pack(c)
    assert img.dtype == torch.uint8 and img.numel() % 256 == 0
    offs = [off for _, off, _, _ in lay if off is not None]
    assert all(o % 256 == 0 for o in offs) and offs == sorted(offs)
    back = stream.unpack(img.clone(), lay)
    for k in ("tiles", "rbase", "ev", "er"):
        a, b = c["q16"][k], back["q16"][k]
        assert a.dtype == b.dtype and a.shape == b.shape
        assert torch.equal(a.view(torch.uint8) if a.numel() else a, b.view(torch.uint8) if b.numel() else b)
    assert back["N"] == 33 and back["K"] == 256 and back["name"] == "o"


def test_unpack_views_share_the_buffer():
    img, lay = stream.pack(_dict())
    buf = img.clone()
    back = stream.unpack(buf, lay)
    back["q16"]["ev"][0] = 42.0
    again = stream.unpack(buf, lay)
    assert float(again["q16"]["ev"][0]) == 42.0
