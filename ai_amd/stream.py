"""Layers streamed from pinned host memory into HBM, for models whose 12-bit
weights do not all stay resident (the reference's "stream" placement: a
byte image per layer, a pinned arena and a loader thread,
ramvi/engine/ramvi_engine/core/engine.py:34-187, 271-320).

MI355X form, without a host thread:

  LayerImage  the packed matrices of one layer (the q16_* tensors the
              kernels read) back to back in one pinned host buffer
              (hipHostMalloc through torch's pin_memory), each at a 256-byte
              aligned offset, with a table (matrix, key, offset, bytes,
              dtype, shape);
  Streamer    S device slots of the largest image; streamed layer i uses
              slot i % S.  Its H2D copies run on a copy stream of their own
              and are ordered against the compute stream by events only:
              copy i waits until the compute of layer i - S has released
              the slot, the compute of layer i waits until copy i has
              filled it.  The whole decode step, copies included, is
              enqueued at once, so it can be captured as one HIP graph, and
              the first S copies overlap the resident layers' compute.

The views of a slot are ordinary matrix dicts (q16_* tensors, N, K): the
linears read them exactly as they read a resident layer.
"""
import torch

KEYS = ("q16_tiles", "q16_rbase", "q16_rp", "q16_er", "q16_ec", "q16_ev")
ALIGN = 256


class LayerImage:
    """One layer's packed matrices in one host buffer (pinned unless
    pin=False, which only the host-side tests use)."""

    def __init__(self, mats, pin=True):
        self.table = []  # (matrix, key, offset, bytes, dtype, shape)
        off = 0
        for name, c in mats.items():
            for k in KEYS:
                t = c[k]
                nb = t.numel() * t.element_size()
                self.table.append((name, k, off, nb, t.dtype, tuple(t.shape)))
                off += -(-nb // ALIGN) * ALIGN
        self.nbytes = max(off, ALIGN)
        self.host = torch.empty(self.nbytes, dtype=torch.uint8, pin_memory=pin)
        for name, k, o, nb, _, _ in self.table:
            if nb:
                self.host[o:o + nb].copy_(mats[name][k].contiguous().view(-1).view(torch.uint8))
        self.meta = {name: {"N": int(c["N"]), "K": int(c["K"])} for name, c in mats.items()}

    def views(self, buf):
        """The layer's matrices as dicts of views into buf (a uint8 tensor of
        at least nbytes): buf holds the image, the views its tensors."""
        if buf.numel() < self.nbytes:
            raise ValueError("the buffer is smaller than the layer image")
        out = {name: dict(m) for name, m in self.meta.items()}
        for name, k, o, nb, dt, shape in self.table:
            out[name][k] = buf[o:o + nb].view(dt).view(shape)
        return out


class Streamer:
    """S device slots fed with the images of the streamed layers (in the
    order they run) on a copy stream; see the module docstring."""

    def __init__(self, images, device, slots=2):
        if slots < 1:
            raise ValueError("at least one slot")
        self.images = list(images)
        self.n, self.S = len(self.images), int(slots)
        size = max(im.nbytes for im in self.images)
        self.slots = [torch.empty(size, dtype=torch.uint8, device=device) for _ in range(self.S)]
        self.copy = torch.cuda.Stream(device)  # default priority
        self.filled = [torch.cuda.Event() for _ in range(self.S)]
        self.drained = [torch.cuda.Event() for _ in range(self.S)]
        self.W = [im.views(self.slots[i % self.S]) for i, im in enumerate(self.images)]
        self.bytes_per_pass = sum(im.nbytes for im in self.images)

    def begin(self):
        """Start of a pass over the layers: the copy stream forks off the
        current stream (after everything enqueued so far, the previous
        pass's use of the slots included) and the first S copies go out."""
        self.copy.wait_stream(torch.cuda.current_stream())
        for i in range(min(self.S, self.n)):
            self._load(i)

    def _load(self, i):
        s = i % self.S
        with torch.cuda.stream(self.copy):
            if i >= self.S:
                self.copy.wait_event(self.drained[s])
            im = self.images[i]
            self.slots[s][:im.nbytes].copy_(im.host, non_blocking=True)
            self.filled[s].record(self.copy)

    def acquire(self, i):
        """Streamed layer i's matrices, once its copy has landed (the current
        stream waits for it)."""
        torch.cuda.current_stream().wait_event(self.filled[i % self.S])
        return self.W[i]

    def release(self, i):
        """Streamed layer i's kernels are enqueued: its slot is free once
        they finish, and the copy of layer i + S goes out behind them."""
        self.drained[i % self.S].record(torch.cuda.current_stream())
        if i + self.S < self.n:
            self._load(i + self.S)

    def end(self):
        """End of a pass: the current stream joins the copy stream."""
        torch.cuda.current_stream().wait_stream(self.copy)
