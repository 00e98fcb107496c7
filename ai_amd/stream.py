"""Layers kept in host memory and streamed into HBM for each pass: the
reference engine's byte image, pinned arena and loader thread
(ramvi/engine/ramvi_engine/core/engine.py:34-187).

    pack(c) -> (bytes, layout)   engine.py:34-45   one uint8 image of a dict's tensors,
                                                   each part padded to 256 bytes
    unpack(buf, layout) -> dict  engine.py:48-56   views into a device copy of the image
    Arena(budget)                engine.py:59-80   pinned host memory in 256 MiB chunks,
                                                   plain memory beyond the budget
    Loader()                     engine.py:83-174  a thread that copies jobs host -> device
                                                   on its own stream in 10 MiB chunks,
                                                   passes errors on, bounds every wait

On MI355X the images are the kernels' packed form (Q16 tiles, row windows,
the packed exception list), so a streamed layer runs the same kernels on the
same bytes as a resident one.  Pinned memory is allocated as such (torch
pin_memory, hipHostMalloc); memory that already exists is never registered:
a non-pinned source goes through a ring of pinned staging buffers.
"""
import queue
import threading
import time

import torch

ALIGN = 256


def _flat(c, prefix=""):
    for k, v in c.items():
        name = prefix + str(k)
        if isinstance(v, dict):
            yield from _flat(v, name + "/")
        else:
            yield name, v


def pack(c):
    """Every tensor of the (nested) dict c in one uint8 image, each part
    starting at a multiple of 256 bytes; other values are kept in the layout
    (engine.py:34-45)."""
    parts, lay, off = [], [], 0
    for k, v in _flat(c):
        if torch.is_tensor(v):
            b = v.contiguous().view(-1).view(torch.uint8)
            lay.append((k, off, v.dtype, tuple(v.shape)))
            pad = (-b.numel()) % ALIGN
            parts += [b, torch.zeros(pad, dtype=torch.uint8, device=b.device)]
            off += b.numel() + pad
        else:
            lay.append((k, None, v, None))
    if not parts:
        return torch.zeros(0, dtype=torch.uint8), lay
    return torch.cat(parts), lay


def unpack(buf, lay):
    """The dict of pack's layout with every tensor a view into buf
    (engine.py:48-56)."""
    c = {}
    for k, off, dt, sh in lay:
        *path, leaf = k.split("/")
        d = c
        for p in path:
            d = d.setdefault(p, {})
        if off is None:
            d[leaf] = dt
        else:
            n = torch.Size(sh).numel() * torch.empty(0, dtype=dt).element_size()
            d[leaf] = buf[off:off + n].view(dt).view(sh)
    return c


class Arena:
    """Pinned host memory in chunks of exactly 256 MiB (engine.py:59-80);
    beyond `budget` bytes the images stay in ordinary memory."""
    CH = 256 * 2**20

    def __init__(self, budget):
        self.budget, self.chunks, self.used, self.pinned, self.plain = budget, [], self.CH, 0, 0

    def put(self, t):
        n = t.numel() * t.element_size()
        if self.used + n > self.CH:
            if (len(self.chunks) + 1) * self.CH > self.budget or n > self.CH:
                self.plain += n
                return t.contiguous().cpu()
            self.chunks.append(torch.empty(self.CH, dtype=torch.uint8, pin_memory=True))
            self.used = 0
        v = self.chunks[-1][self.used:self.used + n].view(t.dtype).view(t.shape)
        v.copy_(t)
        self.used += (n + ALIGN - 1) // ALIGN * ALIGN
        self.pinned += n
        return v


class Loader:
    """Host -> device copies on a thread of their own, with error passing,
    bounded waits and an explicit close (engine.py:83-174).

    A job is a dict {"pairs": [(src uint8 host, dst uint8 device)], "wait":
    earlier release or None, "done": Event, "ev": None, "rel": release}: the
    thread waits for `wait` (the slot's previous user has finished with it),
    makes its stream wait for that release's event, copies every pair in
    chunks of CHUNK bytes, records `ev` and sets `done`.  An error is stored
    in the job (and its release) and ends every later job."""
    TIMEOUT = 60.0
    CHUNK = 10 * 2**20
    STAGE_SLOTS = 4

    def __init__(self, device=None):
        dev = torch.device(device) if device is not None else torch.device("cuda")
        self.dev = dev if dev.index is not None else torch.device("cuda", torch.cuda.current_device())
        self.q, self.cs = queue.Queue(), torch.cuda.Stream(self.dev)
        self._stop = threading.Event()
        self._stage = None
        self.thread = threading.Thread(target=self._run, name="rv12-loader", daemon=True)
        self.thread.start()

    @classmethod
    def wait(cls, job, cancel=None):
        """Wait for a job (at most TIMEOUT s); its error becomes a RuntimeError."""
        end = time.monotonic() + cls.TIMEOUT
        while not job["done"].wait(min(0.05, max(0.0, end - time.monotonic()))):
            if cancel is not None and cancel.is_set():
                raise RuntimeError("streaming closed")
            if time.monotonic() >= end:
                raise TimeoutError("timed out waiting for a streamed layer")
        if job.get("error") is not None:
            raise RuntimeError("streaming a layer failed") from job["error"]

    def _stage_slot(self, n):
        """A pinned staging buffer for a chunk from ordinary memory (a ring of
        4 x 10 MiB, engine.py:105-118); reused only after its last copy ended."""
        if self._stage is None:
            self._stage = [torch.empty(self.CHUNK, dtype=torch.uint8, pin_memory=True)
                           for _ in range(self.STAGE_SLOTS)]
            self._stage_events = [None] * self.STAGE_SLOTS
            self._stage_index = -1
        self._stage_index = (self._stage_index + 1) % self.STAGE_SLOTS
        prev = self._stage_events[self._stage_index]
        if prev is not None:
            self._event(prev)
        return self._stage[self._stage_index][:n]

    def _event(self, event):
        if self._stop.is_set():
            raise RuntimeError("streaming closed")
        event.synchronize()

    def _run(self):
        failure = None
        while True:
            job = self.q.get()
            if job is None:
                return
            try:
                if failure is not None:
                    raise RuntimeError("the loader failed earlier") from failure
                if self._stop.is_set():
                    raise RuntimeError("streaming closed")
                torch.cuda.set_device(self.dev)
                if job["wait"] is not None:
                    self.wait(job["wait"], self._stop)
                    self.cs.wait_event(job["wait"]["ev"])
                pend = []
                for src, dst in job["pairs"]:
                    if src.numel() > dst.numel():
                        raise ValueError("streamed image larger than its device slot")
                    staged = not src.is_pinned()
                    for a in range(0, src.numel(), self.CHUNK):
                        if self._stop.is_set():
                            raise RuntimeError("streaming closed")
                        part = src[a:a + self.CHUNK]
                        if staged:
                            slot = self._stage_slot(part.numel())
                            slot.copy_(part)
                            part = slot
                        with torch.cuda.stream(self.cs):
                            dst[a:a + part.numel()].copy_(part, non_blocking=True)
                            event = torch.cuda.Event()
                            event.record(self.cs)
                        if staged:
                            self._stage_events[self._stage_index] = event
                        pend.append(event)
                        if len(pend) > 2:
                            self._event(pend.pop(0))
                event = torch.cuda.Event()
                event.record(self.cs)
                job["ev"] = event
            except Exception as exc:  # passed to the consumer through the job
                failure = exc
                job["error"] = exc
                if job.get("rel") is not None:
                    job["rel"]["error"] = exc
                    job["rel"]["done"].set()
            finally:
                job["done"].set()

    def close(self):
        """Stop the thread and wait (bounded) for the last copies."""
        self._stop.set()
        self.q.put(None)
        self.thread.join(timeout=5)
        if self.thread.is_alive():
            raise RuntimeError("the loader thread did not end")
        end = time.monotonic() + self.TIMEOUT
        while not self.cs.query():
            if time.monotonic() >= end:
                raise TimeoutError("copies did not finish at close")
            time.sleep(0.001)
