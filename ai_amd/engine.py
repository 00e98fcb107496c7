"""Qwen3 greedy decoding on the 12-bit decode-linear: the reference engine's
call contract for the path (ramvi/engine/ramvi_engine/core/engine.py).

For every layer the four fused matrices are compressed once (engine.py:223-224)
and a token runs them exactly as the reference's `_gpu_layer` does
(engine.py:329-341):

    gemvc1(x,   W.qkv,  qkv, 0, lnw=ln1)      RMSNorm fused in the prologue
    q/k head norms, RoPE, KV write, attention  (one HIP kernel; tkernels.py:164-213)
    gemvc1(att, W.o,    x,   1)               residual accumulate
    gemvc1(x,   W.gu,   gu,  0, lnw=ln2)
    gemvc1(gu,  W.down, x,   2)               silu(g) * u prologue, accumulate

and 2..16 tokens of one sequence as `_batch_layer` does (engine.py:344-356),
`gemvc_tc` for the four matrices with the RMSNorms fused into the prologue.  The lm_head runs
through the same 12-bit linear with the final norm fused (new: the reference
picks greedy tokens with an int8 bound pass and exact CPU rows,
ramvi/engine/ramvi_engine/generation/head.py:29-88), followed by argmax, the
smallest id on ties (head.py:76-79).

A decode step is one HIP graph (the reference captures one per batch bucket,
engine.py:432-444): all layers on the embedding row of the current token,
the head with its fused pick, and one small library kernel
(rv12_decode_advance) for the bookkeeping (the id recorded, the next token's
embedding row written, position and output counter advanced) run on the
device, so the host only replays the graph.
The step's attention (head norms, RoPE, KV write, grouped-query attention)
is one HIP kernel per layer (ai_amd.attn); passes of 2..16 tokens use the
batch kernels of the same library, the blocked prefill its prompt kernels.

A prompt goes through passes of up to 16 tokens (the reference's legacy
prefill, engine.py:471-480), or, in the reference's opt-in blocked mode
(RAMVI_PREFILL=blocked from RAMVI_PREFILL_MIN_TOKENS tokens on,
ramvi/engine/ramvi_engine/kernels/prefill.py), all prompt tokens at once with
each matrix decoded once and multiplied in one GEMM (ai_amd.prefill).

Every layer stays resident in HBM by default (the reference's "gpu"
placement): at about 1.5 bytes per weight the largest model here, Qwen3-32B,
needs 48 GB of the MI355X's 288 GB.  With stream_layers = n the last n layers
are kept as byte images in pinned host memory instead and copied into HBM
slots during every pass (the reference's "stream" placement, ai_amd.stream),
the copies ordered by events inside the same graph.
"""
import os

import torch

from . import _lib
from . import prefill as blocked_prefill
from . import wcomp
from .attn import RopeAttn
from .stream import LayerImage, Streamer

MATS = ("qkv", "o", "gu", "down")
BATCH = 16  # largest batch of one pass, as the reference's graph buckets (engine.py:31)


class Engine:
    """Greedy Qwen3 decoding with every linear on the MI355X 12-bit path.

    ck        checkpoint object (ai_amd.model.Ckpt / RandomCkpt)
    maxt      context length of the KV cache
    kv_dtype  dtype of the KV cache (the reference keeps float32,
              engine.py:234-235; bfloat16 halves its traffic)
    prefill   "legacy" (passes of 16 tokens) or "blocked" (ai_amd.prefill);
              None reads RAMVI_PREFILL as the reference does
    prefill_min  fewest prompt tokens for the blocked prefill (None:
              RAMVI_PREFILL_MIN_TOKENS, 256)
    stream_layers  the last n layers live in pinned host memory and are
              streamed through `slots` HBM slots every pass (ai_amd.stream)
    tune      measure the launch shapes of the four layer linears on this
              device first (ai_amd.tune, cached per library and device), with
              the prologues the engine runs them with: the RMSNorm for qkv and
              gu, silu(g) * u for down (the reference tunes at load,
              core/engine.py:207-208)
    """

    def __init__(self, ck, maxt=2048, kv_dtype=torch.float32, device="cuda", log=None, prefill=None,
                 prefill_min=None, stream_layers=0, slots=2, tune=False):
        if prefill is None:
            blocked_prefill.enabled()  # validates RAMVI_PREFILL
            prefill = os.environ.get("RAMVI_PREFILL", "legacy")
        if prefill not in ("legacy", "blocked"):
            raise ValueError("prefill must be legacy or blocked")
        if prefill_min is None:
            prefill_min = int(os.environ.get("RAMVI_PREFILL_MIN_TOKENS", "256"))
        if prefill_min < 0:
            raise ValueError("prefill_min must not be negative")
        self.prefill_mode, self.prefill_min = prefill, int(prefill_min)
        self.ck = ck
        self.L, self.D, self.H, self.KV, self.HD, self.FF, self.eps = ck.L, ck.D, ck.H, ck.KV, ck.HD, ck.FF, ck.eps
        self.V, self.maxt, self.kv_dtype = ck.V, maxt, kv_dtype
        dev = self.dev = torch.device(device)
        H, KV, HD = self.H, self.KV, self.HD
        if tune:
            from . import tune as tuner
            P = ck.layer_params()
            tuner.tune([(*P["qkv"], 0, True), (*P["o"], 1), (*P["gu"], 0, True), (*P["down"], 2)],
                       log=log or (lambda *a: None))
        self.inv = (1.0 / (ck.theta ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)  # engine.py:204
        self.emb = ck.t("model.embed_tokens.weight", dev)
        if not 0 <= stream_layers <= self.L:
            raise ValueError("stream_layers must be in 0..layers")
        self.first_streamed = self.L - int(stream_layers)
        self.W, self.small, self.Kc, self.Vc, images = [], [], [], [], []
        for i in range(self.L):
            w = ck.layer(i, dev)
            self.small.append({k: w[k] for k in ("ln1", "ln2")} | {k: w[k].float() for k in ("qn", "kn")})
            self.W.append({n: wcomp.compact(wcomp.compress(w[n])) for n in MATS})
            if i >= self.first_streamed:  # to pinned host memory; HBM keeps only the slots
                images.append(LayerImage(self.W[i]))
                self.W[i] = None
            self.Kc.append(torch.zeros(KV, maxt, HD, dtype=kv_dtype, device=dev))
            self.Vc.append(torch.zeros_like(self.Kc[-1]))
            del w
            if log:
                log(f"layer {i + 1}/{self.L} compressed")
        self.streamer = Streamer(images, dev, slots) if images else None
        self.norm = ck.t("model.norm.weight", dev)
        self.normf = self.norm.float()
        self.head = wcomp.compact(wcomp.compress(ck.t(ck.head_name(), dev)))
        torch.cuda.empty_cache()
        f = lambda n: torch.zeros(BATCH, n, device=dev)
        self.xb, self.qkvb, self.attb, self.gub = f(self.D), f((H + 2 * KV) * HD), f(H * HD), f(2 * self.FF)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.tok = torch.zeros(BATCH, dtype=torch.long, device=dev)
        self.nxt = torch.zeros(BATCH, dtype=torch.long, device=dev)
        self.steps = torch.zeros(1, dtype=torch.long, device=dev)
        self.out = torch.zeros(maxt + 1, dtype=torch.long, device=dev)
        self.attn = RopeAttn(H, KV, HD, maxt, kv_dtype, self.eps, dev)
        self.graph = None
        self.pgraph = None  # a full prefill chunk of BATCH tokens
        self.tgraphs = {}   # T -> graph of one pass of T <= BATCH tokens (process)

    # ---------------------------------------------------------------- layers
    def _rope_attn(self, l, T, p0=None):
        """Rows 0..T-1 of qkv at positions pos..pos+T-1: q/k head RMSNorm,
        RoPE, K/V into the cache (rounded to its dtype), causal attention over
        the cache (tkernels.py:82-150, 164-213), all on the device: the
        one-token kernel, or the batch kernels for T > 1."""
        s = self.small[l]
        if T == 1:
            self.attn(self.qkvb[0], s["qn"], s["kn"], self.inv, self.pos, self.Kc[l], self.Vc[l], self.attb[0])
        else:
            self.attn.batch(self.qkvb[:T], s["qn"], s["kn"], self.inv, self.pos, self.Kc[l], self.Vc[l],
                            self.attb[:T], T)

    def _gpu_layer(self, l, x, T, p0=None, W=None):
        """engine.py:329-341: one token with the RMS prologues fused, else the batched layer."""
        W = self.W[l] if W is None else W
        if T > 1:
            return self._batch_layer(l, x, T, p0, W)
        s = self.small[l]
        wcomp.gemvc1(x, W["qkv"], self.qkvb[:1], 0, lnw=s["ln1"], eps=self.eps)
        self._rope_attn(l, 1)
        wcomp.gemvc1(self.attb[:1], W["o"], x, 1)
        wcomp.gemvc1(x, W["gu"], self.gub[:1], 0, lnw=s["ln2"], eps=self.eps)
        wcomp.gemvc1(self.gub[:1], W["down"], x, 2)

    def _batch_layer(self, l, x, T, p0=None, W=None):
        """engine.py:344-356: T <= 16 tokens of one sequence; the RMSNorms
        (rmsg_k in the reference) are fused into the qkv and gu linears."""
        W = self.W[l] if W is None else W
        s = self.small[l]
        wcomp.gemvc_tc(x, W["qkv"], self.qkvb[:T], 0, T, lnw=s["ln1"], eps=self.eps)
        self._rope_attn(l, T, p0)
        wcomp.gemvc_tc(self.attb[:T], W["o"], x, 1, T)
        wcomp.gemvc_tc(x, W["gu"], self.gub[:T], 0, T, lnw=s["ln2"], eps=self.eps)
        wcomp.gemvc_tc(self.gub[:T], W["down"], x, 2, T)

    def _layers(self, x, T, p0=None, fn=None):
        """Every layer in order (fn(l, W) in place of _gpu_layer); the streamed
        layers take their matrices from the streamer's slots."""
        fn = fn or (lambda l, W: self._gpu_layer(l, x, T, p0, W))
        st = self.streamer
        if st:
            st.begin()
        for l in range(self.L):
            if l < self.first_streamed:
                fn(l, self.W[l])
            else:
                i = l - self.first_streamed
                fn(l, st.acquire(i))
                st.release(i)
        if st:
            st.end()

    def _head_row(self, x1):
        """Greedy id of one row into self.nxt[0]: the final norm fused into the
        12-bit lm_head, the pick (smallest id on ties) fused into its epilogue
        (head.py:59-88)."""
        wcomp.greedy(x1, self.head, 1, self.nxt, lnw=self.norm, eps=self.eps)

    def _head_rows(self, x, T):
        """Greedy ids of T rows (T <= 16) into self.nxt[:T]."""
        wcomp.greedy(x, self.head, T, self.nxt, lnw=self.norm, eps=self.eps)

    # ---------------------------------------------------------------- passes
    def _embed(self, T):
        self.xb[:T].copy_(self.emb.index_select(0, self.tok[:T]).float())

    def _step(self):
        """One decode step, all on the device (graph body): the layers on the
        activations xb[0] (the embedding row of the current token), the greedy
        pick, then rv12_decode_advance records the id in out[steps], makes it
        the next token, writes its embedding row into xb[0] and advances pos
        and steps (one kernel in place of torch's lookup, conversion, index
        copy and counter additions)."""
        self._layers(self.xb[:1], 1)
        self._head_row(self.xb[:1])
        _lib.check(_lib.lib().rv12_decode_advance(
            wcomp._ptr(self.nxt), wcomp._ptr(self.emb), self.emb.shape[0], self.emb.shape[1], wcomp._ptr(self.xb),
            wcomp._ptr(self.out), self.out.numel(), wcomp._ptr(self.steps), wcomp._ptr(self.pos),
            wcomp._ptr(self.tok), wcomp._stream(self.xb.device)), "rv12_decode_advance")

    def reset(self):
        for c in self.Kc + self.Vc:
            c.zero_()
        self.pos.zero_()
        self.steps.zero_()
        self.out.zero_()

    def _chunk(self):
        """One full prefill chunk (BATCH tokens at positions pos.., tokens in
        self.tok) through all layers: the body of the prefill graph."""
        self._embed(BATCH)
        self._layers(self.xb[:BATCH], BATCH)

    def _record(self, fn):
        """fn as a HIP graph: two eager warm passes on a side stream
        (workspaces get allocated, engine.py:432-444), then the capture."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        torch.cuda.synchronize()
        return g

    def capture(self):
        """Record the decode step and a full prefill chunk as HIP graphs (the
        reference captures one graph per batch bucket, engine.py:31, 432-444);
        the state the warm passes touched is reset."""
        self.graph = self._record(self._step)
        if self.maxt > BATCH:
            self.pos.zero_()
            self.pgraph = self._record(self._chunk)
        self.reset()

    def prefill(self, tokens):
        """Prompt tokens at positions 0.. in passes of up to 16 (the reference's
        chunked prefill, engine.py:471-480); returns the greedy id after the
        last one (left in self.nxt[0])."""
        P = len(tokens)
        if not 1 <= P < self.maxt:
            raise ValueError("prompt must fit the context")
        t = torch.tensor(tokens, dtype=torch.long, device=self.dev)
        if self.prefill_mode == "blocked" and P >= self.prefill_min:
            return self._prefill_blocked(t)
        for c0 in range(0, P, BATCH):
            T = min(BATCH, P - c0)
            self.pos.fill_(c0)
            self.tok[:T].copy_(t[c0:c0 + T])
            if T == BATCH and self.pgraph is not None:
                self.pgraph.replay()
            else:
                self._embed(T)
                self._layers(self.xb[:T], T, c0)
        last = (P - 1) % BATCH
        self._head_row(self.xb[last:last + 1])
        self.pos.fill_(P)
        return self.nxt[:1]

    def _prefill_blocked(self, t):
        """All prompt tokens t at positions 0.. through every layer at once
        (ai_amd.prefill.layer), then the greedy id after the last one."""
        P = t.numel()
        x = self.emb.index_select(0, t).float()
        self._layers(x, P, fn=lambda l, W: blocked_prefill.layer(self, l, W, x, 0, self.Kc[l], self.Vc[l]))
        self._head_row(x[P - 1:P].contiguous())
        self.pos.fill_(P)
        return self.nxt[:1]

    def process(self, tokens, pos0):
        """The tokens at positions pos0.. (the cache before pos0 already
        filled); returns the greedy id after each of them, or after the last
        only for more than 16 tokens (engine.py:505-526).  Up to 16 tokens run
        as one batched pass (_batch_layer for 2..16), as the reference's
        speculative verification does."""
        T = len(tokens)
        if T < 1 or pos0 < 0 or pos0 + T > self.maxt:
            raise ValueError("the tokens must fit the context")
        t = torch.tensor(tokens, dtype=torch.long, device=self.dev)
        if T > BATCH:
            if pos0 == 0:
                self.prefill(tokens)
                return self.nxt[:1].tolist()
            for c0 in range(0, T, BATCH):
                n = min(BATCH, T - c0)
                self.pos.fill_(pos0 + c0)
                self.tok[:n].copy_(t[c0:c0 + n])
                self._embed(n)
                self._layers(self.xb[:n], n, pos0 + c0)
            last = (T - 1) % BATCH
            self._head_row(self.xb[last:last + 1])
            self.pos.fill_(pos0 + T)
            return self.nxt[:1].tolist()
        self.pos.fill_(pos0)
        self.tok[:T].copy_(t)
        self._pass_graph(T).replay()
        self.pos.fill_(pos0 + T)
        return self.nxt[:T].tolist()

    def _pass(self, T):
        """One pass of T <= 16 tokens (tokens in self.tok, first position in
        self.pos, both on the device): embedding rows, every layer, the greedy
        id after each token into self.nxt[:T]."""
        self._embed(T)
        self._layers(self.xb[:T], T)
        if T == 1:
            self._head_row(self.xb[:1])
        else:
            self._head_rows(self.xb[:T], T)

    def _pass_graph(self, T):
        """The HIP graph of a T-token pass, recorded on first use (the
        reference captures one graph per pass size on first use and replays
        it, engine.py:31, 393-444).  Recording runs the pass eagerly twice
        with the current tokens and position; a pass writes its own cache
        slots only, so those warm runs leave what the replay then writes."""
        g = self.tgraphs.get(T)
        if g is None:
            g = self.tgraphs[T] = self._record(lambda: self._pass(T))
        return g

    def batch_pass_ms(self, T, p0, tokens=None, reps=10):
        """ms per call of process() with T tokens of one sequence at positions
        p0..p0+T-1 (the reference's _batch_layer, engine.py:344-356, replayed
        from the pass's graph), the host's part of each call included (token
        upload, graph launch, reading the ids back); tokens default to the
        first T ids of the vocabulary."""
        if not 1 < T <= BATCH or p0 + T > self.maxt:
            raise ValueError("T must be in 2..16 and the pass must fit the context")
        toks = list(tokens) if tokens is not None else list(range(T))
        self.process(toks, p0)  # records the graph on first use
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            self.process(toks, p0)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def generate(self, prompt, max_new, timing=False):
        """Greedy ids of `max_new` tokens after `prompt`.  With timing=True also
        (prefill ms, decode ms for the max_new - 1 graph replays)."""
        if len(prompt) + max_new > self.maxt:
            raise ValueError("prompt + max_new exceed the context")
        if self.graph is None:
            self.capture()
        self.reset()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        first = self.prefill(prompt)
        self.out[:1].copy_(first)
        self.tok[:1].copy_(first)
        self._embed(1)  # the first step's activations; each step writes the next one's
        self.steps.fill_(1)
        e[1].record()
        for _ in range(max_new - 1):
            self.graph.replay()
        e[2].record()
        torch.cuda.synchronize()
        ids = self.out[:max_new].tolist()
        if timing:
            return ids, e[0].elapsed_time(e[1]), e[1].elapsed_time(e[2])
        return ids
