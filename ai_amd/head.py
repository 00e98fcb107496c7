"""The next-token head on the 12-bit path, with the reference's Head interface
(ramvi/engine/ramvi_engine/generation/head.py:29-88).

    Head(Wu16, TM=16)                          head.py:29-47
    bounds(h, T)                               head.py:49-54 (no bounds are needed here)
    pick(h, T, temperature, top_p, rng, run_bounds)   head.py:56-88

The reference keeps an int8 copy of the vocabulary on the GPU for logit
bounds and computes the exact fp32 logits of the candidate rows on the CPU
from the bf16 rows.  Here the vocabulary is the 12-bit matrix itself (exact
bf16 weights, 1.5 bytes each, resident in HBM) and every logit is an fp32
dot product on the GPU: greedy picks (temperature 0) run the fused pick of
rv12_head_argmax, the largest logit with the smallest id on ties
(head.py:76-79); sampling takes all logits from the same launch and applies
the reference's temperature / top-p rule on the host (head.py:80-88).
"""
import numpy as np
import torch

from . import wcomp


class Head:
    def __init__(self, Wu16, TM=16, device="cuda"):
        """Wu16 [V, D]: bf16 bits (uint16 numpy array or memmap, or a bf16 /
        int16 tensor); compressed once to the 12-bit form on the GPU."""
        if isinstance(Wu16, np.ndarray):
            w = torch.from_numpy(np.ascontiguousarray(Wu16).view(np.int16)).view(torch.bfloat16)
        else:
            w = Wu16 if Wu16.dtype == torch.bfloat16 else Wu16.view(torch.bfloat16)
        self.V, self.D = int(w.shape[0]), int(w.shape[1])
        self.TM = int(TM)
        self.c = wcomp.compact(wcomp.compress(w.to(device)))
        self.ids = torch.zeros(max(self.TM, 16), dtype=torch.int64, device=device)
        self.logits = None

    def bounds(self, h, T):
        """The reference's int8 logit bounds (head.py:49-54): not needed, every
        logit is computed exactly; kept so that callers run unchanged."""
        return None

    def pick(self, h, T, temperature=0.0, top_p=1.0, rng=None, run_bounds=True):
        """Ids for the T rows of h ([T, D] fp32 on the GPU); temperature 0
        picks the most likely id, the smallest on ties."""
        T = int(T)
        x = h[:T].float().contiguous()
        if temperature <= 0:
            wcomp.greedy(x, self.c, T, self.ids)
            return self.ids[:T].tolist()
        if self.logits is None or self.logits.shape[0] < T:
            self.logits = torch.empty(max(T, 1), self.V, device=x.device)
        wcomp.greedy(x, self.c, T, self.ids, logits=self.logits)
        lg = self.logits[:T].cpu().numpy().astype(np.float64)
        out = []
        for t in range(T):
            z = (lg[t] - lg[t].max()) / temperature
            p = np.exp(z)
            p /= p.sum()
            o = np.argsort(-p, kind="stable")
            cs = np.cumsum(p[o])
            keep = o[:int(np.searchsorted(cs, top_p) + 1)]
            pk = p[keep] / p[keep].sum()
            out.append(int(keep[(rng or np.random.default_rng()).choice(len(keep), p=pk)]))
        return out
