"""Write golden input/output vectors of the reference 12-bit codec.

Runs the reference's own `compress` and `decompress`
(ramvi/engine/ramvi_engine/kernels/wcomp.py:13-45) on small bf16 matrices that
exercise the cases the format has to get right: the `base` window tie-break,
nibble order inside a 256-chunk, row-major exception order, the fp32 exception
values, +-0, subnormals, +-inf, NaN, values far outside the exponent window,
outlier rows and outlier columns, and an all-zero matrix.

The two functions are taken out of the reference file by AST extraction, in
the same way the reference's own tests load them
(ramvi/engine/tests/legacy/audit_support.py:16-23), so Triton is never
imported.  This script only runs in a checkout next to /root/reference; the
fixtures it writes (codec_golden.npz) are what the tests read.

    python tests/golden/gen_codec_golden.py
"""
import ast
import os
import sys

import numpy as np
import torch

REF = "/root/reference/ramvi/engine/ramvi_engine/kernels/wcomp.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "codec_golden.npz")


def _load(names):
    tree = ast.parse(open(REF, encoding="utf-8").read())
    ns = {"torch": torch}
    for node in tree.body:
        if getattr(node, "name", None) in names:
            exec(compile(ast.Module(body=[node], type_ignores=[]), REF, "exec"), ns)
    return [ns[n] for n in names]


def _bits(w):
    return w.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def cases():
    out = []
    # 1. the reference's own forced-exception matrices (tests/legacy/test_prefill.py:25-30)
    for seed in (7, 43, 109):
        torch.manual_seed(seed)
        w = torch.randn(9, 512).bfloat16()
        w[3, 11] = 1e-30
        w[4, 92] = 1e20
        out.append((f"prefill_seed{seed}", w, 256))
    # 2. special values scattered over a N(0, 0.02) matrix
    g = torch.Generator().manual_seed(1)
    w = (torch.randn(12, 768, generator=g) * 0.02).bfloat16()
    sp = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1e-30, -1e-30, 1e20, -1e20,
                       1e-39, -1e-39, 9.2e-41, 3.0e38, -3.0e38, 1.0, -1.0]).bfloat16()
    for i in range(sp.numel()):
        w[i % 12, (i * 37) % 768] = sp[i]
    w[5, :] = 0.0  # a whole zero row
    out.append(("special_values", w, 256))
    # 3. tie-break: two disjoint exponent windows with equal counts -> first window wins
    a = torch.full((4, 256), 2.0 ** -20).bfloat16()
    a[:, 128:] = 2.0 ** 10
    out.append(("tie_two_windows", a, 256))
    # tie with partial overlap: exponents spread so several windows share the max
    e = torch.arange(4 * 512) % 20
    t = (2.0 ** (e.float() - 10)).reshape(4, 512).bfloat16()
    out.append(("tie_spread", t, 256))
    # 4. all-zero matrix: base 0, every weight in window with exponent 0
    out.append(("all_zero", torch.zeros(3, 256).bfloat16(), 256))
    # subnormal-heavy matrix: most exponents are 0
    g = torch.Generator().manual_seed(2)
    s = (torch.randn(5, 256, generator=g) * 1e-39).bfloat16()
    s[0, :8] = 1.0
    out.append(("subnormal_heavy", s, 256))
    # 5. huge magnitudes: window reaches the inf/NaN exponent
    g = torch.Generator().manual_seed(3)
    h = (torch.randn(4, 256, generator=g) * 1e37).bfloat16()
    h[0, 0] = float("inf")
    h[1, 3] = float("-inf")
    h[2, 7] = float("nan")
    h[3, 9] = 1e-3
    out.append(("huge_with_inf", h, 256))
    # window that contains exponent 255: base 241, inf/NaN are in-window codes
    e = torch.arange(2 * 256) % 15 + 241
    v = (torch.arange(2 * 256) % 128).int()
    bits = ((e.int() << 7) | v).to(torch.int16).reshape(2, 256)
    wh = bits.view(torch.bfloat16).clone()
    wh[0, 5] = float("inf")
    wh[1, 6] = float("nan")
    wh[1, 7] = -float("inf")
    out.append(("window_hits_inf", wh, 256))
    # 6. outlier rows and outlier columns (x20) on N(0, sigma)
    g = torch.Generator().manual_seed(4)
    o = torch.randn(64, 1024, generator=g) * 0.03
    o[[5, 40], :] *= 20
    o[:, [17, 600]] *= 20
    out.append(("outliers_rows_cols", o.bfloat16(), 256))
    # 7. a non-default chunk length
    g = torch.Generator().manual_seed(5)
    out.append(("chunk128", (torch.randn(6, 384, generator=g) * 0.05).bfloat16(), 128))
    # 8. every bf16 bit pattern once (256 rows x 256 columns)
    allp = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(256, 256)
    out.append(("all_patterns", allp, 256))
    return out


def main():
    if not os.path.exists(REF):
        sys.exit(f"reference not found at {REF}")
    compress, decompress = _load(["compress", "decompress"])
    blob = {}
    names = []
    for name, w, ch in cases():
        c = compress(w, CH=ch)
        d = decompress(c)
        names.append(name)
        blob[f"{name}/w"] = _bits(w)
        blob[f"{name}/ch"] = np.int64(ch)
        blob[f"{name}/m8"] = c["m8"].numpy()
        blob[f"{name}/e4"] = c["e4"].numpy()
        blob[f"{name}/base"] = np.int64(c["base"])
        blob[f"{name}/rp"] = c["rp"].numpy()
        blob[f"{name}/er"] = c["er"].numpy()
        blob[f"{name}/ec"] = c["ec"].numpy()
        blob[f"{name}/ev"] = c["ev"].numpy()
        blob[f"{name}/dec"] = _bits(d)
        print(f"{name:22s} N={c['N']:4d} K={c['K']:4d} base={c['base']:3d} E={c['er'].numel()}")
    blob["names"] = np.array(names)
    np.savez_compressed(OUT, **blob)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
