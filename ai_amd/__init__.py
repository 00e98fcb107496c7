"""ai_amd — MI355X-native 12-bit lossless bf16 decode-linear (RAMVI Engine wcomp path).

    from ai_amd import wcomp
    c = wcomp.compress(W)                 # W: bf16 [N, K] on the GPU
    wcomp.gemvc1(x, c, y, 0, lnw=ln1)     # y = W . rmsnorm(x)

The kernels live in librv12.so (ai_amd/csrc, C ABI in include/rv12.h), built
with `python -m ai_amd.build`.
"""
__all__ = ["wcomp"]
