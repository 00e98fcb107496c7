"""rv12_gemm_static (split-K partials in the library's own device scratch)
against rv12_gemm with a caller-owned workspace: the same kernels and split
order, so the outputs must be equal bit for bit.  Two calls in a row, the
second with a smaller matrix and fewer tokens, reuse the scratch the first
left behind."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _matrix(N, K, seed):
    from ai_amd import wcomp
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(N, K, device="cuda", generator=g) * 0.02
    w[torch.randperm(N, device="cuda", generator=g)[: max(1, N // 100)]] *= 20
    return wcomp.compress(w.bfloat16())


def _both(c, T, mode, cfg, seed, rms):
    from ai_amd import _lib, wcomp
    L = _lib.lib()
    N, K = int(c["N"]), int(c["K"])
    g = torch.Generator(device="cuda").manual_seed(seed)
    xs = 2 * K if mode == 2 else K
    x = torch.randn(T, xs, device="cuda", generator=g)
    y0 = torch.randn(T, N, device="cuda", generator=g)
    lnw = (1 + 0.1 * torch.randn(K, device="cuda", generator=g)).bfloat16() if rms else None
    m = wcomp._matrix(c)
    shape = _lib.Launch()
    assert L.rv12_launch_shape(N, K, T, ctypes.byref(cfg), ctypes.byref(shape)) == 0
    assert shape.splits > 1, "the case must exercise the split-K workspace"
    need = L.rv12_workspace_bytes(N, K, T, shape.splits)
    assert 0 < need <= _lib.STATIC_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    ya, yb = y0.clone(), y0.clone()
    rc = L.rv12_gemm(ctypes.byref(m), p(x), p(ya), T, p(lnw), 1e-6, mode, ctypes.byref(cfg), p(ws), need, st)
    assert rc == 0, _lib.strerror(rc)
    rc = L.rv12_gemm_static(ctypes.byref(m), p(x), p(yb), T, p(lnw), 1e-6, mode, ctypes.byref(cfg), st)
    assert rc == 0, _lib.strerror(rc)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb), float((ya - yb).abs().max())
    assert not torch.equal(ya, y0)


def test_static_scratch_matches_caller_workspace():
    from ai_amd import _lib
    print("case 1: 1000 x 2048, 2 tokens (built-in split), modes 0/1/2, RMS", flush=True)
    c1 = _matrix(1000, 2048, 1)
    for mode in (0, 1, 2):
        _both(c1, 2, mode, _lib.Launch(), 10 + mode, rms=mode == 0)
    print("case 2: 300 x 1024, 1 token, 7 forced splits (smaller, after case 1)", flush=True)
    c2 = _matrix(300, 1024, 2)
    for mode in (0, 2):
        _both(c2, 1, mode, _lib.Launch(1, 1, 4, 7), 20 + mode, rms=mode == 0)
