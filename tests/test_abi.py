"""C-ABI checks that need no GPU: librv12.so loads, exports every entry point
include/rv12.h declares, and rejects bad arguments with the documented status
before any device work (so none of these calls touches a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    src = open(os.path.join(ROOT, "include", "rv12.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(rv12_[a-z0-9_]+)\s*\(", src)))


def test_header_and_binding_agree():
    from ai_amd import _lib
    assert sorted(_lib.EXPORTS) == _header_functions()


def test_library_exports_every_symbol():
    from ai_amd import _lib
    L = _lib.lib()
    for name in _header_functions():
        assert hasattr(L, name), name


def test_abi_version_and_strerror():
    from ai_amd import _lib
    L = _lib.lib()
    assert L.rv12_abi_version() == 8
    for s in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -20):
        assert _lib.strerror(s) and _lib.strerror(s) != "unknown rv12 status"
    assert _lib.strerror(-99) == "unknown rv12 status"


def test_sizes():
    from ai_amd import _lib
    L = _lib.lib()
    assert L.rv12_tiles_bytes(4096, 4096) == 4096 * 4096 * 3 // 2
    assert L.rv12_tiles_bytes(17, 256) == 32 * 256 * 3 // 2
    assert L.rv12_tiles_bytes(16, 100) == 0
    assert L.rv12_workspace_bytes(4096, 4096, 1, 1) == 0
    assert L.rv12_workspace_bytes(4096, 4096, 2, 4) == 4 * (4 * 2 * 4096 + 4 * 2)
    assert L.rv12_workspace_bytes(4096, 4096, 17, 1) == 0
    # the exact launch: the split count rv12_gemm resolves (n, k, t, cfg) to
    lw = lambda n, k, t, cfg=None: L.rv12_launch_workspace_bytes(n, k, t, None if cfg is None else ctypes.byref(cfg))
    assert lw(4096, 4096, 1) == 0
    assert lw(1024, 4096, 2, _lib.Launch(1, 1, 4, 4)) == 4 * (4 * 2 * 1024 + 4 * 2)
    for n, k, t, cfg in ((5120, 5120, 8, None), (1024, 5120, 16, None), (5120, 17408, 16, None),
                         (2048, 5120, 16, _lib.Launch(2, 1, 2, 0))):    # the split count left to the library
        c = _lib.Launch()
        assert L.rv12_launch_shape(n, k, t, None if cfg is None else ctypes.byref(cfg), ctypes.byref(c)) == 0
        assert c.splits > 1 and lw(n, k, t, cfg) == L.rv12_workspace_bytes(n, k, t, c.splits)
    assert lw(4096, 4096, 1, _lib.Launch(4, 1, 4, 2)) == 0                 # rejected: 0
    assert lw(4096, 100, 1) == 0 and lw(4096, 4096, 17) == 0


def test_launch_shapes():
    """The built-in launch table (host code only): the vector kernel at one
    token, and from 2 to 4 tokens where its activations fit the LDS unsplit
    and (3 and 4 tokens) the matrix is small enough for its FMAs to hide
    behind the weight stream; the MFMA kernel beyond; a partial configuration
    is completed, with K split further where it needs it."""
    from ai_amd import _lib
    L = _lib.lib()

    def shape(n, k, t, cfg=None):
        c = _lib.Launch()
        assert L.rv12_launch_shape(n, k, t, None if cfg is None else ctypes.byref(cfg), ctypes.byref(c)) == _lib.RV12_OK
        return (c.kernel, c.rb, c.waves, c.splits)

    assert shape(6144, 4096, 1) == (1, 2, 8, 1)           # Qwen3-8B qkv, one token: 384 row blocks, two per workgroup
    assert shape(4096, 4096, 1) == (1, 1, 8, 1)           # o: 256 row blocks, one per workgroup
    assert shape(1024, 4096, 1) == (1, 1, 8, 1)           # k/v: 64 row blocks, K unsplit at one token
    assert shape(1024, 4096, 2) == (1, 1, 8, 4)           # ... split at two
    assert shape(4096, 1024, 1) == (1, 1, 8, 1)           # Qwen3-0.6B qkv: 32 K steps over 8 waves
    assert shape(6144, 1024, 1) == (1, 2, 8, 1)           # 0.6B gate/up: 384 row blocks, two per workgroup
    assert shape(5120, 8192, 1) == (1, 2, 8, 1)           # 32B o: 320 row blocks of K 8192, two per workgroup
    assert shape(5120, 17408, 1) == (1, 2, 8, 3)          # 14B down: 3 splits fill the last round (480 workgroups)
    assert shape(5120, 25600, 1) == (1, 2, 8, 3)          # 32B down
    assert shape(4096, 12288, 1) == (1, 1, 16, 1)         # down: 16 waves for K >= 8192
    assert shape(151936, 4096, 1) == (1, 2, 4, 1)         # lm_head: two row blocks per workgroup
    # 2 tokens: the vector kernel wherever its activations fit the LDS unsplit
    assert shape(5120, 17408, 2) == (1, 2, 8, 1)          # Qwen3-14B down: 17408 columns x 2 tokens staged
    assert shape(5120, 25600, 2)[0] == 2                  # 32B down: they need a split: MFMA
    assert shape(7168, 5120, 2) == (1, 2, 8, 1)           # 14B qkv: unsplit, 2 row blocks
    assert shape(5120, 8192, 2) == (1, 2, 8, 1)           # 32B o: 2 row blocks of 8 waves
    assert shape(151936, 4096, 2) == (1, 2, 4, 1)         # 8B lm_head
    # 3 tokens: up to 512 row blocks, or K <= 4096 below 4096 row blocks
    assert shape(6144, 4096, 3) == (1, 2, 8, 1)           # 8B qkv: two row blocks, unsplit
    assert shape(1024, 5120, 3) == (1, 1, 8, 4)           # 14B k/v: split below 128 row blocks
    assert shape(24576, 4096, 3) == (1, 2, 8, 1)          # 8B gate/up: two row blocks of 8 waves
    assert shape(5120, 17408, 3)[0] == 2                  # 14B down: its activations need a split: MFMA
    assert shape(17408, 5120, 3)[0] == 2                  # 14B gate/up: MFMA
    assert shape(151936, 4096, 3)[0] == 2                 # 8B lm_head: MFMA
    # 4 tokens: up to 512 row blocks where the grid keeps >= 192 workgroups
    assert shape(4096, 4096, 4) == (1, 1, 8, 1)           # 8B o: 256 workgroups
    assert shape(6144, 4096, 4) == (1, 2, 8, 1)           # 8B qkv: 192 workgroups of two row blocks
    assert shape(1024, 5120, 4) == (1, 1, 8, 4)           # 14B k/v: K split to fill the CUs
    assert shape(5120, 5120, 4)[0] == 2                   # 14B o: 160 workgroups of two row blocks: MFMA
    assert shape(4096, 12288, 4)[0] == 2                  # 8B down: its activations need a split: MFMA
    # the MFMA kernel's time model picks the shapes the MI355X sweeps found best
    assert shape(4096, 4096, 8) == (2, 1, 8, 8)           # 8B o: 256 workgroups of 16 K steps
    assert shape(10240, 5120, 4) == (2, 2, 8, 6)          # 32B qkv: 640 row blocks, two per wave
    assert shape(1024, 5120, 16) == (2, 1, 4, 14)         # 14B k/v: 64 row blocks, 14 splits of 12 steps
    assert shape(5120, 5120, 4) == (2, 1, 8, 6)           # 14B o: 240 workgroups of 27 K steps
    assert shape(5120, 17408, 16) == (2, 2, 8, 12)        # 14B down: two row blocks per wave
    assert shape(5120, 8192, 16) == (2, 2, 8, 11)         # 32B o
    assert shape(5120, 25600, 8) == (2, 2, 8, 12)         # 32B down
    # a partial configuration keeps the built-in split where its staging fits
    # the LDS (3 KB per K step at 16 tokens, 768 B at 4); an explicit split
    # whose staging does not fit is rejected
    assert shape(5120, 5120, 16, _lib.Launch(2, 2, 4, 0)) == (2, 2, 4, 6)
    # the waves splitting K (kernel 3): row blocks per workgroup at most the
    # waves; one workgroup stages all 5120 columns at 4 tokens (147 KB of LDS)
    assert shape(5120, 5120, 4, _lib.Launch(3, 2, 8, 1)) == (3, 2, 8, 1)
    c = _lib.Launch()
    assert L.rv12_launch_shape(5120, 5120, 4, ctypes.byref(_lib.Launch(3, 4, 2, 1)),
                               ctypes.byref(c)) == _lib.RV12_E_CONFIG     # 4 row blocks, 2 waves
    assert L.rv12_launch_shape(5120, 5120, 8, ctypes.byref(_lib.Launch(3, 2, 8, 1)),
                               ctypes.byref(c)) == _lib.RV12_E_CONFIG     # 8 columns: 246 KB
    assert shape(5120, 5120, 4, _lib.Launch(2, 1, 4, 1)) == (2, 1, 4, 1)    # 160 steps of 768 B
    c = _lib.Launch()
    assert L.rv12_launch_shape(5120, 5120, 16, ctypes.byref(_lib.Launch(2, 2, 4, 2)),
                               ctypes.byref(c)) == _lib.RV12_E_CONFIG     # 80 steps of 3 KB

    assert shape(5120, 5120, 1, _lib.Launch(1, 1, 4, 3)) == (1, 1, 4, 3)
    c = _lib.Launch()
    assert L.rv12_launch_shape(64, 100, 1, None, ctypes.byref(c)) == _lib.RV12_E_SHAPE
    assert L.rv12_launch_shape(64, 256, 17, None, ctypes.byref(c)) == _lib.RV12_E_TOKENS
    assert L.rv12_launch_shape(64, 256, 1, None, None) == _lib.RV12_E_NULL
    assert L.rv12_launch_shape(64, 256, 1, ctypes.byref(_lib.Launch(4, 1, 4, 1)), ctypes.byref(c)) == _lib.RV12_E_CONFIG


def _mat(n=64, k=256, tiles=0x1000, n_exc=0, rbase=0x1800):
    from ai_amd import _lib
    return _lib.Matrix(tiles, rbase, 0x2000, 0x3000 if n_exc else 0, 0x4000 if n_exc else 0,
                       0x5000 if n_exc else 0, n, k, n_exc)


def test_gemm_argument_errors():
    """Every case returns before any device work (the pointers are fake)."""
    from ai_amd import _lib
    L = _lib.lib()
    x, y, ws = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x20000), ctypes.c_void_p(0x30000)

    def call(m, t=1, mode=0, cfg=None, lnw=None, xx=x, yy=y, wsb=0):
        return L.rv12_gemm(ctypes.byref(m) if m is not None else None, xx, yy, t, lnw, 1e-6, mode,
                           ctypes.byref(cfg) if cfg else None, ws, wsb, None)

    assert call(None) == _lib.RV12_E_NULL
    assert call(_mat(tiles=0)) == _lib.RV12_E_NULL
    assert call(_mat(), xx=None) == _lib.RV12_E_NULL
    assert call(_mat(k=100)) == _lib.RV12_E_SHAPE
    assert call(_mat(n=0)) == _lib.RV12_E_SHAPE
    assert call(_mat(rbase=0)) == _lib.RV12_E_NULL
    assert call(_mat(k=1 << 21)) == _lib.RV12_E_SHAPE
    assert call(_mat(), mode=3) == _lib.RV12_E_MODE
    assert call(_mat(), t=0) == _lib.RV12_E_TOKENS
    assert call(_mat(), t=17) == _lib.RV12_E_TOKENS
    assert call(_mat(tiles=0x1004)) == _lib.RV12_E_ALIGN
    assert call(_mat(), xx=ctypes.c_void_p(0x10004)) == _lib.RV12_E_ALIGN
    assert call(_mat(), cfg=_lib.Launch(0, 3, 4, 1)) == _lib.RV12_E_CONFIG
    assert call(_mat(), cfg=_lib.Launch(0, 1, 17, 1)) == _lib.RV12_E_CONFIG
    assert call(_mat(), cfg=_lib.Launch(0, 1, 4, 65)) == _lib.RV12_E_CONFIG
    assert call(_mat(k=256), cfg=_lib.Launch(0, 1, 4, 9)) == _lib.RV12_E_CONFIG  # more splits than K steps
    assert call(_mat(), cfg=_lib.Launch(4, 1, 4, 1)) == _lib.RV12_E_CONFIG       # no kernel 4
    assert call(_mat(), t=5, cfg=_lib.Launch(1, 1, 4, 1)) == _lib.RV12_E_CONFIG  # vector kernel: T <= 4
    assert call(_mat(), t=2, cfg=_lib.Launch(2, 1, 16, 1)) == _lib.RV12_E_CONFIG  # MFMA kernel: <= 8 waves
    # a split launch needs a workspace of rv12_workspace_bytes()
    need = L.rv12_workspace_bytes(64, 256, 1, 2)
    assert call(_mat(), cfg=_lib.Launch(0, 1, 4, 2), wsb=need - 4) == _lib.RV12_E_WORKSPACE
    # exceptions declared without their arrays
    m = _mat(n_exc=5)
    m.er = 0
    assert call(m) == _lib.RV12_E_NULL


def test_head_argmax_argument_errors_and_workspace():
    """The greedy pick's checks (before any device work) and its workspace:
    split partials, the logits (the output of an unfused launch; what the
    fused one reads as y), the fused pick's per-workgroup pairs at 1-2 tokens,
    the chunk pairs of a two-pass pick (each part 256-byte aligned)."""
    from ai_amd import _lib
    L = _lib.lib()
    P = ctypes.c_void_p
    x, ids, ws, lg = P(0x10000), P(0x20000), P(0x30000), P(0x50000)

    def call(m, t=1, xx=x, ii=ids, logits=None, cfg=None, wsb=1 << 20):
        return L.rv12_head_argmax(ctypes.byref(m) if m is not None else None, xx, t, None, 1e-6, logits, ii,
                                  ctypes.byref(cfg) if cfg else None, ws, wsb, None)

    assert call(None) == _lib.RV12_E_NULL
    assert call(_mat(), ii=None) == _lib.RV12_E_NULL
    assert call(_mat(), xx=None) == _lib.RV12_E_NULL
    assert call(_mat(), t=0) == _lib.RV12_E_TOKENS
    assert call(_mat(), t=17) == _lib.RV12_E_TOKENS
    assert call(_mat(), ii=P(0x20004)) == _lib.RV12_E_ALIGN
    assert call(_mat(), logits=P(0x50004)) == _lib.RV12_E_ALIGN
    assert call(_mat(k=100)) == _lib.RV12_E_SHAPE
    assert call(_mat(), cfg=_lib.Launch(4, 1, 4, 1)) == _lib.RV12_E_CONFIG
    need = L.rv12_head_workspace_bytes(64, 256, 1, None)
    assert need > 0 and call(_mat(), wsb=need - 1) == _lib.RV12_E_WORKSPACE
    a = lambda b: (b + 255) // 256 * 256
    hw = lambda n, k, t, cfg=None: L.rv12_head_workspace_bytes(n, k, t, None if cfg is None else ctypes.byref(cfg))
    # Qwen3-8B head at one token: the vector kernel, 9496 workgroups (two row
    # blocks each), more pairs than one pick chunk (8192): two passes
    c = _lib.Launch()
    assert L.rv12_launch_shape(151936, 4096, 1, None, ctypes.byref(c)) == 0 and c.kernel == 1 and c.splits == 1
    m = (151936 // 16 + c.rb - 1) // c.rb
    nc = (m + 8191) // 8192 if m > 8192 else 0
    assert hw(151936, 4096, 1) == a(4 * 151936) + 2 * a(4 * m) + 2 * a(4 * nc)
    # 16 tokens (MFMA): split partials, logits, 19 chunk pairs per token
    assert L.rv12_launch_shape(151936, 4096, 16, None, ctypes.byref(c)) == 0 and c.kernel == 2
    split = L.rv12_workspace_bytes(151936, 4096, 16, c.splits)
    assert hw(151936, 4096, 16) == a(split) + a(16 * 151936 * 4) + 2 * a(16 * 19 * 4)
    # a split vector launch is not fused: logits, one chunk (no pair pass)
    assert hw(1000, 4096, 1, _lib.Launch(1, 1, 4, 4)) == a(L.rv12_workspace_bytes(1000, 4096, 1, 4)) + a(1000 * 4)
    assert hw(64, 100, 1) == 0 and hw(64, 256, 17) == 0


def test_pack_decode_encode_argument_errors():
    from ai_amd import _lib
    L = _lib.lib()
    P = ctypes.c_void_p
    w, rb, rx, rp, tl = P(0x1000), P(0x2000), P(0x3000), P(0x4000), P(0x9000)
    need = L.rv12_tiles_bytes(64, 256)
    assert L.rv12_pack_plan(None, 64, 256, rb, rx, None) == _lib.RV12_E_NULL
    assert L.rv12_pack_plan(w, 64, 100, rb, rx, None) == _lib.RV12_E_SHAPE
    assert L.rv12_pack_plan(P(0x1002), 64, 256, rb, rx, None) == _lib.RV12_E_ALIGN
    assert L.rv12_pack(w, 64, 256, rb, rp, 0, None, need, None, None, None, None) == _lib.RV12_E_NULL
    assert L.rv12_pack(w, 64, 256, rb, rp, 5, tl, need, None, None, None, None) == _lib.RV12_E_NULL
    assert L.rv12_pack(w, 64, 256, rb, rp, 0, tl, need - 1, None, None, None, None) == _lib.RV12_E_SIZE
    assert L.rv12_pack(w, 0, 256, rb, rp, 0, tl, need, None, None, None, None) == _lib.RV12_E_SHAPE
    cod = _lib.Codec(0x1000, 0x2000, 0x3000, 0, 0, 0, 64, 256, 256, 100, 0)
    assert L.rv12_codec_to_bf16(ctypes.byref(cod), None, None) == _lib.RV12_E_NULL
    bad = _lib.Codec(0x1000, 0x2000, 0x3000, 0, 0, 0, 64, 256, 24, 100, 0)
    assert L.rv12_codec_to_bf16(ctypes.byref(bad), tl, None) == _lib.RV12_E_SHAPE
    bad = _lib.Codec(0x1000, 0x2000, 0x3000, 0, 0, 0, 64, 256, 256, 300, 0)
    assert L.rv12_codec_to_bf16(ctypes.byref(bad), tl, None) == _lib.RV12_E_BASE
    bad = _lib.Codec(0x1000, 0x2000, 0x3000, 0, 0, 0, 64, 256, 256, 100, 3)
    assert L.rv12_codec_to_bf16(ctypes.byref(bad), tl, None) == _lib.RV12_E_NULL
    m = _mat()
    out = ctypes.c_void_p(0x40000)
    assert L.rv12_decode_rows(ctypes.byref(m), 5, 3, out, 0, None) == _lib.RV12_E_SHAPE
    assert L.rv12_decode_rows(ctypes.byref(m), 0, 65, out, 0, None) == _lib.RV12_E_SHAPE
    assert L.rv12_decode_rows(ctypes.byref(m), 0, 4, None, 0, None) == _lib.RV12_E_NULL
    assert L.rv12_decode_rows(ctypes.byref(m), 2, 2, None, 0, None) == _lib.RV12_OK
    assert L.rv12_decode_rows(ctypes.byref(m), 3, 3, out, 0, None) == _lib.RV12_OK  # empty range: no work
    assert L.rv12_encode_stats(None, 4, 4, ctypes.c_void_p(0x1000), None) == _lib.RV12_E_NULL
    assert L.rv12_encode(ctypes.c_void_p(0x1000), 4, 256, 256, 250, ctypes.c_void_p(0x2000),
                         ctypes.c_void_p(0x3000), ctypes.c_void_p(0x4000), None) == _lib.RV12_E_BASE
    assert L.rv12_encode(ctypes.c_void_p(0x1000), 4, 250, 256, 10, ctypes.c_void_p(0x2000),
                         ctypes.c_void_p(0x3000), ctypes.c_void_p(0x4000), None) == _lib.RV12_E_SHAPE


def test_static_scratch_entry_rejects_oversized_workspace():
    """rv12_gemm_static checks the launch's workspace against its static
    scratch (8 MiB) before any device call."""
    from ai_amd import _lib
    L = _lib.lib()
    assert L.rv12_gemm_static(None, None, None, 1, None, 1e-6, 0, None, None) == _lib.RV12_E_NULL
    m = _lib.Matrix(0x1000, 0x2000, 0x3000, 0, 0, 0, 8192, 2048, 0)
    cfg = _lib.Launch(1, 1, 4, 64)   # 64 splits x 4 tokens x 8192 rows of partials: 8 MiB + sums of squares
    assert L.rv12_workspace_bytes(8192, 2048, 4, 64) > _lib.STATIC_SCRATCH_BYTES
    p = ctypes.c_void_p(0x10000)
    assert L.rv12_gemm_static(ctypes.byref(m), p, p, 4, None, 1e-6, 0, ctypes.byref(cfg), None) == _lib.RV12_E_SCRATCH
    assert L.rv12_gemm_static(ctypes.byref(m), p, p, 17, None, 1e-6, 0, None, None) == _lib.RV12_E_TOKENS


def test_python_mirror_fails_loudly_without_a_gpu():
    """compress takes a CPU tensor as the reference's does, but runs on the
    GPU: with none it raises (there is no CPU path); the linears want device
    tensors."""
    import torch
    from ai_amd import wcomp
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError):
        wcomp.compress(torch.zeros(4, 256, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        wcomp.gemvc1(torch.zeros(256), {"N": 4, "K": 256}, torch.zeros(4), 0)


def test_attention_argument_errors():
    """Every attention argument fault is a status before any device work; the
    workspace size follows the partial layout [n_kv][splits][G][HD + 2]."""
    from ai_amd import _lib
    L = _lib.lib()
    A = lambda **kw: _lib.Attn(*[kw.get(k, d) for k, d in (("n_heads", 32), ("n_kv", 8), ("head_dim", 128),
                                                              ("maxt", 2304), ("kv_bf16", 1), ("splits", 36),
                                                              ("eps", 1e-6), ("scale", 128 ** -0.5))])
    assert L.rv12_attn_workspace_bytes(ctypes.byref(A())) == 4 * 8 * 36 * 4 * 130
    assert L.rv12_attn_workspace_bytes(ctypes.byref(A(maxt=64, splits=1))) == 0
    p = ctypes.c_void_p(0x1000)

    def call(a, ws=0x100000, ws_bytes=1 << 30, **null):
        args = {k: (None if k in null else p) for k in ("qkv", "qn", "kn", "inv", "pos", "kc", "vc", "out")}
        return L.rv12_rope_attn(ctypes.byref(a), *args.values(), ctypes.c_void_p(ws), ctypes.c_size_t(ws_bytes), None)

    assert call(A(head_dim=96)) == _lib.RV12_E_SHAPE
    assert call(A(n_heads=24)) == _lib.RV12_E_SHAPE          # 3 q heads per kv head
    assert call(A(n_heads=4)) == _lib.RV12_E_SHAPE           # fewer q heads than kv heads
    assert call(A(maxt=0)) == _lib.RV12_E_SHAPE
    assert call(A(splits=0)) == _lib.RV12_E_CONFIG
    assert call(A(splits=129, maxt=8192)) == _lib.RV12_E_CONFIG
    assert call(A(splits=28)) == _lib.RV12_E_CONFIG          # 83 positions per split
    assert call(A(maxt=10241, splits=128)) == _lib.RV12_E_CONFIG  # 81 positions per split
    assert call(A(maxt=257, splits=1)) == _lib.RV12_E_CONFIG    # one split covers at most 256 positions
    assert L.rv12_attn_workspace_bytes(ctypes.byref(A(maxt=256, splits=1))) == 0  # no partials, no combine
    assert call(A(), out=None) == _lib.RV12_E_NULL
    assert call(A(), pos=None) == _lib.RV12_E_NULL
    assert call(A(), ws=0) == _lib.RV12_E_WORKSPACE
    assert call(A(), ws_bytes=1000) == _lib.RV12_E_WORKSPACE


def test_prefill_attention_argument_errors():
    """The prompt attention's faults are statuses before any device work; its
    workspace holds the q rows (t * n_heads * head_dim floats); the splits
    of the decode attention do not apply, its 32-bit offset limits do."""
    from ai_amd import _lib
    L = _lib.lib()
    A = lambda **kw: _lib.Attn(*[kw.get(k, d) for k, d in (("n_heads", 32), ("n_kv", 8), ("head_dim", 128),
                                                              ("maxt", 2304), ("kv_bf16", 1), ("splits", 36),
                                                              ("eps", 1e-6), ("scale", 128 ** -0.5))])
    ws = lambda a, t: L.rv12_prefill_attn_workspace_bytes(ctypes.byref(a), t)
    assert ws(A(), 2048) == 2048 * 32 * 128 * 4
    assert ws(A(splits=0, maxt=20000), 2048) == 2048 * 32 * 128 * 4  # no split rule
    assert ws(A(), 0) == 0 and ws(A(), (1 << 15) + 1) == 0 and ws(A(n_heads=8), 1 << 15) > 0
    assert ws(A(n_heads=128, n_kv=16), 1 << 15) == 0                 # q rows past 2^31 bytes
    assert ws(A(maxt=1 << 22, kv_bf16=0), 16) == 0                   # cache offsets past 2^31
    assert ws(A(head_dim=96), 16) == 0 and ws(A(n_heads=24), 16) == 0
    p = ctypes.c_void_p(0x1000)

    def call(a, t=16, ws=0x100000, ws_bytes=1 << 30, **null):
        args = {k: (None if k in null else p) for k in ("qkv", "qn", "kn", "inv", "pos", "kc", "vc", "out")}
        return L.rv12_prefill_rope_attn(ctypes.byref(a), t, *args.values(), ctypes.c_void_p(ws),
                                        ctypes.c_size_t(ws_bytes), None)

    assert call(A(head_dim=96)) == _lib.RV12_E_SHAPE
    assert call(A(n_heads=24)) == _lib.RV12_E_SHAPE
    assert call(A(), t=0) == _lib.RV12_E_TOKENS
    assert call(A(), kc=None) == _lib.RV12_E_NULL
    assert call(A(), ws=0) == _lib.RV12_E_WORKSPACE
    assert call(A(), ws_bytes=1000) == _lib.RV12_E_WORKSPACE


def test_build_manifest_checked_at_load(monkeypatch):
    """librv12.so loads only while it matches its manifest: the binary's and
    every source's sha256, the code-generation flags and the ABI version (as
    the reference's native/write_manifest.py + cpu/gcpu.py:121-160)."""
    import json
    from ai_amd import build
    assert build.manifest_problem() is None
    m = json.load(open(build.MANIFEST))
    assert set(m["sources"]) == {f"ai_amd/csrc/{n}" for n in build.SOURCES + build.HEADERS} | {"include/rv12.h"}
    assert "-packed-fp32-ops" in m["flags"] and "--offload-arch=gfx950" in m["flags"]
    changed = dict(build.inputs(), **{"ai_amd/csrc/rv12_gemv.hip": "0" * 64})
    monkeypatch.setattr(build, "inputs", lambda: changed)
    assert "sources changed" in build.manifest_problem()
    monkeypatch.undo()
    monkeypatch.setattr(build, "CODEGEN", build.CODEGEN[:-4])
    assert "other flags" in build.manifest_problem()


def test_decode_advance_argument_errors():
    """The decode step's bookkeeping entry reports NULL pointers, empty shapes
    and misaligned pointers as statuses before any device work (tok alone
    may be NULL)."""
    from ai_amd import _lib
    L = _lib.lib()

    def call(vocab=151936, hidden=4096, out_len=64, odd=(), **null):
        names = ("ids", "emb", "x", "out", "steps", "pos", "tok")
        a = {k: (None if k in null else ctypes.c_void_p(0x1000 + (2 if k in odd else 0))) for k in names}
        return L.rv12_decode_advance(a["ids"], a["emb"], vocab, hidden, a["x"], a["out"], out_len, a["steps"],
                                     a["pos"], a["tok"], None)

    for k in ("ids", "emb", "x", "out", "steps", "pos"):
        assert call(**{k: None}) == _lib.RV12_E_NULL, k
    assert call(vocab=0) == _lib.RV12_E_SHAPE
    assert call(hidden=0) == _lib.RV12_E_SHAPE
    assert call(out_len=-1) == _lib.RV12_E_SHAPE
    for k in ("ids", "out", "steps", "pos", "tok", "x"):
        assert call(odd=(k,)) == _lib.RV12_E_ALIGN, k


def test_attention_wrapper_checks_the_caches():
    """RopeAttn rejects caches of another dtype, shape or layout than the one
    it was built for, and rows too few for T, before any library call (the
    C ABI sees only pointers, so such a cache would be written out of
    bounds).  CPU tensors: every case raises before a launch."""
    import torch
    from ai_amd.attn import RopeAttn
    H, KV, HD, maxt = 4, 2, 64, 96
    f32 = lambda *s: torch.zeros(*s, dtype=torch.float32)
    qkv, qn, kn, inv, out = f32((H + 2 * KV) * HD), f32(HD), f32(HD), f32(HD // 2), f32(H * HD)
    pos = torch.zeros(1, dtype=torch.int64)
    for kv_dtype, other in ((torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16)):
        a = RopeAttn(H, KV, HD, maxt, kv_dtype, 1e-6, "cpu")
        good = torch.zeros(KV, maxt, HD, dtype=kv_dtype)
        cases = [torch.zeros(KV, maxt, HD, dtype=other), torch.zeros(KV, maxt - 1, HD, dtype=kv_dtype),
                 torch.zeros(KV + 1, maxt, HD, dtype=kv_dtype),
                 torch.zeros(KV, HD, maxt, dtype=kv_dtype).transpose(1, 2)]
        for bad in cases:
            with pytest.raises(ValueError, match="kc and vc"):
                a(qkv, qn, kn, inv, pos, bad, good, out)
            with pytest.raises(ValueError, match="kc and vc"):
                a.batch(qkv.repeat(2), qn, kn, inv, pos, good, bad, out.repeat(2), 2)
            with pytest.raises(ValueError, match="kc and vc"):
                a.prefill(qkv.repeat(2), qn, kn, inv, pos, bad, good, out.repeat(2), 2)
        with pytest.raises(ValueError, match="rows"):
            a.batch(qkv, qn, kn, inv, pos, good, good, out, 2)
        with pytest.raises(ValueError, match="int64"):
            a(qkv, qn, kn, inv, pos.int(), good, good, out)
