"""12-bit lossless bf16 weights and the fused decode-linear, on MI355X.

Operator API of the reference module ramvi/engine/ramvi_engine/kernels/wcomp.py
with the same names, argument meaning and error behaviour:

    compress(W, CH=256) -> dict          wcomp.py:13-32  (same dict, bit for bit)
    decompress(c) -> bf16[N, K]          wcomp.py:35-45
    gemvc1(x, c, y, mode, BN, w, lnw, eps)    wcomp.py:118-126
    gemvc_tc(x, c, y, mode, T, BN, w, S)      wcomp.py:233-242
    greedy(x, c, T, out, lnw, eps, logits)    head.py:59-88 (the greedy pick, on the 12-bit head)
    CFG1, CFGT, _SK                      wcomp.py:115, 222-230

plus decode_rows(c, first, last) (prefill_kernels.py:100-110) and prepare(c),
which re-tiles a dict built elsewhere (the reference's own compress, a file)
for the kernels.  Every call goes through librv12.so; there is no other path.

The dict (Codec12) stores the reference keys base, rp, er, ec, ev, N, K, CH
(bit for bit what the reference's compress builds) and the packed form the
kernels read as top-level tensors q16_tiles (the weights in the Q16 layout,
1.5 bytes per weight), q16_rbase (one exponent window per row) and that
layout's own exception list q16_rp / q16_er / q16_ec / q16_ev; the
reference's m8 / e4 are derived on request (c["m8"]), so the device holds
about 1.5 bytes per weight and the reference's _pack / _unpack stream exactly
the kernels' bytes.
Launch parameters keep the reference meaning: BN = rows per workgroup
(rounded up to 16, 32 or 64), w = waves per workgroup, S = K splits.
"""
import ctypes

import torch

from . import _lib
from ._lib import KERNEL_MFMA, KERNEL_MFMA_KSPLIT, KERNEL_VECTOR, Codec, Launch, Matrix, check, lib

CFG1 = {}  # (N, K, MODE) -> (BN, waves) or (BN, waves, S); filled by ai_amd.tune
CFGT = {}  # (N, K, MODE) -> (BN, waves, S); filled by ai_amd.tune
VECTOR_TOKENS = 2  # a given BN names the vector kernel up to 2 tokens, the bf16 MFMA kernel above
_SK = {}   # (N, device) -> workspace tensor (split-K partial sums)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _need_cuda(t, what):
    if not (torch.is_tensor(t) and t.is_cuda):
        raise ValueError(f"{what} must be a tensor on the GPU")


def _window_base(hist):
    """First argmax of the 15-wide exponent window counts (wcomp.py:19-21)."""
    h = hist.to(torch.int64).cpu()
    cs = torch.cat([torch.zeros(1, dtype=torch.int64), h.cumsum(0)])
    return int((cs[15:] - cs[:-15]).argmax())


PACKED = ("q16_tiles", "q16_rbase", "q16_rp", "q16_er", "q16_ec", "q16_ev")


class Codec12(dict):
    """The dict compress() returns.  Stored: the reference keys base, rp, er,
    ec, ev, N, K, CH (bit for bit the reference's) and the kernels' packed
    form as top-level tensors q16_tiles, q16_rbase, q16_rp, q16_er, q16_ec,
    q16_ev, about 1.5 bytes per weight in all.  The reference's m8 and e4 (1.5
    bytes per weight more) are not kept: c["m8"] and c["e4"] re-derive them
    on the GPU from the packed form, bit for bit what the reference compress
    builds (keep_codec() stores them).  So the reference Engine's budget of
    about 1.5 bytes per weight holds (planning/plan.py:38), and its
    _pack / _unpack (core/engine.py:34-56), which carry the top-level tensors,
    carry exactly what the kernels read."""

    def __missing__(self, k):
        if k in ("m8", "e4") and "q16_tiles" in self:
            return _reference_arrays(self)[0 if k == "m8" else 1]
        raise KeyError(k)

    def keep_codec(self):
        """Store m8 / e4 in the dict (the reference's full codec)."""
        m8, e4 = _reference_arrays(self)
        self["m8"], self["e4"] = m8, e4
        return self


def _reference_arrays(c):
    """(m8, e4) of the reference codec from the packed form: the exact bf16
    weights, encoded again with the stored base (the same encoder compress
    runs), on the dict's device."""
    home = c["q16_tiles"].device
    dev = home if home.type == "cuda" else torch.device("cuda")
    g = c if home.type == "cuda" else {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in c.items()}
    W = decode_rows(g, 0, int(c["N"]), torch.bfloat16)
    N, K, CH = int(c["N"]), int(c["K"]), int(c["CH"])
    m8 = torch.empty(N, K, dtype=torch.uint8, device=dev)
    e4 = torch.empty(N, K // 2, dtype=torch.uint8, device=dev)
    row_exc = torch.empty(N, dtype=torch.int32, device=dev)
    check(lib().rv12_encode(_ptr(W), N, K, CH, int(c["base"]), _ptr(m8), _ptr(e4), _ptr(row_exc), _stream(dev)),
          "compress")
    return m8.to(home), e4.to(home)


def compress(W, CH=256):
    """W [N, K] bf16 -> codec dict (wcomp.py:13-32): the reference keys and the
    packed form (Codec12).  W on the GPU, or on the CPU as the reference
    allows: the work then runs on the current GPU and the dict's tensors are
    returned on the CPU (a GPU is required either way)."""
    if not torch.is_tensor(W):
        raise ValueError("W must be a tensor")
    home = W.device
    if home.type != "cuda":
        if not torch.cuda.is_available():
            raise RuntimeError("compress: librv12 runs on the GPU and none is available")
        W = W.to("cuda")
    if W.dtype != torch.bfloat16 or W.dim() != 2:
        raise ValueError("W must be a 2-D bfloat16 tensor")
    N, K = W.shape
    assert K % CH == 0
    dev = W.device
    W = W.contiguous()
    if W.data_ptr() % 16:
        W = W.clone()
    st = _stream(dev)
    L = lib()
    hist = torch.empty(256, dtype=torch.int32, device=dev)
    check(L.rv12_encode_stats(_ptr(W), N, K, _ptr(hist), st), "compress")
    base = _window_base(hist)
    m8 = torch.empty(N, K, dtype=torch.uint8, device=dev)
    e4 = torch.empty(N, K // 2, dtype=torch.uint8, device=dev)
    row_exc = torch.empty(N, dtype=torch.int32, device=dev)
    check(L.rv12_encode(_ptr(W), N, K, CH, base, _ptr(m8), _ptr(e4), _ptr(row_exc), st), "compress")
    rp = torch.zeros(N + 1, dtype=torch.int32, device=dev)
    rp[1:] = row_exc.cumsum(0)
    E = int(rp[-1])
    er = torch.empty(E, dtype=torch.int32, device=dev)
    ec = torch.empty(E, dtype=torch.int32, device=dev)
    ev = torch.empty(E, dtype=torch.float32, device=dev)
    if E:
        check(L.rv12_encode_exc(_ptr(W), N, K, base, _ptr(rp), _ptr(er), _ptr(ec), _ptr(ev), st), "compress")
    c = Codec12(base=base, rp=rp, er=er, ec=ec, ev=ev, N=N, K=K, CH=CH)
    if K % 32 == 0 and CH % 16 == 0:
        c.update(pack(W))
        del m8, e4
    else:  # no packed form for this K: the dict keeps the reference arrays
        c["m8"], c["e4"] = m8, e4
    if home.type != "cuda":
        for k, v in list(c.items()):
            if torch.is_tensor(v):
                c[k] = v.to(home)
    return c


def pack(W):
    """bf16 W [N, K] on the GPU -> the kernels' packed form (keys q16_*): Q16
    tiles with one exponent window per row and that layout's own exception
    list."""
    N, K = W.shape
    dev = W.device
    L = lib()
    st = _stream(dev)
    rbase = torch.empty(N, dtype=torch.int32, device=dev)
    row_exc = torch.empty(N, dtype=torch.int32, device=dev)
    check(L.rv12_pack_plan(_ptr(W), N, K, _ptr(rbase), _ptr(row_exc), st), "pack")
    rp = torch.zeros(N + 1, dtype=torch.int32, device=dev)
    rp[1:] = row_exc.cumsum(0)
    E = int(rp[-1])
    nbytes = L.rv12_tiles_bytes(N, K)
    if nbytes == 0:
        raise ValueError("K must be a positive multiple of 32")
    tiles = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    er = torch.empty(E, dtype=torch.int32, device=dev)
    ec = torch.empty(E, dtype=torch.int32, device=dev)
    ev = torch.empty(E, dtype=torch.float32, device=dev)
    check(L.rv12_pack(_ptr(W), N, K, _ptr(rbase), _ptr(rp), E, _ptr(tiles), nbytes, _ptr(er), _ptr(ec), _ptr(ev),
                      st), "pack")
    return {"q16_tiles": tiles, "q16_rbase": rbase, "q16_rp": rp, "q16_er": er, "q16_ec": ec, "q16_ev": ev}


def to_bf16(c):
    """The bf16 matrix a reference codec dict (m8, e4, ...) encodes, bit for
    bit (NaN payloads kept)."""
    dev = c["m8"].device
    N, K = int(c["N"]), int(c["K"])
    W = torch.empty(N, K, dtype=torch.bfloat16, device=dev)
    cod = Codec(_ptr(c["m8"]), _ptr(c["e4"]), _ptr(c["rp"]), _ptr(c["er"]), _ptr(c["ec"]), _ptr(c["ev"]),
                N, K, int(c["CH"]), int(c["base"]), int(c["er"].numel()))
    check(lib().rv12_codec_to_bf16(ctypes.byref(cod), _ptr(W), _stream(dev)), "to_bf16")
    return W


def prepare(c, device=None):
    """Ready a dict for the kernels, in place: one built elsewhere (the
    reference's own compress, a file; numpy or CPU arrays) is moved to the GPU
    and packed; a packed one on the CPU (compress of a CPU tensor, the
    reference's _unpack of a host image) has its tensors moved to the GPU.
    Idempotent."""
    if "q16_tiles" in c:
        if not c["q16_tiles"].is_cuda:
            dev = torch.device(device) if device is not None else torch.device("cuda")
            for k, v in list(c.items()):
                if torch.is_tensor(v):
                    c[k] = v.to(dev)
        return c
    dev = torch.device(device) if device is not None else (
        c["m8"].device if torch.is_tensor(c["m8"]) and c["m8"].is_cuda else torch.device("cuda"))
    for k, dt in (("m8", torch.uint8), ("e4", torch.uint8), ("rp", torch.int32), ("er", torch.int32),
                  ("ec", torch.int32), ("ev", torch.float32)):
        v = c[k]
        if not torch.is_tensor(v):
            v = torch.as_tensor(v)
        c[k] = v.to(device=dev, dtype=dt).contiguous()
    c.update(pack(to_bf16(c)))
    return c


def compact(c):
    """Drop stored m8 / e4 (the kernels read only the packed form)."""
    prepare(c)
    dict.pop(c, "m8", None)
    dict.pop(c, "e4", None)
    return c


def _matrix(c):
    if "q16_tiles" not in c or not c["q16_tiles"].is_cuda:
        prepare(c)
    return Matrix(_ptr(c["q16_tiles"]), _ptr(c["q16_rbase"]), _ptr(c["q16_rp"]), _ptr(c["q16_er"]),
                  _ptr(c["q16_ec"]), _ptr(c["q16_ev"]), int(c["N"]), int(c["K"]), int(c["q16_er"].numel()))


def decode_rows(c, first, last, dtype=torch.float32):
    """Rows [first, last) decoded exactly: float32 (as prefill_kernels.decode_rows)
    or bfloat16 (the original bit patterns, NaN payloads included)."""
    m = _matrix(c)
    dev = c["q16_tiles"].device
    out = torch.empty((last - first, int(c["K"])), dtype=dtype, device=dev)
    f32 = 1 if dtype == torch.float32 else 0
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("dtype must be float32 or bfloat16")
    check(lib().rv12_decode_rows(ctypes.byref(m), int(first), int(last), _ptr(out), f32, _stream(dev)),
          "decode_rows")
    return out


def weight_rows(c, first, last):
    """Exact float32 rows (prefill.py:23-42, compressed branch)."""
    return decode_rows(c, first, last, torch.float32)


def decompress(c):
    """bf16[N, K] (wcomp.py:35-45).  Bit-identical to the weights compress()
    saw; the reference's final `.bfloat16()` would additionally map every NaN
    payload to one canonical NaN."""
    return decode_rows(c, 0, int(c["N"]), torch.bfloat16)


def _launch(BN, w, S, T):
    """Launch struct for the reference's tuning triple.  BN = rows per
    workgroup: row blocks of 16 per workgroup in the vector kernel (T <= 2);
    above 2 tokens the MFMA kernel, with row blocks per wave times waves when
    BN covers at least one row block per wave, else BN / 16 row blocks shared
    by the waves, which split K between them (kernel 3).  A given BN names its
    kernel; without one the library picks (rv12_launch_shape: the vector
    kernel at one token, and at 2 to 4 tokens where its activations fit the
    LDS unsplit and, at 3 and 4 tokens, on matrices small enough for its FMAs
    to hide behind the weight stream)."""
    rb = kernel = 0
    if BN:
        vec = T <= VECTOR_TOKENS
        waves = int(w or 8)
        ks = not vec and BN // 16 < waves
        per = BN // 16 if vec or ks else BN // (16 * waves)
        rb = 1 if per <= 1 else (2 if per <= 2 else 4)
        kernel = KERNEL_VECTOR if vec else (KERNEL_MFMA_KSPLIT if ks else KERNEL_MFMA)
    return Launch(kernel, rb, int(w or 0), int(S or 0))


_BUILTIN_KERNEL = {}  # (N, K, T) -> the kernel of the built-in launch shape


def _builtin_kernel(N, K, T):
    k = _BUILTIN_KERNEL.get((N, K, T))
    if k is None:
        k = _BUILTIN_KERNEL[(N, K, T)] = launch_shape(N, K, T)[0]
    return k


def launch_shape(N, K, T, cfg=None):
    """(kernel, rb, waves, splits) a linear of N x K at T tokens runs with for
    the Launch cfg (None: the built-in choice); kernel 1 = vector FMA, 2 =
    bf16 MFMA with rows per wave, 3 = bf16 MFMA with K split over the waves
    (rv12_launch_shape)."""
    c = Launch()
    check(lib().rv12_launch_shape(int(N), int(K), int(T), None if cfg is None else ctypes.byref(cfg),
                                  ctypes.byref(c)), "launch_shape")
    return c.kernel, c.rb, c.waves, c.splits


_SK_RETIRED = []  # workspaces replaced by larger ones: kept alive for graphs that captured them


def _sk_buf(N, S, dev, K=None, T=16, cfg=None):
    """Workspace for split partial sums, cached per (N, device)
    (wcomp.py:226-230): at least what the launch (N, K, T, cfg) resolves to
    needs, and what the built-in 16-token launch needs, so one buffer serves
    every batch size; a buffer that must grow is retired, not freed, because a
    captured HIP graph may still hold its address (the retired ones go with
    _SK when the caches are cleared)."""
    L = lib()
    K = int(K or 32 * max(S, 1))
    need = max(L.rv12_launch_workspace_bytes(int(N), K, int(T), None if cfg is None else ctypes.byref(cfg)),
               L.rv12_workspace_bytes(int(N), K, 16, 0))
    k = (N, str(dev))
    if k not in _SK or _SK[k].numel() < need:
        if k in _SK:
            _SK_RETIRED.append(_SK[k])
        _SK[k] = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    return _SK[k]


def clear_caches():
    """Drop every cached workspace, the retired ones too (the engine's
    caches are cleared with the last session, model_loader.py:385-390)."""
    _SK.clear()
    _HEAD_WS.clear()
    _SK_RETIRED.clear()


def _linear(x, c, y, mode, T, BN, w, S, lnw, eps, where):
    _need_cuda(x, "x")
    _need_cuda(y, "y")
    if x.dtype != torch.float32 or y.dtype != torch.float32:
        raise ValueError(f"{where}: x and y must be float32")
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError(f"{where}: x and y must be contiguous")
    N, K = int(c["N"]), int(c["K"])
    if BN is not None and N % BN:
        raise ValueError("число строк не кратно BN (N is not a multiple of BN)")  # wcomp.py:123
    xs = 2 * K if mode == 2 else K
    if x.numel() < T * xs or y.numel() < T * N:
        raise ValueError(f"{where}: x needs {T}x{xs} and y {T}x{N} floats")
    if lnw is not None:
        _need_cuda(lnw, "lnw")
        if lnw.dtype != torch.bfloat16 or lnw.numel() < K or not lnw.is_contiguous():
            raise ValueError(f"{where}: lnw must be a contiguous bf16 vector of K entries")
    m = _matrix(c)
    cfg = _launch(BN, w, S, T)
    launch_shape(N, K, T, cfg)  # validates the configuration (ValueError)
    ws = _sk_buf(N, 0, x.device, K, T, cfg)
    rc = lib().rv12_gemm(ctypes.byref(m), _ptr(x), _ptr(y), int(T), _ptr(lnw), float(eps), int(mode),
                         ctypes.byref(cfg), _ptr(ws), ws.numel(), _stream(x.device))
    check(rc, where)


_HEAD_WS = {}  # (N, device) -> workspace tensor of the greedy pick


def greedy(x, c, T, out, lnw=None, eps=1e-6, logits=None):
    """Greedy ids of T rows (1 <= T <= 16) over the 12-bit head c into the
    int64 device tensor out[:T]: the row of the largest logit, the smallest id
    on ties (head.py:59-88, tie rule :76-79), NaN counting as the largest
    value.  x' as gemvc1 mode 0 (lnw: the final RMSNorm fused).  logits (fp32
    [T, N]) also receives the logits when given.  Device-side only: no host
    synchronisation, so it can be captured in a HIP graph once its workspace
    exists (the first call allocates it)."""
    _need_cuda(x, "x")
    _need_cuda(out, "out")
    T = int(T)
    if not 1 <= T <= 16:
        raise ValueError("T must be in [1, 16]")
    N, K = int(c["N"]), int(c["K"])
    if x.dtype != torch.float32 or not x.is_contiguous() or x.numel() < T * K:
        raise ValueError(f"greedy: x must be contiguous float32 with {T}x{K} entries")
    if out.dtype != torch.int64 or not out.is_contiguous() or out.numel() < T:
        raise ValueError("greedy: out must be a contiguous int64 tensor of at least T entries")
    if logits is not None:
        _need_cuda(logits, "logits")
        if logits.dtype != torch.float32 or not logits.is_contiguous() or logits.numel() < T * N:
            raise ValueError(f"greedy: logits must be contiguous float32 with {T}x{N} entries")
    if lnw is not None:
        _need_cuda(lnw, "lnw")
        if lnw.dtype != torch.bfloat16 or lnw.numel() < K or not lnw.is_contiguous():
            raise ValueError("greedy: lnw must be a contiguous bf16 vector of K entries")
    L = lib()
    need = max(L.rv12_head_workspace_bytes(N, K, T, None), L.rv12_head_workspace_bytes(N, K, 16, None))
    k = (N, K, str(x.device))
    if k not in _HEAD_WS or _HEAD_WS[k].numel() < need:
        if k in _HEAD_WS:
            _SK_RETIRED.append(_HEAD_WS[k])
        _HEAD_WS[k] = torch.empty(need, dtype=torch.uint8, device=x.device)
    ws = _HEAD_WS[k]
    rc = L.rv12_head_argmax(ctypes.byref(_matrix(c)), _ptr(x), T, _ptr(lnw), float(eps), _ptr(logits), _ptr(out),
                            None, _ptr(ws), ws.numel(), _stream(x.device))
    check(rc, "greedy")


def gemvc1(x, c, y, mode, BN=None, w=None, lnw=None, eps=1e-6):
    """T = 1: y (=|+=) W x' with the MODE / RMS prologue (wcomp.py:67-126)."""
    N, K = int(c["N"]), int(c["K"])
    S = None
    if BN is None:
        cfg = CFG1.get((N, K, mode))
        if cfg:
            BN, w = cfg[0], cfg[1]
            S = cfg[2] if len(cfg) > 2 else None
    _linear(x, c, y, mode, 1, BN, w, S, lnw, eps, "gemvc1")


def gemvc_tc(x, c, y, mode, T, BN=None, w=None, S=None, lnw=None, eps=1e-6):
    """1 <= T <= 16 token rows: y[t] (=|+=) W x'[t] (wcomp.py:155-242).  lnw
    (an addition: bf16 [K]) fuses each row's RMSNorm into the prologue, as
    gemvc1 does at one token, in place of a separate rmsg_k pass."""
    N, K = int(c["N"]), int(c["K"])
    if not 1 <= int(T) <= 16:
        raise ValueError("T must be in [1, 16]")
    # CFGT is tuned at 16 tokens, for the MFMA kernel: it applies from 3
    # tokens on where the built-in choice is that kernel too
    if BN is None and int(T) > VECTOR_TOKENS and _builtin_kernel(N, K, int(T)) != KERNEL_VECTOR:
        cfg = CFGT.get((N, K, mode))
        if cfg:
            BN, w, S = cfg
    _linear(x, c, y, mode, int(T), BN, w, S, lnw, eps, "gemvc_tc")
