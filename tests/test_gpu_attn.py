"""The decode-step attention kernel (rv12_rope_attn) against the same math in
float32 torch: head RMSNorm, rotate-half RoPE, the cache write rounded to the
cache dtype, grouped-query softmax attention over 0..pos."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _torch_ref(qkv, qn, kn, inv, pos, kc, vc, H, KV, HD, eps, k_at_pos=None):
    """k_at_pos: the step's key as the kernel stored it (one bf16 rounding of
    the same fp32 value can land one ulp away; the test checks that apart)."""
    G = H // KV
    q = qkv[:H * HD].view(H, HD)
    k = qkv[H * HD:(H + KV) * HD].view(KV, HD)
    v = qkv[(H + KV) * HD:].view(KV, HD)
    rms = lambda x, w: w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))
    q, k = rms(q, qn), rms(k, kn)
    ang = (torch.tensor(float(pos), device=inv.device) * inv).double()  # the angle in float32, as the kernel forms it
    cos = torch.cat([ang, ang]).cos().float()
    sin = torch.cat([ang, ang]).sin().float()
    rot = lambda t: torch.cat([-t[..., HD // 2:], t[..., :HD // 2]], -1)
    q, k = q * cos + rot(q) * sin, k * cos + rot(k) * sin
    kr, vr = k.to(kc.dtype), v.to(vc.dtype)
    K = kc[:, :pos + 1].float().clone()
    V = vc[:, :pos + 1].float().clone()
    K[:, pos], V[:, pos] = (kr if k_at_pos is None else k_at_pos).float(), vr.float()
    s = torch.matmul(q.view(KV, G, HD).double(), K.double().transpose(1, 2).contiguous()) * HD ** -0.5
    a = torch.softmax(s, -1)
    out = torch.matmul(a, V.double().contiguous()).reshape(H * HD).float()
    return out, kr, vr


@pytest.mark.parametrize("H,KV,HD", [(32, 8, 128), (16, 8, 128), (8, 4, 64), (64, 8, 128), (8, 8, 64)])
@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
def test_rope_attn_matches_torch(H, KV, HD, kv_dtype):
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    maxt = 300
    g = torch.Generator(device=dev).manual_seed(H * 100 + HD)
    eps = 1e-6
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    qn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    kn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    for splits in (5, 8, 19, 53):
        # one object per split count: its workspace serves every call, as in
        # a decode loop; 53 splits take the combine's one-batch path for 33-64
        # splits (the Qwen3-32B decode at a 4224-position cache)
        att = RopeAttn(H, KV, HD, maxt, kv_dtype, eps, dev, splits=splits)
        for pos in (0, 1, 37, 130, maxt - 1):
            print("case", H, KV, HD, kv_dtype, splits, pos, flush=True)
            qkv = torch.randn((H + 2 * KV) * HD, device=dev, generator=g) * 3
            kc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
            vc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
            kc0, vc0 = kc.clone(), vc.clone()
            out = torch.zeros(H * HD, device=dev)
            att(qkv, qn, kn, inv, torch.tensor([pos], device=dev), kc, vc, out)
            torch.cuda.synchronize()
            ref, kr, vr = _torch_ref(qkv, qn, kn, inv, pos, kc0, vc0, H, KV, HD, eps, k_at_pos=kc[:, pos].clone())
            assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), float((out - ref).abs().max())
            # the cache: slot pos holds the rounded k (within one bf16 ulp) and v,
            # every other slot is untouched
            tol = 2.0 ** -7 if kv_dtype == torch.bfloat16 else 1e-5  # one bf16 ulp
            assert torch.allclose(kc[:, pos].float(), kr.float(), rtol=tol, atol=1e-6)
            assert torch.equal(vc[:, pos].float(), vr.float())
            keep = torch.ones(maxt, dtype=torch.bool)
            keep[pos] = False
            assert torch.equal(kc[:, keep], kc0[:, keep]) and torch.equal(vc[:, keep], vc0[:, keep])


@pytest.mark.parametrize("H,KV,HD", [(32, 8, 128), (16, 8, 128), (8, 4, 64), (64, 8, 128), (8, 8, 64)])
@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
def test_long_span_single_split_matches_torch(H, KV, HD, kv_dtype):
    """A cache of up to 256 positions takes one split (the 1024-thread
    workgroup over up to 256 positions, one per q head, no combine pass):
    against the float64 reference at positions inside and past the first 80,
    with the cache slot written once per kv head as in the split kernel, and
    equal within float32 rounding to the same step over 5 splits."""
    from ai_amd.attn import RopeAttn, default_splits
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(H * 10 + HD + 7)
    eps = 1e-6
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    qn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    kn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    for maxt in (81, 192, 256):
        assert default_splits(KV, maxt) == 1
        att = RopeAttn(H, KV, HD, maxt, kv_dtype, eps, dev, splits=1)
        split = RopeAttn(H, KV, HD, maxt, kv_dtype, eps, dev, splits=5)
        for pos in (0, 1, 63, 64, 79, 80, 130, maxt - 1):
            if pos >= maxt:
                continue
            print("case", H, KV, HD, kv_dtype, maxt, pos, flush=True)
            qkv = torch.randn((H + 2 * KV) * HD, device=dev, generator=g) * 3
            kc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
            vc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
            kc0, vc0 = kc.clone(), vc.clone()
            out = torch.zeros(H * HD, device=dev)
            att(qkv, qn, kn, inv, torch.tensor([pos], device=dev), kc, vc, out)
            k5, v5 = kc0.clone(), vc0.clone()
            o5 = torch.zeros(H * HD, device=dev)
            split(qkv, qn, kn, inv, torch.tensor([pos], device=dev), k5, v5, o5)
            torch.cuda.synchronize()
            ref, kr, vr = _torch_ref(qkv, qn, kn, inv, pos, kc0, vc0, H, KV, HD, eps, k_at_pos=kc[:, pos].clone())
            assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), float((out - ref).abs().max())
            assert torch.allclose(out, o5, rtol=1e-5, atol=1e-6), float((out - o5).abs().max())
            tol = 2.0 ** -7 if kv_dtype == torch.bfloat16 else 1e-5  # one bf16 ulp
            assert torch.allclose(kc[:, pos].float(), kr.float(), rtol=tol, atol=1e-6)
            assert torch.equal(vc[:, pos].float(), vr.float())
            keep = torch.ones(maxt, dtype=torch.bool)
            keep[pos] = False
            assert torch.equal(kc[:, keep], kc0[:, keep]) and torch.equal(vc[:, keep], vc0[:, keep])


@pytest.mark.parametrize("maxt,splits", [(32, 4), (100, 1)])
def test_position_outside_cache_gives_zeros(maxt, splits):
    """A position outside the cache writes no cache row and gives zeros; with
    the split kernel (4 splits) and with the short-cache workgroup per q head
    (one split over 100 positions); then a position inside the cache."""
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    H, KV, HD = 8, 4, 64
    att = RopeAttn(H, KV, HD, maxt, torch.float32, 1e-6, dev, splits=splits)
    kc = torch.randn(KV, maxt, HD, device=dev)
    vc = torch.randn(KV, maxt, HD, device=dev)
    kc0, vc0 = kc.clone(), vc.clone()
    out = torch.full((H * HD,), 7.0, device=dev)
    inv = torch.ones(HD // 2, device=dev)
    ones = torch.ones(HD, device=dev)
    qkv = torch.randn((H + 2 * KV) * HD, device=dev)
    att(qkv, ones, ones, inv, torch.tensor([maxt], device=dev), kc, vc, out)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(out))
    assert torch.equal(kc, kc0) and torch.equal(vc, vc0)
    # the same workspace then serves a position inside the cache
    att(qkv, ones, ones, inv, torch.tensor([maxt - 1], device=dev), kc, vc, out)
    torch.cuda.synchronize()
    ref, _, _ = _torch_ref(qkv, ones, ones, inv, maxt - 1, kc0, vc0, H, KV, HD, 1e-6, k_at_pos=kc[:, maxt - 1].clone())
    assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), float((out - ref).abs().max())
    keep = torch.ones(maxt, dtype=torch.bool)
    keep[maxt - 1] = False
    assert torch.equal(kc[:, keep], kc0[:, keep]) and torch.equal(vc[:, keep], vc0[:, keep])


def test_single_split_and_split_limits():
    """One split (a short cache) matches several; more than 64 positions per
    split, or more than 128 splits, is rejected before any launch."""
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    H, KV, HD, maxt = 16, 8, 128, 64
    g = torch.Generator(device=dev).manual_seed(5)
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    ones = torch.ones(HD, device=dev)
    qkv = torch.randn((H + 2 * KV) * HD, device=dev, generator=g)
    kc = torch.randn(KV, maxt, HD, device=dev, generator=g)
    vc = torch.randn(KV, maxt, HD, device=dev, generator=g)
    outs = []
    for splits in (1, 2, 5):
        k, v = kc.clone(), vc.clone()
        out = torch.zeros(H * HD, device=dev)
        RopeAttn(H, KV, HD, maxt, torch.float32, 1e-6, dev, splits=splits)(
            qkv, ones, ones, inv, torch.tensor([maxt - 1], device=dev), k, v, out)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.allclose(outs[0], outs[1], rtol=1e-5, atol=1e-6)
    assert torch.allclose(outs[0], outs[2], rtol=1e-5, atol=1e-6)
    for mt, splits in ((300, 2), (10241, 128), (300, 129), (257, 1)):  # one split: at most 256 positions
        with pytest.raises(ValueError):
            RopeAttn(H, KV, HD, mt, torch.float32, 1e-6, dev, splits=splits)(
                qkv, ones, ones, inv, torch.tensor([0], device=dev), kc, vc, torch.zeros(H * HD, device=dev))


def test_random_draws_of_positions_and_splits():
    """48 seeded draws of head layout, head size, cache dtype, cache length
    (1-2048), position and split count over the range the library accepts
    (one split up to 256 positions, else at most 80 positions per split and
    at most 128 splits), each against the float64 reference; the step's
    value lands in its cache slot."""
    import numpy as np
    from ai_amd.attn import RopeAttn, default_splits
    dev = "cuda"
    eps = 1e-6
    rng = np.random.default_rng(77)
    layouts = [(32, 8, 128), (16, 8, 128), (8, 4, 64), (64, 8, 128), (8, 8, 64), (4, 1, 128), (16, 2, 64)]
    for d in range(48):
        H, KV, HD = layouts[int(rng.integers(len(layouts)))]
        kv_dtype = torch.bfloat16 if rng.integers(2) else torch.float32
        maxt = int(rng.integers(1, 2049))
        lo = -(-maxt // 80)
        choices = [default_splits(KV, maxt, kv_dtype == torch.bfloat16, HD), lo, min(128, lo + int(rng.integers(0, 40)))]
        if maxt <= 256:
            choices.append(1)
        splits = int(choices[int(rng.integers(len(choices)))])
        pos = int(rng.integers(0, maxt))
        print("draw", d, H, KV, HD, kv_dtype, maxt, splits, pos, flush=True)
        g = torch.Generator(device=dev).manual_seed(700 + d)
        inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
        qn = 1 + 0.1 * torch.randn(HD, device=dev, generator=g)
        kn = 1 + 0.1 * torch.randn(HD, device=dev, generator=g)
        qkv = torch.randn((H + 2 * KV) * HD, device=dev, generator=g) * 3
        kc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
        vc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
        kc0, vc0 = kc.clone(), vc.clone()
        out = torch.zeros(H * HD, device=dev)
        RopeAttn(H, KV, HD, maxt, kv_dtype, eps, dev, splits=splits)(
            qkv, qn, kn, inv, torch.tensor([pos], device=dev), kc, vc, out)
        torch.cuda.synchronize()
        ref, kr, vr = _torch_ref(qkv, qn, kn, inv, pos, kc0, vc0, H, KV, HD, eps, k_at_pos=kc[:, pos].clone())
        assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), (d, float((out - ref).abs().max()))
        assert torch.equal(vc[:, pos].float(), vr.float()), d


def test_long_cache_many_splits():
    """10240 positions over 128 splits, bf16 cache, against the float64
    reference at a few positions."""
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    H, KV, HD, maxt = 32, 8, 128, 10240
    g = torch.Generator(device=dev).manual_seed(11)
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    qn = 1 + 0.1 * torch.randn(HD, device=dev, generator=g)
    kn = 1 + 0.1 * torch.randn(HD, device=dev, generator=g)
    att = RopeAttn(H, KV, HD, maxt, torch.bfloat16, 1e-6, dev)
    assert att.a.splits == 128
    for pos in (5, 4100, maxt - 1):
        print("pos", pos, flush=True)
        qkv = torch.randn((H + 2 * KV) * HD, device=dev, generator=g) * 3
        kc = torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16()
        vc = torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16()
        kc0, vc0 = kc.clone(), vc.clone()
        out = torch.zeros(H * HD, device=dev)
        att(qkv, qn, kn, inv, torch.tensor([pos], device=dev), kc, vc, out)
        torch.cuda.synchronize()
        ref, _, _ = _torch_ref(qkv, qn, kn, inv, pos, kc0, vc0, H, KV, HD, 1e-6, k_at_pos=kc[:, pos].clone())
        assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), float((out - ref).abs().max())


def test_graph_replays_advance_the_position():
    """The call captured in a HIP graph with the position advanced on the
    device: every replay (eager work and a synchronisation between them)
    matches the reference at its own position."""
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    H, KV, HD, maxt = 32, 8, 128, 256
    g = torch.Generator(device=dev).manual_seed(12)
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    ones = torch.ones(HD, device=dev)
    att = RopeAttn(H, KV, HD, maxt, torch.bfloat16, 1e-6, dev)
    qkv = torch.randn((H + 2 * KV) * HD, device=dev, generator=g)
    kc = torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16()
    vc = torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16()
    pos = torch.tensor([100], device=dev)
    out = torch.zeros(H * HD, device=dev)

    def step():
        att(qkv, ones, ones, inv, pos, kc, vc, out)
        pos.add_(1)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # eager warm call at position 100
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    pos.fill_(120)
    for r in range(5):
        kc0, vc0 = kc.clone(), vc.clone()
        graph.replay()
        torch.cuda.synchronize()
        p = 120 + r
        assert int(pos) == p + 1
        ref, _, _ = _torch_ref(qkv, ones, ones, inv, p, kc0, vc0, H, KV, HD, 1e-6, k_at_pos=kc[:, p].clone())
        assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), (r, float((out - ref).abs().max()))
        qkv.mul_(0.9)  # eager work between the replays


def _torch_batch_ref(qkv, qn, kn, inv, p0, kc, vc, H, KV, HD, eps, k_new=None):
    """T rows of qkv at positions p0..p0+T-1: the rounded k/v of all T
    positions in the caches (k_new: the keys as the kernel stored them, one
    bf16 rounding apart at most), then token t attends over 0..p0+t."""
    T = qkv.shape[0]
    G = H // KV
    q = qkv[:, :H * HD].view(T, H, HD)
    k = qkv[:, H * HD:(H + KV) * HD].view(T, KV, HD)
    v = qkv[:, (H + KV) * HD:].view(T, KV, HD)
    rms = lambda x, w: w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))
    q, k = rms(q, qn), rms(k, kn)
    pos = torch.arange(p0, p0 + T, device=inv.device, dtype=torch.float32)
    ang = (pos[:, None] * inv[None]).double()
    cos = torch.cat([ang, ang], -1).cos().float()[:, None]
    sin = torch.cat([ang, ang], -1).sin().float()[:, None]
    rot = lambda t: torch.cat([-t[..., HD // 2:], t[..., :HD // 2]], -1)
    q, k = q * cos + rot(q) * sin, k * cos + rot(k) * sin
    kr, vr = k.to(kc.dtype), v.to(vc.dtype)
    K = kc.float().clone()
    V = vc.float().clone()
    K[:, p0:p0 + T] = (kr if k_new is None else k_new).float().transpose(0, 1)
    V[:, p0:p0 + T] = vr.float().transpose(0, 1)
    out = torch.empty(T, H * HD, device=qkv.device)
    for t in range(T):
        n = p0 + t + 1
        s = torch.matmul(q[t].view(KV, G, HD).double(), K[:, :n].double().transpose(1, 2).contiguous()) * HD ** -0.5
        a = torch.softmax(s, -1)
        out[t] = torch.matmul(a, V[:, :n].double().contiguous()).reshape(H * HD).float()
    return out, kr, vr


@pytest.mark.parametrize("H,KV,HD", [(32, 8, 128), (16, 8, 128), (8, 4, 64), (64, 8, 128), (8, 8, 64)])
@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
def test_batch_attention_matches_torch(H, KV, HD, kv_dtype):
    """rv12_rope_attn_batch (the batched companions qk_rope_cache_k + attn_k)
    for T = 2, 5, 16 tokens at the start, the middle and the end of the cache,
    one split and several: outputs within 1e-4 of the float64 restatement,
    the T cache slots written (k within one bf16 ulp, v exact), the others
    untouched."""
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    maxt = 300
    g = torch.Generator(device=dev).manual_seed(H * 10 + HD + 7)
    eps = 1e-6
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    qn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    kn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    for splits in (4, 19, 60):
        att = RopeAttn(H, KV, HD, maxt, kv_dtype, eps, dev, splits=splits)
        for T in (2, 5, 16):
            for p0 in (0, 37, maxt - T):
                print("case", H, KV, HD, kv_dtype, splits, T, p0, flush=True)
                qkv = torch.randn(T, (H + 2 * KV) * HD, device=dev, generator=g) * 3
                kc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
                vc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
                kc0, vc0 = kc.clone(), vc.clone()
                out = torch.zeros(T, H * HD, device=dev)
                att.batch(qkv, qn, kn, inv, torch.tensor([p0], device=dev), kc, vc, out, T)
                torch.cuda.synchronize()
                ref, kr, vr = _torch_batch_ref(qkv, qn, kn, inv, p0, kc0, vc0, H, KV, HD, eps,
                                               k_new=kc[:, p0:p0 + T].transpose(0, 1).clone())
                assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), float((out - ref).abs().max())
                tol = 2.0 ** -7 if kv_dtype == torch.bfloat16 else 1e-5
                assert torch.allclose(kc[:, p0:p0 + T].float(), kr.float().transpose(0, 1), rtol=tol, atol=1e-6)
                assert torch.equal(vc[:, p0:p0 + T].float(), vr.float().transpose(0, 1))
                keep = torch.ones(maxt, dtype=torch.bool)
                keep[p0:p0 + T] = False
                assert torch.equal(kc[:, keep], kc0[:, keep]) and torch.equal(vc[:, keep], vc0[:, keep])


def test_random_draws_of_batches():
    """32 seeded draws of the batched pass (rv12_rope_attn_batch): head
    layout, head size, cache dtype, cache length (16-2048), token count
    (1-16), first position and split count, each against the float64
    restatement; the T cache slots written, the others untouched."""
    import numpy as np
    from ai_amd.attn import RopeAttn, default_splits
    dev = "cuda"
    eps = 1e-6
    rng = np.random.default_rng(1616)
    layouts = [(32, 8, 128), (16, 8, 128), (8, 4, 64), (64, 8, 128), (8, 8, 64), (4, 1, 128), (16, 2, 64)]
    for d in range(32):
        H, KV, HD = layouts[int(rng.integers(len(layouts)))]
        kv_dtype = torch.bfloat16 if rng.integers(2) else torch.float32
        maxt = int(rng.integers(16, 2049))
        T = int(rng.integers(1, 17))
        p0 = int(rng.integers(0, maxt - T + 1))
        lo = -(-maxt // 80)
        choices = [default_splits(KV, maxt, kv_dtype == torch.bfloat16, HD), lo, min(128, lo + int(rng.integers(0, 40)))]
        if maxt <= 256:
            choices.append(1)
        splits = int(choices[int(rng.integers(len(choices)))])
        print("draw", d, H, KV, HD, kv_dtype, maxt, T, p0, splits, flush=True)
        g = torch.Generator(device=dev).manual_seed(1600 + d)
        inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
        qn = 1 + 0.1 * torch.randn(HD, device=dev, generator=g)
        kn = 1 + 0.1 * torch.randn(HD, device=dev, generator=g)
        qkv = torch.randn(T, (H + 2 * KV) * HD, device=dev, generator=g) * 3
        kc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
        vc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
        kc0, vc0 = kc.clone(), vc.clone()
        out = torch.zeros(T, H * HD, device=dev)
        RopeAttn(H, KV, HD, maxt, kv_dtype, eps, dev, splits=splits).batch(
            qkv, qn, kn, inv, torch.tensor([p0], device=dev), kc, vc, out, T)
        torch.cuda.synchronize()
        ref, kr, vr = _torch_batch_ref(qkv, qn, kn, inv, p0, kc0, vc0, H, KV, HD, eps,
                                       k_new=kc[:, p0:p0 + T].transpose(0, 1).clone())
        assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), (d, float((out - ref).abs().max()))
        assert torch.equal(vc[:, p0:p0 + T].float(), vr.float().transpose(0, 1)), d
        keep = torch.ones(maxt, dtype=torch.bool)
        keep[p0:p0 + T] = False
        assert torch.equal(kc[:, keep], kc0[:, keep]) and torch.equal(vc[:, keep], vc0[:, keep]), d


def test_batch_equals_single_steps_and_graph_replays():
    """A batch of 8 equals 8 single-token steps from the same cache (each step
    sees the keys the previous ones wrote), and a captured batch replayed with
    the position advanced on the device gives the eager results; a batch
    past the cache's end gives zeros and writes nothing."""
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    H, KV, HD, maxt, T = 32, 8, 128, 512, 8
    g = torch.Generator(device=dev).manual_seed(5)
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    qn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    kn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    att = RopeAttn(H, KV, HD, maxt, torch.bfloat16, 1e-6, dev)
    qkv = torch.randn(T, (H + 2 * KV) * HD, device=dev, generator=g)
    kc = torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16()
    vc = torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16()
    kc1, vc1 = kc.clone(), vc.clone()
    p0 = 200
    out = torch.zeros(T, H * HD, device=dev)
    att.batch(qkv, qn, kn, inv, torch.tensor([p0], device=dev), kc, vc, out, T)
    one = torch.zeros(T, H * HD, device=dev)
    for t in range(T):
        att(qkv[t].contiguous(), qn, kn, inv, torch.tensor([p0 + t], device=dev), kc1, vc1, one[t])
    torch.cuda.synchronize()
    # the same keys up to one bf16 rounding (the two kernels may contract the
    # RoPE products differently), the same values
    assert torch.allclose(kc.float(), kc1.float(), rtol=2.0 ** -7, atol=1e-6) and torch.equal(vc, vc1)
    assert torch.allclose(out, one, rtol=1e-4, atol=1e-5), float((out - one).abs().max())
    # graph: replays at positions p0, p0 + T, p0 + 2T against eager calls
    pos = torch.tensor([p0], device=dev)
    kg, vg = kc.clone(), vc.clone()
    og = torch.zeros(T, H * HD, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        att.batch(qkv, qn, kn, inv, pos, kg, vg, og, T)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        att.batch(qkv, qn, kn, inv, pos, kg, vg, og, T)
        pos.add_(T)
    ke, ve = kg.clone(), vg.clone()
    pe = p0
    for _ in range(3):
        graph.replay()
        oe = torch.zeros(T, H * HD, device=dev)
        att.batch(qkv, qn, kn, inv, torch.tensor([pe], device=dev), ke, ve, oe, T)
        pe += T
        torch.cuda.synchronize()
        assert torch.equal(og, oe) and torch.equal(kg, ke) and torch.equal(vg, ve)
    # past the end: zeros, caches untouched
    k0, v0 = kc.clone(), vc.clone()
    bad = torch.full((T, H * HD), 7.0, device=dev)
    att.batch(qkv, qn, kn, inv, torch.tensor([maxt - T + 1], device=dev), kc, vc, bad, T)
    torch.cuda.synchronize()
    assert torch.equal(bad, torch.zeros_like(bad)) and torch.equal(kc, k0) and torch.equal(vc, v0)


def _prefill_ref(q, kc, vc, p0, T, H, KV, HD):
    """Causal attention of T roped q rows [T, H, HD] at positions p0.. over
    the caches' positions 0..p0 + t, in float64 (the softmax of masked
    scores; prefill_kernels.py:29-51 in exact arithmetic)."""
    G = H // KV
    n = p0 + T
    K = kc[:, :n].double()
    V = vc[:, :n].double()
    qh = q.double().view(T, KV, G, HD).permute(1, 2, 0, 3).reshape(KV, G * T, HD)
    s = torch.matmul(qh, K.transpose(1, 2).contiguous()).view(KV, G, T, n) * HD ** -0.5
    cols = torch.arange(n, device=q.device)
    rows = p0 + torch.arange(T, device=q.device)
    s.masked_fill_(cols[None, None, None, :] > rows[None, None, :, None], float("-inf"))
    a = torch.softmax(s, -1).view(KV, G * T, n)
    o = torch.matmul(a, V.contiguous()).view(KV, G, T, HD).permute(2, 0, 1, 3).reshape(T, H * HD)
    return o.float()


@pytest.mark.parametrize("H,KV,HD", [(32, 8, 128), (16, 8, 128), (8, 4, 64), (64, 8, 128), (8, 8, 64)])
@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
def test_prefill_attention_matches_float64(H, KV, HD, kv_dtype):
    """rv12_prefill_rope_attn (the blocked prefill's qk_rope_cache_k + att_k)
    for T = 1, 17, 300 prompt tokens at positions 0.. and 45.. of the cache:
    the q/k/v prologue as in the batch kernel (k within one bf16 ulp, v
    exact, other slots untouched), outputs within 1e-4 of the float64 causal
    attention over the keys the kernel stored."""
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    maxt = 400
    g = torch.Generator(device=dev).manual_seed(H * 7 + HD + 3)
    eps = 1e-6
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    qn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    kn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    att = RopeAttn(H, KV, HD, maxt, kv_dtype, eps, dev)
    for T in (1, 17, 300):
        for p0 in (0, 45):
            print("case", H, KV, HD, kv_dtype, T, p0, flush=True)
            qkv = torch.randn(T, (H + 2 * KV) * HD, device=dev, generator=g) * 3
            kc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
            vc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
            kc0, vc0 = kc.clone(), vc.clone()
            out = torch.full((T, H * HD), 7.0, device=dev)
            att.prefill(qkv, qn, kn, inv, torch.tensor([p0], device=dev), kc, vc, out, T)
            torch.cuda.synchronize()
            # the prologue: the batch reference's q rows, k/v slots
            _, kr, vr = _torch_batch_ref(qkv[:1], qn, kn, inv, p0, kc0, vc0, H, KV, HD, eps)
            q = qkv[:, :H * HD].view(T, H, HD)
            k = qkv[:, H * HD:(H + KV) * HD].view(T, KV, HD)
            rms = lambda x, w: w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))
            q, k = rms(q, qn), rms(k, kn)
            pos = torch.arange(p0, p0 + T, device=dev, dtype=torch.float32)
            ang = (pos[:, None] * inv[None]).double()
            cos = torch.cat([ang, ang], -1).cos().float()[:, None]
            sin = torch.cat([ang, ang], -1).sin().float()[:, None]
            rot = lambda t: torch.cat([-t[..., HD // 2:], t[..., :HD // 2]], -1)
            q, k = q * cos + rot(q) * sin, k * cos + rot(k) * sin
            v = qkv[:, (H + KV) * HD:].view(T, KV, HD)
            tol = 2.0 ** -7 if kv_dtype == torch.bfloat16 else 1e-5
            assert torch.allclose(kc[:, p0:p0 + T].float(), k.to(kv_dtype).float().transpose(0, 1), rtol=tol, atol=1e-6)
            assert torch.equal(vc[:, p0:p0 + T].float(), v.to(kv_dtype).float().transpose(0, 1))
            keep = torch.ones(maxt, dtype=torch.bool)
            keep[p0:p0 + T] = False
            assert torch.equal(kc[:, keep], kc0[:, keep]) and torch.equal(vc[:, keep], vc0[:, keep])
            ref = _prefill_ref(q, kc, vc, p0, T, H, KV, HD)
            assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), float((out - ref).abs().max())


def test_random_draws_of_prompt_blocks():
    """24 seeded draws of the blocked prefill's attention
    (rv12_prefill_rope_attn): head layout, head size, cache dtype, block of
    1-600 tokens at a random first position of a cache of up to 2048, each
    against the float64 causal attention over the keys the kernel stored;
    the block's cache slots written, the others untouched."""
    import numpy as np
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    eps = 1e-6
    rng = np.random.default_rng(6006)
    layouts = [(32, 8, 128), (16, 8, 128), (8, 4, 64), (64, 8, 128), (8, 8, 64), (4, 1, 128), (16, 2, 64)]
    for d in range(24):
        H, KV, HD = layouts[int(rng.integers(len(layouts)))]
        kv_dtype = torch.bfloat16 if rng.integers(2) else torch.float32
        T = int(rng.integers(1, 601))
        maxt = int(rng.integers(T, 2049))
        p0 = int(rng.integers(0, maxt - T + 1))
        print("draw", d, H, KV, HD, kv_dtype, T, maxt, p0, flush=True)
        g = torch.Generator(device=dev).manual_seed(6000 + d)
        inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
        qn = 1 + 0.1 * torch.randn(HD, device=dev, generator=g)
        kn = 1 + 0.1 * torch.randn(HD, device=dev, generator=g)
        qkv = torch.randn(T, (H + 2 * KV) * HD, device=dev, generator=g) * 3
        kc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
        vc = torch.randn(KV, maxt, HD, device=dev, generator=g).to(kv_dtype)
        kc0, vc0 = kc.clone(), vc.clone()
        out = torch.full((T, H * HD), 7.0, device=dev)
        RopeAttn(H, KV, HD, maxt, kv_dtype, eps, dev).prefill(
            qkv, qn, kn, inv, torch.tensor([p0], device=dev), kc, vc, out, T)
        torch.cuda.synchronize()
        q = qkv[:, :H * HD].view(T, H, HD)
        rms = lambda x, w: w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))
        q = rms(q, qn)
        pos = torch.arange(p0, p0 + T, device=dev, dtype=torch.float32)
        ang = (pos[:, None] * inv[None]).double()
        cos = torch.cat([ang, ang], -1).cos().float()[:, None]
        sin = torch.cat([ang, ang], -1).sin().float()[:, None]
        q = q * cos + torch.cat([-q[..., HD // 2:], q[..., :HD // 2]], -1) * sin
        v = qkv[:, (H + KV) * HD:].view(T, KV, HD)
        assert torch.equal(vc[:, p0:p0 + T].float(), v.to(kv_dtype).float().transpose(0, 1)), d
        keep = torch.ones(maxt, dtype=torch.bool)
        keep[p0:p0 + T] = False
        assert torch.equal(kc[:, keep], kc0[:, keep]) and torch.equal(vc[:, keep], vc0[:, keep]), d
        ref = _prefill_ref(q, kc, vc, p0, T, H, KV, HD)
        assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5), (d, float((out - ref).abs().max()))


def test_prefill_attention_equals_batch_and_rejects_bad_blocks():
    """A prompt block of 16 equals the batch kernel's 16 tokens from the same
    cache (both within 1e-4 of each other); a block past the cache's end
    gives zeros and writes nothing; unsupported blocks are refused before
    any launch."""
    import ctypes
    from ai_amd import _lib
    from ai_amd.attn import RopeAttn
    dev = "cuda"
    H, KV, HD, maxt, T = 32, 8, 128, 512, 16
    g = torch.Generator(device=dev).manual_seed(9)
    inv = (1.0 / (1e6 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))).to(dev)
    qn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    kn = (1 + 0.1 * torch.randn(HD, device=dev, generator=g))
    att = RopeAttn(H, KV, HD, maxt, torch.bfloat16, 1e-6, dev)
    qkv = torch.randn(T, (H + 2 * KV) * HD, device=dev, generator=g)
    kc = torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16()
    vc = torch.randn(KV, maxt, HD, device=dev, generator=g).bfloat16()
    kb, vb = kc.clone(), vc.clone()
    p0 = 300
    out = torch.zeros(T, H * HD, device=dev)
    att.prefill(qkv, qn, kn, inv, torch.tensor([p0], device=dev), kc, vc, out, T)
    ob = torch.zeros(T, H * HD, device=dev)
    att.batch(qkv, qn, kn, inv, torch.tensor([p0], device=dev), kb, vb, ob, T)
    torch.cuda.synchronize()
    assert torch.equal(kc, kb) and torch.equal(vc, vb)
    assert torch.allclose(out, ob, rtol=1e-4, atol=1e-5), float((out - ob).abs().max())
    k0, v0 = kc.clone(), vc.clone()
    bad = torch.full((T, H * HD), 7.0, device=dev)
    att.prefill(qkv, qn, kn, inv, torch.tensor([maxt - T + 1], device=dev), kc, vc, bad, T)
    torch.cuda.synchronize()
    assert torch.equal(bad, torch.zeros_like(bad)) and torch.equal(kc, k0) and torch.equal(vc, v0)
    L = _lib.lib()
    a = att.a
    assert L.rv12_prefill_attn_workspace_bytes(ctypes.byref(a), 0) == 0
    assert L.rv12_prefill_attn_workspace_bytes(ctypes.byref(a), (1 << 15) + 1) == 0
    assert L.rv12_prefill_attn_workspace_bytes(ctypes.byref(a), T) == T * H * HD * 4
    rc = L.rv12_prefill_rope_attn(ctypes.byref(a), T, None, None, None, None, None, None, None, None, None, 0, None)
    assert rc == _lib.RV12_E_NULL
