"""ecd_decode_attn_noalloc (split partials in the library's static device workspace) against
the allocating pair it replaces, ecd_decode_attn + ecd_attn_combine with caller buffers: the
outputs are bit-identical on two calls in a row, the second smaller than the first (the
workspace keeps the first call's contents), and under hipGraph capture after a first eager call
on the device."""
import math

import numpy as np
import pytest

from helpers import randn16, rng

pytestmark = pytest.mark.gpu


def _allocating(q, kc, vc, pos, S, Hq, Hk, L, HD, ns):
    import torch
    from estudiocanciones_amd.kernels import _attn, _attn_combine
    R = q.shape[0]
    o = torch.empty_like(q)
    pm = torch.empty(R * Hq * ns, device=q.device)
    pl = torch.empty_like(pm)
    pa = torch.empty(R * Hq * ns, HD, device=q.device)
    _attn[(R, Hk, ns)](q, kc, vc, pos, o, pm, pl, pa, S, Hq, Hk, L, 1 / math.sqrt(HD), HD=HD,
                       G=Hq // Hk, NSPLIT=ns)
    _attn_combine[(R * Hq,)](pm, pl, pa, o, HD=HD, NSPLIT=ns)
    return o


@pytest.mark.parametrize("order", ["large-then-small", "backbone-then-decoder"])
def test_noalloc_attention_matches_allocating_pair(dev, order):
    import torch
    from estudiocanciones_amd.kernels import decode_attn_noalloc
    if order == "large-then-small":
        cases = [(16, 1, 24, 8, 128, 3000, 16), (3, 1, 24, 8, 128, 700, 7)]
    else:
        cases = [(8, 1, 24, 8, 128, 1200, 16), (16, 2, 8, 4, 384, 300, 4)]
    for k, (R, S, Hq, Hk, HD, L, ns) in enumerate(cases):
        print(f"[noalloc] call {k}: R={R} S={S} Hq={Hq} Hk={Hk} HD={HD} L={L} ns={ns}", flush=True)
        B = R // S
        T = lambda a: torch.from_numpy(a).to(dev)
        q = T(randn16(80 + k, R, Hq * HD))
        kc = T(randn16(81 + k, B, Hk, L, HD))
        vc = T(randn16(82 + k, B, Hk, L, HD))
        p = rng(83 + k).integers(0, L, R).astype(np.int64)
        p[0] = L - 1
        pos = T(p)
        want = _allocating(q, kc, vc, pos, S, Hq, Hk, L, HD, ns)
        out = torch.full_like(q, float("nan"))
        got = decode_attn_noalloc(q, kc, vc, pos, S, Hq, Hk, L, 1 / math.sqrt(HD), nsplit=ns,
                                  out=out)
        torch.cuda.synchronize()
        assert got is out
        assert torch.equal(got, want), f"call {k}"


def test_noalloc_attention_refuses_oversized(dev):
    import torch
    from estudiocanciones_amd.kernels import decode_attn_noalloc
    R, Hq, Hk, HD, L = 64, 32, 8, 512, 64
    q = torch.zeros(R, Hq * HD, dtype=torch.float16, device=dev)
    kc = torch.zeros(R, Hk, L, HD, dtype=torch.float16, device=dev)
    pos = torch.zeros(R, dtype=torch.int64, device=dev)
    with pytest.raises(MemoryError):
        decode_attn_noalloc(q, kc, kc, pos, 1, Hq, Hk, L, 0.1, nsplit=32)


def test_noalloc_attention_under_graph_capture(dev):
    """After one eager call on the device, the call is captured into a hipGraph (nothing
    allocated in the capture); every replay, with other eager work and syncs in between and new
    inputs copied into the captured buffers, equals the allocating pair bit for bit."""
    import torch
    from estudiocanciones_amd.kernels import decode_attn_noalloc
    R, S, Hq, Hk, HD, L, ns = 8, 1, 24, 8, 128, 1500, 16
    B = R // S
    T = lambda a: torch.from_numpy(a).to(dev)
    q = T(randn16(90, R, Hq * HD))
    kc = T(randn16(91, B, Hk, L, HD))
    vc = T(randn16(92, B, Hk, L, HD))
    pos = T(rng(93).integers(0, L, R).astype(np.int64))
    out = torch.empty_like(q)
    sc = 1 / math.sqrt(HD)
    decode_attn_noalloc(q, kc, vc, pos, S, Hq, Hk, L, sc, nsplit=ns, out=out)  # eager first call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        decode_attn_noalloc(q, kc, vc, pos, S, Hq, Hk, L, sc, nsplit=ns, out=out)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        decode_attn_noalloc(q, kc, vc, pos, S, Hq, Hk, L, sc, nsplit=ns, out=out)
    for k in range(4):
        print(f"[noalloc-graph] replay {k}", flush=True)
        q.copy_(T(randn16(100 + k, R, Hq * HD)))
        pos.copy_(T(rng(110 + k).integers(0, L, R).astype(np.int64)))
        # eager work on the same workspace between replays (a smaller call)
        decode_attn_noalloc(q[:3], kc[:3], vc[:3], pos[:3], S, Hq, Hk, L, sc, nsplit=7)
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        want = _allocating(q, kc, vc, pos, S, Hq, Hk, L, HD, ns)
        assert torch.equal(out, want), f"replay {k}"
