"""The one-launch layer tail (ecd_layer_tail): O projection + residual, rms -> w1|w3 -> SiLU*mul,
w2 + residual and the next layer's rms -> q|k|v -> RoPE -> cache write, per layer, checked
against the oracle's per-op composition (Stack.decode, app/engine.py:180-211) and against the
per-op kernels; repeated launches reuse the gate region; a captured graph replays bit-equal.

Weights are random, quantised per row on the GPU (bit-exact with the oracle's quantiser) and
handed to the oracle as codes and bf16 scales."""
import numpy as np
import pytest

from helpers import (ATOL, RTOL, assert_close16, assert_within_noise, clear_warmup_timeout,
                     randn16, rng)
from oracle import kernels as OK
from oracle.model import OLinear, OStack

pytestmark = pytest.mark.gpu


def N(t):
    return t.detach().cpu().numpy()


def _host(t):
    import torch
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def _stacks(dev, cfg, seed, B, L, stream):
    """(oracle stack, GPU stack) with the same quantised weights; GPU weights packed before
    alloc so the stack sets up its layer-tail buffers."""
    import torch
    from estudiocanciones_amd.engine import Linear, Stack
    from estudiocanciones_amd.quant import _stack_norms, _stack_shapes, q8_rows
    from oracle.numerics import bf16_to_f32, f16
    from oracle.quant import scale_f16
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = {}
    for name, (Nn, K) in _stack_shapes("backbone", cfg):
        w[name + ".q8"], w[name + ".s8"] = q8_rows(torch.randn(Nn, K, generator=g, device=dev) * 0.02)
    for name, d in _stack_norms("backbone", cfg):
        w[name] = (1.0 + 0.02 * torch.randn(d, generator=g, device=dev)).to(torch.bfloat16)
    wn = {k: _host(v) for k, v in w.items()}

    def op(name, norm=False):
        if norm:
            return f16(bf16_to_f32(wn[name]))
        return OLinear(wn[name + ".q8"], scale_f16(wn[name + ".s8"]))

    def gp(name, norm=False):
        if norm:
            return w[name].to(torch.float16)
        return Linear(q8=w[name + ".q8"], s8=w[name + ".s8"].to(torch.float16))

    ost = OStack(op, "backbone", cfg)
    ost.alloc(B, L)
    st = Stack(gp, "backbone", cfg)
    for b in st.blocks:
        b.qkv.pack(stream=stream)
        b.o.pack(stream=stream)
        b.w13.pack(interleave=True, stream=stream)
        b.w2.pack(stream=stream)
    st.alloc(B, L, dev, torch.float16)
    return ost, st


def _fill(ost, st, seed, upto):
    import torch
    g = torch.Generator(device=st.blocks[0].kc.device)
    g.manual_seed(seed)
    for ob, gb in zip(ost.blocks, st.blocks):
        for oc, gc in ((ob.kc, gb.kc), (ob.vc, gb.vc)):
            t = torch.randn(gc[:, :, :upto].shape, generator=g, device=gc.device).half()
            gc[:, :, :upto] = t
            oc[:, :, :upto] = N(t)


BB3 = dict(layers=3, heads=24, kv_heads=8, max_seq=8192, dim=3072, ffn=8192)
DEC3 = dict(layers=3, heads=8, kv_heads=2, max_seq=2048, dim=1024, ffn=8192)
DEC_REF2 = dict(layers=2, heads=8, kv_heads=4, max_seq=2048, dim=3072, ffn=8192)


@pytest.mark.parametrize("cfg,B,L,pos_kind,stream,kv_nt", [
    (BB3, 8, 1024, "spread", True, False),  # backbone shape, 8 rows, positions 0 .. L - 1
    (BB3, 8, 1024, "spread", True, True),   # the same, every cache slot read nontemporal
    (BB3, 2, 1024, "last", True, False),    # the C0 rows
    (BB3, 8, 4096, "last", True, False),    # long splits: the new slot in a split's ninth tile
    (DEC3, 8, 8, "spread", False, False),   # 1024-wide decoder, per-frame cache of 8 slots
    (DEC_REF2, 8, 8, "last", False, False),  # the reference's decoder: 3072 wide, head_dim 384
    (DEC_REF2, 8, 8, "spread", False, False),
    (BB3, 8, 8, "spread", False, False),    # backbone shape over an 8-slot cache (VALU attention)
])
def test_tail_stack_vs_oracle(dev, cfg, B, L, pos_kind, stream, kv_nt):
    import torch
    from estudiocanciones_amd.kernels import layer_tail_supported
    ost, st = _stacks(dev, cfg, seed=cfg["dim"] + B, B=B, L=L, stream=stream)
    st.tail_kv_nt = kv_nt
    hd = cfg["dim"] // cfg["heads"]
    assert layer_tail_supported(B, cfg["dim"], cfg["ffn"], cfg["heads"], cfg["kv_heads"], hd)
    assert st.tail is not None
    _fill(ost, st, seed=5, upto=L)
    if pos_kind == "last":
        pos = np.full(B, L - 1, np.int64)
    else:
        pos = rng(6).integers(0, L, B).astype(np.int64)
        pos[0], pos[-1] = 0, L - 1
    x = randn16(7, B, cfg["dim"])

    def run_oracle():
        out = ost.decode(x, pos, 1)
        return out, [(b.kc[np.arange(B), :, pos].copy(), b.vc[np.arange(B), :, pos].copy())
                     for b in ost.blocks]

    want, wslot = run_oracle()
    OK.GEMV_ACC[0] = np.float32
    try:
        alt, aslot = run_oracle()
    finally:
        OK.GEMV_ACC[0] = np.float64
    # the oracle wrote its own slots twice; the GPU stack starts from the same caches
    got = st.decode(torch.from_numpy(x).to(dev), torch.from_numpy(pos).to(dev), 1)
    torch.cuda.synchronize()
    assert not st.tail_error()
    assert_within_noise(N(got), want, alt, what=f"tail stack {cfg['dim']} B={B}")
    bi = torch.arange(B, device=dev)
    pt = torch.from_numpy(pos).to(dev)
    for i, b in enumerate(st.blocks):
        gk, gv = N(b.kc[bi, :, pt]), N(b.vc[bi, :, pt])
        if i == 0:  # one kernel deep: the kernel bar
            assert_close16(gk, wslot[0][0], what="layer 0 k slot")
            assert_close16(gv, wslot[0][1], what="layer 0 v slot")
        else:       # written by the previous layer's tail launch
            assert_within_noise(gk, wslot[i][0], aslot[i][0], what=f"layer {i} k slot")
            assert_within_noise(gv, wslot[i][1], aslot[i][1], what=f"layer {i} v slot")


@pytest.mark.parametrize("cfg,L,stream", [(dict(BB3, layers=2), 512, True),
                                          (dict(DEC3, layers=2), 8, False),
                                          (DEC_REF2, 8, False)])
def test_tail_matches_per_op_kernels_and_repeats(dev, cfg, L, stream):
    """The tail path (head launch + tails) against the per-op fused kernels on the same stack
    (same numerics up to the fp32 summation order), then five more launches from identical
    state give identical bits (the gate region and, for the 1024-wide shape, the split-w2
    counters are reused), and a captured graph of the decode replays bit-equal."""
    import torch
    B = 8
    ost, st = _stacks(dev, cfg, seed=11, B=B, L=L, stream=stream)
    _fill(ost, st, seed=12, upto=L)
    kv0 = [(b.kc.clone(), b.vc.clone()) for b in st.blocks]

    def reset():
        for b, (k, v) in zip(st.blocks, kv0):
            b.kc.copy_(k)
            b.vc.copy_(v)

    x = torch.from_numpy(randn16(13, B, cfg["dim"])).to(dev)
    pos = torch.from_numpy(rng(14).integers(0, L, B).astype(np.int64)).to(dev)
    st.use_tail = False
    ref = st.decode(x, pos, 1).clone()
    st.use_tail = True
    outs = []
    for _ in range(6):
        reset()
        outs.append(st.decode(x, pos, 1).clone())
    torch.cuda.synchronize()
    assert not st.tail_error()
    # the attention splits differ (the launches split a pair's cache over their own waves, the
    # decode kernel over its split count), layer 0 included: the same function up to the fp32
    # summation order, so the fp16 kernel bar holds for all but a few elements, and 3x it for all
    got, want = N(outs[0]).astype(np.float32), N(ref).astype(np.float32)
    err, bound = np.abs(got - want), ATOL + RTOL * np.abs(want)
    assert (err > bound).mean() <= 1e-3, f"tail vs per-op kernels: {(err > bound).sum()} past the bar"
    assert (err <= 3 * bound).all(), f"tail vs per-op kernels: max abs err {err.max():.3e}"
    for o in outs[1:]:
        assert torch.equal(o, outs[0]), "repeated tail launches differ"
    # graph capture and replay
    reset()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        st.decode(x, pos, 1)
    torch.cuda.current_stream(dev).wait_stream(s)
    clear_warmup_timeout(st, "tail path")
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        gout = st.decode(x, pos, 1)
    for _ in range(3):
        reset()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, outs[0]), "graph replay of the tail path differs from eager"
        assert not st.tail_error()


@pytest.mark.parametrize("cfg,L", [(dict(BB3, layers=2), 512), (dict(DEC3, layers=2), 8),
                                   (DEC_REF2, 8)])
def test_tail_timeout_sets_err_and_reset_recovers(dev, cfg, L):
    """The error path, forced from the host: with every wait of the launches giving up at its
    first look (gates, hand-off and merge polls), the launches still end and the error word
    reports it; after Stack.tail_reset the same decode matches the per-op path again."""
    import torch
    B = 8
    ost, st = _stacks(dev, cfg, seed=21, B=B, L=L, stream=False)
    _fill(ost, st, seed=22, upto=L)
    kv0 = [(b.kc.clone(), b.vc.clone()) for b in st.blocks]

    def reset():
        for b, (k, v) in zip(st.blocks, kv0):
            b.kc.copy_(k)
            b.vc.copy_(v)

    x = torch.from_numpy(randn16(23, B, cfg["dim"])).to(dev)
    pos = torch.from_numpy(rng(24).integers(0, L, B).astype(np.int64)).to(dev)
    st.use_tail = False
    ref = st.decode(x, pos, 1).clone()
    st.use_tail = True
    reset()
    st.tail_no_wait = True
    st.decode(x, pos, 1)
    torch.cuda.synchronize()
    e = st.tail_error()
    # bit 0 and the bits of the waits that gave up (gates, parts, hand-off, slots, merge)
    assert e & 1 and e & 0x3FE and not e & ~0x3FF, hex(e)
    st.tail_no_wait = False
    st.tail_reset()
    reset()
    got = N(st.decode(x, pos, 1)).astype(np.float32)
    torch.cuda.synchronize()
    assert not st.tail_error()
    want = N(ref).astype(np.float32)
    err, bound = np.abs(got - want), ATOL + RTOL * np.abs(want)
    assert (err > bound).mean() <= 1e-3 and (err <= 3 * bound).all()


@pytest.mark.parametrize("cfg,first", [(DEC3, True), (DEC3, False), (DEC_REF2, True),
                                       (DEC_REF2, False)])
def test_tail_two_rows_per_cache_vs_oracle(dev, cfg, first):
    """Two rows per cache (the depth decoder's first pass: S = 2, 2B rows at consecutive
    positions p, p + 1 of each cache) through the head launch and the 16-row tails: the output
    against the oracle's per-op composition and against the per-op kernels, and the slots each
    layer's launch wrote.  Both decoders: 1024 wide (head_dim 128) and the reference's 3072 wide
    (head_dim 384, the W2 phase's 16-row tile in two rounds)."""
    import torch
    B, L = 8, 8
    ost, st = _stacks(dev, cfg, seed=31 + int(first) + cfg["dim"], B=B, L=L, stream=False)
    assert st.tail2 is not None and st.tail2["att"]
    _fill(ost, st, seed=32, upto=L)
    kv0 = [(b.kc.clone(), b.vc.clone()) for b in st.blocks]
    p = np.zeros(B, np.int64) if first else rng(33).integers(0, L - 1, B)
    pos = np.stack([p, p + 1], 1).reshape(-1).astype(np.int64)
    x = randn16(34, 2 * B, cfg["dim"])
    rows = np.arange(2 * B) // 2

    def run_oracle():
        out = ost.decode(x, pos, 2)
        return out, [(b.kc[rows, :, pos].copy(), b.vc[rows, :, pos].copy()) for b in ost.blocks]

    want, wslot = run_oracle()
    OK.GEMV_ACC[0] = np.float32
    try:
        alt, aslot = run_oracle()
    finally:
        OK.GEMV_ACC[0] = np.float64
    xt, pt = torch.from_numpy(x).to(dev), torch.from_numpy(pos).to(dev)
    st.use_tail = False
    ref = N(st.decode(xt, pt, 2)).astype(np.float32)
    for b, (k, v) in zip(st.blocks, kv0):
        b.kc.copy_(k)
        b.vc.copy_(v)
    st.use_tail = True
    got = st.decode(xt, pt, 2)
    torch.cuda.synchronize()
    assert not st.tail_error()
    assert_within_noise(N(got), want, alt, what=f"two rows per cache, first={first}")
    g = N(got).astype(np.float32)
    err, bound = np.abs(g - ref), ATOL + RTOL * np.abs(ref)
    assert (err > bound).mean() <= 1e-3 and (err <= 3 * bound).all()
    ri, pi = torch.from_numpy(rows).to(dev), pt
    for i, b in enumerate(st.blocks):
        gk, gv = N(b.kc[ri, :, pi]), N(b.vc[ri, :, pi])
        assert_within_noise(gk, wslot[i][0], aslot[i][0], what=f"layer {i} k slots")
        assert_within_noise(gv, wslot[i][1], aslot[i][1], what=f"layer {i} v slots")


@pytest.mark.parametrize("cfg,L,stream,kv_nt,S", [
    (dict(BB3, layers=14), 1024, True, False, 1),  # backbone shape, two launches of 7 layers
    (dict(BB3, layers=7), 4096, True, True, 1),    # long splits (staged third tile), NT slot loads
    (dict(DEC3, layers=4), 8, False, False, 1),   # 1024-wide decoder, VALU attention
    (dict(DEC3, layers=4), 8, False, False, 2),   # its first pass: two rows per cache
    (dict(DEC_REF2, layers=3), 8, False, False, 1),  # the reference decoder, head_dim 384
    (dict(DEC_REF2, layers=3), 8, False, False, 2),
])
def test_layer_stack_equals_per_layer_tails(dev, cfg, L, stream, kv_nt, S):
    """All layer tails of a decode step as one launch (ecd_layer_stack) against one launch per
    layer: the same arithmetic in the same order, so the output and every cache slot the step
    wrote are bit-equal; repeated stack launches and a captured graph of the step too."""
    import torch
    from estudiocanciones_amd.kernels import layer_stack_supported
    B = 8
    ost, st = _stacks(dev, cfg, seed=41 + S + cfg["dim"], B=B, L=L, stream=stream)
    st.tail_kv_nt = kv_nt
    _fill(ost, st, seed=42, upto=L)
    t = st.tail if S == 1 else st.tail2
    hd = cfg["dim"] // cfg["heads"]
    assert t["plan"] is not None
    assert layer_stack_supported(cfg["layers"], B * S, cfg["dim"], cfg["ffn"], cfg["heads"],
                                 cfg["kv_heads"], hd, L, stream, kv_nt)
    kv0 = [(b.kc.clone(), b.vc.clone()) for b in st.blocks]

    def reset():
        for b, (k, v) in zip(st.blocks, kv0):
            b.kc.copy_(k)
            b.vc.copy_(v)

    if S == 1:
        p = rng(43).integers(0, L, B).astype(np.int64)
        p[0], p[-1] = 0, L - 1
    else:
        p = rng(43).integers(0, L - 1, B)
        p = np.stack([p, p + 1], 1).reshape(-1).astype(np.int64)
    pos = torch.from_numpy(p).to(dev)
    x = torch.from_numpy(randn16(44, B * S, cfg["dim"])).to(dev)

    def run(stack):
        reset()
        st.use_stack = stack
        out = st.decode(x, pos, S).clone()
        torch.cuda.synchronize()
        assert not st.tail_error()
        return out, [(b.kc.clone(), b.vc.clone()) for b in st.blocks]

    # the backbone's stack takes its layers 7 per launch
    assert not layer_stack_supported(4, B, 3072, 8192, 24, 8, 128, 1024, True, False)
    want, wkv = run(False)
    for rep in range(3):
        got, gkv = run(True)
        assert torch.equal(got, want), f"stack launch {rep} differs from the per-layer launches"
        for i, ((gk, gv), (wk, wv)) in enumerate(zip(gkv, wkv)):
            assert torch.equal(gk, wk) and torch.equal(gv, wv), f"layer {i} caches differ"
    # graph capture and replay of the stack path
    reset()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        st.decode(x, pos, S)
    torch.cuda.current_stream(dev).wait_stream(s)
    clear_warmup_timeout(st, "stack path")
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        gout = st.decode(x, pos, S)
    for _ in range(3):
        reset()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, want), "graph replay of the stack path differs"
        assert not st.tail_error()


@pytest.mark.parametrize("nblocks,N,S", [(4, 8197, 1), (2, 8197, 1), (4, 3000, 1), (4, 8197, 2)])
def test_layer_stack_with_codebook_head(dev, nblocks, N, S):
    """A 1024-wide decoder stack whose last layer ends in a codebook head (rms(x', norm) ->
    int8 head GEMV into logits rows of stride 8256): against the stack's output through the
    separate RMS-prologue GEMV.  Same numerics up to the fp32 summation order of the rms sum,
    so the fp16 bar holds for all but a few logits, 3x it for all; the caches match bit for bit.
    8197 columns: 513 tiles, the first workgroup takes a third.  S = 2: the first decoder
    pass's shape (two rows per cache, 16 rows)."""
    import torch
    from estudiocanciones_amd.engine import Linear
    from estudiocanciones_amd.kernels import rms_gemv_packed
    from estudiocanciones_amd.quant import q8_rows
    B, L = 8, 8
    ost, st = _stacks(dev, dict(DEC3, layers=nblocks), seed=51 + nblocks, B=B, L=L, stream=False)
    _fill(ost, st, seed=52, upto=L)
    g = torch.Generator(device=dev)
    g.manual_seed(53)
    q8, s8 = q8_rows(torch.randn(N, 1024, generator=g, device=dev) * 0.02)
    head = Linear(q8=q8, s8=s8.to(torch.float16)).pack()
    y = torch.empty(S * B, -(-N // 64) * 64, device=dev, dtype=torch.float16)[:, :N]
    st.head_plans({3: (head, y)})
    kv0 = [(b.kc.clone(), b.vc.clone()) for b in st.blocks]

    def reset():
        for b, (k, v) in zip(st.blocks, kv0):
            b.kc.copy_(k)
            b.vc.copy_(v)

    if S == 1:
        p = rng(54).integers(0, L, B).astype(np.int64)
    else:  # a row pair per cache at consecutive slots
        p = rng(54).integers(0, L - 1, B)
        p = np.stack([p, p + 1], 1).reshape(-1).astype(np.int64)
    pos = torch.from_numpy(p).to(dev)
    x = torch.from_numpy(randn16(55, S * B, 1024)).to(dev)
    h = st.decode(x, pos, S, final_norm=False)
    want = N_(rms_gemv_packed(h, st.norm, head.qp, head.s8, N, 1024)).astype(np.float32)
    wkv = [(b.kc.clone(), b.vc.clone()) for b in st.blocks]
    for rep in range(2):
        reset()
        got = st.decode_head(x, pos, S, 3)
        torch.cuda.synchronize()
        assert got is not None and got.data_ptr() == y.data_ptr()
        assert not st.tail_error()
        gv = N_(got).astype(np.float32)
        err, bound = np.abs(gv - want), ATOL + RTOL * np.abs(want)
        assert (err > bound).mean() <= 1e-3, f"head in the stack: {(err > bound).sum()} past the bar"
        assert (err <= 3 * bound).all(), f"head in the stack: max abs err {err.max():.3e}"
        for i, ((gk, gv2), (wk, wv)) in enumerate(zip([(b.kc, b.vc) for b in st.blocks], wkv)):
            assert torch.equal(gk, wk) and torch.equal(gv2, wv), f"layer {i} caches differ"
    # no plan for this head index: the caller falls back
    assert st.decode_head(x, pos, S, 4) is None


def N_(t):
    return t.detach().cpu().numpy()
