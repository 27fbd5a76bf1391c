"""Layer-, stack- and frame-level parity of the gfx950 engine against the oracle.

* one backbone layer at the 3B shape (B=2, D=3072, 24q/8kv, hd 128, FFN 8192, L=1024)
* teacher-forced frames of a small model: KL(oracle || gpu) < 1e-4 on all 8 heads
* sampling with injected Exponential(1) draws reproduces the oracle's tokens
* a captured hipGraph replays bit-identically to the eager step
* the prompt pass matches the oracle's causal prefill
"""
import numpy as np
import pytest

from helpers import (AUDIO_VOCAB, N_CB, assert_close16, model_weights_np, randn16, rng,
                     tiny_cfgs, to_torch)
from oracle.model import OModel, OStack, frame_loop_trim

pytestmark = pytest.mark.gpu


def N(t):
    return t.detach().cpu().numpy()


def kl_rows(p_logits, q_logits):
    """mean over rows of KL(softmax(p) || softmax(q)), float64."""
    p = np.asarray(p_logits, np.float64)
    q = np.asarray(q_logits, np.float64)
    lp = p - p.max(-1, keepdims=True)
    lp -= np.log(np.exp(lp).sum(-1, keepdims=True))
    lq = q - q.max(-1, keepdims=True)
    lq -= np.log(np.exp(lq).sum(-1, keepdims=True))
    return float((np.exp(lp) * (lp - lq)).sum(-1).mean())


def build_pair(dev, bb, dec, n_takes, L, seed=0):
    import torch
    from estudiocanciones_amd.engine import HeartMuLaLite
    wn = model_weights_np(bb, dec, seed=seed)
    om = OModel(wn, bb, dec)
    om.alloc(n_takes, L)
    gm = HeartMuLaLite(to_torch(wn, dev), device=dev, backbone=bb, decoder=dec)
    gm.alloc(n_takes, L)
    return om, gm


def test_backbone_layer_c0(dev):
    """One Llama layer decode step at the 3B backbone shape (B=2, pos 1023, cache filled)."""
    import torch
    from estudiocanciones_amd.engine import Stack
    cfg = dict(layers=1, heads=24, kv_heads=8, max_seq=8192, dim=3072, ffn=8192)
    dec = dict(layers=0, heads=2, kv_heads=1, max_seq=2048, dim=256, ffn=512)
    from estudiocanciones_amd.quant import weight_shapes
    wn = {}
    g = rng(0)
    from oracle.numerics import bf16_bits
    from oracle.quant import q8_rows
    lin, dense = weight_shapes(cfg, dec)
    for name, (Nn, K) in lin.items():
        if name.startswith("backbone."):
            wn[name + ".q8"], wn[name + ".s8"] = q8_rows(
                g.standard_normal((Nn, K), dtype=np.float32) * np.float32(0.02))
    for name, shp in dense.items():
        if name.startswith("backbone."):
            wn[name] = bf16_bits(1.0 + 0.02 * g.standard_normal(shp, dtype=np.float32))
    B, L = 2, 1024
    ost = OStack(lambda n, norm=False: _op(wn, n, norm), "backbone", cfg)
    ost.alloc(B, L)
    kc = randn16(2, B, 8, L, 128)
    vc = randn16(3, B, 8, L, 128)
    ost.blocks[0].kc[:] = kc
    ost.blocks[0].vc[:] = vc
    x = randn16(1, B, 3072)
    pos = np.full(B, L - 1, np.int64)
    want = ost.decode(x, pos, 1)

    wt = to_torch(wn, dev)
    from estudiocanciones_amd.engine import Linear

    def p(name, norm=False):
        if norm:
            return wt[name].to(torch.float16)
        return Linear(q8=wt[name + ".q8"], s8=wt[name + ".s8"].to(torch.float16))

    st = Stack(p, "backbone", cfg)
    st.alloc(B, L, dev, torch.float16)
    st.blocks[0].kc.copy_(torch.from_numpy(kc))
    st.blocks[0].vc.copy_(torch.from_numpy(vc))
    got = st.decode(torch.from_numpy(x).to(dev), torch.from_numpy(pos).to(dev), 1)
    assert_close16(N(got), want, what="backbone layer C0")
    assert_close16(N(st.blocks[0].kc), ost.blocks[0].kc, what="cache after layer")


def _op(wn, name, norm):
    from oracle.model import OLinear
    from oracle.numerics import bf16_to_f32, f16
    from oracle.quant import scale_f16
    if norm:
        return f16(bf16_to_f32(wn[name]))
    return OLinear(wn[name + ".q8"], scale_f16(wn[name + ".s8"]))


@pytest.mark.parametrize("n_takes", [1, 4])
def test_frames_teacher_forced_kl(dev, n_takes):
    """Frames under teacher forcing: the 8 logit sets per frame match the oracle (KL < 1e-4)."""
    import torch
    bb, dec = tiny_cfgs()
    L = 48
    om, gm = build_pair(dev, bb, dec, n_takes, L)
    B = gm.B
    g = rng(5)
    tok = g.integers(0, AUDIO_VOCAB, (B, N_CB)).astype(np.int64)
    worst = 0.0
    for f in range(6):
        forced = g.integers(0, AUDIO_VOCAB, (B, N_CB)).astype(np.int64)
        forced[B // 2:] = forced[: B - B // 2] if B > 1 else forced
        _, olog = om.step(tok, f, forced=forced)
        glog = []
        tt = torch.from_numpy(tok).to(dev)
        pt = torch.full((B, 1), f, dtype=torch.long, device=dev)
        gm._step(tt, pt, None, 1.5, 50, 1.0, forced=torch.from_numpy(forced).to(dev), logits_out=glog)
        for i in range(N_CB):
            assert_close16(N(glog[i]), olog[i], what=f"frame {f} head {i} logits")
            worst = max(worst, kl_rows(olog[i], N(glog[i]).astype(np.float32)))
        tok = forced
    assert worst < 1e-4, worst


def test_sampling_with_injected_noise(dev):
    """CFG + top-50 + Exponential race with the same draws picks the oracle's tokens."""
    import torch
    bb, dec = tiny_cfgs()
    om, gm = build_pair(dev, bb, dec, 2, 32, seed=1)
    B, Nt = gm.B, gm.N
    g = rng(6)
    tok = g.integers(0, AUDIO_VOCAB, (B, N_CB)).astype(np.int64)
    tok[Nt:] = tok[:Nt]
    for f in range(3):
        noise = g.exponential(1.0, (N_CB, Nt, AUDIO_VOCAB)).astype(np.float32)
        otok, _ = om.step(tok, f, noise=noise)
        gt = gm._step(torch.from_numpy(tok).to(dev), torch.full((B, 1), f, dtype=torch.long, device=dev),
                      None, 1.5, 50, 1.0, noise=torch.from_numpy(noise).to(dev))
        assert np.array_equal(N(gt), otok), (N(gt), otok)
        tok = otok


@pytest.mark.parametrize("n_takes", [2, 3])
def test_next_rows_table_equals_projection(dev, n_takes):
    """Decoder passes 1..6 take their input from the precomputed projection rows (written by
    the sampler) instead of the projection launch: logits and tokens bit-equal to those of the
    projection path, with and without CFG.  With the precomputed layer-0 q|k|v as well (the
    sampler then writes the cache slot and runs layer 0's attention) and the first pass's
    input from the fused codebook-0 + projection GEMV and the sampler, the tokens are the same
    and every head's logits agree to KL < 1e-4, through the layer tails and through the
    decoder's per-op kernels alike."""
    import torch
    bb, dec = tiny_cfgs()
    _, gm = build_pair(dev, bb, dec, n_takes, 32, seed=4)
    assert gm._next_rows is not None and gm._xnext.shape[0] == gm.B
    assert gm._next_qkv is not None and gm._onext.shape[0] == gm.B
    B, Nt = gm.B, gm.N
    g = rng(8)
    tok = torch.from_numpy(g.integers(0, AUDIO_VOCAB, (B, N_CB))).to(dev)
    noise = torch.from_numpy(g.exponential(1.0, (N_CB, Nt, AUDIO_VOCAB)).astype(np.float32)).to(dev)
    rows, qkv, c0p = gm._next_rows, gm._next_qkv, gm._c0proj
    assert c0p is not None
    runs = {}
    for name, r, q, cp, tail in (("proj", None, None, None, True), ("rows", rows, None, None, True),
                                 ("rows_c0proj", rows, None, c0p, True),
                                 ("qkv", rows, qkv, c0p, True), ("qkv_perop", rows, qkv, c0p, False)):
        gm._next_rows, gm._next_qkv = r, q
        gm._c0proj = cp
        gm.decoder.use_tail = tail
        lg = []
        out = gm._step(tok, torch.full((B, 1), 3, dtype=torch.long, device=dev), None, 1.5, 50,
                       1.0, noise=noise, logits_out=lg)
        torch.cuda.synchronize()
        runs[name] = (out.clone(), [x.clone() for x in lg])
    gm._next_rows, gm._next_qkv, gm._c0proj = rows, qkv, c0p
    gm.decoder.use_tail = True
    assert torch.equal(runs["rows"][0], runs["proj"][0])
    for a, b in zip(runs["rows"][1], runs["proj"][1]):
        assert torch.equal(a, b)
    for name in ("rows_c0proj", "qkv", "qkv_perop"):
        assert torch.equal(runs[name][0], runs["proj"][0]), name
        for i, (a, b) in enumerate(zip(runs[name][1], runs["proj"][1])):
            kl = kl_rows(N(b).astype(np.float64), N(a).astype(np.float64))
            assert kl < 1e-4, (name, i, kl)


def test_graph_replay_matches_eager(dev):
    """The whole frame captured as one hipGraph replays bit-identically to eager execution."""
    import torch
    bb, dec = tiny_cfgs()
    _, gm = build_pair(dev, bb, dec, 4, 40, seed=2)
    B = gm.B
    g = rng(7)
    static = dict(tok=torch.zeros(B, N_CB, dtype=torch.long, device=dev),
                  pos=torch.zeros(B, 1, dtype=torch.long, device=dev),
                  forced=torch.zeros(B, N_CB, dtype=torch.long, device=dev))
    logits_g = []
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gm._step(static["tok"], static["pos"], None, 1.5, 50, 1.0, forced=static["forced"])
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(graph):
        gm._step(static["tok"], static["pos"], None, 1.5, 50, 1.0, forced=static["forced"],
                 logits_out=logits_g)
    for f in range(4):
        tok = torch.from_numpy(g.integers(0, AUDIO_VOCAB, (B, N_CB))).to(dev)
        forced = torch.from_numpy(g.integers(0, AUDIO_VOCAB, (B, N_CB))).to(dev)
        snap = [(b.kc.clone(), b.vc.clone()) for b in gm.backbone.blocks]
        logits_e = []
        gm._step(tok, torch.full((B, 1), f, dtype=torch.long, device=dev), None, 1.5, 50, 1.0,
                 forced=forced, logits_out=logits_e)
        ref = [l.clone() for l in logits_e]
        for b, (k, v) in zip(gm.backbone.blocks, snap):
            b.kc.copy_(k)
            b.vc.copy_(v)
        static["tok"].copy_(tok)
        static["pos"].fill_(f)
        static["forced"].copy_(forced)
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(logits_g, ref):
            assert torch.equal(a, b)


@pytest.mark.parametrize("P", [12, 48])
def test_prefill_matches_oracle(dev, P):
    """Prompt pass (B=2) vs the oracle's causal prefill: 24 rows run the decode kernels, 96 rows
    the MFMA GEMM path (more than 64 rows)."""
    import torch
    bb, dec = tiny_cfgs()
    om, gm = build_pair(dev, bb, dec, 1, 64, seed=3)
    B, D = gm.B, bb["dim"]
    x = randn16(8, B, P, D)
    pos = np.arange(P, dtype=np.int64)
    want = om.backbone.prefill(x, pos)
    got = gm.backbone(torch.from_numpy(x).to(dev), torch.from_numpy(pos).to(dev)[None].expand(B, P))
    assert_close16(N(got), want, what="prefill output")
    for ob, gb in zip(om.backbone.blocks, gm.backbone.blocks):
        assert_close16(N(gb.kc)[:, :, :P], ob.kc[:, :, :P], what="prefill k cache")
        assert_close16(N(gb.vc)[:, :, :P], ob.vc[:, :, :P], what="prefill v cache")


def test_generate_small_song(dev):
    """End-to-end generate(): prompt pass, graph-per-song frame loop, EOS trim."""
    import torch
    from estudiocanciones_amd.engine import HeartMuLaLite
    bb, dec = tiny_cfgs()
    wn = model_weights_np(bb, dec, seed=4)
    gm = HeartMuLaLite(to_torch(wn, dev), device=dev, backbone=bb, decoder=dec)
    text = rng(9).integers(0, 64, 10)
    out = gm.generate(text, 3, max_ms=80 * 30, seed=1, n=2)
    assert isinstance(out, list) and len(out) == 2
    for o in out:
        assert o.shape[0] == N_CB and 1 <= o.shape[1] <= 31
        assert int(o.min()) >= 0 and int(o.max()) < AUDIO_VOCAB
    one = gm.generate(text, 3, max_ms=80 * 5, seed=1, use_graphs=False)
    assert one.shape[0] == N_CB
    assert gm.generate(text, 3, max_ms=800, abort=lambda: True) is None


@pytest.mark.parametrize("use_graphs", [True, False])
@pytest.mark.parametrize("ends", [(3, 26, 51, None), (3, 26, 40, 12)], ids=["one-never", "all-end"])
def test_generate_forced_eos_trim(dev, use_graphs, ends):
    """The song loop (app/engine.py:401-446) with every frame's tokens forced: EOS first appears
    at the given frames (None: never); later EOS tokens and one in the prompt frame change
    nothing.  The returned takes and the frames run equal the oracle's restatement of the EOS
    scan (every 25 frames) and the per-take trim."""
    import torch
    from estudiocanciones_amd.engine import HeartMuLaLite
    bb, dec = tiny_cfgs()
    wn = model_weights_np(bb, dec, seed=4)
    gm = HeartMuLaLite(to_torch(wn, dev), device=dev, backbone=bb, decoder=dec)
    n, n_frames = 4, 60
    g = rng(12)
    frames = g.integers(0, 8193, (n_frames + 1, 2 * n, N_CB)).astype(np.int64)
    for c, t in enumerate(ends):
        if t is not None:
            frames[t, c, 5] = 8193 + c
            frames[min(t + 2, n_frames), c, 0] = 8196
    frames[0, 3, 1] = 8193
    frames[:, n:] = frames[:, :n]
    want, ran = frame_loop_trim(frames[:, :n], n_frames)
    got = gm.generate(rng(9).integers(0, 64, 10), 3, max_ms=80 * n_frames, seed=1, n=n,
                      use_graphs=use_graphs, forced=torch.from_numpy(frames).to(dev))
    assert gm.frames_run == ran
    for c in range(n):
        assert np.array_equal(N(got[c]), want[c]), c


def test_generate_graph_equals_eager(dev):
    """Sampled songs (no forcing): the captured loop and the eager loop give the same tokens for
    the same seed, and a second run repeats them."""
    from estudiocanciones_amd.engine import HeartMuLaLite
    bb, dec = tiny_cfgs()
    wn = model_weights_np(bb, dec, seed=4)
    gm = HeartMuLaLite(to_torch(wn, dev), device=dev, backbone=bb, decoder=dec)
    text = rng(9).integers(0, 64, 10)
    a = gm.generate(text, 3, max_ms=80 * 30, seed=5, n=2)
    b = gm.generate(text, 3, max_ms=80 * 30, seed=5, n=2, use_graphs=False)
    c = gm.generate(text, 3, max_ms=80 * 30, seed=5, n=2)
    for x, y, z in zip(a, b, c):
        assert np.array_equal(N(x), N(y)) and np.array_equal(N(x), N(z))


@pytest.mark.parametrize("stack", ["backbone", "decoder"])
def test_generate_raises_on_tail_timeout(dev, stack):
    """The song loop reads the layer tails' error words with the EOS frames: with every wait of
    one stack's tail launches giving up at its first look (forced from the host, so every kernel
    still exits normally), generate() raises RuntimeError instead of returning tokens; the next
    song on the same model runs and matches its eager loop."""
    import torch
    from estudiocanciones_amd.engine import HeartMuLaLite
    from estudiocanciones_amd.quant import synthetic_weights
    cfg = dict(layers=2, heads=8, kv_heads=2, max_seq=2048, dim=1024, ffn=8192)
    gm = HeartMuLaLite(synthetic_weights(cfg, cfg, device=dev, seed=31, text_vocab=64),
                       device=dev, backbone=cfg, decoder=cfg)
    text = rng(9).integers(0, 64, 10)
    st = getattr(gm, stack)
    st.tail_no_wait = True
    with pytest.raises(RuntimeError, match="timed out"):
        gm.generate(text, 3, max_ms=80 * 3, seed=2, n=4)
    assert gm.backbone.tail is None and gm.decoder.tail is None  # released
    st.tail_no_wait = False
    a = gm.generate(text, 3, max_ms=80 * 30, seed=5, n=4)
    assert not gm.graphs
    gm.alloc(4, 16)
    assert gm.backbone.tail is not None and gm.decoder.tail is not None, "tails not in use"
    b = gm.generate(text, 3, max_ms=80 * 30, seed=5, n=4, use_graphs=False)
    for x, y in zip(a, b):
        assert np.array_equal(N(x), N(y))
