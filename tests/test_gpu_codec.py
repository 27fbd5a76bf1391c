"""Kernels of the codec's flow-matching estimator (app/heartcodec/models/transformer.py) and its
Euler solver (app/heartcodec/models/flow_matching.py) against the oracle (oracle/codec.py) and
fp32 numpy products with the same fp16 rounding points as torch's fp16 layers.

Bars: copies, RoPE rotation and the Euler update bit-exact; single kernels within
|got - want| <= 2e-3 + 1e-2 |want|; the whole estimator and solver (many fp16 layers, fp32
accumulation in a different order than the oracle's float64) within 2e-2 of the output's
largest magnitude, with correlation above 0.9999."""
import numpy as np
import pytest

from helpers import assert_close16, randn16, rng
from oracle import codec as OC
from oracle.numerics import f16

pytestmark = pytest.mark.gpu


def D_(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def N_(t):
    return t.detach().cpu().numpy()


def _exact(got, want, what):
    """Bit-exact comparison that names the first differing elements."""
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bad = np.argwhere(got.view(np.uint16) != want.view(np.uint16))
    if len(bad):
        show = [(tuple(i), float(got[tuple(i)]), float(want[tuple(i)])) for i in bad[:6]]
        raise AssertionError(f"{what}: {len(bad)} of {got.size} differ; first {show}")


def _call(name, *args):
    import torch
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd.kernels import stream_ptr
    _ffi.call(name, *args, stream_ptr(torch.device("cuda")))


# ---------------------------------------------------------------- fp16 GEMM
@pytest.mark.parametrize("M,N,K,bias,alpha,res", [
    (17, 100, 64, True, 1.0, False),          # ragged M and N, one K chunk
    (1488, 1536, 3072, True, 3 ** -0.5, False),  # ProjectLayer conv (k = 3) as a GEMM, scaled
    (200, 1536, 7680, False, 1.0, True),      # connection_proj width (K = 3 x 2560), residual
    (96, 3072, 1536, True, 1.0, True),
])
def test_gemm_f16_linear(dev, M, N, K, bias, alpha, res):
    """F.linear(x, w, b) numerics: fp32 accumulation and bias, one fp16 rounding; then the
    optional fp16 scale and fp16 residual add."""
    from estudiocanciones_amd.kernels import gemm_f16_packed, pack_f16
    g = rng(400 + K)
    x = randn16(401 + M, M, K)
    w = (g.standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float16)
    b = (g.standard_normal(N, dtype=np.float32) * 0.1) if bias else None
    r = randn16(402 + M, M, N) if res else None
    want = x.astype(np.float32) @ w.astype(np.float32).T
    if bias:
        want = want + b
    want = f16(want)
    if alpha != 1.0:
        want = f16(want.astype(np.float32) * np.float32(alpha))
    if res:
        want = f16(want.astype(np.float32) + r.astype(np.float32))
    got = gemm_f16_packed(D_(x, dev), pack_f16(D_(w, dev)), N, K, D_(b, dev) if bias else None,
                          alpha, D_(r, dev) if res else None)
    assert_close16(N_(got), want, what=f"gemm f16 M={M} N={N} K={K}")


@pytest.mark.parametrize("M,F,K", [(40, 256, 128), (1488, 4096, 1536)])
def test_gemm_f16_silu(dev, M, F, K):
    """LlamaMLP's F.silu(gate(x)) * up(x) in fp16 (transformer.py:178-181)."""
    import torch
    from estudiocanciones_amd.kernels import gemm_f16_silu_packed, pack_f16
    g = rng(410 + F)
    x = randn16(411 + M, M, K)
    gate = (g.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    up = (g.standard_normal((F, K), dtype=np.float32) * 0.02).astype(np.float16)
    a = f16(x.astype(np.float32) @ gate.astype(np.float32).T).astype(np.float32)
    u = f16(x.astype(np.float32) @ up.astype(np.float32).T).astype(np.float32)
    want = f16(f16(a / (1.0 + np.exp(-a))).astype(np.float32) * u)
    wp = pack_f16(torch.cat([D_(gate, dev), D_(up, dev)], 0).contiguous(), interleave=True)
    got = gemm_f16_silu_packed(D_(x, dev), wp, F, K)
    assert_close16(N_(got), want, what=f"gemm f16 silu M={M} F={F}")


@pytest.mark.parametrize("M,N,K,silu", [(200, 1536, 1536, 0), (77, 1000, 640, 0), (300, 2048, 512, 1),
                                         (130, 200, 64, 0), (65, 96, 192, 0), (90, 256, 128, 1)])
def test_gemm_f16_tile_configs_agree(dev, M, N, K, silu):
    """Every block tile / pipeline variant (2 or 3 LDS stages; K of 1-3 chunks exercises the short
    pipelines) accumulates each output in the same order: all agree bit for bit with the first,
    and the library default with the fp32 product."""
    import torch
    from estudiocanciones_amd.kernels import pack_f16
    g = rng(420 + N)
    x = randn16(421 + M, M, K)
    w = (g.standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float16)
    b = None if silu else D_((g.standard_normal(N, dtype=np.float32) * 0.1), dev)
    r = None if silu else D_(randn16(422, M, N), dev)
    xt, wp = D_(x, dev), pack_f16(D_(w, dev), interleave=bool(silu))
    No = N // 2 if silu else N
    outs = []
    for cfg in range(0, 17):
        y = torch.empty(M, No, dtype=torch.float16, device=dev)
        _call("ecd_gemm_f16p_tuned", xt.data_ptr(), K, wp.data_ptr(),
              None if b is None else b.data_ptr(), 1.0 if silu else 0.75,
              None if r is None else r.data_ptr(), N, y.data_ptr(), No, M, N, K, silu, cfg)
        outs.append(N_(y))
    for cfg, o in enumerate(outs[2:], 2):
        _exact(o, outs[1], f"gemm f16 cfg {cfg} vs cfg 1 (M={M} N={N} K={K} silu={silu})")
    _exact(outs[0], outs[1], "library default vs cfg 1")
    if not silu:
        want = f16(x.astype(np.float32) @ w.astype(np.float32).T + N_(b))
        want = f16(f16(want.astype(np.float32) * np.float32(0.75)).astype(np.float32) + N_(r))
        assert_close16(outs[0], want, what="gemm f16 default")


# ---------------------------------------------------------------- RoPE
@pytest.mark.parametrize("L,HD", [(744, 64), (744, 128), (37, 64)])
def test_codec_rope_table(dev, L, HD):
    import torch
    tab = torch.empty(L, HD, dtype=torch.float16, device=dev)
    _call("ecd_codec_rope_table", tab.data_ptr(), L, HD)
    sin, cos = OC.rope_table(L, HD)
    got = N_(tab).reshape(L, HD // 2, 2)
    # the angles are fp16 values on both sides; only last-bit differences of fp32 sin/cos can
    # flip a rounding
    np.testing.assert_allclose(got[..., 0], cos, atol=1e-3, rtol=0)
    np.testing.assert_allclose(got[..., 1], sin, atol=1e-3, rtol=0)


@pytest.mark.parametrize("B,L,H,HD", [(2, 37, 3, 64), (2, 50, 2, 128)])
def test_codec_rope_heads_bit_exact(dev, B, L, H, HD):
    import torch
    D = H * HD
    qkv = randn16(500 + HD, B * L, 3 * D)
    sin, cos = OC.rope_table(L, HD)
    tab = np.stack([cos, sin], -1).astype(np.float16)
    q = torch.empty(B * L, D, dtype=torch.float16, device=dev)
    k = torch.empty(B, H, L, HD, dtype=torch.float16, device=dev)
    v = torch.empty_like(k)
    qt, tt = D_(qkv, dev), D_(tab, dev)
    _call("ecd_codec_rope_heads", qt.data_ptr(), 3 * D, tt.data_ptr(), q.data_ptr(),
          k.data_ptr(), v.data_ptr(), B, L, H, HD)
    heads = lambda a: a.reshape(B, L, H, HD).transpose(0, 2, 1, 3)
    want_q = OC.apply_rope_vec(heads(qkv[:, :D]), sin, cos)
    want_k = OC.apply_rope_vec(heads(qkv[:, D:2 * D]), sin, cos)
    assert np.array_equal(N_(q), want_q.transpose(0, 2, 1, 3).reshape(B * L, D))
    assert np.array_equal(N_(k), want_k)
    assert np.array_equal(N_(v), heads(qkv[:, 2 * D:]))


@pytest.mark.parametrize("B,L,H,HD,K", [(2, 37, 3, 64, 192), (1, 130, 2, 128, 256), (2, 9, 5, 64, 64)])
def test_gemm_f16_rope_fused(dev, B, L, H, HD, K):
    """The q | k | v GEMM with RoPE in its epilogue equals the GEMM followed by the standalone
    RoPE kernel bit for bit (q rows, k and v heads), with and without a bias."""
    import torch
    from estudiocanciones_amd.kernels import pack_f16
    D, M = H * HD, B * L
    g = rng(560 + HD + L)
    x = randn16(561 + L, M, K)
    w = f16(g.standard_normal((3 * D, K)) * 0.05)
    sin, cos = OC.rope_table(L, HD)
    tab = D_(np.stack([cos, sin], -1).astype(np.float16), dev)
    xt, wp = D_(x, dev), pack_f16(D_(w, dev))
    for bias in (None, D_((g.standard_normal(3 * D) * 0.1).astype(np.float32), dev)):
        bp = None if bias is None else bias.data_ptr()
        qkv = torch.empty(M, 3 * D, dtype=torch.float16, device=dev)
        _call("ecd_gemm_f16p", xt.data_ptr(), K, wp.data_ptr(), bp, 1.0, None, 0, qkv.data_ptr(),
              3 * D, M, 3 * D, K)
        outs = []
        for fused in (False, True):
            q = torch.empty(M, D, dtype=torch.float16, device=dev)
            k = torch.empty(B, H, L, HD, dtype=torch.float16, device=dev)
            v = torch.empty_like(k)
            if fused:
                _call("ecd_gemm_f16p_rope", xt.data_ptr(), K, wp.data_ptr(), bp, tab.data_ptr(),
                      q.data_ptr(), k.data_ptr(), v.data_ptr(), M, L, H, HD, K)
            else:
                _call("ecd_codec_rope_heads", qkv.data_ptr(), 3 * D, tab.data_ptr(), q.data_ptr(),
                      k.data_ptr(), v.data_ptr(), B, L, H, HD)
            outs.append((N_(q), N_(k), N_(v)))
        for name, a, b in zip("qkv", outs[0], outs[1]):
            _exact(b, a, f"fused rope {name} (H={H} HD={HD} bias={bias is not None})")


# ---------------------------------------------------------------- norms + adaLN
@pytest.mark.parametrize("norm,resid,per_batch,D", [(0, False, False, 1536), (0, True, True, 3072),
                                                    (1, True, False, 1536), (1, False, True, 128),
                                                    (0, True, False, 4096)])
def test_codec_norm_mod(dev, norm, resid, per_batch, D):
    import torch
    B, L = 2, 29
    g = rng(600 + D + norm)
    x = randn16(601 + D, B * L, D, std=2.0)
    h = randn16(602 + D, B * L, D)
    w = f16(1 + 0.1 * g.standard_normal(D))
    tab = f16(g.standard_normal((3, D)) * 0.3)          # gate, shift, scale rows
    tm = f16(g.standard_normal((B if per_batch else 1, 3, D)) * 0.3)
    ld = 3 * D if per_batch else 0
    xt, ht, wt, tabt, tmt = (D_(a, dev) for a in (x, h, w, tab, tm))
    y = torch.empty(B * L, D, dtype=torch.float16, device=dev)
    a = lambda t, i: t.data_ptr() + 2 * i * D
    _call("ecd_codec_norm_mod", xt.data_ptr(), ht.data_ptr() if resid else None,
          a(tabt, 0) if resid else None, a(tmt, 0) if resid else None, ld,
          wt.data_ptr() if norm == 0 else None, a(tabt, 1), a(tmt, 1), a(tabt, 2), a(tmt, 2), ld,
          y.data_ptr(), B * L, L, D, norm, 1e-6)
    bt = lambda v: np.repeat(v, L, 0) if per_batch else v
    m = f16(tab[None].astype(np.float32) + tm.astype(np.float32))       # [B or 1, 3, D]
    gate, shift, scale = bt(m[:, 0]), bt(m[:, 1]), bt(m[:, 2])
    xw = x
    if resid:
        xw = f16(x.astype(np.float32) + f16(gate.astype(np.float32) * h.astype(np.float32)))
        assert np.array_equal(N_(xt), xw), "gated residual must be bit-exact"
    n = OC.rms_norm(xw, w) if norm == 0 else OC.layer_norm(xw)
    assert_close16(N_(y), OC.modulate(n, shift, scale), what=f"norm_mod norm={norm} D={D}")


# ---------------------------------------------------------------- conv columns
def test_codec_cols3_bit_exact(dev):
    """Segments as solve_euler feeds them: x and incontext shared by both halves, mu zeroed in
    the unconditional half, plus a per-row segment (connection_proj's s)."""
    import ctypes
    import torch
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd.kernels import stream_ptr
    B, L = 1, 23
    x, ic, mu = randn16(700, B * L, 16), randn16(701, B * L, 16), randn16(702, B * L, 32)
    s = randn16(703, 2 * B * L, 24)
    segs = [(x, 16, B, 0), (ic, 16, B, 0), (mu, 32, B, B), (s, 24, 2 * B, 0)]
    dt = [D_(a[0], dev) for a in segs]
    C = 88
    out = torch.full((2 * B * L, 3 * C), 7.0, dtype=torch.float16, device=dev)
    n = len(segs)
    _ffi.call("ecd_codec_cols3", (ctypes.c_void_p * n)(*[t.data_ptr() for t in dt]),
              (ctypes.c_long * n)(*[sg[1] for sg in segs]), (ctypes.c_int * n)(*[sg[1] for sg in segs]),
              (ctypes.c_int * n)(*[sg[2] for sg in segs]), (ctypes.c_int * n)(*[sg[3] for sg in segs]),
              None, n, out.data_ptr(), 2 * B, L, stream_ptr(dev))
    inp = np.concatenate([np.concatenate([x, x]), np.concatenate([ic, ic]),
                          np.concatenate([np.zeros_like(mu), mu]), s], 1).reshape(2 * B, L, C)
    pad = np.zeros((2 * B, L + 2, C), np.float16)
    pad[:, 1:-1] = inp
    want = np.concatenate([pad[:, j:j + L] for j in range(3)], -1).reshape(2 * B * L, 3 * C)
    assert np.array_equal(N_(out), want)


# ---------------------------------------------------------------- timestep path pieces
def test_codec_timestep_and_silu(dev):
    import torch
    t = OC.t_span(10)
    out = torch.empty(11, 512, dtype=torch.float16, device=dev)
    tt = D_(t, dev)
    _call("ecd_codec_timestep", tt.data_ptr(), out.data_ptr(), 11)
    assert_close16(N_(out), OC.timestep_sinusoid(t), what="timestep sinusoid")
    x = randn16(710, 7, 300, std=4.0)
    y = torch.empty(7, 300, dtype=torch.float16, device=dev)
    xt = D_(x, dev)
    _call("ecd_codec_silu", xt.data_ptr(), y.data_ptr(), x.size)
    assert_close16(N_(y), OC.silu(x), what="silu")


# ---------------------------------------------------------------- Euler update
@pytest.mark.parametrize("cfg,mode,L", [(1, 0, 10), (0, 0, 0), (1, 1, 7), (1, 0, 0)])
def test_codec_euler_bit_exact(dev, cfg, mode, L):
    B, Ln, C = 1, 30, 256
    x, nz, ic = randn16(720, B, Ln, C), randn16(721, B, Ln, C), randn16(722, B, Ln, C)
    d = randn16(723, (2 if cfg else 1) * B, Ln, C)
    dt, g, tb = np.float32(0.1), 1.25, np.float32(0.3)
    xt, nzt, ict, dt_ = D_(x, dev), D_(nz, dev), D_(ic, dev), D_(d, dev)   # keep all alive
    _call("ecd_codec_euler", xt.data_ptr(), nzt.data_ptr(), ict.data_ptr(), dt_.data_ptr(), cfg,
          B, Ln, C, L, float(dt), g, float(tb), mode)
    f32 = lambda a: np.asarray(a, np.float32)
    if cfg:
        u, c = d[:B], d[B:]
        v = f16(f32(u) + f32(f16(np.float32(g) * f32(f16(f32(c) - f32(u))))))
    else:
        v = d
    want = f16(f32(x) + f32(f16(dt * f32(v))))
    if L:
        if mode == 1:
            want[:, :L] = ic[:, :L]
        else:
            a = np.float32(np.float32(1) - np.float32(np.float32(1 - 1e-6) * tb))
            want[:, :L] = f16(f32(f16(a * f32(nz[:, :L]))) + f32(f16(tb * f32(ic[:, :L]))))
    _exact(N_(xt), want, f"euler cfg={cfg} mode={mode} L={L}")


# ---------------------------------------------------------------- estimator and solver
TINY = dict(heads=2, head_dim=64, in_channels=192, out_channels=64, layers=2, layers_2=1)


def _estimator(dev, p, cfg):
    import torch
    from estudiocanciones_amd.codec import LlamaTransformer
    sd = {k: torch.from_numpy(v) for k, v in p.items()}
    return LlamaTransformer(sd, num_attention_heads=cfg["heads"],
                            attention_head_dim=cfg["head_dim"], in_channels=cfg["in_channels"],
                            out_channels=cfg["out_channels"], num_layers=cfg["layers"],
                            num_layers_2=cfg["layers_2"], device=dev)


def _close_model(got, want, what):
    got, want = got.astype(np.float64), want.astype(np.float64)
    assert np.all(np.isfinite(got)), what
    err = np.abs(got - want).max() / np.abs(want).max()
    corr = np.corrcoef(got.ravel(), want.ravel())[0, 1]
    assert err < 2e-2 and corr > 0.9999, f"{what}: rel max err {err:.3g}, corr {corr:.6f}"


@pytest.mark.parametrize("B,L,t", [(2, 40, (0.3, 0.3)), (1, 70, (0.0,)), (3, 17, (0.1, 0.5, 0.9))])
def test_codec_estimator_forward(dev, B, L, t):
    p = OC.random_weights(TINY, seed=21)
    est = _estimator(dev, p, TINY)
    hidden = randn16(730 + L, B, L, TINY["in_channels"])
    tt = np.array(t, np.float32)
    got = est(D_(hidden, dev), D_(tt, dev))
    _close_model(N_(got), OC.estimator(p, TINY, hidden, tt), f"estimator B={B} T={L}")


@pytest.mark.parametrize("g,L_ic", [(1.25, 0), (1.25, 9), (1.0, 5)])
def test_codec_solve_euler(dev, g, L_ic):
    from estudiocanciones_amd.codec import solve_euler
    p = OC.random_weights(TINY, seed=22)
    est = _estimator(dev, p, TINY)
    Ln, C, Cmu = 36, 64, 64
    x0, ic, mu = randn16(740, 1, Ln, C), randn16(741, 1, Ln, C), randn16(742, 1, Ln, Cmu)
    ic[:, L_ic:] = 0
    ts = OC.t_span(4)
    got = solve_euler(est, D_(x0, dev), D_(ic, dev), L_ic, ts, D_(mu, dev), g)
    want = OC.solve_euler(lambda h, t: OC.estimator(p, TINY, h, t), x0, ic, L_ic, ts, mu, g)
    _close_model(N_(got), want, f"solve_euler g={g} L={L_ic}")


# ---------------------------------------------------------------- code embedding, inference_codes
def test_codec_vq_embed(dev):
    """Sum of the 8 quantizers' codebook rows (-1 and out-of-range codes dropped), zero-padded to
    the GEMM's K, from a strided [B, Q, Tc] window of a longer code tensor."""
    import torch
    B, Q, Tfull, Tc, V, Dc, Wp = 2, 8, 40, 29, 100, 32, 64
    g = rng(760)
    books = f16(g.standard_normal((Q, V, Dc)) * 0.5)
    codes_full = g.integers(0, V, (B, Q, Tfull))
    codes_full[0, 2, 7] = -1
    codes_full[1, 5, 3] = V + 3
    win = codes_full[:, :, 5:5 + Tc]
    ct = D_(codes_full, dev)[:, :, 5:5 + Tc]
    out = torch.full((B * Tc, Wp), 9.0, dtype=torch.float16, device=dev)
    bt = D_(books, dev)
    for clamp in (0, 1):
        _call("ecd_codec_vq_embed", ct.data_ptr(), ct.stride(0), ct.stride(1), bt.data_ptr(),
              out.data_ptr(), B, Q, Tc, V, Dc, Wp, clamp)
        want = np.zeros((B, Tc, Wp))
        for q in range(Q):
            idx = np.clip(win[:, q], 0, V - 1) if clamp else win[:, q]
            ok = (idx >= 0) & (idx < V)
            want[..., :Dc] += books[q].astype(np.float64)[np.where(ok, idx, 0)] * ok[..., None]
        assert_close16(N_(out), f16(want).reshape(B * Tc, Wp), what=f"vq embed clamp={clamp}")
        assert np.all(N_(out)[:, Dc:] == 0)


def _code_embedding(dev, p):
    import torch
    from estudiocanciones_amd.codec import CodeEmbedding
    return CodeEmbedding({k: torch.from_numpy(v) for k, v in p.items()}, device=dev)


def test_code_embedding_host(dev):
    p = OC.random_vq_weights(8, 64, 32, 128, seed=33)
    codes = rng(34).integers(0, 64, (2, 8, 21))
    got = _code_embedding(dev, p)(D_(codes, dev))
    want = OC.code_embedding(p, codes)[:, ::2].reshape(2 * 21, 128)
    assert_close16(N_(got), want, what="code embedding")


@pytest.mark.parametrize("scenario,L_ic", [("start_seg", 0), ("other_seg", 8)])
def test_codec_inference_codes(dev, scenario, L_ic):
    """codes -> latents through the embedding, the half-rate mu read as its 2x upsampling, the
    CFG solve and the final in-context copy, against the oracle."""
    from estudiocanciones_amd.codec import inference_codes
    p_est = OC.random_weights(TINY, seed=35)
    p_fm = OC.random_vq_weights(8, 64, 32, 64, seed=36)
    est = _estimator(dev, p_est, TINY)
    emb = _code_embedding(dev, p_fm)
    Tc = 18
    codes = rng(37).integers(0, 64, (1, 8, Tc))
    true_lat = randn16(38, 1, 2 * Tc, 64)
    noise = randn16(39, 1, 2 * Tc, 64)
    got = inference_codes(emb, est, D_(codes, dev), D_(true_lat, dev), 2 * Tc, L_ic, 1.25, 3,
                          scenario, noise=D_(noise, dev))
    want = OC.inference_codes(p_fm, p_est, TINY, codes, true_lat, 2 * Tc, L_ic, 1.25, 3, scenario,
                              noise)
    _close_model(N_(got), want, f"inference_codes {scenario}")
    if L_ic:
        _exact(N_(got)[:, :L_ic], true_lat[:, :L_ic], "in-context prefix copied")


def test_codec_detokenize_latents(dev):
    """The window loop of detokenize up to the latents: 250 codes at a 7.44 s window (93 codes,
    hop 80, overlap 13 codes = 26 frames) are padded to 253 by repetition and decoded as three
    windows, each later one continuing the previous window's last 26 frames; codes outside the
    codebook are clamped."""
    import torch
    from estudiocanciones_amd.codec import detokenize_latents
    p_est = OC.random_weights(TINY, seed=40)
    p_fm = OC.random_vq_weights(8, 64, 32, 64, seed=41)
    est = _estimator(dev, p_est, TINY)
    emb = _code_embedding(dev, p_fm)
    codes = rng(42).integers(0, 64, (8, 250))
    codes[2, 17] = 70
    codes[5, 100] = -4
    duration, frames = 7.44, 186
    noises = [randn16(43 + w, 1, frames, 64) for w in range(3)]
    it = iter(noises)
    got = detokenize_latents(emb, est, D_(codes, dev), duration, 2, 1.25,
                             randn=lambda shape: D_(next(it), dev))
    want = OC.detokenize_latents(p_fm, p_est, TINY, codes, duration, 2, 1.25, noises)
    assert len(got) == len(want) == 3
    for w, (g, wv) in enumerate(zip(got, want)):
        _close_model(N_(g), wv, f"detokenize window {w}")
    _exact(N_(got[1])[:, :26], N_(got[0])[:, -26:], "window 1 continues window 0")


# ---------------------------------------------------------------- waveform decoder
DEC = dict(latent_hidden_dim=64, init_channel=64, upsample_factors=(2, 3))


@pytest.mark.parametrize("offs,rep,row0,nrows", [((-6, -5, -4, -3, -2, -1, 0), 1, 0, None),
                                                 ((-18, -15, -12, -9, -6, -3, 0), 1, 0, None),
                                                 ((-2, -1, 0, 1, 2), 1, 7, 40),
                                                 ((0, -1), 1, 0, None),
                                                 ((-6, -5, -4, -3, -2, -1, 0), 2, 33, 50)])
def test_codec_cols_taps_bit_exact(dev, offs, rep, row0, nrows):
    import ctypes
    import torch
    B, T, C = 2, 44, 24
    src = randn16(800 + len(offs), B * (T // rep), C)
    n = nrows or B * T
    out = torch.full((n, len(offs) * C), 5.0, dtype=torch.float16, device=dev)
    st = D_(src, dev)
    _call("ecd_codec_cols_taps", st.data_ptr(), C, (ctypes.c_int * len(offs))(*offs), len(offs),
          out.data_ptr(), B, T, C, rep, 0, row0, n)
    x = src.reshape(B, T // rep, C)
    want = np.zeros((B * T, len(offs) * C), np.float16)
    for b in range(B):
        for t in range(T):
            for j, o in enumerate(offs):
                if 0 <= t + o < T:
                    want[b * T + t, j * C:(j + 1) * C] = x[b, (t + o) // rep]
    _exact(N_(out), want[row0:row0 + n], f"cols taps {offs} rep {rep}")


@pytest.mark.parametrize("offs,C,N,ypad,prelu,rep", [((-18, -15, -12, -9, -6, -3, 0), 64, 64, 60, True, 1),
                                                      ((0, -1), 128, 192, 20, False, 1),
                                                      ((-6, -5, -4, -3, -2, -1, 0), 128, 1, -1, False, 1),
                                                      ((0,), 64, 64, 60, True, 1),
                                                      ((-2, -1, 0, 1, 2), 64, 96, 60, False, 1),
                                                      ((-6, -5, -4, -3, -2, -1, 0), 64, 64, 60, True, 2),
                                                      ((-3, -1, 0, 1, 3), 64, 96, -1, False, 2)])
def test_gemm_f16_conv_implicit_taps(dev, offs, C, N, ypad, prelu, rep):
    """A convolution over implicit tap columns of a zero-padded activation equals the GEMM over
    materialised columns bit for bit (same accumulation order), with padded or plain output and
    the residual read through the same row map; centred taps read the next sequence's pad rows
    and, after the last sequence, the trailing zero rows; rep = 2 reads a source upsampled 2x by
    row repeat (the PostProcessor), odd taps from the second set of lane rows."""
    import ctypes
    import torch
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd.kernels import pack_f16, stream_ptr
    B, T, P = 2, 204 if rep == 2 else 203, 60
    Tin = T // rep
    k = len(offs)
    K = k * C
    g = rng(840 + C + N + rep)
    x = randn16(841 + rep, B, Tin, C)
    xp = np.zeros((B * (P + Tin) + 8, C), np.float16)
    for b in range(B):
        xp[b * (P + Tin) + P:b * (P + Tin) + P + Tin] = x[b]
    w = f16(g.standard_normal((N, K)) * 0.05)
    bias = (g.standard_normal(N) * 0.1).astype(np.float32)
    wp, bt = pack_f16(D_(w, dev)), D_(bias, dev)
    st = stream_ptr(dev)
    off = (ctypes.c_int * k)(*offs)
    xpt = D_(xp, dev)
    cols = torch.empty(B * T, K, dtype=torch.float16, device=dev)
    _ffi.call("ecd_codec_cols_taps", xpt.data_ptr(), C, off, k, cols.data_ptr(), B, T, C, rep, P, 0,
              B * T, st)
    yrows = B * (ypad + T) + 8 if ypad >= 0 else B * T
    r = randn16(842, yrows, N)
    y_ref = D_(r, dev)
    y_imp = D_(r, dev)
    epi = 2 if prelu else 0
    _ffi.call("ecd_gemm_f16p_conv", cols.data_ptr(), K, wp.data_ptr(), bt.data_ptr(), 0.25,
              y_ref.data_ptr(), N, y_ref.data_ptr(), N, B * T, N, K, T, 0, ypad, None, 0, 1, epi, st)
    _ffi.call("ecd_gemm_f16p_conv", xpt.data_ptr(), C, wp.data_ptr(), bt.data_ptr(), 0.25,
              y_imp.data_ptr(), N, y_imp.data_ptr(), N, B * T, N, K, T, P, ypad, off, k, rep, epi, st)
    _exact(N_(y_imp), N_(y_ref), f"implicit taps {offs} C={C} N={N} ypad={ypad} rep={rep}")
    # every block tile (sizes, LDS stages, pipelined or not) reads the implicit taps identically
    for cfg in range(1, 17):
        y_cfg = D_(r, dev)
        _ffi.call("ecd_gemm_f16p_conv_tuned", xpt.data_ptr(), C, wp.data_ptr(), bt.data_ptr(), 0.25,
                  y_cfg.data_ptr(), N, y_cfg.data_ptr(), N, B * T, N, K, T, P, ypad, off, k, rep,
                  epi, cfg, st)
        _exact(N_(y_cfg), N_(y_ref), f"implicit taps {offs} rep {rep}, tile cfg {cfg}")


def test_codec_weight_norm_and_latent_split(dev):
    import torch
    g = rng(810)
    v = f16(g.standard_normal((24, 16, 7)))
    gg = f16(np.abs(g.standard_normal((24, 1, 1))) + 0.5)
    w = torch.empty(24, 16, 7, dtype=torch.float16, device=dev)
    vt, gt = D_(v, dev), D_(gg, dev)
    _call("ecd_codec_weight_norm", vt.data_ptr(), gt.data_ptr(), w.data_ptr(), 24, 16 * 7)
    assert_close16(N_(w), OC.weight_norm(v, gg), what="weight norm")
    lat = randn16(811, 1, 50, 128, std=2.0)
    lat[0, 0, :4] = f16(np.array([0.5, 1.5, -0.5, 2.5]) / 9)     # ties of round(9 x)
    out = torch.empty(2, 50, 64, dtype=torch.float16, device=dev)
    lt = D_(lat, dev)
    _call("ecd_codec_latent_split", lt.data_ptr(), out.data_ptr(), 50, 2, 64)
    _exact(N_(out), OC.round9(lat[0].reshape(50, 2, 64).transpose(1, 0, 2)), "latent split")


def test_gemm_f16_prelu(dev):
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd.kernels import pack_f16, stream_ptr
    import torch
    M, N, K = 300, 192, 448
    x = randn16(820, M, K)
    w = f16(rng(821).standard_normal((N, K)) * 0.05)
    b = (rng(822).standard_normal(N) * 0.1).astype(np.float32)
    r = randn16(823, M, N)
    xt, rt, bt = D_(x, dev), D_(r, dev), D_(b, dev)
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    _ffi.call("ecd_gemm_f16p_prelu", xt.data_ptr(), K, pack_f16(D_(w, dev)).data_ptr(), bt.data_ptr(),
              0.25, rt.data_ptr(), N, y.data_ptr(), N, M, N, K, stream_ptr(dev))
    want = f16(f32_(x) @ f32_(w).T + b)
    want = f16(f32_(OC.prelu(want, 0.25)) + f32_(r))
    assert_close16(N_(y), want, what="gemm prelu")


def f32_(a):
    return np.asarray(a, np.float32)


def test_codec_scalar_decoder_real_widths(dev):
    """ScalarModel.decode at the real configuration (latent 256 split into 2 groups of 128,
    channels 2048 -> 1024 -> ... -> 64, upsampling 5, 4, 4, 4, 3, post 2x: x1920) over a short
    window of 6 latent frames, against the oracle."""
    import torch
    from estudiocanciones_amd.codec import ScalarDecoder
    cfg = dict(latent_hidden_dim=128, init_channel=64, upsample_factors=(5, 4, 4, 4, 3))
    p = OC.random_decoder_weights(cfg, seed=850)
    dec = ScalarDecoder({k: torch.from_numpy(np.asarray(v)) for k, v in p.items()}, device=dev)
    T = 6
    lat = randn16(851, 1, T, 256)
    got = dec.decode(D_(lat, dev))
    want = OC.scalar_decode(p, cfg, lat)
    assert got.shape == want.shape == (2, T * 1920, 1)
    _close_model(N_(got), want, "scalar decoder, real widths")


@pytest.mark.parametrize("T,rows_bytes", [(12, 64 * 1024), (37, 64 * 1024), (300, 4096)])
def test_codec_scalar_decoder(dev, T, rows_bytes):
    """ScalarModel.decode at a small configuration (latent 64 x 2 channel groups, channels
    256 -> 128 -> 64, upsampling 2 and 3, post 2x) against the oracle.  The first conv's tap
    columns are cut into row chunks of at least 256 rows; at T = 300 with a small chunk budget
    each sequence's 300 rows run as two chunks, so a chunk starting past row 0 runs too."""
    import torch
    from estudiocanciones_amd.codec import ScalarDecoder
    p = OC.random_decoder_weights(DEC, seed=830)
    dec = ScalarDecoder({k: torch.from_numpy(np.asarray(v)) for k, v in p.items()},
                        latent_hidden_dim=64, init_channel=64, upsample_factors=(2, 3),
                        upsample_kernel_sizes=(4, 6), device=dev)
    dec.ROWS_BYTES = rows_bytes
    lat = randn16(831 + T, 1, T, 128)
    got = dec.decode(D_(lat, dev))
    want = OC.scalar_decode(p, DEC, lat)
    assert got.shape == want.shape == (2, T * 12, 1)
    _close_model(N_(got), want, f"scalar decoder T={T}")


def test_codec_scalar_decoder_reuse(dev):
    """One decoder over windows of changing length (20, 9, 20 frames): its padded buffers are
    rebuilt per shape, and every output equals a fresh decoder's bit for bit (the padding rows
    stay zero across calls)."""
    import torch
    from estudiocanciones_amd.codec import ScalarDecoder
    p = OC.random_decoder_weights(DEC, seed=840)
    sd = {k: torch.from_numpy(np.asarray(v)) for k, v in p.items()}
    cfg = dict(latent_hidden_dim=64, init_channel=64, upsample_factors=(2, 3),
               upsample_kernel_sizes=(4, 6), device=dev)
    dec = ScalarDecoder(sd, **cfg)
    for i, T in enumerate((20, 9, 20)):
        lat = D_(randn16(841 + i, 1, T, 128), dev)
        got = N_(dec.decode(lat))
        want = N_(ScalarDecoder(sd, **cfg).decode(lat))
        _exact(got, want, f"reused decoder, window {i} (T={T})")


def test_codec_detokenize_audio(dev):
    """codes -> waveform: three 7.44 s windows (latents on the GPU), each decoded by the waveform
    decoder (small configuration: one channel group, 12 samples per latent frame, so
    sample_rate 300 stands in for 48 kHz) and crossfaded over the overlap, against the oracle."""
    import torch
    from estudiocanciones_amd.codec import ScalarDecoder, detokenize
    p_est = OC.random_weights(TINY, seed=60)
    p_fm = OC.random_vq_weights(8, 64, 32, 64, seed=61)
    dcfg = dict(latent_hidden_dim=64, init_channel=64, upsample_factors=(2, 3))
    p_dec = OC.random_decoder_weights(dcfg, seed=62)
    est = _estimator(dev, p_est, TINY)
    emb = _code_embedding(dev, p_fm)
    dec = ScalarDecoder({k: torch.from_numpy(np.asarray(v)) for k, v in p_dec.items()},
                        latent_hidden_dim=64, init_channel=64, upsample_factors=(2, 3),
                        upsample_kernel_sizes=(4, 6), device=dev)
    codes = rng(63).integers(0, 64, (8, 250))
    noises = [randn16(64 + w, 1, 186, 64) for w in range(3)]
    it = iter(noises)
    got = detokenize(emb, est, dec, D_(codes, dev), 7.44, 2, 1.25, 300,
                     randn=lambda shape: D_(next(it), dev))
    want = OC.detokenize(p_fm, p_est, TINY, p_dec, dcfg, codes, 7.44, 2, 1.25, 300, noises)
    assert got.shape == want.shape == (1, 6000)   # one 64-wide channel group
    _close_model(got, want, "detokenize audio")
