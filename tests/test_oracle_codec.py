"""Pins of the codec estimator / Euler oracle (oracle/codec.py) on the CPU.

Each check is independent of the oracle's own formulas: closed forms, invariants, special
cases, and float64 library routines (torch's conv1d, layer_norm, scaled_dot_product_attention,
linear) composed along the reference's module structure.  A dropped term, a wrong sign,
a swapped modulation chunk, a flipped convolution or a transposed head layout fails one."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import codec as OC
from oracle.numerics import f16

TINY = dict(heads=2, head_dim=64, in_channels=192, out_channels=64, layers=2, layers_2=1)


def test_mlp_hidden_widths():
    # 4 * dim * 2 / 3 rounded up to 256 (transformer.py:170-172) at the real widths
    assert OC.mlp_hidden(1536) == 4096
    assert OC.mlp_hidden(3072) == 8192
    assert OC.mlp_hidden(128) == 512          # 341 -> 512
    assert OC.mlp_hidden(256) == 768          # 682 -> 768


@pytest.mark.parametrize("HD", [64, 128])
def test_rope_table_closed_form(HD):
    sin, cos = OC.rope_table(744, HD)
    assert sin.shape == cos.shape == (744, HD // 2)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    th = 10000.0 ** (-np.arange(0, HD, 2) / HD)
    # small positions: only the fp16 roundings of theta and t * theta separate the table from
    # the exact rotation angle t * theta
    t = np.arange(1, 9)[:, None]
    np.testing.assert_allclose(cos[1:9], np.cos(t * th), atol=6e-3)
    np.testing.assert_allclose(sin[1:9], np.sin(t * th), atol=6e-3)
    np.testing.assert_allclose(sin.astype(np.float64) ** 2 + cos.astype(np.float64) ** 2, 1,
                               atol=2e-3)


def test_apply_rope_is_complex_rotation_of_interleaved_pairs():
    g = np.random.default_rng(1)
    x = f16(g.standard_normal((2, 3, 40, 64)))
    sin, cos = OC.rope_table(40, 64)
    got = OC.apply_rope_vec(x, sin, cos).astype(np.float64)
    z = (x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2]) * (cos + 1j * sin.astype(np.float64))
    np.testing.assert_allclose(got[..., 0::2], z.real, atol=8e-3, rtol=4e-3)
    np.testing.assert_allclose(got[..., 1::2], z.imag, atol=8e-3, rtol=4e-3)
    # position 0 is the identity
    assert np.array_equal(OC.apply_rope_vec(x, sin, cos)[:, :, 0], x[:, :, 0])


def test_rms_norm_closed_form():
    g = np.random.default_rng(2)
    x = f16(g.standard_normal((5, 256)) * 3)
    w = f16(1 + 0.1 * g.standard_normal(256))
    want = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    want = want * w
    np.testing.assert_allclose(OC.rms_norm(x, w), want, rtol=4e-3, atol=2e-3)
    # a constant row normalises to w * sign
    c = f16(np.full((1, 64), -2.5))
    np.testing.assert_allclose(OC.rms_norm(c, np.ones(64, np.float16)), -1.0, atol=1e-3)


def test_layer_norm_matches_library():
    g = np.random.default_rng(3)
    x = f16(g.standard_normal((6, 192)) * 2 + 0.7)
    want = F.layer_norm(torch.from_numpy(x.astype(np.float64)), (192,), eps=1e-6).numpy()
    np.testing.assert_allclose(OC.layer_norm(x), want, atol=2e-3, rtol=2e-3)


def test_modulate_special_cases():
    g = np.random.default_rng(4)
    n = f16(g.standard_normal((3, 16)))
    sh = f16(g.standard_normal(16))
    # scale = -1 removes the normalised input: only the shift is left, exactly
    assert np.array_equal(OC.modulate(n, sh, f16(-np.ones(16))), np.broadcast_to(sh, (3, 16)))
    # scale = 0, shift = 0 is the identity
    assert np.array_equal(OC.modulate(n, np.zeros(16, np.float16), np.zeros(16, np.float16)), n)


def test_sdpa_matches_library_and_is_permutation_invariant():
    g = np.random.default_rng(5)
    q, k, v = (f16(g.standard_normal((2, 3, 33, 64))) for _ in range(3))
    t = lambda a: torch.from_numpy(a.astype(np.float64))
    want = F.scaled_dot_product_attention(t(q), t(k), t(v)).numpy()
    got = OC.sdpa(q, k, v)
    np.testing.assert_allclose(got, want, atol=2e-3, rtol=2e-3)
    perm = g.permutation(33)
    assert np.array_equal(OC.sdpa(q, k[:, :, perm], v[:, :, perm]), got)


def test_project_layer_matches_conv1d():
    g = np.random.default_rng(6)
    p = {"c.ffn_1.weight": f16(g.standard_normal((48, 40, 3)) / 8),
         "c.ffn_1.bias": f16(g.standard_normal(48) * 0.1),
         "c.ffn_2.weight": f16(g.standard_normal((48, 48)) / 7),
         "c.ffn_2.bias": f16(g.standard_normal(48) * 0.1)}
    x = f16(g.standard_normal((2, 21, 40)))
    t = lambda a: torch.from_numpy(np.asarray(a).astype(np.float64))
    y = F.conv1d(t(x).transpose(1, 2), t(p["c.ffn_1.weight"]), t(p["c.ffn_1.bias"]),
                 padding=1).transpose(1, 2) * 3 ** -0.5
    want = F.linear(y, t(p["c.ffn_2.weight"]), t(p["c.ffn_2.bias"])).numpy()
    np.testing.assert_allclose(OC.project_layer(p, "c.", x), want, atol=6e-3, rtol=6e-3)


def test_timestep_sinusoid_closed_form():
    e = OC.timestep_sinusoid(np.array([0.0, 0.3, 1.0], np.float32))
    assert e.shape == (3, 512)
    assert np.all(e[0, :256] == 1) and np.all(e[0, 256:] == 0)
    fr = 10000.0 ** (-np.arange(256) / 256)
    np.testing.assert_allclose(e[1, :256], np.cos(0.3 * fr * 1000), atol=3e-3)
    np.testing.assert_allclose(e[2, 256:], np.sin(fr * 1000), atol=3e-3)


def test_t_span_is_uniform_grid():
    ts = OC.t_span(10)
    assert ts.dtype == np.float32 and ts[0] == 0 and ts[-1] == 1
    np.testing.assert_allclose(ts, np.linspace(0, 1, 11), atol=1e-7)


@pytest.mark.parametrize("g", [1.0, 1.25])
def test_solve_euler_constant_velocity(g):
    """A velocity field independent of x integrates to x0 + (u + g (c - u)) * 1; with zero
    velocity the in-context rows end at the blend of the last step's time."""
    rng = np.random.default_rng(7)
    B, T, C, L = 1, 12, 8, 4
    x0 = f16(rng.standard_normal((B, T, C)))
    ic = f16(rng.standard_normal((B, T, C)))
    mu = f16(rng.standard_normal((B, T, 16)))
    u = f16(rng.standard_normal((B, T, C)) * 0.5)
    c = f16(rng.standard_normal((B, T, C)) * 0.5)

    def est(inp, t):
        assert inp.shape[-1] == 2 * C + 16 and len(t) == inp.shape[0]
        if g > 1:
            assert np.all(inp[:B, :, 2 * C:] == 0)          # unconditional half: mu zeroed
            assert np.array_equal(inp[B:, :, 2 * C:], mu)
            return np.concatenate([u, c], 0)
        return c

    x = OC.solve_euler(est, x0, ic, 0, OC.t_span(10), mu, g)
    v = (u + g * (c.astype(np.float64) - u)) if g > 1 else c.astype(np.float64)
    np.testing.assert_allclose(x, x0 + v, atol=1.5e-2)
    z = OC.solve_euler(lambda inp, t: np.zeros((inp.shape[0], T, C), np.float16), x0, ic, L,
                       OC.t_span(10), mu, g)
    assert np.array_equal(z[:, L:], x0[:, L:])
    tl = 0.9
    np.testing.assert_allclose(z[:, :L], (1 - tl) * x0[:, :L] + tl * ic[:, :L], atol=4e-3)


# ---------------------------------------------------------------- composition in float64
def _torch_estimator(p, cfg, hidden, t):
    """The reference's module structure evaluated with float64 torch library calls."""
    T_ = lambda a: torch.from_numpy(np.asarray(a).astype(np.float64))
    H, HD = cfg["heads"], cfg["head_dim"]

    def rms(x, w):
        return T_(w) * x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)

    def rope(x):                                         # x [B, H, T, hd], interleaved pairs
        hd, n = x.shape[-1], x.shape[-2]
        th = 10000.0 ** (-torch.arange(0, hd, 2, dtype=torch.float64) / hd)
        ang = torch.arange(n, dtype=torch.float64)[:, None] * th
        z = torch.view_as_complex(x.reshape(*x.shape[:-1], hd // 2, 2).contiguous())
        return torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)).reshape(x.shape)

    def attn(pre, x, hd):
        B, n, D = x.shape
        sh = lambda a: a.view(B, n, H, hd).transpose(1, 2)
        q = rope(sh(F.linear(x, T_(p[pre + "q_proj.weight"]))))
        k = rope(sh(F.linear(x, T_(p[pre + "k_proj.weight"]))))
        v = sh(F.linear(x, T_(p[pre + "v_proj.weight"])))
        o = F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(B, n, D)
        return F.linear(o, T_(p[pre + "o_proj.weight"]))

    def block(pre, x, tmod, hd):
        B, _, D = x.shape
        m = (T_(p[pre + "scale_shift_table"])[None] + tmod.reshape(B, 6, D)).chunk(6, 1)
        n = rms(x, p[pre + "attn_norm.weight"]) * (1 + m[1]) + m[0]
        x = x + m[2] * attn(pre + "attn.", n, hd)
        n = rms(x, p[pre + "mlp_norm.weight"]) * (1 + m[4]) + m[3]
        h = F.silu(F.linear(n, T_(p[pre + "mlp.gate.weight"]))) * F.linear(n, T_(p[pre + "mlp.up.weight"]))
        return x + m[5] * F.linear(h, T_(p[pre + "mlp.down.weight"]))

    def proj(pre, x):
        y = F.conv1d(x.transpose(1, 2), T_(p[pre + "ffn_1.weight"]), T_(p[pre + "ffn_1.bias"]),
                     padding=1).transpose(1, 2) * 3 ** -0.5
        return F.linear(y, T_(p[pre + "ffn_2.weight"]), T_(p[pre + "ffn_2.bias"]))

    def ada(pre, tt):
        half = torch.arange(256, dtype=torch.float64)
        a = tt[:, None] * torch.exp(-math.log(10000) * half / 256)[None] * 1000
        e = torch.cat([torch.cos(a), torch.sin(a)], -1)
        te = pre + "emb.timestep_embedder."
        e = F.linear(F.silu(F.linear(e, T_(p[te + "linear_1.weight"]), T_(p[te + "linear_1.bias"]))),
                     T_(p[te + "linear_2.weight"]), T_(p[te + "linear_2.bias"]))
        return F.linear(F.silu(e), T_(p[pre + "linear.weight"]), T_(p[pre + "linear.bias"])), e

    def fin(x, table, emb):
        sh, sc = (T_(table)[None] + emb[:, None]).chunk(2, 1)
        return F.layer_norm(x, (x.shape[-1],), eps=1e-6) * (1 + sc) + sh

    hs = T_(hidden)
    tt = T_(t)
    s = proj("proj_in.", hs)
    tm, e = ada("adaln_single.", tt)
    for i in range(cfg["layers"]):
        s = block(f"transformer_blocks.{i}.", s, tm, HD)
    s = fin(s, p["scale_shift_table"], e)
    x = proj("connection_proj.", torch.cat([hs, s], -1))
    tm2, e2 = ada("adaln_single_2.", tt)
    for i in range(cfg["layers_2"]):
        x = block(f"transformer_blocks_2.{i}.", x, tm2, 2 * HD)
    x = fin(x, p["scale_shift_table_2"], e2)
    return proj("proj_out.", x).numpy()


def test_estimator_matches_float64_library_composition():
    p = OC.random_weights(TINY, seed=11)
    g = np.random.default_rng(12)
    hidden = f16(g.standard_normal((2, 24, TINY["in_channels"])))
    t = np.array([0.3, 0.3], np.float32)
    got = OC.estimator(p, TINY, hidden, t).astype(np.float64)
    want = _torch_estimator(p, TINY, hidden, t)
    assert got.shape == want.shape == (2, 24, TINY["out_channels"])
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 2e-2, err
    assert np.corrcoef(got.ravel(), want.ravel())[0, 1] > 0.9999


def test_code_embedding_matches_library():
    """Per-quantizer F.embedding summed, the two linears and nearest 2x interpolation in float64
    torch; a -1 code (the library's padding) contributes nothing."""
    Q, V, Dc, dim = 8, 64, 32, 96
    p = OC.random_vq_weights(Q, V, Dc, dim, seed=31)
    g = np.random.default_rng(32)
    codes = g.integers(0, V, (2, Q, 13))
    codes[1, 3, 5] = -1
    got = OC.code_embedding(p, codes).astype(np.float64)
    t = lambda a: torch.from_numpy(np.asarray(a).astype(np.float64))
    ci = torch.from_numpy(codes)
    e = sum(F.embedding(ci[:, q].clamp(min=0), t(p[f"vq_embed.layers.{q}._codebook.embed"][0]))
            * (ci[:, q] >= 0)[..., None] for q in range(Q))
    h = F.linear(F.linear(e, t(p["vq_embed.project_out.weight"]), t(p["vq_embed.project_out.bias"])),
                 t(p["cond_feature_emb.weight"]), t(p["cond_feature_emb.bias"]))
    want = F.interpolate(h.permute(0, 2, 1), scale_factor=2, mode="nearest").permute(0, 2, 1).numpy()
    assert got.shape == (2, 26, dim)
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)
    # a -1 code is the same as a code whose codebook row is all zeros
    unused = next(c for c in range(V) if c not in set(codes[:, 3].ravel().tolist()))
    p0 = dict(p)
    book = p["vq_embed.layers.3._codebook.embed"].copy()
    book[0, unused] = 0
    p0["vq_embed.layers.3._codebook.embed"] = book
    codes0 = codes.copy()
    codes0[1, 3, 5] = unused
    assert np.array_equal(OC.code_embedding(p0, codes0), got.astype(np.float16))


# ---------------------------------------------------------------- waveform decoder
DEC = dict(latent_hidden_dim=64, init_channel=64, upsample_factors=(2, 3))


def test_decoder_pieces_match_library():
    g = np.random.default_rng(50)
    t = lambda a: torch.from_numpy(np.asarray(a).astype(np.float64))
    x = f16(g.standard_normal((2, 30, 16)))
    w = f16(g.standard_normal((24, 16, 7)) / 10)
    b = f16(g.standard_normal(24) * 0.1)
    for d, causal in ((1, True), (3, True), (1, False)):
        xc = t(x).transpose(1, 2)
        if causal:
            want = F.conv1d(F.pad(xc, (6 * d, 0)), t(w), t(b), dilation=d)
        else:
            want = F.conv1d(xc, t(w), t(b), padding=3 * d, dilation=d)
        np.testing.assert_allclose(OC.conv1d(x, w, b, d, causal), want.transpose(1, 2).numpy(),
                                   atol=1e-2, rtol=1e-2)
    wt = f16(g.standard_normal((16, 12, 6)) / 6)
    bt = f16(g.standard_normal(12) * 0.1)
    want = F.conv_transpose1d(t(x).transpose(1, 2), t(wt), t(bt), stride=3)[:, :, :-3]
    np.testing.assert_allclose(OC.conv_transpose_causal(x, wt, bt, 3),
                               want.transpose(1, 2).numpy(), atol=1e-2, rtol=1e-2)
    np.testing.assert_allclose(OC.prelu(x, 0.25), F.prelu(t(x), t([0.25])).numpy(), atol=1e-3)
    v = f16(g.standard_normal((12, 5, 3)))
    gg = f16(np.abs(g.standard_normal((12, 1, 1))) + 0.5)
    np.testing.assert_allclose(OC.weight_norm(v, gg), torch._weight_norm(t(v), t(gg), 0).numpy(),
                               atol=2e-3, rtol=2e-3)
    # round(9 x) / 9: a grid of ninths is a fixed point up to fp16 rounding, ties go to even
    q = f16(np.arange(-18, 19) / 9.0)
    np.testing.assert_allclose(OC.round9(q), q, atol=1e-3)
    assert OC.round9(f16([0.5 / 9]))[0] == 0 and OC.round9(f16([1.5 / 9]))[0] == f16(2 / 9)


def test_decoder_matches_library_composition():
    p = OC.random_decoder_weights(DEC, seed=51)
    lat = f16(np.random.default_rng(52).standard_normal((1, 12, 128)))
    got = OC.scalar_decode(p, DEC, lat).astype(np.float64)
    t = lambda a: torch.from_numpy(np.asarray(a).astype(np.float64))
    wn = lambda pre: torch._weight_norm(t(p[pre + "parametrizations.weight.original1"]),
                                        t(p[pre + "parametrizations.weight.original0"]), 0)
    x = t(lat).reshape(1, 12, 2, 64).permute(0, 2, 1, 3).reshape(2, 12, 64).transpose(1, 2)
    x = torch.round(9 * x) / 9
    x = F.conv1d(x, wn("decoder.0."), t(p["decoder.0.bias"]), padding=2)
    for i, s in enumerate(DEC["upsample_factors"]):
        pre = f"decoder.{1 + i}."
        x = F.conv_transpose1d(x, wn(pre + "up_conv.layer."), t(p[pre + "up_conv.layer.bias"]),
                               stride=s)[:, :, :-s]
        for u, d in enumerate((1, 3, 5, 7, 9)):
            q = f"{pre}convs.{u}."
            h = F.prelu(F.conv1d(F.pad(x, (6 * d, 0)), wn(q + "conv1."), t(p[q + "conv1.bias"]),
                                 dilation=d), t(p[q + "activation1.weight"]))
            h = F.prelu(F.conv1d(h, wn(q + "conv2."), t(p[q + "conv2.bias"])),
                        t(p[q + "activation2.weight"]))
            x = h + x
    n = 1 + len(DEC["upsample_factors"])
    x = x.transpose(1, 2).repeat(1, 1, 2).reshape(2, -1, 64).transpose(1, 2)
    x = F.prelu(F.conv1d(F.pad(x, (6, 0)), t(p[f"decoder.{n}.conv.weight"]),
                         t(p[f"decoder.{n}.conv.bias"])), t(p[f"decoder.{n}.activation.weight"]))
    x = F.conv1d(F.pad(x, (6, 0)), wn(f"decoder.{n + 1}."), t(p[f"decoder.{n + 1}.bias"]))
    want = x.transpose(1, 2).numpy()
    assert got.shape == want.shape == (2, 12 * 6 * 2, 1)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 3e-2 and np.corrcoef(got.ravel(), want.ravel())[0, 1] > 0.999, err
