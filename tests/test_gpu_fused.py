"""Fused packed-weight GEMVs against the oracle's unfused composition of the reference kernels:
rms -> gemv, rms -> qkv -> rope/cache, rms -> w1|w3 -> silu*mul, embedding -> projection."""
import math

import numpy as np
import pytest

from helpers import assert_close16, randn16, rng
from oracle import kernels as OK
from oracle.numerics import bf16_to_f32, f16
from oracle.quant import q8_rows
from oracle.rope import rope_cache

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def N_(t):
    return t.detach().cpu().numpy()


def qweights(seed, n, k, std=0.02):
    q, sb = q8_rows(rng(seed).standard_normal((n, k), dtype=np.float32) * np.float32(std))
    return q, f16(bf16_to_f32(sb))


@pytest.mark.parametrize("M,N,K,res", [(8, 16384, 3072, False), (8, 3072, 8192, True),
                                       (16, 1024, 3072, False), (8, 8197, 1024, False),
                                       (1, 64, 64, True), (40, 300, 256, True)])
def test_gemv_packed(dev, M, N, K, res):
    from estudiocanciones_amd.kernels import gemv_packed, pack_i8
    q, s = qweights(1, N, K)
    x = randn16(2, M, K)
    r = randn16(3, M, N) if res else None
    wp = pack_i8(T(q, dev))
    y = gemv_packed(T(x, dev), wp, T(s, dev), N, K, T(r, dev) if res else None)
    assert_close16(N_(y), OK.gemv_i8(x, q, s, r), what=f"packed gemv M={M} N={N} K={K}")


def test_gemv_packed_every_tile_config_and_chunk_count(dev):
    """Every (tiles per block, waves per block) pair over K values that give each wave 0, 1, 2,
    3-4, 5-8 and more than 8 chunks (the register-x kernel's bounds and the LDS-tile fallback),
    both numerics (M <= 16 and M > 16) and a row count that is not a multiple of 16."""
    import torch
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd.kernels import pack_i8, stream_ptr
    for K in (64, 192, 1024, 4096, 8192, 9216):
        for N in (100, 1000):
            q, s = qweights(K + N, N, K)
            wp = pack_i8(T(q, dev))
            st = T(s, dev)
            for M in (8, 20):
                x = randn16(K + M, M, K)
                r = randn16(K + M + 1, M, N)
                want = OK.gemv_i8(x, q, s, r)
                xt, rt = T(x, dev), T(r, dev)
                for nt, kw in ((1, 8), (1, 16), (2, 8), (2, 16), (4, 8), (4, 16)):
                    y = torch.empty(M, N, dtype=torch.float16, device=dev)
                    _ffi.call("ecd_gemv_i8p", xt.data_ptr(), K, wp.data_ptr(), st.data_ptr(),
                              rt.data_ptr(), N, y.data_ptr(), N, M, N, K, int(M > 16), nt, kw,
                              stream_ptr(dev))
                    assert_close16(N_(y), want, what=f"M={M} N={N} K={K} nt={nt} kw={kw}")


@pytest.mark.parametrize("M,N,K", [(8, 8197, 1024), (8, 8197, 512), (16, 9000, 64), (20, 8197, 1024),
                                   (8, 300, 1024), (8, 8197, 3072), (8, 11269, 3072),
                                   (8, 12300, 1024)])
def test_rms_gemv_packed_shapes(dev, M, N, K):
    """RMS prologue on the shapes that take the register-x kernel (8 waves, <= 2 chunks per
    wave) and on those that stay on the LDS tile; 513-767 tiles run 3 tiles per workgroup (the
    codebook heads, and codebook 0's head with the decoder projection)."""
    from estudiocanciones_amd.kernels import pack_i8, rms_gemv_packed
    q, s = qweights(7 + K, N, K)
    x = randn16(8 + K, M, K, std=2.0)
    nw = (1 + 0.02 * rng(9).standard_normal(K)).astype(np.float16)
    y = rms_gemv_packed(T(x, dev), T(nw, dev), pack_i8(T(q, dev)), T(s, dev), N, K)
    assert_close16(N_(y), OK.gemv_i8(OK.rms(x, nw), q, s), what=f"rms+gemv M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K,ks,res", [(8, 1024, 8192, 4, True), (16, 1024, 8192, 4, False),
                                          (8, 100, 4096, 2, True), (20, 300, 2048, 8, True),
                                          (3, 64, 1024, 16, False)])
def test_gemv_packed_splitk(dev, M, N, K, ks, res):
    """K split over ks workgroups (fp32 partials, in-order reduction) vs the oracle; M > 16 keeps
    the dense numerics."""
    from estudiocanciones_amd.kernels import gemv_packed_splitk, pack_i8
    q, s = qweights(50 + ks, N, K)
    x = randn16(51 + M, M, K)
    r = randn16(52 + M, M, N) if res else None
    y = gemv_packed_splitk(T(x, dev), pack_i8(T(q, dev)), T(s, dev), N, K, ks, T(r, dev) if res else None)
    assert_close16(N_(y), OK.gemv_i8(x, q, s, r), what=f"splitk M={M} N={N} K={K} ks={ks}")


@pytest.mark.parametrize("M,N,K,res", [(17, 100, 64, True), (128, 1000, 1024, False),
                                       (300, 3072, 1024, True), (512, 1536, 3072, False),
                                       (129, 257, 192, True)])
def test_gemm_packed_dense_numerics(dev, M, N, K, res):
    """The prompt-pass GEMM: the dense numerics (fp16(q * s) weights, fp32 sums) of int8_mm for
    M > 16, ragged M and N, residual added in fp16."""
    from estudiocanciones_amd.kernels import gemm_packed, pack_i8
    q, s = qweights(30 + K, N, K)
    x = randn16(31 + M, M, K)
    r = randn16(32 + M, M, N) if res else None
    y = gemm_packed(T(x, dev), pack_i8(T(q, dev)), T(s, dev), N, K, T(r, dev) if res else None)
    want = OK.gemv_i8(x, q, s, r)  # M > 16: the oracle's dense numerics
    assert_close16(N_(y), want, what=f"gemm M={M} N={N} K={K}")


@pytest.mark.parametrize("M,F,K", [(96, 512, 256), (2048, 8192, 1024)])
def test_gemm_silu_packed(dev, M, F, K):
    """GEMM on row-interleaved w1|w3 with the SiLU * mul epilogue vs silu_mul(int8_mm(...))."""
    import torch
    from estudiocanciones_amd.kernels import gemm_silu_packed, pack_i8
    q, s = qweights(40 + F, 2 * F, K)
    x = randn16(41 + M, M, K, std=0.5)
    st = T(s, dev)
    sp = torch.stack([st[:F], st[F:]], 1).reshape(-1).contiguous()
    mm = gemm_silu_packed(T(x, dev), pack_i8(T(q, dev), True), sp, F, K)
    want = OK.silu_mul(OK.gemv_i8(x, q, s))
    assert_close16(N_(mm), want, what=f"gemm+silu M={M} F={F}")


def test_rms_gemv_packed(dev):
    from estudiocanciones_amd.kernels import pack_i8, rms_gemv_packed
    M, N, K = 8, 8197, 3072
    q, s = qweights(4, N, K)
    x = randn16(5, M, K, std=2.0)
    nw = (1 + 0.02 * rng(6).standard_normal(K)).astype(np.float16)
    y = rms_gemv_packed(T(x, dev), T(nw, dev), pack_i8(T(q, dev)), T(s, dev), N, K)
    assert_close16(N_(y), OK.gemv_i8(OK.rms(x, nw), q, s), what="rms+gemv")


@pytest.mark.parametrize("M,S,Hq,Hk,HD,D,L", [(8, 1, 24, 8, 128, 3072, 64), (16, 2, 8, 2, 128, 1024, 8),
                                              (16, 2, 8, 4, 384, 3072, 8), (24, 12, 2, 1, 128, 256, 32)])
def test_rms_qkv_rope(dev, M, S, Hq, Hk, HD, D, L):
    import torch
    from estudiocanciones_amd.kernels import pack_i8, rms_qkv_rope
    B = M // S
    Nq = (Hq + 2 * Hk) * HD
    q8, s = qweights(7, Nq, D)
    x = randn16(8, M, D, std=2.0)
    nw = (1 + 0.02 * rng(9).standard_normal(D)).astype(np.float16)
    if S == 1:
        pos = rng(10).integers(0, L, M).astype(np.int64)
    else:
        pos = np.tile(np.arange(S, dtype=np.int64), B)
    rope = rope_cache(HD, L)
    kc0 = randn16(11, B, Hk, L, HD)
    vc0 = randn16(12, B, Hk, L, HD)
    kc, vc = kc0.copy(), vc0.copy()
    qkv = OK.gemv_i8(OK.rms(x, nw), q8, s)
    q_want = OK.rope_kv_write(qkv, rope, pos, kc, vc, S, Hq, Hk, HD)
    kct, vct = T(kc0, dev), T(vc0, dev)
    q = torch.empty(M, Hq * HD, dtype=torch.float16, device=dev)
    rms_qkv_rope(T(x, dev), T(nw, dev), pack_i8(T(q8, dev)), T(s, dev), T(rope, dev), T(pos, dev), q,
                 kct, vct, S, Hq, Hk, L, HD)
    assert_close16(N_(q), q_want, what="fused q")
    assert_close16(N_(kct), kc, what="fused k cache")
    assert_close16(N_(vct), vc, what="fused v cache")


@pytest.mark.parametrize("M,S,Hq,Hk,HD,D,L,bad", [
    (300, 1, 24, 8, 128, 3072, 64, False),   # the backbone's q|k|v, ragged rows, one row per cache
    (256, 128, 8, 2, 128, 1024, 160, False),  # two prompts of 128 positions sharing their caches
    (64, 32, 8, 4, 384, 3072, 40, False),    # head_dim 384
    (96, 1, 2, 1, 64, 256, 64, True),        # positions outside [0, L): no slot, q at the clamp
])
def test_gemm_rope_packed(dev, M, S, Hq, Hk, HD, D, L, bad):
    """The prompt pass's q|k|v GEMM with RoPE and the cache write in its epilogue: bit-equal to
    the GEMM followed by the RoPE kernel (q and both caches, untouched slots included), and
    within the fp16 bar of the oracle's dense GEMM + rope_kv_write."""
    import torch
    from estudiocanciones_amd.kernels import (_rope_cache, gemm_packed, gemm_rope_packed,
                                              next_power_of_2, pack_i8)
    B = M // S
    Nq = (Hq + 2 * Hk) * HD
    q8, s = qweights(50 + HD, Nq, D)
    x = randn16(51 + M, M, D, std=0.5)
    if S == 1:
        pos = rng(52).integers(0, L, M).astype(np.int64)
    else:
        pos = np.tile(np.arange(S, dtype=np.int64), B)
    if bad:
        pos[::7] = -1
        pos[3::7] = L + 5
    rope = rope_cache(HD, L)
    kc0 = randn16(53, B, Hk, L, HD)
    vc0 = randn16(54, B, Hk, L, HD)
    wp, st, rt, pt = pack_i8(T(q8, dev)), T(s, dev), T(rope, dev), T(pos, dev)
    kc, vc = T(kc0, dev), T(vc0, dev)
    q = torch.empty(M, Hq * HD, dtype=torch.float16, device=dev)
    gemm_rope_packed(T(x, dev), wp, st, rt, pt, q, kc, vc, S, Hq, Hk, L, HD, D)
    kc2, vc2 = T(kc0, dev), T(vc0, dev)
    q2 = torch.empty_like(q)
    qkv = gemm_packed(T(x, dev), wp, st, Nq, D)
    _rope_cache[(M, Hq + Hk)](qkv, rt, pt, q2, kc2, vc2, S, Hq, Hk, L, HD=HD,
                              HALF=next_power_of_2(HD // 2))
    assert torch.equal(q, q2), "q differs from GEMM + RoPE kernel"
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2), "cache differs from GEMM + RoPE kernel"
    if not bad:
        kw, vw = kc0.copy(), vc0.copy()
        q_want = OK.rope_kv_write(OK.gemv_i8(x, q8, s), rope, pos, kw, vw, S, Hq, Hk, HD)
        assert_close16(N_(q), q_want, what="gemm+rope q")
        assert_close16(N_(kc), kw, what="gemm+rope k cache")
        assert_close16(N_(vc), vw, what="gemm+rope v cache")


@pytest.mark.parametrize("M,D,F", [(8, 3072, 8192), (16, 1024, 8192), (40, 256, 512)])
def test_rms_w13_silu(dev, M, D, F):
    import torch
    from estudiocanciones_amd.kernels import pack_i8, rms_w13_silu
    q8, s = qweights(13, 2 * F, D)
    x = randn16(14, M, D, std=2.0)
    nw = (1 + 0.02 * rng(15).standard_normal(D)).astype(np.float16)
    want = OK.silu_mul(OK.gemv_i8(OK.rms(x, nw), q8, s))
    st = T(s, dev)
    s_il = torch.stack([st[:F], st[F:]], 1).reshape(-1).contiguous()
    mm = rms_w13_silu(T(x, dev), T(nw, dev), pack_i8(T(q8, dev), interleave=True), s_il, F)
    assert_close16(N_(mm), want, what="fused w13+silu")


@pytest.mark.parametrize("B,even", [(8, True), (8, False), (4, False)])
def test_embed_gemv(dev, B, even):
    from estudiocanciones_amd.kernels import embed_gemv_packed, pack_i8
    V, D, Nout, cb = 8197, 3072, 1024, 3
    tq, ts = qweights(16, 8 * V, D, std=1.0)
    wq, ws = qweights(17, Nout, D)
    tok = rng(18).integers(0, V, (B, 8)).astype(np.int64)
    tokc = tok[:, cb:cb + 1]
    e = OK.embed_rows(tq, ts, tokc[:, 0] + cb * V)
    ev = randn16(19, B, D) if even else None
    x = np.stack([ev, e], 1).reshape(2 * B, D) if even else e
    want = OK.gemv_i8(x, wq, ws)
    tt = T(tok, dev)[:, cb:cb + 1]                      # strided token column, like samples[:, i]
    y = embed_gemv_packed(tt, T(tq, dev), T(ts, dev), cb, V, pack_i8(T(wq, dev)), T(ws, dev), Nout,
                          even=T(ev, dev) if even else None)
    assert_close16(N_(y), want, what="embed+projection")


def test_fused_layer_c0(dev):
    """One 3B backbone layer (B=2, L=1024, pos 1023) through the fused kernels vs the oracle."""
    import torch
    from estudiocanciones_amd.engine import Linear, Stack
    from oracle.model import OLinear, OStack
    from oracle.numerics import bf16_bits
    from estudiocanciones_amd.quant import weight_shapes
    cfg = dict(layers=1, heads=24, kv_heads=8, max_seq=8192, dim=3072, ffn=8192)
    lin, dense = weight_shapes(cfg, dict(layers=0, heads=2, kv_heads=1, dim=256))
    g = rng(20)
    wn = {}
    for name, (n, k) in lin.items():
        if name.startswith("backbone."):
            wn[name + ".q8"], wn[name + ".s8"] = q8_rows(g.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    for name, shp in dense.items():
        if name.startswith("backbone."):
            wn[name] = bf16_bits(1.0 + 0.02 * g.standard_normal(shp, dtype=np.float32))

    def op(name, norm=False):
        if norm:
            return f16(bf16_to_f32(wn[name]))
        return OLinear(wn[name + ".q8"], f16(bf16_to_f32(wn[name + ".s8"])))

    B, L = 2, 1024
    ost = OStack(op, "backbone", cfg)
    ost.alloc(B, L)
    kc, vc = randn16(21, B, 8, L, 128), randn16(22, B, 8, L, 128)
    ost.blocks[0].kc[:], ost.blocks[0].vc[:] = kc, vc
    x = randn16(23, B, 3072)
    pos = np.full(B, L - 1, np.int64)
    want = ost.decode(x, pos, 1)

    def gp(name, norm=False):
        if norm:
            return T(f16(bf16_to_f32(wn[name])), dev)
        return Linear(q8=T(wn[name + ".q8"], dev), s8=T(f16(bf16_to_f32(wn[name + ".s8"])), dev))

    st = Stack(gp, "backbone", cfg)
    for b in st.blocks:
        b.qkv.pack(), b.o.pack(), b.w13.pack(interleave=True), b.w2.pack()
    st.alloc(B, L, dev, torch.float16)
    st.blocks[0].kc.copy_(T(kc, dev))
    st.blocks[0].vc.copy_(T(vc, dev))
    got = st.decode(T(x, dev), T(pos, dev), 1)
    assert_close16(N_(got), want, what="fused backbone layer")
    assert_close16(N_(st.blocks[0].kc), ost.blocks[0].kc, what="fused layer k cache")
