"""Per-kernel parity of the gfx950 HIP kernels (through the C ABI) against the oracle.

Bars: int8 codes and bf16/fp16 scales bit-exact; fp16 kernel outputs within
max-abs 2e-3 or 1e-2 relative (|got - want| <= 2e-3 + 1e-2 |want|)."""
import math

import numpy as np
import pytest

from helpers import assert_close16, randn16, rng
from oracle import kernels as OK
from oracle.numerics import bf16_to_f32, f16
from oracle.quant import q8_rows as o_q8_rows
from oracle.rope import rope_cache as o_rope_cache

pytestmark = pytest.mark.gpu


def T(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def N(t):
    return t.detach().cpu().numpy()


# ---------------------------------------------------------------- quantiser
@pytest.mark.parametrize("shape", [(64, 3072), (7, 1000), (1, 1)])
def test_q8_rows_bit_exact(dev, shape):
    import torch
    from estudiocanciones_amd.quant import q8_rows
    g = rng(11)
    w = g.standard_normal(shape, dtype=np.float32) * np.float32(0.02)
    if shape[0] > 3:
        w[1] = 0.0                                   # all-zero row -> scale 1e-8/127
        w[2, :] = np.float32(127 * 0.5)              # exact ties at k + 0.5 after division
        w[2, 0] = np.float32(127)
    q, s = q8_rows(T(w, dev))
    qo, so = o_q8_rows(w)
    assert np.array_equal(N(q), qo)
    assert np.array_equal(N(s.view(torch.int16)).view(np.uint16), so)


def test_q8_rows_fp16_scale(dev):
    import torch
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd.kernels import stream_ptr
    w = rng(12).standard_normal((33, 256), dtype=np.float32) * np.float32(0.05)
    wt = T(w, dev)
    q = torch.empty(33, 256, dtype=torch.int8, device=dev)
    s16 = torch.empty(33, dtype=torch.float16, device=dev)
    _ffi.call("ecd_quantize_rows_i8", wt.data_ptr(), q.data_ptr(), None, s16.data_ptr(), 33, 256,
              stream_ptr(dev))
    qo, so = o_q8_rows(w)
    assert np.array_equal(N(q), qo)
    assert np.array_equal(N(s16), f16(bf16_to_f32(so)))


# ---------------------------------------------------------------- GEMV
GEMV_CASES = [
    # M, N, K, res
    (1, 64, 64, False),
    (2, 5120, 3072, False),
    (2, 3072, 3072, True),
    (4, 16384, 3072, False),
    (8, 3072, 8192, True),
    (8, 8197, 3072, False),
    (16, 1536, 1024, False),
    (16, 1024, 3072, False),
    (8, 8197, 1024, False),
    (3, 100, 200, True),        # K not a multiple of 64: generic kernel
    (5, 77, 128, False),
]


@pytest.mark.parametrize("M,Nn,K,res", GEMV_CASES)
def test_int8_mm_gemv(dev, M, Nn, K, res):
    from estudiocanciones_amd.kernels import int8_mm
    x = randn16(1, M, K)
    w = rng(2).standard_normal((Nn, K), dtype=np.float32) * np.float32(0.02)
    q, sb = o_q8_rows(w)
    s = f16(bf16_to_f32(sb))
    r = randn16(3, M, Nn) if res else None
    y = int8_mm(T(x, dev), T(q, dev), T(s, dev), T(r, dev) if res else None)
    assert_close16(N(y), OK.gemv_i8(x, q, s, r), what=f"gemv M={M} N={Nn} K={K}")


@pytest.mark.parametrize("M,Nn,K", [(40, 256, 512), (17, 1024, 3072), (64, 300, 256)])
def test_int8_mm_dense_numerics(dev, M, Nn, K):
    """M > 16 rows follow the reference's dequantise-then-GEMM rounding."""
    from estudiocanciones_amd.kernels import int8_mm
    x = randn16(4, M, K)
    w = rng(5).standard_normal((Nn, K), dtype=np.float32) * np.float32(0.02)
    q, sb = o_q8_rows(w)
    s = f16(bf16_to_f32(sb))
    r = randn16(6, M, Nn)
    y = int8_mm(T(x, dev), T(q, dev), T(s, dev), T(r, dev))
    assert_close16(N(y), OK.gemv_i8(x, q, s, r), what=f"dense M={M}")


def test_int8_mm_strided_rows(dev):
    """x given as every other row of a [2B, K] buffer (the [1::2] view of the engine)."""
    from estudiocanciones_amd.kernels import int8_mm
    xb = randn16(7, 16, 1024)
    w = rng(8).standard_normal((8197, 1024), dtype=np.float32) * np.float32(0.02)
    q, sb = o_q8_rows(w)
    s = f16(bf16_to_f32(sb))
    xt = T(xb, dev)[1::2]
    y = int8_mm(xt, T(q, dev), T(s, dev))
    assert_close16(N(y), OK.gemv_i8(xb[1::2], q, s), what="strided gemv")


@pytest.mark.parametrize("nt,kw", [(1, 1), (1, 4), (1, 16), (2, 8), (4, 4)])
def test_gemv_tile_configs_agree(dev, nt, kw):
    import torch
    from estudiocanciones_amd import _ffi
    from estudiocanciones_amd.kernels import stream_ptr
    M, Nn, K = 8, 2048, 4096
    x = randn16(9, M, K)
    w = rng(10).standard_normal((Nn, K), dtype=np.float32) * np.float32(0.02)
    q, sb = o_q8_rows(w)
    s = f16(bf16_to_f32(sb))
    xt, qt, st = T(x, dev), T(q, dev), T(s, dev)
    y = torch.empty(M, Nn, dtype=torch.float16, device=dev)
    _ffi.call("ecd_gemv_i8_tuned", xt.data_ptr(), K, qt.data_ptr(), st.data_ptr(), None, 0,
              y.data_ptr(), Nn, M, Nn, K, 0, nt, kw, stream_ptr(dev))
    assert_close16(N(y), OK.gemv_i8(x, q, s), what=f"gemv nt={nt} kw={kw}")


# ---------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("R,D", [(1, 3072), (8, 3072), (16, 1024), (3, 100)])
def test_rms(dev, R, D):
    from estudiocanciones_amd.kernels import rms
    x = randn16(20, R, D, std=3.0)
    w = (1 + 0.02 * rng(21).standard_normal(D)).astype(np.float16)
    y = rms(T(x, dev), T(w, dev))
    assert_close16(N(y), OK.rms(x, w), what="rms")


# ---------------------------------------------------------------- RoPE table
@pytest.mark.parametrize("hd,L", [(128, 4096), (384, 64), (64, 17)])
def test_rope_table(dev, hd, L):
    from estudiocanciones_amd.engine import rope_cache
    t = N(rope_cache(hd, L, device=dev))
    want = o_rope_cache(hd, L)
    np.testing.assert_allclose(t, want, rtol=0, atol=2e-6)


# ---------------------------------------------------------------- RoPE + KV write
@pytest.mark.parametrize("R,S,Hq,Hk,HD,L", [(8, 1, 24, 8, 128, 64), (16, 2, 8, 4, 384, 8),
                                            (6, 3, 4, 2, 64, 32)])
def test_rope_kv_write(dev, R, S, Hq, Hk, HD, L):
    import torch
    from estudiocanciones_amd.kernels import _rope_cache
    B = R // S
    qkv = randn16(30, R, (Hq + 2 * Hk) * HD)
    pos = rng(31).integers(0, L, R).astype(np.int64)
    if S > 1:   # rows of one batch entry hold distinct positions
        pos = np.tile(np.arange(S, dtype=np.int64), B) + rng(32).integers(0, L - S, 1)[0]
    rope = o_rope_cache(HD, L)
    kc0 = randn16(33, B, Hk, L, HD)
    vc0 = randn16(34, B, Hk, L, HD)
    kc, vc = kc0.copy(), vc0.copy()
    q_want = OK.rope_kv_write(qkv, rope, pos, kc, vc, S, Hq, Hk, HD)
    kct, vct = T(kc0, dev), T(vc0, dev)
    q = torch.empty(R, Hq * HD, dtype=torch.float16, device=dev)
    _rope_cache[(R, Hq + Hk)](T(qkv, dev), T(rope, dev), T(pos, dev), q, kct, vct, S, Hq, Hk, L,
                              HD=HD, HALF=HD // 2)
    assert_close16(N(q), q_want, what="rope q")
    assert_close16(N(kct), kc, what="k cache")
    assert np.array_equal(N(vct), vc), "v cache must be an exact copy"


# ---------------------------------------------------------------- decode attention
ATTN_CASES = [
    # R, S, Hq, Hk, HD, L, nsplit
    (2, 1, 24, 8, 128, 1024, 16),
    (8, 1, 24, 8, 128, 750, 16),
    (8, 1, 24, 8, 128, 4096, 16),
    (16, 2, 8, 4, 384, 8, 1),
    (8, 1, 8, 4, 384, 8, 16),
    (16, 2, 8, 2, 128, 8, 1),
    (4, 1, 8, 2, 128, 300, 7),
    (3, 1, 6, 1, 64, 40, 1),
    # the engine's split counts for few rows (one row: 64 splits; 40 and 100 exercise the
    # combine's register path and its loop path)
    (1, 1, 24, 8, 128, 4096, 64),
    (2, 1, 24, 8, 128, 2048, 40),
    (1, 1, 24, 8, 128, 3000, 100),
    # one split over a short cache (<= 16 slots): the VALU kernel
    (8, 1, 8, 4, 384, 8, 1),
    (8, 1, 12, 4, 256, 16, 1),
    (8, 1, 8, 2, 128, 5, 1),
]


MERGED_CASES = [
    # R, S, Hq, Hk, HD, L, kb (workgroups of 8 splits per (row, kv head))
    (1, 1, 24, 8, 128, 4096, 32),  # one row: the engine's 32 workgroups per pair
    (8, 1, 24, 8, 128, 4096, 4),   # batch 8 at the target length
    (8, 1, 24, 8, 128, 750, 4),    # ragged positions: some workgroups see empty splits only
    (2, 1, 24, 8, 128, 300, 3),
    (4, 2, 8, 2, 128, 1024, 8),    # two rows per cache at consecutive positions
    (2, 1, 8, 4, 384, 1000, 5),    # head_dim 384
    (3, 1, 12, 4, 256, 700, 2),
    (8, 1, 8, 1, 128, 512, 1),     # one workgroup per pair, 8 query heads per kv head
]


@pytest.mark.parametrize("R,S,Hq,Hk,HD,L,kb", MERGED_CASES)
def test_decode_attn_merged(dev, R, S, Hq, Hk, HD, L, kb):
    """The split attention and its merge in one launch (ecd_decode_attn_merged) against the
    oracle's split attention with the same 8 kb splits and the exact softmax, twice in a row
    (the second call on new queries): the pair counters are zero after each call."""
    import torch
    from estudiocanciones_amd import _ffi
    B = R // S
    kc = randn16(141, B, Hk, L, HD)
    vc = randn16(142, B, Hk, L, HD)
    g = rng(143)
    if S == 1:
        pos = g.integers(0, L, R).astype(np.int64)
        pos[0] = L - 1
    else:
        pos = np.tile(np.arange(S, dtype=np.int64), B) + (L - S) // 2
    kt, vt, pt = T(kc, dev), T(vc, dev), T(pos, dev)
    G = Hq // Hk
    ws = torch.full((R * Hk * kb * G * (2 + HD),), float("nan"), device=dev)
    cnt = torch.zeros(R * Hk, dtype=torch.int32, device=dev)
    for call in range(2):
        q = randn16(140 + call, R, Hq * HD)
        o = torch.empty(R, Hq * HD, dtype=torch.float16, device=dev)
        _ffi.call("ecd_decode_attn_merged", T(q, dev).data_ptr(), kt.data_ptr(), vt.data_ptr(),
                  pt.data_ptr(), o.data_ptr(), ws.data_ptr(), cnt.data_ptr(), R, S, Hq, Hk, L, HD,
                  kb, 1.0 / math.sqrt(HD), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert int(cnt.abs().sum()) == 0, f"pair counters left at {cnt.tolist()}"
        want = OK.decode_attn_out(q, kc, vc, pos, S, Hq, Hk, HD, nsplit=8 * kb)
        assert_close16(N(o), want, what=f"merged attn R={R} L={L} HD={HD} kb={kb} call {call}")
        exact = OK.attention_exact(q, kc, vc, pos, S, Hq, Hk, HD)
        assert_close16(N(o), exact, what="merged attn vs exact softmax")


@pytest.mark.parametrize("R,S,Hq,Hk,HD,L,ns", ATTN_CASES)
def test_decode_attn(dev, R, S, Hq, Hk, HD, L, ns):
    import torch
    from estudiocanciones_amd.kernels import _attn, _attn_combine
    B = R // S
    q = randn16(40, R, Hq * HD)
    kc = randn16(41, B, Hk, L, HD)
    vc = randn16(42, B, Hk, L, HD)
    g = rng(43)
    if S == 1:
        pos = g.integers(0, L, R).astype(np.int64)
        pos[0] = L - 1
    else:
        pos = np.tile(np.arange(S, dtype=np.int64), B) + (L - S) // 2
    want = OK.decode_attn_out(q, kc, vc, pos, S, Hq, Hk, HD, nsplit=ns)
    qt, kt, vt, pt = T(q, dev), T(kc, dev), T(vc, dev), T(pos, dev)
    o = torch.empty(R, Hq * HD, dtype=torch.float16, device=dev)
    if ns > 1:
        pm = torch.empty(R * Hq * ns, device=dev)
        pl = torch.empty_like(pm)
        pa = torch.empty(R * Hq * ns, HD, device=dev)
    else:
        pm = pl = pa = o
    scale = 1.0 / math.sqrt(HD)
    _attn[(R, Hk, ns)](qt, kt, vt, pt, o, pm, pl, pa, S, Hq, Hk, L, scale, HD=HD, G=Hq // Hk,
                       NSPLIT=ns)
    if ns > 1:
        _attn_combine[(R * Hq,)](pm, pl, pa, o, HD=HD, NSPLIT=ns)
    assert_close16(N(o), want, what=f"attn R={R} L={L} HD={HD} ns={ns}")
    exact = OK.attention_exact(q, kc, vc, pos, S, Hq, Hk, HD)
    assert_close16(N(o), exact, what="attn vs exact softmax")


def test_decode_attn_split_invariance(dev):
    """Any split count gives the same attention (up to fp32 re-association)."""
    import torch
    from estudiocanciones_amd.kernels import _attn, _attn_combine
    R, Hq, Hk, HD, L = 4, 24, 8, 128, 2000
    q = T(randn16(50, R, Hq * HD), dev)
    kc = T(randn16(51, R, Hk, L, HD), dev)
    vc = T(randn16(52, R, Hk, L, HD), dev)
    pos = T(np.array([1999, 1000, 17, 0], np.int64), dev)
    outs = []
    for ns in (1, 2, 5, 16, 32):
        o = torch.empty(R, Hq * HD, dtype=torch.float16, device=dev)
        pm = torch.empty(R * Hq * ns, device=dev)
        pl = torch.empty_like(pm)
        pa = torch.empty(R * Hq * ns, HD, device=dev)
        _attn[(R, Hk, ns)](q, kc, vc, pos, o, pm, pl, pa, 1, Hq, Hk, L, 1 / math.sqrt(HD), HD=HD,
                           NSPLIT=ns)
        if ns > 1:
            _attn_combine[(R * Hq,)](pm, pl, pa, o, HD=HD, NSPLIT=ns)
        outs.append(N(o))
    for o in outs[1:]:
        assert_close16(o, outs[0], what="split invariance")


@pytest.mark.parametrize("B,S,Hq,Hk,L,off,HD", [(2, 100, 24, 8, 128, 0, 128),
                                                 (1, 64, 8, 2, 160, 37, 128),
                                                 (3, 17, 4, 4, 40, 5, 128),
                                                 (1, 130, 8, 4, 256, 0, 128),
                                                 (2, 100, 6, 6, 128, 0, 64),
                                                 (1, 70, 8, 2, 100, 9, 64)])
def test_prefill_attn(dev, B, S, Hq, Hk, L, off, HD):
    """Causal prompt-pass attention on MFMA against the exact softmax and against the decode
    kernel (one split per row) on the same inputs: row s attends [0, off + s]; S not a
    multiple of the 64-row block, G = 1..4, a prompt placed after cached slots."""
    import torch
    from estudiocanciones_amd.kernels import _attn, prefill_attn
    R = B * S
    q = randn16(60, R, Hq * HD)
    kc = randn16(61, B, Hk, L, HD)
    vc = randn16(62, B, Hk, L, HD)
    pos = np.tile(np.arange(S, dtype=np.int64) + off, B)
    exact = OK.attention_exact(q, kc, vc, pos, S, Hq, Hk, HD)
    qt, kt, vt, pt = T(q, dev), T(kc, dev), T(vc, dev), T(pos, dev)
    got = prefill_attn(qt, kt, vt, pt, S, Hq, Hk)
    assert_close16(N(got), exact, what=f"prefill attn B={B} S={S} G={Hq // Hk}")
    o = torch.empty(R, Hq * HD, dtype=torch.float16, device=dev)
    _attn[(R, Hk, 1)](qt, kt, vt, pt, o, o, o, o, S, Hq, Hk, L, 1 / math.sqrt(HD), HD=HD,
                      NSPLIT=1)
    assert_close16(N(got), N(o), what="prefill attn vs decode kernel")


def test_prefill_attn_positions_clamped(dev):
    """Positions outside the cache: a negative one attends nothing (zero output), one past the
    cache attends the whole cache, like the decode kernel's clamp; other rows are unaffected."""
    from estudiocanciones_amd.kernels import prefill_attn
    B, S, Hq, Hk, L, HD = 1, 70, 4, 2, 96, 128
    q = randn16(80, B * S, Hq * HD)
    kc = randn16(81, B, Hk, L, HD)
    vc = randn16(82, B, Hk, L, HD)
    pos = np.arange(S, dtype=np.int64) + 10
    pos[3], pos[40] = -5, 1 << 40
    got = N(prefill_attn(T(q, dev), T(kc, dev), T(vc, dev), T(pos, dev), S, Hq, Hk))
    assert not np.any(got[3]), "a negative position attends nothing"
    ok = pos >= 0
    want = OK.attention_exact(q[ok], kc, vc, np.minimum(pos[ok], L - 1), int(ok.sum()), Hq, Hk, HD)
    assert_close16(got[ok], want, what="clamped positions")


@pytest.mark.parametrize("B,Ls,H,HD", [(2, 100, 4, 64), (2, 70, 2, 128)])
def test_prefill_attn_full_sequence(dev, B, Ls, H, HD):
    """Every position at the last slot: non-causal attention over the whole sequence (the codec
    estimator's SDPA without a mask), against the exact softmax."""
    from estudiocanciones_amd.kernels import prefill_attn
    R = B * Ls
    q = randn16(70, R, H * HD)
    kc = randn16(71, B, H, Ls, HD)
    vc = randn16(72, B, H, Ls, HD)
    pos = np.full(R, Ls - 1, np.int64)
    exact = OK.attention_exact(q, kc, vc, pos, Ls, H, H, HD)
    got = prefill_attn(T(q, dev), T(kc, dev), T(vc, dev), T(pos, dev), Ls, H, H)
    assert_close16(N(got), exact, what=f"full attention T={Ls} HD={HD}")


# ---------------------------------------------------------------- SiLU * mul
@pytest.mark.parametrize("R,F", [(8, 8192), (16, 8192), (2, 1000)])
def test_silu_mul(dev, R, F):
    import torch
    from estudiocanciones_amd.kernels import _silu_mul, cdiv
    x = randn16(60, R, 2 * F, std=3.0)
    y = torch.empty(R, F, dtype=torch.float16, device=dev)
    _silu_mul[(R, cdiv(F, 1024))](T(x, dev), y, F, BLOCK=1024)
    assert_close16(N(y), OK.silu_mul(x), what="silu_mul")


# ---------------------------------------------------------------- embeddings
def test_embed_sum_and_gather(dev):
    import torch
    from estudiocanciones_amd.engine import AUDIO_VOCAB, Emb
    D = 256
    w = rng(70).standard_normal((8 * AUDIO_VOCAB, D), dtype=np.float32)
    q, sb = o_q8_rows(w)
    s = f16(bf16_to_f32(sb))
    emb = Emb(q8=T(q, dev), s8=T(s, dev))
    tok = rng(71).integers(0, AUDIO_VOCAB, (8, 8)).astype(np.int64)
    h = emb.sum_codebooks(T(tok, dev), AUDIO_VOCAB)
    assert_close16(N(h), OK.embed_sum(q, s, tok, AUDIO_VOCAB), atol=0, rtol=1e-3, what="embed sum")
    c = T(tok[:, 3:4].copy(), dev)
    e = emb.gather(c, 3, AUDIO_VOCAB)
    assert np.array_equal(N(e), OK.embed_rows(q, s, tok[:, 3] + 3 * AUDIO_VOCAB))
    even = T(randn16(72, 8, D), dev)
    x = emb.gather(c, 3, AUDIO_VOCAB, even=even)
    assert np.array_equal(N(x)[0::2], N(even))
    assert np.array_equal(N(x)[1::2], N(e))
    idx = T(np.array([[0, 5], [AUDIO_VOCAB * 8 - 1, 2]], np.int64), dev)
    assert np.array_equal(N(emb(idx)), OK.embed_rows(q, s, N(idx)))


@pytest.mark.parametrize("M,Nn,K,res", [(2048, 3072, 3072, True), (300, 8197, 1024, False),
                                        (40, 100, 192, True)])
def test_int8_mm_many_rows_runs_the_mfma_gemm(dev, M, Nn, K, res):
    """int8_mm with more than 16 rows (the reference's dense fallback, app/kernels.py:46-49) on
    the row-major [N, K] weights: the MFMA GEMM, dense numerics, partial feature tiles."""
    from estudiocanciones_amd.kernels import int8_mm
    x = randn16(90, M, K)
    w = rng(91).standard_normal((Nn, K), dtype=np.float32) * np.float32(0.02)
    q, sb = o_q8_rows(w)
    s = f16(bf16_to_f32(sb))
    r = randn16(92, M, Nn) if res else None
    y = int8_mm(T(x, dev), T(q, dev), T(s, dev), T(r, dev) if res else None)
    assert_close16(N(y), OK.gemv_i8(x, q, s, r), what=f"int8_mm M={M} N={Nn} K={K}")
