"""Pins for the kernel-level oracle (app/kernels.py): brute force on tiny inputs with explicit
loops, closed forms and special cases that a dropped term, transposed operand, wrong head
mapping or wrong rounding point fails."""
import math

import numpy as np

from oracle import kernels as K
from oracle.numerics import f16
from oracle.quant import q8_rows, scale_f16
from oracle.rope import rope_cache

rng = np.random.default_rng


# ---------------------------------------------------------------- GEMV
def _gemv_loops(x, q, s, res, dense):
    """Explicit-loop restatement used only here: float64 sums, the reference's fp16 points."""
    M, Kd = x.shape
    N = q.shape[0]
    y = np.zeros((M, N), np.float16)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(Kd):
                w = float(q[n, k])
                if dense:
                    w = float(np.float16(np.float32(np.float16(w)) * np.float32(s[n])))
                acc += float(x[m, k]) * w
            v = np.float32(acc) if dense else np.float32(acc) * np.float32(s[n])
            o = np.float16(v)
            if res is not None:
                o = np.float16(np.float32(o) + np.float32(res[m, n]))
            y[m, n] = o
    return y


def test_gemv_brute_force_both_numerics():
    g = rng(0)
    q = g.integers(-127, 128, (3, 5)).astype(np.int8)             # N=3, K=5: a transpose fails
    s = (g.random(3) * 0.03).astype(np.float16)
    for M in (2, 17):                                              # GEMV numerics / dense numerics
        x = g.standard_normal((M, 5)).astype(np.float16)
        r = g.standard_normal((M, 3)).astype(np.float16)
        got = K.gemv_i8(x, q, s, r)
        assert np.array_equal(got, _gemv_loops(x, q, s, r, M > 16))


def test_gemv_dense_and_scaled_numerics_differ():
    """For M > 16 the reference dequantises first (fp16(q * s)), which rounds differently."""
    g = rng(1)
    q = g.integers(-127, 128, (64, 256)).astype(np.int8)
    s = (g.random(64) * 0.02 + 1e-3).astype(np.float16)
    x = g.standard_normal((17, 256)).astype(np.float16)
    dense = K.gemv_i8(x, q, s)
    scaled = np.concatenate([K.gemv_i8(x[i:i + 1], q, s) for i in range(17)])
    assert not np.array_equal(dense, scaled)
    np.testing.assert_allclose(dense.astype(np.float32), scaled.astype(np.float32), atol=2e-2, rtol=2e-2)


def test_gemv_linearity_and_scale():
    g = rng(2)
    q = g.integers(-127, 128, (40, 96)).astype(np.int8)
    s = (g.random(40) * 0.02).astype(np.float16)
    x1 = g.standard_normal((4, 96)).astype(np.float16)
    x2 = g.standard_normal((4, 96)).astype(np.float16)
    y12 = K.gemv_i8(f16(x1.astype(np.float32) + x2.astype(np.float32)), q, s).astype(np.float32)
    y1, y2 = K.gemv_i8(x1, q, s).astype(np.float32), K.gemv_i8(x2, q, s).astype(np.float32)
    np.testing.assert_allclose(y12, y1 + y2, atol=3e-2, rtol=1e-2)
    ref = (x1.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    np.testing.assert_allclose(y1, ref, atol=2e-3, rtol=2e-3)


# ---------------------------------------------------------------- RMSNorm
def test_rms_closed_form():
    D = 3072
    x = np.full((2, D), 3.0, np.float16)
    x[1] = -0.5
    w = np.ones(D, np.float16)
    y = K.rms(x, w)
    inv0 = 1.0 / math.sqrt(9.0 + 1e-5)
    inv1 = 1.0 / math.sqrt(0.25 + 1e-5)
    assert np.all(y[0] == np.float16(np.float32(3.0) * np.float32(inv0)))   # mean, not sum
    assert np.all(y[1] == np.float16(np.float32(-0.5) * np.float32(inv1)))
    xr = rng(3).standard_normal((3, 1024)).astype(np.float16)
    wr = (1 + 0.1 * rng(4).standard_normal(1024)).astype(np.float16)
    a = K.rms(xr, wr).astype(np.float32)
    b = K.rms(f16(xr.astype(np.float32) * 4), wr).astype(np.float32)        # scale invariant
    np.testing.assert_allclose(a, b, atol=2e-3, rtol=2e-3)
    np.testing.assert_allclose(((a / wr.astype(np.float32)) ** 2).mean(-1), 1.0, atol=1e-2)  # mean x^2 = 1


# ---------------------------------------------------------------- attention
def _cache(seed, B, Hk, L, HD):
    g = rng(seed)
    return (g.standard_normal((B, Hk, L, HD)).astype(np.float16),
            g.standard_normal((B, Hk, L, HD)).astype(np.float16))


def test_attention_single_token_and_uniform_keys():
    B, Hq, Hk, HD, L = 2, 6, 2, 64, 32
    kc, vc = _cache(5, B, Hk, L, HD)
    q = rng(6).standard_normal((B, Hq * HD)).astype(np.float16)
    o = K.decode_attn_out(q, kc, vc, np.zeros(B, np.int64), 1, Hq, Hk, HD).reshape(B, Hq, HD)
    for b in range(B):
        for h in range(Hq):
            assert np.array_equal(o[b, h], vc[b, h // 3, 0])       # one token: output = v[0]
    kc[:] = 0.25                                                    # all scores equal
    o = K.decode_attn_out(q, kc, vc, np.full(B, 9, np.int64), 1, Hq, Hk, HD).reshape(B, Hq, HD)
    mean = vc[:, :, :10].astype(np.float64).mean(2)
    for h in range(Hq):
        np.testing.assert_allclose(o[:, h].astype(np.float64), mean[:, h // 3], atol=2e-3)


def test_attention_matches_textbook_softmax_and_gqa_mapping():
    B, S, Hq, Hk, HD, L = 2, 2, 8, 4, 128, 50
    kc, vc = _cache(7, B, Hk, L, HD)
    q = rng(8).standard_normal((B * S, Hq * HD)).astype(np.float16)
    pos = np.array([20, 21, 48, 49], np.int64)
    exact = K.attention_exact(q, kc, vc, pos, S, Hq, Hk, HD)
    for ns, blk in ((1, 64), (16, 64), (5, 16)):
        o = K.decode_attn_out(q, kc, vc, pos, S, Hq, Hk, HD, nsplit=ns, blk=blk)
        np.testing.assert_allclose(o.astype(np.float64), exact, atol=2e-3, rtol=1e-2)
    # brute force of one (row, head) with explicit loops, GQA head h -> kv head h // (Hq / Hk)
    r, h = 3, 5
    kh = h // 2
    sc = [sum(float(q[r, h * HD + d]) * float(kc[r // S, kh, t, d]) for d in range(HD)) / math.sqrt(HD)
          for t in range(pos[r] + 1)]
    mx = max(sc)
    p = [math.exp(v - mx) for v in sc]
    want = [sum(p[t] * float(vc[r // S, kh, t, d]) for t in range(len(p))) / sum(p) for d in range(HD)]
    np.testing.assert_allclose(exact.reshape(B * S, Hq, HD)[r, h], want, atol=1e-9)
    wrong = (h % Hk)                                                # a h % Hk mapping reads kv head 1
    assert wrong != kh


def test_combine_ignores_empty_splits():
    pm = np.array([[1.0, -np.inf, 0.5]], np.float32)
    pl = np.array([[2.0, 0.0, 1.0]], np.float32)
    pa = np.array([[[2.0, 4.0], [9.0, 9.0], [1.0, 1.0]]], np.float32)
    o = K.attn_combine(pm, pl, pa)
    w0, w2 = 1.0, math.exp(-0.5)
    want = [(2 * w0 + 1 * w2) / (2 * w0 + 1 * w2), (4 * w0 + 1 * w2) / (2 * w0 + 1 * w2)]
    np.testing.assert_allclose(o[0].astype(np.float64), want, rtol=1e-3)


# ---------------------------------------------------------------- SiLU * mul, embeddings
def test_silu_mul_known_values():
    a = np.array([0.0, 1.0, -1.0, 8.0, -20.0], np.float16)
    b = np.array([3.0, 2.0, 2.0, 0.5, 1.0], np.float16)
    y = K.silu_mul(np.concatenate([a, b])[None])[0].astype(np.float64)
    silu = [0.0, 1 / (1 + math.exp(-1)), -1 / (1 + math.exp(1)), 8 / (1 + math.exp(-8)), -20 / (1 + math.exp(20))]
    want = [float(np.float16(np.float16(v) * np.float16(bb))) for v, bb in zip(silu, b.astype(float))]
    assert y.tolist() == want


def test_embeddings_gather_and_codebook_offsets():
    V, D = 10, 6
    w = rng(9).standard_normal((3 * V, D)).astype(np.float32)
    q8, sb = q8_rows(w)
    s16 = scale_f16(sb)
    tok = np.array([[1, 2, 3], [9, 0, 5]], np.int64)
    got = K.embed_sum(q8, s16, tok, V).astype(np.float64)
    for b in range(2):
        acc = np.zeros(D, np.float32)
        for c in range(3):
            row = tok[b, c] + c * V                                  # codebook c offset by c * vocab
            acc += np.float16(q8[row].astype(np.float16) * s16[row]).astype(np.float32)
        np.testing.assert_array_equal(got[b], np.float16(acc).astype(np.float64))
    e = K.embed_rows(q8, s16, np.array([7]))
    np.testing.assert_allclose(e[0].astype(np.float64), w[7], atol=float(s16[7]) * 0.6 + 2e-3)


def test_rope_kv_write_touches_only_its_slots():
    S, Hq, Hk, HD, L = 2, 4, 2, 64, 12
    R = 4
    qkv = rng(10).standard_normal((R, (Hq + 2 * Hk) * HD)).astype(np.float16)
    kc = np.zeros((R // S, Hk, L, HD), np.float16)
    vc = np.zeros_like(kc)
    pos = np.array([3, 4, 7, 8], np.int64)
    K.rope_kv_write(qkv, rope_cache(HD, L), pos, kc, vc, S, Hq, Hk, HD)
    written = np.argwhere(np.abs(vc).sum(-1) > 0)
    assert sorted(map(tuple, written.tolist())) == sorted(
        [(b, h, p) for b, ps in ((0, (3, 4)), (1, (7, 8))) for p in ps for h in range(Hk)])
    assert np.array_equal(vc[1, 1, 8], qkv[3, (Hq + Hk + 1) * HD:(Hq + Hk + 2) * HD])   # v copied as is
